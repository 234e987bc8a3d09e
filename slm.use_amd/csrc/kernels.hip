// gfx950 (CDNA4) kernels for the token loop of SLM.use: one code object, loaded by the
// host runtime with hipModuleLoadData. Compiled with -ffp-contract=off so that every
// expression rounds exactly as written wherever it is inlined.
//
// Each operation computes every output element in an order that does not depend on how
// many tokens a call carries (m = 1 decode or an m = 256 prompt chunk), so a prompt read
// in chunks leaves bit-identical state to one read token by token:
//   - linear: one fixed MFMA chain per output (v_mfma_f32_16x16x4f32 over 16-column
//     blocks, chained from zero within 64-column slices; slice sums added in order within
//     768-column splits, split sums added in order); the m <= 16 kernel, the m > 16
//     kernel and the fused one-token kernel run the same chain;
//   - attend: keys are grouped by absolute position into 16-key tiles, 64-key segments
//     and 256-key superblocks; a segment is an online softmax over its tiles, segments
//     fold into superblocks in order and superblocks into the result in order;
//   - gla: one kernel for every m, tokens in order;
//   - rms / l2norm: the 16-accumulator dot of the reference CPU backend (src/cpu.rs:9-21),
//     so these two are bit-identical to it;
//   - the rest is element-wise.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fusion.h"
typedef float f4 __attribute__((ext_vector_type(4)));

#define KERNEL extern "C" __global__

#define GRID_LOOP(i, n)                                                              \
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < (n);    \
         i += (long long)gridDim.x * blockDim.x)

static constexpr float NEG_INF = -__builtin_inff();

__device__ __forceinline__ long long dyn_or(const long long* dyn, long long imm) {
    return dyn ? dyn[0] : imm;
}

// Loads and stores through pointers the compiler cannot see are global (for instance
// pointers read from LDS), as global rather than flat memory instructions.
#define GAS __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ T gld(const T* p) {
    return *(const GAS T*)p;
}
template <typename T>
__device__ __forceinline__ void gst(T* p, T v) {
    *(GAS T*)p = v;
}
// A value into an fp16 ring, rounded to nearest even.
__device__ __forceinline__ void gst16(_Float16* p, float v) {
    *(GAS _Float16*)p = (_Float16)v;
}

// Device-scope loads and stores (sc1: past the per-XCD L2 for what other workgroups of the
// same launch read or wrote), used by the phases of a one-launch step (slm_step) for every
// value one phase hands to another; with C false, the plain access.
template <bool C, typename T>
__device__ __forceinline__ T ldc(const T* p) {
    if constexpr (C) return __hip_atomic_load((const GAS T*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else return *(const GAS T*)p;
}
template <bool C, typename T>
__device__ __forceinline__ void stc(T* p, T v) {
    if constexpr (C) __hip_atomic_store((GAS T*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else *(GAS T*)p = v;
}

// A bounded wait of a fused kernel that gave up: lane 0 ORs 1 into the fault word (host
// memory), which the runtime reports at the next read or flush. The kernel goes on, so a
// mistake cannot hang the GPU; its results are then not valid.
__device__ __forceinline__ void wait_gave_up(int* fault, int lane) {
    if (fault && lane == 0) __hip_atomic_fetch_or(fault, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// The wait at the start of a phase of slm_step: until every workgroup's flag has reached
// `target` (workgroup w stores epoch + p + 1 into flags[w] once it is done with phase p),
// polled by one wave with device-scope loads; no wait when `flags` is null (the first
// phase). Gives up after `spin` polls and returns true then (the fault word set).
struct StepWait {
    const unsigned* flags;
    unsigned target;
    int spin;
    int* fault;
};
__device__ __forceinline__ bool step_wait(const StepWait& w, int lane) {
    if (!w.flags) return false;
    // two polls in flight: each check waits only for the older one
    constexpr int NJ = SLM_STEP_WG / 64;
    auto poll = [&](unsigned (&f)[NJ]) {
#pragma unroll
        for (int j = 0; j < NJ; j++)
            f[j] = __hip_atomic_load(w.flags + 64 * j + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    auto done = [&](const unsigned (&f)[NJ]) {
        bool ok = true;
#pragma unroll
        for (int j = 0; j < NJ; j++) ok = ok && (int)(f[j] - w.target) >= 0;
        return __all(ok) != 0;
    };
    unsigned fa[NJ], fb[NJ];
    int it = 0;
    if (w.spin > 0) poll(fa);
    for (; it < w.spin; it += 2) {
        poll(fb);
        if (done(fa)) break;
        poll(fa);
        if (done(fb)) break;
    }
    // (later loads stay after the polls: the compiler may not lift them above this fence, and
    // the hardware issues them only once the loop has seen the flags)
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    bool gave_up = it >= w.spin;
    if (gave_up) wait_gave_up(w.fault, lane);
    return gave_up;
}

// A workgroup barrier that orders LDS only (what memory loads are in flight stay in flight).
__device__ __forceinline__ void lds_bar() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// The wait of a step phase whose body runs on every wave of the workgroup: wave 0 polls, the
// workgroup learns the outcome at an LDS barrier (`gave` in LDS). True: the wait gave up.
__device__ __forceinline__ bool step_wait_wg(const StepWait& w, int* gave, int tid) {
    if ((tid >> 6) == 0) {
        bool g = step_wait(w, tid & 63);
        if (tid == 0) *gave = g;
    }
    lds_bar();
    return *gave != 0;
}

__device__ __forceinline__ f4 mfma4(float a, float b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// fp16 mode (the --fp16 analogue, mlx.rs:19-23): a 16-column block of a linear's chain is one
// v_mfma_f32_16x16x16f16 instead of four 16x16x4 f32 MFMAs. Its operands are the same
// registers (lane (i, g) holds columns 4g .. 4g + 3 of row / token i), rounded to fp16 to
// nearest even; the sums stay fp32.
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ h4 to_h4(f4 v) {
    return h4{(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
}
__device__ __forceinline__ f4 block16h(f4 a, f4 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(to_h4(a), to_h4(b), c, 0, 0, 0);
}
// The same block with the first operand already in fp16 (weights stored as halves): the
// halves a rounding to nearest even of the fp32 weights gives, so the same MFMA inputs.
__device__ __forceinline__ f4 block16hw(h4 a, f4 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, to_h4(b), c, 0, 0, 0);
}
// Four fp16 weights widened to fp32 (exactly): what block16h rounds back to the same halves.
__device__ __forceinline__ f4 wide4(h4 v) { return f4{(float)v.x, (float)v.y, (float)v.z, (float)v.w}; }

// fp16 mode's values (mlx.rs:19-23, 53-67: every buffer Float16): each operation's result is
// rounded to fp16 (to nearest even) as it is written, at the points where mlx.rs's fp16
// arrays round: a product or sum of two arrays, a scalar turned into the dtype
// (mlx.rs:25-27), the norm's fp32 quotient before its weight (mlx.rs:178-185). Sums inside a
// reduction (a linear's chain, a norm's dot, attention, the GLA's column sums) stay fp32.
// Kernels that run in both modes read the mode word slm_h16 (set by the host); those that
// run only in fp16 mode, or take a descriptor, decide it at compile time or from a field.
__constant__ int slm_h16;
// (the fp32 value goes through an opaque register first: otherwise the compiler may turn
// (half)(a·b) into one v_fma_mixlo_f16, a single rounding of the exact product, in some
// kernels and not in others, and the same expression would differ by an fp16 step)
__device__ __forceinline__ float r16(float v) {
    asm("" : "+v"(v));
    return (float)(_Float16)v;
}
template <bool H>
__device__ __forceinline__ float h16(float v) { return H ? r16(v) : v; }
// The element-wise expressions of both modes (fp32: cpu.rs's; fp16: mlx.rs's roundings).
template <bool H>
__device__ __forceinline__ float e_add(float a, float b) { return h16<H>(a + b); }
template <bool H>
__device__ __forceinline__ float e_mix(float a, float b, float t) {  // mlx.rs:165-169
    return H ? r16(a + r16(r16(b - a) * r16(t))) : a + t * (b - a);
}
template <bool H>
__device__ __forceinline__ float e_scale(float a, float f) {  // mlx.rs:157-163
    return H ? r16(a * r16(f)) : a * f;
}
template <bool H>
__device__ __forceinline__ float e_silu(float g, float u) {  // mlx.rs:188-192: g·sigmoid(g), then ·u
    if (H) return r16(r16(g * r16(1.0f / (1.0f + expf(-g)))) * u);
    return u * g / (1.0f + expf(-g));
}
template <bool H>
__device__ __forceinline__ float e_rms(float a, float r, float w) {  // mlx.rs:178-185
    return H ? r16(r16(a * r) * w) : a * r * w;
}
template <bool H>  // rope's two halves (mlx.rs:227-230): a·c − b·s, a·s + b·c
__device__ __forceinline__ float e_rope_l(float a, float b, float c, float s) {
    return H ? r16(r16(a * c) - r16(b * s)) : a * c - b * s;
}
template <bool H>
__device__ __forceinline__ float e_rope_r(float a, float b, float c, float s) {
    return H ? r16(r16(a * s) + r16(b * c)) : a * s + b * c;
}

// ---------------------------------------------------------------------------------------
// element-wise operations (src/cpu.rs:66-185, 209-268, 331-350)
// ---------------------------------------------------------------------------------------

KERNEL void slm_copy(float* __restrict__ y, const float* __restrict__ x, long long n) {
    GRID_LOOP(i, n) y[i] = x[i];
}

// Zeroes new buffers (a kernel, not a memset, so it may sit inside a captured graph).
KERNEL void slm_fill(float* __restrict__ y, long long n, float v) {
    GRID_LOOP(i, n) y[i] = v;
}

// fp32 -> fp16 to nearest even: the halves fp16 mode's linears round their weights to, kept
// as a shadow copy of a weight buffer so those linears stream half the bytes.
KERNEL void slm_to_half(_Float16* __restrict__ y, const float* __restrict__ x, long long n) {
    GRID_LOOP(i, n) y[i] = (_Float16)x[i];
}

// Copies n floats of device memory into mapped host memory, then the last workgroup to finish
// stores `seq` into the host flag: every workgroup releases its stores at system scope before
// it counts itself on the device counter (never reset: this launch's workgroups take the
// values base .. last), and the one that takes `last` releases at system scope again before
// the flag, so a host that sees the flag sees all n values. No waits: every workgroup ends.
KERNEL void __launch_bounds__(256) slm_to_host(float* __restrict__ dst, const float* __restrict__ src,
                                               long long n, unsigned long long* ctr,
                                               unsigned long long last, unsigned long long* flag,
                                               unsigned long long seq) {
    long long n4 = n >> 2;
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n4; i += (long long)gridDim.x * 256)
        ((f4*)dst)[i] = ((const f4*)src)[i];
    if (blockIdx.x == 0 && threadIdx.x < (n & 3)) dst[4 * n4 + threadIdx.x] = src[4 * n4 + threadIdx.x];
    __threadfence_system();
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long k = __hip_atomic_fetch_add(ctr, 1ull, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        if (k == last) {
            __threadfence_system();
            __hip_atomic_store(flag, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
}

KERNEL void slm_add(float* __restrict__ y, const float* __restrict__ a,
                    const float* __restrict__ b, long long n) {
    if (slm_h16) GRID_LOOP(i, n) y[i] = e_add<true>(a[i], b[i]);
    else GRID_LOOP(i, n) y[i] = a[i] + b[i];
}

KERNEL void slm_add_row(float* __restrict__ y, const float* __restrict__ x,
                        const float* __restrict__ row, long long n, long long d) {
    if (slm_h16) GRID_LOOP(i, n) y[i] = e_add<true>(x[i], row[i % d]);
    else GRID_LOOP(i, n) y[i] = x[i] + row[i % d];
}

KERNEL void slm_mix(float* __restrict__ y, const float* __restrict__ a,
                    const float* __restrict__ b, long long n, float t) {
    if (slm_h16) GRID_LOOP(i, n) y[i] = e_mix<true>(a[i], b[i], t);
    else GRID_LOOP(i, n) y[i] = a[i] + t * (b[i] - a[i]);
}

// y = silu(g)·u = u·g / (1 + e^-g), cpu.rs:209-215.
KERNEL void slm_silu_mul(float* __restrict__ y, const float* __restrict__ g,
                         const float* __restrict__ u, long long n) {
    if (slm_h16) GRID_LOOP(i, n) y[i] = e_silu<true>(g[i], u[i]);
    else GRID_LOOP(i, n) {
        float v = g[i];
        y[i] = u[i] * v / (1.0f + expf(-v));
    }
}

// y[i] = f[i]·x[i] with rows of d; one factor `f0` when `f` is null.
KERNEL void slm_scale_rows(float* __restrict__ y, const float* __restrict__ x,
                           const float* __restrict__ f, float f0, long long n, long long d) {
    if (slm_h16) GRID_LOOP(i, n) y[i] = e_scale<true>(x[i], f ? f[i / d] : f0);
    else GRID_LOOP(i, n) y[i] = x[i] * (f ? f[i / d] : f0);
}

KERNEL void slm_shift(float* __restrict__ y, const float* __restrict__ first,
                      const float* __restrict__ x, long long n, long long d) {
    GRID_LOOP(i, n) y[i] = i < d ? first[i] : x[i - d];
}

KERNEL void slm_columns(float* __restrict__ y, const float* __restrict__ x, long long n,
                        long long stride, long long off, long long len) {
    GRID_LOOP(i, n) y[i] = x[(i / len) * stride + off + i % len];
}

// y[i] = w[ids[i]]; ids are 64-bit (a device copy of the host list).
KERNEL void slm_gather(float* __restrict__ y, const float* __restrict__ w,
                       const long long* __restrict__ ids, long long n, long long d) {
    GRID_LOOP(i, n) y[i] = w[ids[i / d] * d + i % d];
}

// Greedy pick on the device (sample.rs:48-53: b = 0, then b = i whenever x[i] > x[b]): the
// first index holding the largest value that is not a NaN, 0 when x[0] is a NaN or no value
// compares. One workgroup: M = the maximum (fmaxf skips NaNs; the order of a maximum does not
// matter), then the smallest index with x[i] == M. Writes the index to tok[0] (the next
// step's gather reads it there) and to ids[slot] (slot from the device when `dslot`).
KERNEL void __launch_bounds__(1024) slm_argmax(const float* __restrict__ x, long long n,
                                               long long* __restrict__ tok, unsigned* __restrict__ ids,
                                               const long long* __restrict__ dslot, long long slot_imm) {
    __shared__ float wm[16];
    __shared__ int wi[16];
    int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float M = NEG_INF;
    for (long long i = tid; i < n; i += 1024) M = fmaxf(M, x[i]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
    if (lane == 0) wm[wave] = M;
    __syncthreads();
    M = wm[0];
#pragma unroll
    for (int w = 1; w < 16; w++) M = fmaxf(M, wm[w]);
    int b = 0x7fffffff;
    for (long long i = tid; i < n; i += 1024)
        if (x[i] == M) {
            b = (int)i;
            break;
        }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) b = min(b, __shfl_xor(b, off));
    if (lane == 0) wi[wave] = b;
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 16; w++) b = min(b, wi[w]);
        b = min(b, wi[0]);
        long long r = b < n ? b : 0;
        if (!(x[0] == x[0])) r = 0;  // a NaN first: nothing compares greater
        tok[0] = r;
        if (ids) ids[dslot ? dslot[0] : slot_imm] = (unsigned)r;
    }
}

// Ring write: src [m][heads][dh] → cache [heads][cap][dh] at slots (pos+i) % cap.
KERNEL void slm_store(float* __restrict__ cache, const float* __restrict__ src,
                      const long long* __restrict__ dyn, long long pos_imm, long long n,
                      long long cap, long long heads, long long dh) {
    long long pos = dyn_or(dyn, pos_imm);
    GRID_LOOP(t, n) {
        long long tok = t / (heads * dh), h = (t / dh) % heads, e = t % dh;
        long long slot = (pos + tok) % cap;
        cache[(h * cap + slot) * dh + e] = src[t];
    }
}

// A cache [heads][cap][dh] laid out at twice the capacity (model.rs:383-398's relayout): head
// h's cap·dh values to the start of its 2·cap·dh in y (zero after); fp32 and fp16 caches.
template <typename T>
__device__ __forceinline__ void grow_body(T* __restrict__ y, const T* __restrict__ x, long long heads,
                                          long long n) {
    GRID_LOOP(t, heads * n) y[(t / n) * 2 * n + t % n] = x[t];
}
KERNEL void slm_grow(float* y, const float* x, long long heads, long long n) { grow_body(y, x, heads, n); }
KERNEL void slm_grow16(_Float16* y, const _Float16* x, long long heads, long long n) { grow_body(y, x, heads, n); }

// slm_store into a ring of fp16 values (fp16 mode's caches): each value rounded to nearest even.
KERNEL void slm_store16(_Float16* __restrict__ cache, const float* __restrict__ src,
                        const long long* __restrict__ dyn, long long pos_imm, long long n,
                        long long cap, long long heads, long long dh) {
    long long pos = dyn_or(dyn, pos_imm);
    GRID_LOOP(t, n) {
        long long tok = t / (heads * dh), h = (t / dh) % heads, e = t % dh;
        long long slot = (pos + tok) % cap;
        cache[(h * cap + slot) * dh + e] = (_Float16)src[t];
    }
}

// Half-split rotation, cpu.rs:239-268.
KERNEL void slm_rope(float* __restrict__ y, const float* __restrict__ x,
                     const float* __restrict__ cs, const float* __restrict__ sn, long long m,
                     long long heads, long long dh) {
    long long half = dh / 2;
    GRID_LOOP(t, m * heads * half) {
        long long row = t / (heads * half), h = (t / half) % heads, i = t % half;
        long long at = (row * heads + h) * dh;
        float c = cs[row * half + i], s = sn[row * half + i];
        float a = x[at + i], b = x[at + half + i];
        if (slm_h16) {
            y[at + i] = e_rope_l<true>(a, b, c, s);
            y[at + half + i] = e_rope_r<true>(a, b, c, s);
        } else {
            y[at + i] = a * c - b * s;
            y[at + half + i] = a * s + b * c;
        }
    }
}

// Rows pos .. pos+m-1 of a resident [positions][half] cos/sin table (computed on the host
// with the same libm calls as cpu.rs:217-237).
KERNEL void slm_rope_table(float* __restrict__ cs, float* __restrict__ sn,
                           const float* __restrict__ tc, const float* __restrict__ ts,
                           const long long* __restrict__ dyn, long long pos_imm, long long n,
                           long long half) {
    long long pos = dyn_or(dyn, pos_imm);
    GRID_LOOP(i, n) {
        cs[i] = tc[pos * half + i];
        sn[i] = ts[pos * half + i];
    }
}

// ---------------------------------------------------------------------------------------
// rms and l2norm: 16 lanes per group, the 16-accumulator dot of cpu.rs:9-21
// ---------------------------------------------------------------------------------------

// Sum of squares of in[0..size) in the reference's order: lane j keeps the running sum of
// elements j, j+16, ...; the 16 sums are added left to right from -0.0, then the tail.
// `in` may be global or LDS memory.
__device__ __forceinline__ float dot16_self(const float* in, int size, int l) {
    int chunks = size / 16;
    float acc = 0.0f;
    int c = 0;
    for (; c + 8 <= chunks; c += 8) {  // eight reads in flight, then the sums in order
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = in[(c + u) * 16 + l];
#pragma unroll
        for (int u = 0; u < 8; u++) acc = acc + v[u] * v[u];
    }
    for (; c < chunks; c++) {
        float v = in[c * 16 + l];
        acc = acc + v * v;
    }
    float s = -0.0f;
    for (int t = 0; t < 16; t++) s = s + __shfl(acc, t, 16);
    float tail = -0.0f;
    for (int j = chunks * 16; j < size; j++) tail = tail + in[j] * in[j];
    return s + tail;
}

// Up to 16 groups per workgroup: the groups are staged in LDS with coalesced loads (rows
// padded to an odd stride against bank conflicts), then 16 lanes per group run the
// reference's sums. mode 0: rms (cpu.rs:187-207), r = 1/sqrt(dot/size + eps), y = x·r·w;
// mode 1: l2norm (cpu.rs:270-282), r = 1/max(sqrt(dot), 1e-12), y = x·r.
template <int MODE>
__device__ void norm_body(float* __restrict__ y, const float* __restrict__ x,
                          const float* __restrict__ w, int groups, int size, float eps, int G) {
    extern __shared__ float buf[];
    int stride = size | 1;
    long long g0 = (long long)blockIdx.x * G;
    int ng = (int)min((long long)G, groups - g0);
    const float* src = x + g0 * size;
    for (int i = threadIdx.x; i < ng * size; i += blockDim.x) buf[(i / size) * stride + i % size] = src[i];
    __syncthreads();
    int grp = threadIdx.x >> 4, l = threadIdx.x & 15;
    if (grp >= ng) return;  // the 16 lanes of a group leave together
    const float* in = buf + grp * stride;
    float d = dot16_self(in, size, l);
    float r = MODE == 0 ? 1.0f / sqrtf(d / (float)size + eps) : 1.0f / fmaxf(sqrtf(d), 1e-12f);
    float* out = y + (g0 + grp) * size;
    if (slm_h16)
        for (int j = l; j < size; j += 16) out[j] = MODE == 0 ? e_rms<true>(in[j], r, w[j]) : r16(in[j] * r);
    else
        for (int j = l; j < size; j += 16) out[j] = MODE == 0 ? in[j] * r * w[j] : in[j] * r;
}

// Wide groups (size a multiple of 4, at most 4096, vectors 16-byte aligned): one wave per
// group, four groups per workgroup. The wave stages its group in LDS with float4 loads,
// sums the squares in the order of dot16_self (dot16_wave, defined with the fused kernels
// below), then scales the float4s it loaded. Same expressions as norm_body.
__device__ float dot16_wave(const float* in, int size, int lane);
template <int MODE>
__device__ void norm_wave_body(float* __restrict__ y, const float* __restrict__ x,
                               const float* __restrict__ w, int groups, int size, float eps) {
    extern __shared__ float buf[];
    int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    long long grp = (long long)blockIdx.x * 4 + wave;
    if (grp >= groups) return;  // the wave's group is past the end (its lanes leave together)
    float* row = buf + wave * size;
    const f4* src = (const f4*)(x + grp * size);
    int n4 = size >> 2;
    for (int c = lane; c < n4; c += 64) ((f4*)row)[c] = src[c];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    float d = dot16_wave(row, size, lane);
    float r = MODE == 0 ? 1.0f / sqrtf(d / (float)size + eps) : 1.0f / fmaxf(sqrtf(d), 1e-12f);
    f4* out = (f4*)(y + grp * size);
    bool h = slm_h16;
    for (int c = lane; c < n4; c += 64) {
        f4 v = ((const f4*)row)[c], o;
        if (MODE == 0) {
            f4 wv = ((const f4*)w)[c];
#pragma unroll
            for (int e = 0; e < 4; e++) o[e] = h ? e_rms<true>(v[e], r, wv[e]) : v[e] * r * wv[e];
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++) o[e] = h ? r16(v[e] * r) : v[e] * r;
        }
        out[c] = o;
    }
}

KERNEL void __launch_bounds__(256) slm_rms_wave(float* y, const float* x, const float* w,
                                                int groups, int size, float eps) {
    norm_wave_body<0>(y, x, w, groups, size, eps);
}

KERNEL void __launch_bounds__(256) slm_l2norm_wave(float* y, const float* x, int groups,
                                                   int size) {
    norm_wave_body<1>(y, x, nullptr, groups, size, 0.0f);
}

KERNEL void __launch_bounds__(256) slm_rms(float* y, const float* x, const float* w, int groups,
                                           int size, float eps, int G) {
    norm_body<0>(y, x, w, groups, size, eps, G);
}

KERNEL void __launch_bounds__(256) slm_l2norm(float* y, const float* x, int groups, int size,
                                              int G) {
    norm_body<1>(y, x, nullptr, groups, size, 0.0f, G);
}

// ---------------------------------------------------------------------------------------
// gated linear attention (ops.rs:191-205, cpu.rs:284-329)
// ---------------------------------------------------------------------------------------
//
// Sixteen lanes per state column b (lanes 16c .. 16c+15 of a wave); lane j owns rows
// j·RPL .. j·RPL+RPL-1 of S[h][:, b] in registers. Tokens run in order:
// d = 1/(1 + e^(decay + bias)), S[a][b] = d·S[a][b] + k[a]·v[b], y[b] = Σ_a q[a]·S[a][b],
// where each lane sums its rows in order and the sixteen lane sums are added pairwise
// by lane distance 1, 2, 4, 8 (gla_colsum). The prompt kernel and the one-token kernel
// (gla1_body) run the same expressions.

// xor-1 and xor-2 lane swaps within quads (DPP quad_perm [1,0,3,2] and [2,3,0,1])
__device__ __forceinline__ float dpp_xor1(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_xor2(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false));
}
// The column total of the sixteen lane sums, in every lane of the sixteen.
__device__ __forceinline__ float gla_colsum(float p) {
    p = p + dpp_xor1(p);
    p = p + dpp_xor2(p);
    p = p + __shfl_xor(p, 4);
    p = p + __shfl_xor(p, 8);
    return p;
}

// The same total in the column's first lane only (what the prompt kernel stores): distance
// 4 and 8 through DPP row shifts (lane 16c + i reads lane 16c + i + n), so lane 16c adds the
// same pairs in the same order as gla_colsum. (Lanes whose source is past the row read zero,
// bound_ctrl, which lets each shift fuse into its add; only lane 16c's total is used, and its
// sources are always inside the row.)
__device__ __forceinline__ float gla_colsum0(float p) {
    p = p + dpp_xor1(p);
    p = p + dpp_xor2(p);
    p = p + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(p), 0x104, 0xF, 0xF, true));
    p = p + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(p), 0x108, 0xF, 0xF, true));
    return p;
}

// One lane's rows for one token: st = d·st + k·v, and the lane's sum of q·st in order.
// One state element's update for one token, st·d + k·v (fp16 mode: mlx.rs:321's state.multiply,
// ki.multiply and add, each rounded); and the decay factor sigmoid(−(raw + bias)) (mlx.rs:313).
template <bool H>
__device__ __forceinline__ float gla_upd(float dc, float s, float k, float v) {
    return H ? r16(r16(dc * s) + r16(k * v)) : dc * s + k * v;
}
template <bool H>
__device__ __forceinline__ float gla_decay(float raw, float bias) {
    return H ? r16(1.0f / (1.0f + expf(r16(raw + bias)))) : 1.0f / (1.0f + expf(raw + bias));
}

template <int RPL, bool H = false>
__device__ __forceinline__ float gla_rows(float (&st)[RPL], const float* kk, const float* qq,
                                          float dc, float vb, int j, int dh) {
    float part = 0.0f;
    if ((j + 1) * RPL <= dh) {
#pragma unroll
        for (int rr = 0; rr < RPL; rr++) {
            int a = j * RPL + rr;
            st[rr] = gla_upd<H>(dc, st[rr], kk[a], vb);
            part = part + qq[a] * st[rr];
        }
    } else {
#pragma unroll
        for (int rr = 0; rr < RPL; rr++) {
            int a = j * RPL + rr;
            if (a < dh) {
                st[rr] = gla_upd<H>(dc, st[rr], kk[a], vb);
                part = part + qq[a] * st[rr];
            }
        }
    }
    return part;
}

// gla_rows when every lane's RPL rows are inside the head: the rows' k and q read as float4s.
template <int RPL, bool H = false>
__device__ __forceinline__ float gla_rows_full(float (&st)[RPL], const float* kk, const float* qq,
                                               float dc, float vb, int j) {
    float kv[RPL], qv[RPL];
    if constexpr (RPL % 4 == 0) {
#pragma unroll
        for (int c = 0; c < RPL / 4; c++) {
            f4 a = *(const f4*)(kk + j * RPL + 4 * c), b = *(const f4*)(qq + j * RPL + 4 * c);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                kv[4 * c + e] = a[e];
                qv[4 * c + e] = b[e];
            }
        }
    } else {
#pragma unroll
        for (int rr = 0; rr < RPL; rr++) {
            kv[rr] = kk[j * RPL + rr];
            qv[rr] = qq[j * RPL + rr];
        }
    }
    float part = 0.0f;
#pragma unroll
    for (int rr = 0; rr < RPL; rr++) {
        st[rr] = gla_upd<H>(dc, st[rr], kv[rr], vb);
        part = part + qv[rr] * st[rr];
    }
    return part;
}

// One token's operands for a lane of the prompt kernel's pipelined path: its RPL rows of k
// and q and the column's v.
template <int RPL>
struct GlaOps {
    float k[RPL], q[RPL], v;
};
// gla_rows_full's expressions on operands already in registers.
template <int RPL>
__device__ __forceinline__ float gla_step(float (&st)[RPL], const GlaOps<RPL>& o, float dc) {
    float part = 0.0f;
#pragma unroll
    for (int rr = 0; rr < RPL; rr++) {
        st[rr] = dc * st[rr] + o.k[rr] * o.v;
        part = part + o.q[rr] * st[rr];
    }
    return part;
}

// The prompt kernel: grid (heads, groups of SLM_GLA_COLS columns), one wave a workgroup (so a
// CU's LDS serves one wave's reads); each workgroup stages q and k of its head and v of its
// columns for SLM_GLA_T tokens at a time in LDS.
template <int RPL, bool H>
__device__ void gla_body(float* __restrict__ y, float* __restrict__ S,
                         const float* __restrict__ q, const float* __restrict__ k,
                         const float* __restrict__ v, const float* __restrict__ decay,
                         const float* __restrict__ bias, int m, int heads, int dh, int vec) {
    extern __shared__ __attribute__((aligned(16))) float lds[];  // 2 x ([SLM_GLA_T][q (dh) | k (dh) | v (SLM_GLA_COLS)], then [SLM_GLA_T] d)
    constexpr int NC = SLM_GLA_COLS;
    int h = blockIdx.x, c0 = blockIdx.y * NC, tid = threadIdx.x, nt = blockDim.x;
    int b = c0 + (tid >> 4), j = tid & 15;
    bool live = b < dh;
    float* Sh = S + (long long)h * dh * dh;
    float st[RPL];
#pragma unroll
    for (int rr = 0; rr < RPL; rr++) {
        int a = j * RPL + rr;
        st[rr] = (live && a < dh) ? Sh[(long long)a * dh + b] : 0.0f;
    }
    float bh = bias[h];
    bool full = 16 * RPL == dh && c0 + NC <= dh;  // uniform
    int rowl = 2 * dh + NC, bufl = SLM_GLA_T * (rowl + 1);
    // Two LDS buffers of SLM_GLA_T token rows (then their decays): the next group's rows are
    // copied straight into one (and its decay inputs loaded into registers) while the
    // tokens of the other run. Thread tid copies piece pc (of `vec` floats) of tokens
    // tt0, tt0 + tpar, ...: piece tid·vec of the buffer, so a wave's copies are contiguous.
    // (A row longer than the workgroup, lpt > nt: thread tid copies pieces tid, tid + nt, ...
    // of every token instead.)
    int lpt = rowl / vec, tpar = max(1, nt / lpt);
    int tt0 = tid / lpt, pc = (tid % lpt) * vec;
    bool loader = tid < tpar * lpt;
    auto piece_src = [&](int pf) {  // token 0's source of the piece at float pf of a row
        const float* sp = q + (long long)h * dh;  // (a piece past the head's columns copies q)
        if (pf < dh) sp = q + (long long)h * dh + pf;
        else if (pf < 2 * dh) sp = k + (long long)h * dh + pf - dh;
        else if (c0 + pf - 2 * dh < dh) sp = v + (long long)h * dh + c0 + pf - 2 * dh;
        return sp;
    };
    const float* src0 = piece_src(pc);
    int wbase = (tid & ~63) * vec;  // this wave's first piece
    auto copy = [&](const float* src, float* dst) {
        if (vec == 4)
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                             (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
        else
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                             (__attribute__((address_space(3))) void*)dst, 4, 0, 0);
    };
    auto issue = [&](int i0, int buf) {
        int nt_tok = min(SLM_GLA_T, m - i0);
        float* base = lds + buf * bufl + wbase;
        if (lpt > nt) {
            for (int tt = 0; tt < nt_tok; tt++)
                for (int r = 0; r * nt < lpt; r++)
                    if (r * nt + tid < lpt)
                        copy(piece_src((r * nt + tid) * vec) + (long long)(i0 + tt) * heads * dh,
                             base + tt * rowl + r * nt * vec);
            return;
        }
        if (!loader) return;
        // tokens tt0, tt0 + tpar, ...: the source and destination advance by fixed strides
        const float* src = src0 + (long long)(i0 + tt0) * heads * dh;
        const long long sstep = (long long)tpar * heads * dh;
        float* dst = base;
        const int dstep = tpar * rowl;
        if (vec == 4)
            for (int tt = tt0; tt < nt_tok; tt += tpar, src += sstep, dst += dstep)
                __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                                 (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
        else
            for (int tt = tt0; tt < nt_tok; tt += tpar, src += sstep, dst += dstep)
                __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                                 (__attribute__((address_space(3))) void*)dst, 4, 0, 0);
    };
    float dnext = 0.0f;  // thread tt: the decay input of token tt of the next group
    issue(0, 0);
    if (tid < min(SLM_GLA_T, m)) dnext = decay[(long long)tid * heads + h];
    // The outputs of a pipelined group's last eight tokens are stored only after the next
    // group's copies are issued, so that the wait for those copies does not also wait for
    // stores issued just before it.
    float pend[8];
    float* pend_y = nullptr;  // (the first of the eight tokens' outputs of this lane's column)
    const int ys = heads * dh;  // token stride of y
    auto store_pend = [&]() {
        if (pend_y && j == 0)
#pragma unroll
            for (int u = 0; u < 8; u++) pend_y[u * ys] = pend[u];
        pend_y = nullptr;
    };
    for (int i0 = 0, buf = 0; i0 < m; i0 += SLM_GLA_T, buf ^= 1) {
        int nt_tok = min(SLM_GLA_T, m - i0);
        const float* rows = lds + buf * bufl;
        float* dcs = lds + buf * bufl + SLM_GLA_T * rowl;
        __builtin_amdgcn_s_waitcnt(0);  // this thread's copies of the group are in
        if (tid < nt_tok) dcs[tid] = gla_decay<H>(dnext, bh);
        // every thread's copies and decays are in, and every thread is done with the group
        // before (whose buffer the next copies overwrite)
        __syncthreads();
        if (i0 + SLM_GLA_T < m) {
            issue(i0 + SLM_GLA_T, buf ^ 1);
            if (tid < min(SLM_GLA_T, m - i0 - SLM_GLA_T)) dnext = decay[(long long)(i0 + SLM_GLA_T + tid) * heads + h];
        }
        store_pend();
        // eight tokens at a time: their state updates in order, then their eight column
        // sums side by side (no token's sum waits for the next token's update)
        if constexpr (RPL <= 8) if (full && nt_tok == SLM_GLA_T) {
            // every lane's rows inside the head (dh = 16·RPL), every column live, a whole
            // group: the operands of token t + 2 are read from LDS while token t runs (four
            // register sets in turn), so no token waits for its reads; each read is a lane
            // base plus a constant offset
            constexpr int DH = 16 * RPL, ROWL = 2 * DH + NC;
            const float* qb = rows + j * RPL;
            const float* vb = rows + 2 * DH + (b - c0);
            // LDS reads per token (k and q rows, v); a token's reads are in once at most the two
            // later tokens' reads are pending
            constexpr int GLA_NRD = (RPL % 4 == 0 ? RPL / 2 : 2 * RPL) + 1;
            constexpr int GLA_WAIT = 2 * GLA_NRD < 15 ? 2 * GLA_NRD : 15;
            GlaOps<RPL> ops[4];
            auto load = [&](GlaOps<RPL>& o, int t) {
                if constexpr (RPL % 4 == 0) {
#pragma unroll
                    for (int c = 0; c < RPL / 4; c++) {
                        f4 ka = *(const f4*)(qb + t * ROWL + DH + 4 * c), qa = *(const f4*)(qb + t * ROWL + 4 * c);
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            o.k[4 * c + e] = ka[e];
                            o.q[4 * c + e] = qa[e];
                        }
                    }
                } else {
#pragma unroll
                    for (int rr = 0; rr < RPL; rr++) {
                        o.k[rr] = qb[t * ROWL + DH + rr];
                        o.q[rr] = qb[t * ROWL + rr];
                    }
                }
                o.v = vb[t * ROWL];
            };
            // the group's decay factors, read once (four at a time: the decays start 16-byte
            // aligned, as SLM_GLA_T is a multiple of 4)
            static_assert(SLM_GLA_T % 8 == 0, "the prompt GLA runs whole blocks of eight tokens");
            float dg[SLM_GLA_T];
#pragma unroll
            for (int t = 0; t < SLM_GLA_T; t += 4) {
                f4 d4 = *(const f4*)(dcs + t);
#pragma unroll
                for (int e = 0; e < 4; e++) dg[t + e] = d4[e];
            }
            __builtin_amdgcn_s_waitcnt(0xC07F);  // (nothing pending: the counts below are exact)
#pragma unroll
            for (int u = 0; u < 2; u++) load(ops[u], u);
            // step t updates the state with token t and sums token t - 1 over the state that
            // token left (the same expressions as gla_rows_full, in two halves that do not
            // wait for each other)
            float part[8];
            float* yg = y + ((long long)i0 * heads + h) * dh + b;  // token i0's output, column b
#pragma unroll
            for (int t = 0; t <= SLM_GLA_T; t++) {
                if (t < SLM_GLA_T) {
                    // (past the group's last token the last row is read again, unused)
                    load(ops[(t + 2) & 3], min(t + 2, SLM_GLA_T - 1));
                    __builtin_amdgcn_s_waitcnt(0xC07F | (GLA_WAIT << 8));
                }
                __builtin_amdgcn_sched_barrier(0);
                float sn[RPL];
                if (t < SLM_GLA_T) {
                    const GlaOps<RPL>& o = ops[t & 3];
#pragma unroll
                    for (int rr = 0; rr < RPL; rr++) sn[rr] = gla_upd<H>(dg[t], st[rr], o.k[rr], o.v);
                }
                if (t > 0) {
                    const GlaOps<RPL>& o = ops[(t - 1) & 3];
                    float pp = 0.0f;
#pragma unroll
                    for (int rr = 0; rr < RPL; rr++) pp = pp + o.q[rr] * st[rr];
                    part[(t - 1) & 7] = pp;
                }
                if (t < SLM_GLA_T)
#pragma unroll
                    for (int rr = 0; rr < RPL; rr++) st[rr] = sn[rr];
                __builtin_amdgcn_sched_barrier(0);
                if (t > 0 && (t & 7) == 0) {
#pragma unroll
                    for (int u = 0; u < 8; u++) part[u] = h16<H>(gla_colsum0(part[u]));
                    if (t == SLM_GLA_T) {
#pragma unroll
                        for (int u = 0; u < 8; u++) pend[u] = part[u];
                        pend_y = yg + (t - 8) * ys;
                    } else if (j == 0) {
#pragma unroll
                        for (int u = 0; u < 8; u++) yg[(t - 8 + u) * ys] = part[u];
                    }
                }
            }
            continue;
        }
        for (int t0 = 0; t0 < nt_tok; t0 += 8) {
            int nu = min(8, nt_tok - t0);
            float part[8];
            if (full && nu == 8) {  // (every lane's rows inside the head, every column live)
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const float* row = rows + (t0 + u) * rowl;
                    part[u] = gla_rows_full<RPL, H>(st, row + dh, row, dcs[t0 + u], row[2 * dh + (b - c0)], j);
                }
            } else {
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    part[u] = 0.0f;
                    if (u < nu && live) {
                        const float* row = rows + (t0 + u) * rowl;
                        part[u] = gla_rows<RPL, H>(st, row + dh, row, dcs[t0 + u], row[2 * dh + (b - c0)], j, dh);
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < 8; u++) part[u] = h16<H>(gla_colsum0(part[u]));
            if (live && j == 0)
#pragma unroll
                for (int u = 0; u < 8; u++)
                    if (u < nu) y[((long long)(i0 + t0 + u) * heads + h) * dh + b] = part[u];
        }
    }
    store_pend();
#pragma unroll
    for (int rr = 0; rr < RPL; rr++) {
        int a = j * RPL + rr;
        if (live && a < dh) Sh[(long long)a * dh + b] = st[rr];
    }
}

// (slm_glah_*: fp16 mode's)
#define GLA_K(NAME, R, H)                                                              \
    KERNEL void __launch_bounds__(16 * SLM_GLA_COLS)                                    \
        NAME(float* y, float* S, const float* q, const float* k, const float* v,        \
             const float* decay, const float* bias, int m, int heads, int dh,           \
             int vec) {                                                                 \
        gla_body<R, H>(y, S, q, k, v, decay, bias, m, heads, dh, vec);                  \
    }
#define GLA(R) GLA_K(slm_gla_##R, R, false) GLA_K(slm_glah_##R, R, true)
GLA(1)
GLA(2)
GLA(4)
GLA(8)
GLA(16)

// ---------------------------------------------------------------------------------------
// linear: y[i][r] = Σ_c w[r][c]·x[i][c] (ops.rs:116-126)
// ---------------------------------------------------------------------------------------
//
// The canonical chain, shared by every linear kernel (and the fused one). For
// v_mfma_f32_16x16x4f32 lane l holds A[l%16][l/16], B[l/16][l%16] and D[4(l/16)+r][l%16]
// in element r. Rows of w are A's rows, tokens are B's columns. Columns go in blocks of
// 16: lane group g = l/16 loads the four columns 16kb+4g .. 16kb+4g+3 of its row (of w)
// and of its token (of x), and MFMA e (e = 0..3) takes element e of both, so MFMA e of
// block kb sums the columns {16kb + 4g + e : g = 0..3}. Blocks are chained in order
// within a slice of SLM_KS = 4 blocks (64 columns) starting from zero; the slice sums of
// a split of SLM_SPLIT = 12 slices (768 columns) are added in order, Q = ((P0 + P1) + P2)
// + ..., and the split sums are added in order: y = ((Q0 + Q1) + Q2) + ...  Columns past
// `cols` load as zero.

template <bool VEC>
__device__ __forceinline__ f4 ld4(const float* __restrict__ p, long long row, long long nrows,
                                  long long cols, long long c) {
    f4 r = {0.0f, 0.0f, 0.0f, 0.0f};
    if (row < nrows) {
        const float* src = p + row * cols;
        if (VEC) {
            if (c < cols) r = *(const f4*)(src + c);
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (c + e < cols) r[e] = src[c + e];
        }
    }
    return r;
}

// m <= 16: one workgroup per 16 rows; wave w takes slices w, w+W, w+2W, ... four at a
// time, loading them before their chains start (four independent chains interleave);
// slice partials meet in LDS and one pass adds them in order.
// Row `row`, columns c .. c + 3 of fp16 weights (cols a multiple of 64), widened; zeros past
// the last row.
__device__ __forceinline__ f4 ld4w16(const float* __restrict__ p, long long row, long long nrows,
                                     long long cols, long long c) {
    f4 r = {0.0f, 0.0f, 0.0f, 0.0f};
    if (row < nrows && c < cols) r = wide4(*(const h4*)((const _Float16*)p + row * cols + c));
    return r;
}

template <bool VEC, bool H, bool W16 = false>
__device__ void linear_small_body(float* __restrict__ y, const float* __restrict__ w,
                                  const float* __restrict__ x, int rows, int cols, int m) {
    extern __shared__ float part[];  // [slices][16 rows][16 tokens]
    int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    int i = lane & 15, g = lane >> 4;
    long long r0 = (long long)blockIdx.x * 16;
    int kblocks = (cols + 15) >> 4, nsl = (kblocks + SLM_KS - 1) / SLM_KS;
    for (int s0 = wave; s0 < nsl; s0 += 4 * waves) {
        f4 wa[4][SLM_KS], xb[4][SLM_KS];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            int s = s0 + j * waves;
#pragma unroll
            for (int u = 0; u < SLM_KS; u++) {
                int kb = s * SLM_KS + u;
                wa[j][u] = f4{0.0f, 0.0f, 0.0f, 0.0f};
                xb[j][u] = f4{0.0f, 0.0f, 0.0f, 0.0f};
                if (s < nsl && kb < kblocks) {
                    long long c = (long long)kb * 16 + g * 4;
                    if constexpr (W16) wa[j][u] = ld4w16(w, r0 + i, rows, cols, c);
                    else wa[j][u] = ld4<VEC>(w, r0 + i, rows, cols, c);
                    xb[j][u] = ld4<VEC>(x, i, m, cols, c);
                }
            }
        }
        f4 acc[4];
#pragma unroll
        for (int j = 0; j < 4; j++) acc[j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (H) {
#pragma unroll
            for (int u = 0; u < SLM_KS; u++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    int s = s0 + j * waves;
                    if (s < nsl && s * SLM_KS + u < kblocks) acc[j] = block16h(wa[j][u], xb[j][u], acc[j]);
                }
        } else {
#pragma unroll
            for (int u = 0; u < SLM_KS; u++)
#pragma unroll
                for (int e = 0; e < 4; e++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        int s = s0 + j * waves;
                        if (s < nsl && s * SLM_KS + u < kblocks) acc[j] = mfma4(wa[j][u][e], xb[j][u][e], acc[j]);
                    }
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            int s = s0 + j * waves;
            if (s < nsl) {
#pragma unroll
                for (int r = 0; r < 4; r++) part[s * 256 + (4 * g + r) * 16 + i] = acc[j][r];
            }
        }
    }
    __syncthreads();
    for (int t = threadIdx.x; t < 256; t += blockDim.x) {
        int rr = t >> 4, tt = t & 15;
        float tot = 0.0f;
        for (int s0 = 0; s0 < nsl; s0 += SLM_SPLIT) {
            float q = part[s0 * 256 + t];
            int s1 = min(s0 + SLM_SPLIT, nsl);
            for (int s = s0 + 1; s < s1; s++) q = q + part[s * 256 + t];
            tot = s0 == 0 ? q : tot + q;
        }
        if (r0 + rr < rows && tt < m) y[(long long)tt * rows + r0 + rr] = h16<H>(tot);
    }
}

KERNEL void __launch_bounds__(512) slm_linear_small_v(float* y, const float* w, const float* x,
                                                      int rows, int cols, int m) {
    linear_small_body<true, false>(y, w, x, rows, cols, m);
}
KERNEL void __launch_bounds__(512) slm_linear_small_s(float* y, const float* w, const float* x,
                                                      int rows, int cols, int m) {
    linear_small_body<false, false>(y, w, x, rows, cols, m);
}
KERNEL void __launch_bounds__(512) slm_linear_small_vh(float* y, const float* w, const float* x,
                                                       int rows, int cols, int m) {
    linear_small_body<true, true>(y, w, x, rows, cols, m);
}
// fp16 mode with the weights stored as halves (w: rows x cols fp16)
KERNEL void __launch_bounds__(512) slm_linear_small_vhw(float* y, const float* w, const float* x,
                                                        int rows, int cols, int m) {
    linear_small_body<true, true, true>(y, w, x, rows, cols, m);
}

// m > 16: a 64-row × 64-token tile per workgroup, 32 × 32 per wave (2 × 2 MFMA tiles).
template <bool VEC>
__device__ void linear_big_body(float* __restrict__ y, const float* __restrict__ w,
                                const float* __restrict__ x, int rows, int cols, int m) {
    int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int i = lane & 15, g = lane >> 4;
    long long rb = (long long)blockIdx.x * 64 + (wave & 1) * 32;
    long long tb = (long long)blockIdx.y * 64 + (wave >> 1) * 32;
    int kblocks = (cols + 15) >> 4, nsl = (kblocks + SLM_KS - 1) / SLM_KS;
    f4 tot[2][2], sp[2][2];
    for (int s = 0; s < nsl; s++) {
        f4 acc[2][2];
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int v = 0; v < 2; v++) acc[u][v] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        int kb1 = min(s * SLM_KS + SLM_KS, kblocks);
        for (int kb = s * SLM_KS; kb < kb1; kb++) {
            long long c = (long long)kb * 16 + g * 4;
            f4 a[2], b[2];
#pragma unroll
            for (int u = 0; u < 2; u++) a[u] = ld4<VEC>(w, rb + 16 * u + i, rows, cols, c);
#pragma unroll
            for (int v = 0; v < 2; v++) b[v] = ld4<VEC>(x, tb + 16 * v + i, m, cols, c);
#pragma unroll
            for (int e = 0; e < 4; e++)
#pragma unroll
                for (int u = 0; u < 2; u++)
#pragma unroll
                    for (int v = 0; v < 2; v++) acc[u][v] = mfma4(a[u][e], b[v][e], acc[u][v]);
        }
        bool open = s % SLM_SPLIT == 0, close = s % SLM_SPLIT == SLM_SPLIT - 1 || s == nsl - 1;
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int v = 0; v < 2; v++) {
                sp[u][v] = open ? acc[u][v] : sp[u][v] + acc[u][v];
                if (close) tot[u][v] = s < SLM_SPLIT ? sp[u][v] : tot[u][v] + sp[u][v];
            }
    }
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
        for (int v = 0; v < 2; v++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                long long row = rb + 16 * u + 4 * g + r, tok = tb + 16 * v + i;
                if (row < rows && tok < m) y[tok * rows + row] = tot[u][v][r];
            }
}

KERNEL void __launch_bounds__(256) slm_linear_big_v(float* y, const float* w, const float* x,
                                                    int rows, int cols, int m) {
    linear_big_body<true>(y, w, x, rows, cols, m);
}
KERNEL void __launch_bounds__(256) slm_linear_big_s(float* y, const float* w, const float* x,
                                                    int rows, int cols, int m) {
    linear_big_body<false>(y, w, x, rows, cols, m);
}

// m > 16, columns a multiple of 4, 16-byte aligned rows: the prompt GEMM. A 64-row × 64-token
// tile per workgroup, 32 × 32 per wave; the weights and tokens of one slice (64 columns)
// at a time are staged in LDS (row stride 68 floats), the next slice's loads in flight
// while one computes. blockIdx.z is the split: with several splits each workgroup adds
// one split's slices and writes its partial to part[split][token][row] (added in order by
// slm_fold); with one it writes y. Same chain and sums as linear_big_body.
#define GEMM_LS 68
KERNEL void __launch_bounds__(256) slm_gemm(float* __restrict__ y, float* __restrict__ part,
                                            const float* __restrict__ w,
                                            const float* __restrict__ x, int rows, int cols,
                                            int m) {
    __shared__ float sw[2][64 * GEMM_LS];
    __shared__ float sx[2][64 * GEMM_LS];
    int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int i = lane & 15, g = lane >> 4;
    int wr = (wave & 1) * 32, wt = (wave >> 1) * 32;
    long long r0 = (long long)blockIdx.x * 64, t0 = (long long)blockIdx.y * 64;
    int kblocks = (cols + 15) >> 4, nsl = (kblocks + SLM_KS - 1) / SLM_KS;
    int s_first = blockIdx.z * SLM_SPLIT, s_end = min(nsl, s_first + SLM_SPLIT);
    // staging: f4 number fi = tid + 256q of a 64 x 64 tile: row fi / 16, column 4 (fi % 16)
    f4 rw[4], rx[4];
    auto fetch = [&](int s) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            int fi = tid + 256 * q, row = fi >> 4, c = s * 64 + 4 * (fi & 15);
            bool cin = c < cols;
            rw[q] = f4{0.0f, 0.0f, 0.0f, 0.0f};
            rx[q] = f4{0.0f, 0.0f, 0.0f, 0.0f};
            if (cin && r0 + row < rows) rw[q] = *(const f4*)(w + (r0 + row) * cols + c);
            if (cin && t0 + row < m) rx[q] = *(const f4*)(x + (t0 + row) * cols + c);
        }
    };
    auto stash = [&](int b) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            int fi = tid + 256 * q, row = fi >> 4, c = 4 * (fi & 15);
            *(f4*)(&sw[b][row * GEMM_LS + c]) = rw[q];
            *(f4*)(&sx[b][row * GEMM_LS + c]) = rx[q];
        }
    };
    f4 tot[2][2], sp[2][2];
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
        for (int v = 0; v < 2; v++) {
            tot[u][v] = f4{0.0f, 0.0f, 0.0f, 0.0f};
            sp[u][v] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    fetch(s_first);
    stash(0);
    __syncthreads();
    for (int s = s_first; s < s_end; s++) {
        int b = (s - s_first) & 1;
        if (s + 1 < s_end) fetch(s + 1);
        f4 acc[2][2];
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int v = 0; v < 2; v++) acc[u][v] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int q = 0; q < SLM_KS; q++) {
            if (s * SLM_KS + q >= kblocks) break;
            f4 a[2], bb[2];
#pragma unroll
            for (int u = 0; u < 2; u++) a[u] = *(const f4*)(&sw[b][(wr + 16 * u + i) * GEMM_LS + 16 * q + 4 * g]);
#pragma unroll
            for (int v = 0; v < 2; v++) bb[v] = *(const f4*)(&sx[b][(wt + 16 * v + i) * GEMM_LS + 16 * q + 4 * g]);
#pragma unroll
            for (int e = 0; e < 4; e++)
#pragma unroll
                for (int u = 0; u < 2; u++)
#pragma unroll
                    for (int v = 0; v < 2; v++) acc[u][v] = mfma4(a[u][e], bb[v][e], acc[u][v]);
        }
        // slice sums in order within the split, split sums in order (one split here)
        bool open = (s - s_first) == 0;
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int v = 0; v < 2; v++) sp[u][v] = open ? acc[u][v] : sp[u][v] + acc[u][v];
        if (s + 1 < s_end) {
            stash(b ^ 1);
            __syncthreads();
        }
    }
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
        for (int v = 0; v < 2; v++) tot[u][v] = sp[u][v];
    // out: D[4g + r][i] is row wr + 16u + 4g + r, token wt + 16v + i; through LDS so the
    // stores run along rows
    __syncthreads();
    float* so = &sw[0][0];  // [64 tokens][65]
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
        for (int v = 0; v < 2; v++)
#pragma unroll
            for (int r = 0; r < 4; r++) so[(wt + 16 * v + i) * 65 + wr + 16 * u + 4 * g + r] = tot[u][v][r];
    __syncthreads();
    float* out = gridDim.z > 1 ? part + (long long)blockIdx.z * m * rows : y;
    for (int e = tid; e < 64 * 64; e += 256) {
        int tok = e >> 6, row = e & 63;
        if (t0 + tok < m && r0 + row < rows) out[(t0 + tok) * rows + r0 + row] = so[tok * 65 + row];
    }
}

// The same GEMM with a deeper pipeline, for cols a multiple of 64 and 16-byte aligned rows:
// tiles of BM rows x 64 tokens, 64-column slices copied straight into LDS (no registers) by
// the four waves, GEMM_STAGES slices in flight, one barrier per slice. Two stages (80 KB of
// LDS for 96-row tiles) let two workgroups share a CU, from concurrent prompt chunks; three
// measured the same on one stream and 2 % slower on three. In LDS, row r of a
// slice is 16 chunks of 16 bytes with chunk c at position c ^ (r & 15), so the MFMA operand
// reads (sixteen rows at one chunk) fall on distinct banks; the copy puts each lane's chunk
// there by permuting the global addresses it reads. Waves 2 x 2 over the tile, each
// (BM / 2) x 32. The arithmetic is slm_gemm's: the same MFMA chain per slice, slices added
// in order within the split, one split per blockIdx.z.
#define GEMM_STAGES 2
__device__ __forceinline__ int gsw(int row, int chunk) { return row * 64 + 4 * (chunk ^ (row & 15)); }

template <int N>
__device__ __forceinline__ void vm_wait() {  // s_waitcnt vmcnt(N), other counters untouched
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// The attention-input epilogue (ROPE, BM = dh = 64, rows = 3·d): y [m][3d] is written as
// usual, and tile r0 is one head of q, k or v: q and k are also written rotated (slm_rope's
// expressions with the cos/sin rows of each token) into ep.q / ep.k [m][d], v as it is into
// ep.v, and k and v into the rings at slot (pos + t) mod cap (slm_store).
struct GemmEpi {
    float* q;
    float* k;
    float* v;
    float* kring;
    float* vring;
    const float* cs;  // [m][32]
    const float* sn;
    float* g;  // (L2: the gate columns)
    const long long* kdyn;  // each ring store's position on the device (or null: kpos, vpos)
    const long long* vdyn;
    long long kpos, vpos, cap;
    int d, ring16;  // ring16: the rings hold fp16 values
};
// With SILU the weight rows are the two halves of a gate|amp matrix (rows = 2·half): tile
// rows 0 .. BM/2 − 1 are gate rows r0h + j and rows BM/2 .. BM − 1 the amp rows half + r0h + j
// (r0h = blockIdx.x·BM/2), and the tile writes amp·gate / (1 + e^−gate) (slm_silu_mul's
// expression) for its BM/2 output columns of y [m][half]; one split only.
// With W16 the weights are fp16 (rows x cols halves, H too): a stage holds the tile's BM rows of
// 64 halves (128 bytes: eight 16-byte chunks, chunk c at position c ^ (row & 7)), eight rows
// per copy instruction; copies past the stage's count repeat earlier ones (the same bytes to
// the same place), so every wave issues the same number.
// With KG = 2 the workgroup has two groups of WAVES waves: group 0 runs the first half of
// the split's slices and group 1 the second half, each through LDS buffers of its own, side
// by side (twice the MFMA chains per SIMD); group 1 hands its slice sums to group 0, which
// adds them after its own, in slice order (the same sums as one group). Plain outputs only.
// RGX (when not 0) sets the number of row groups of the waves (RG); the token groups are the
// rest (WAVES / RG), each 64 / (WAVES / RG) tokens wide.
template <int BM, int WAVES, bool H, bool SILU, int ROPE = 0, bool W16 = false, int KG = 1, int RGX = 0>
__device__ void gemm2_body(float* __restrict__ y, float* __restrict__ part,
                           const float* __restrict__ w, const float* __restrict__ x, int rows,
                           int cols, int m, GemmEpi ep = GemmEpi{}) {
    static_assert(!W16 || H, "fp16 weights run the fp16 chain");
    constexpr int SW = W16 ? BM * 32 : BM * 64, SX = 64 * 64, STAGE = SW + SX;  // floats per stage
    constexpr int RG = RGX ? RGX : WAVES == 16 ? 4 : 2;         // groups of rows over the waves
    constexpr int NV = 4 / (WAVES / RG);                        // 16-token MFMA tiles per wave
    static_assert(WAVES % RG == 0 && NV * (WAVES / RG) == 4, "waves over rows and tokens");
    constexpr int MU = BM / (16 * RG);                          // 16-row MFMA tiles per wave
    constexpr int NW = W16 ? BM / 8 : BM / 4;                   // copy instructions of the w tile
    constexpr int NT = NW + 16;                                 // ... and of the x tile
    constexpr int NDMA = (NT + WAVES - 1) / WAVES;              // copies per wave per stage
    static_assert(W16 || (BM + 64) % (4 * WAVES) == 0, "copies per wave");
    static_assert(MU >= 1 && NDMA * WAVES < 2 * NT && BM % 8 == 0, "rows per wave, repeated copies");
    static_assert(KG == 1 || (KG == 2 && !SILU && ROPE == 0), "slice groups: plain outputs");
    constexpr int NTH = 64 * WAVES * KG;                        // threads
    extern __shared__ __attribute__((aligned(16))) float lds[];  // [KG][GEMM_STAGES][w: BM x 64 | x: 64 x 64]
    int tid = threadIdx.x, lane = tid & 63;
    int kg = __builtin_amdgcn_readfirstlane((tid >> 6) / WAVES), wave = __builtin_amdgcn_readfirstlane((tid >> 6) % WAVES);
    int i = lane & 15, g = lane >> 4;
    // waves: RG groups of the rows times (64 / 16NV) groups of tokens
    int wr = (wave % RG) * (BM / RG), wt = (wave / RG) * 16 * NV;
    long long r0 = (long long)blockIdx.x * BM, t0 = (long long)blockIdx.y * 64;
    long long r0h = (long long)blockIdx.x * (BM / 2), half = rows / 2;  // (SILU)
    int nsl = cols >> 6;
    int s_first = blockIdx.z * SLM_SPLIT, s_end = min(nsl, s_first + SLM_SPLIT), ns = s_end - s_first;
    float* gl = lds + kg * GEMM_STAGES * STAGE;  // this group's buffers
    // Stage copy: instruction k of this wave covers rows 4k' .. 4k'+3 of the stage's (BM + 64)
    // rows (w rows first, then x rows), k' = wave + WAVES k; lane L takes row 4k' + L/16,
    // position L % 16, i.e. chunk (L % 16) ^ (row & 15) of that row.
    auto issue = [&](int sl, int buf) {
        if constexpr (W16) {
#pragma unroll
            for (int k = 0; k < NDMA; k++) {
                int kk = wave + WAVES * k;
                if (kk >= NT) kk -= NT;
                const void* src;
                if (kk < NW) {  // eight weight rows of 64 halves
                    int rl = 8 * kk + (lane >> 3), chunk = (lane & 7) ^ (rl & 7);
                    long long wr_ = r0 + rl;
                    bool ok = wr_ < rows;
                    if constexpr (SILU) {
                        long long j = r0h + (rl < BM / 2 ? rl : rl - BM / 2);
                        ok = j < half;
                        wr_ = rl < BM / 2 ? j : half + j;
                    }
                    src = (const _Float16*)w + (ok ? wr_ * cols : 0) + (long long)sl * 64 + 8 * chunk;
                } else {  // four token rows of 64 floats
                    int rl = 4 * (kk - NW) + (lane >> 4), chunk = (lane & 15) ^ (rl & 15);
                    bool ok = t0 + rl < m;
                    src = x + (ok ? (t0 + rl) * cols : 0) + (long long)sl * 64 + 4 * chunk;
                }
                float* dst = gl + buf * STAGE + kk * 256;  // uniform: 1 KB per instruction
                __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                                 (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
            }
            return;
        }
#pragma unroll
        for (int k = 0; k < NDMA; k++) {
            int rr = 4 * (wave + WAVES * k) + (lane >> 4), pos = lane & 15;
            int rl = rr < BM ? rr : rr - BM;  // row within the w or x tile
            int chunk = pos ^ (rl & 15);
            const float* src;
            if (rr < BM) {
                long long wr_ = r0 + rl;
                bool ok = wr_ < rows;
                if constexpr (SILU) {
                    long long j = r0h + (rl < BM / 2 ? rl : rl - BM / 2);
                    ok = j < half;
                    wr_ = rl < BM / 2 ? j : half + j;
                }
                src = w + (ok ? wr_ * cols : 0) + (long long)sl * 64 + 4 * chunk;
            } else {
                bool ok = t0 + rl < m;
                src = x + (ok ? (t0 + rl) * cols : 0) + (long long)sl * 64 + 4 * chunk;
            }
            float* dst = gl + buf * STAGE + (4 * (wave + WAVES * k)) * 64;  // uniform: 4 rows
            // a row past the end copies row 0 instead (its outputs are never stored), so every
            // copy runs and the waits below count them exactly
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                             (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
        }
    };
    f4 sp[MU][NV];
#pragma unroll
    for (int u = 0; u < MU; u++)
#pragma unroll
        for (int v = 0; v < NV; v++) sp[u][v] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    // A slice's operands go from LDS into registers one slice ahead: while the MFMAs of slice
    // q run, the reads of slice q + 1 are in flight (the LDS reads of all waves take about half
    // as long as their MFMAs), and the copies of slices q + 2 and q + 3.
    f4 p1[KG == 2 ? SLM_SPLIT / 2 : 1][MU][NV];  // (group 1) its slice sums
    struct Ops {
        f4 a[SLM_KS][MU];
        h4 aw[SLM_KS][MU];
        f4 bb[SLM_KS][NV];
    };
    auto load_ops = [&](int buf, Ops& o) {
        const float* sw = gl + buf * STAGE;
        const float* sx = sw + SW;
#pragma unroll
        for (int q = 0; q < SLM_KS; q++) {
#pragma unroll
            for (int u = 0; u < MU; u++) {
                int row = wr + 16 * u + i;
                if constexpr (W16)  // lane (i, g) of block q: halves 16q + 4g .. + 3 of its row, chunk 2q + g / 2
                    o.aw[q][u] = *(const h4*)((const char*)sw + row * 128 + 16 * ((2 * q + (g >> 1)) ^ (row & 7)) +
                                              8 * (g & 1));
                else
                    o.a[q][u] = *(const f4*)(sw + gsw(row, 4 * q + g));
            }
#pragma unroll
            for (int v = 0; v < NV; v++) o.bb[q][v] = *(const f4*)(sx + gsw(wt + 16 * v + i, 4 * q + g));
        }
    };
    auto run_ops = [&](const Ops& o, int q0) {
        f4 acc[MU][NV];
#pragma unroll
        for (int u = 0; u < MU; u++)
#pragma unroll
            for (int v = 0; v < NV; v++) acc[u][v] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (W16) {
#pragma unroll
            for (int q = 0; q < SLM_KS; q++)
#pragma unroll
                for (int u = 0; u < MU; u++)
#pragma unroll
                    for (int v = 0; v < NV; v++) acc[u][v] = block16hw(o.aw[q][u], o.bb[q][v], acc[u][v]);
        } else if constexpr (H) {
#pragma unroll
            for (int q = 0; q < SLM_KS; q++)
#pragma unroll
                for (int u = 0; u < MU; u++)
#pragma unroll
                    for (int v = 0; v < NV; v++) acc[u][v] = block16h(o.a[q][u], o.bb[q][v], acc[u][v]);
        } else {
#pragma unroll
            for (int q = 0; q < SLM_KS; q++)
#pragma unroll
                for (int e = 0; e < 4; e++)
#pragma unroll
                    for (int u = 0; u < MU; u++)
#pragma unroll
                        for (int v = 0; v < NV; v++) acc[u][v] = mfma4(o.a[q][u][e], o.bb[q][v][e], acc[u][v]);
        }
        // slice sums in order within the split (group 1 keeps its own for group 0)
        if (KG == 1 || kg == 0) {
#pragma unroll
            for (int u = 0; u < MU; u++)
#pragma unroll
                for (int v = 0; v < NV; v++) sp[u][v] = q0 == 0 ? acc[u][v] : sp[u][v] + acc[u][v];
        } else {  // (constant indices only: p1 stays in registers)
#pragma unroll
            for (int j = 0; j < (KG == 2 ? SLM_SPLIT / 2 : 1); j++)
                if (j == q0)
#pragma unroll
                    for (int u = 0; u < MU; u++)
#pragma unroll
                        for (int v = 0; v < NV; v++) p1[j][u][v] = acc[u][v];
        }
    };
    // a barrier without the fence of __syncthreads, which would wait for every copy in flight;
    // this wave's LDS reads issued before it are done (the second wait, a no-op, tells the
    // compiler so: it would otherwise count the reads of two slices in flight, more than the
    // counter holds, and wait for all of them before the first MFMA)
    auto barrier = [&]() {
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt, expcnt untouched
    };
    static_assert(GEMM_STAGES >= 2, "the copy waits below count GEMM_STAGES buffers");
    // (two slices of operands in registers do not fit 16 waves of 128-row tiles: those read
    // each slice after its barrier)
    constexpr bool PIPE = !(BM == 128 && WAVES == 16);
    static_assert(PIPE || KG == 1, "slice groups run the pipelined loop");
    if constexpr (!PIPE) {
#pragma unroll
        for (int p = 0; p < GEMM_STAGES - 1; p++)
            if (p < ns) issue(s_first + p, p);
        for (int q0 = 0; q0 < ns; q0++) {
            if (q0 + 1 < ns) vm_wait<NDMA * (GEMM_STAGES - 2)>();
            else vm_wait<0>();
            barrier();
            if (q0 + GEMM_STAGES - 1 < ns)
                issue(s_first + q0 + GEMM_STAGES - 1, (q0 + GEMM_STAGES - 1) % GEMM_STAGES);
            Ops o;
            load_ops(q0 % GEMM_STAGES, o);
            run_ops(o, q0);
        }
    } else {
        // This group's slices: g_ns from g_first (group 0: the first nst of the split; group 1
        // the rest, possibly none). Both groups run nst steps (the same barriers).
        int nst = (ns + KG - 1) / KG;
        int g_first = kg == 0 ? s_first : s_first + nst, g_ns = kg == 0 ? nst : ns - nst;
        int c_first = g_ns > 0 ? g_first : s_first, c_last = (g_ns > 0 ? g_ns : 1) - 1;
        // Every step issues one slice's copies (past the group's last slice, the last one again
        // into the free buffer), so every wait below counts the same: no branches, and the
        // compiler's waits for the LDS reads stay exact.
#pragma unroll
        for (int p = 0; p < GEMM_STAGES; p++) issue(c_first + min(p, c_last), p);
        // slice 0 is in (this wave's copies of the later stages may still run), then everyone's is
        vm_wait<(GEMM_STAGES - 1) * NDMA>();
        barrier();
        Ops R0, R1;
        load_ops(0, R0);
        // step q (q + 1 < nst): slice q + 1 is in (everyone's copies) and slice q's buffer is
        // free (everyone's reads of it were waited for before the barrier): copy slice
        // q + GEMM_STAGES there, read slice q + 1, run slice q, whose operands the barrier
        // waited for
        auto step = [&](int q, Ops& cur, Ops& nxt) {
            vm_wait<(GEMM_STAGES - 2) * NDMA>();
            barrier();
            issue(c_first + min(q + GEMM_STAGES, c_last), q % GEMM_STAGES);
            load_ops((q + 1) % GEMM_STAGES, nxt);
            __builtin_amdgcn_sched_barrier(0);  // the reads stay ahead of the MFMAs
            if (q < g_ns) run_ops(cur, q);
        };
        // unrolled over the group's slices (nst <= SLM_SPLIT / KG), so that the two register
        // sets alternate without copies
#pragma unroll
        for (int q0 = 0; q0 < SLM_SPLIT / KG; q0 += 2) {
            if (q0 + 1 < nst) {
                step(q0, R0, R1);
                if (q0 + 2 < nst) {
                    step(q0 + 1, R1, R0);
                } else {
                    if (q0 + 1 < g_ns) run_ops(R1, q0 + 1);
                    break;
                }
            } else {
                if (q0 < g_ns) run_ops(R0, q0);
                break;
            }
        }
        vm_wait<0>();  // the repeated copies are in before the buffers are reused below
        if constexpr (KG == 2) {
            // group 1's slice sums through LDS to group 0, which adds them after its own
            __syncthreads();
            f4* xp = (f4*)lds;  // [slice][wave][u][v][lane]
            if (kg == 1) {
#pragma unroll
                for (int j = 0; j < SLM_SPLIT / 2; j++)
                    if (j < g_ns)
#pragma unroll
                        for (int u = 0; u < MU; u++)
#pragma unroll
                            for (int v = 0; v < NV; v++)
                                xp[(((j * WAVES + wave) * MU + u) * NV + v) * 64 + lane] = p1[j][u][v];
            }
            __syncthreads();
            if (kg == 0) {
                int n1 = ns - nst;
#pragma unroll
                for (int j = 0; j < SLM_SPLIT / 2; j++)
                    if (j < n1)
#pragma unroll
                        for (int u = 0; u < MU; u++)
#pragma unroll
                            for (int v = 0; v < NV; v++)
                                sp[u][v] = sp[u][v] + xp[(((j * WAVES + wave) * MU + u) * NV + v) * 64 + lane];
            }
        }
    }
    // out: D[4g + r][i] is row wr + 16u + 4g + r, token wt + 16v + i; through LDS so the
    // stores run along rows
    __syncthreads();
    float* so = lds;  // [64 tokens][BM + 1]
    if (KG == 1 || kg == 0) {
#pragma unroll
        for (int u = 0; u < MU; u++)
#pragma unroll
            for (int v = 0; v < NV; v++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    // (fp16 mode: the linear's output rounded; a split's partials are not)
                    float o = sp[u][v][r];
                    so[(wt + 16 * v + i) * (BM + 1) + wr + 16 * u + 4 * g + r] = H && gridDim.z == 1 ? r16(o) : o;
                }
    }
    __syncthreads();
    if constexpr (ROPE == 2) {
        // The linear-attention input (rows = 4·d): q and k leave L2-normalised per head (the
        // sum of slm_l2norm, dot16_wave, over the tile's 64 values of a token), v and the gate
        // as they are; one wave per token, so the sums' lanes are all active.
        static_assert(BM == 64, "one head of 64 dims per tile");
        int region = (int)(r0 / ep.d), head = (int)((r0 % ep.d) >> 6);
        float* dst = region == 0 ? ep.q : region == 1 ? ep.k : region == 2 ? ep.v : ep.g;
        for (int tok = wave; tok < 64; tok += WAVES) {
            long long t = t0 + tok;
            if (t >= m) break;
            const float* sr = so + tok * (BM + 1);
            float v = sr[lane];
            y[t * rows + r0 + lane] = v;
            if (region < 2) {
                float dd = dot16_wave(sr, 64, lane);
                v = h16<H>(v * (1.0f / fmaxf(sqrtf(dd), 1e-12f)));
            }
            dst[t * ep.d + head * 64 + lane] = v;
        }
        return;
    }
    if constexpr (ROPE == 1) {
        static_assert(BM == 64, "one head of 64 dims per tile");
        int region = (int)(r0 / ep.d), head = (int)((r0 % ep.d) >> 6);
        long long pos = 0;
        if (region == 1) pos = ep.kdyn ? ep.kdyn[0] : ep.kpos;
        if (region == 2) pos = ep.vdyn ? ep.vdyn[0] : ep.vpos;
        float* dst = region == 0 ? ep.q : region == 1 ? ep.k : ep.v;
        float* ring = region == 1 ? ep.kring : ep.vring;
        for (int e = tid; e < 64 * 64; e += 64 * WAVES) {
            int tok = e >> 6, j = e & 63;
            long long t = t0 + tok;
            if (t >= m) continue;
            const float* sr = so + tok * (BM + 1);
            float v = sr[j];
            y[t * rows + r0 + j] = v;
            if (region < 2) {
                int i = j & 31;
                float c = ep.cs[t * 32 + i], sn = ep.sn[t * 32 + i];
                float a = sr[i], b = sr[32 + i];
                v = j < 32 ? e_rope_l<H>(a, b, c, sn) : e_rope_r<H>(a, b, c, sn);
            }
            dst[t * ep.d + head * 64 + j] = v;
            if (region > 0) {
                long long at = ((long long)head * ep.cap + (pos + t) % ep.cap) * 64 + j;
                if (ep.ring16) ((_Float16*)ring)[at] = (_Float16)v;  // an fp16 ring
                else ring[at] = v;
            }
        }
        return;
    }
    if constexpr (SILU) {
        constexpr int HB = BM / 2;
        for (int e = tid; e < 64 * HB; e += 64 * WAVES) {
            int tok = e / HB, j = e % HB;
            if (t0 + tok < m && r0h + j < half) {
                float gt = so[tok * (BM + 1) + j], up = so[tok * (BM + 1) + HB + j];
                y[(t0 + tok) * half + r0h + j] = e_silu<H>(gt, up);
            }
        }
        return;
    }
    float* out = gridDim.z > 1 ? part + (long long)blockIdx.z * m * rows : y;
    for (int e = tid; e < 64 * BM; e += NTH) {
        int tok = e / BM, row = e % BM;
        if (t0 + tok < m && r0 + row < rows) out[(t0 + tok) * rows + r0 + row] = so[tok * (BM + 1) + row];
    }
}

#define GEMM2_K(NAME, BM, WAVES, H, S, W16)                                               \
    KERNEL void __launch_bounds__(64 * WAVES) NAME(float* y, float* part, const float* w,  \
                                                   const float* x, int rows, int cols, int m) { \
        gemm2_body<BM, WAVES, H, S, 0, W16>(y, part, w, x, rows, cols, m);                 \
    }
// fp32, fp16 mode, fp16 mode with fp16 weights (..w); plain and with the SiLU pair (..s..)
#define GEMM2(BM, WAVES)                                         \
    GEMM2_K(slm_gemm2_##BM, BM, WAVES, false, false, false)      \
    GEMM2_K(slm_gemm2h_##BM, BM, WAVES, true, false, false)      \
    GEMM2_K(slm_gemm2hw_##BM, BM, WAVES, true, false, true)      \
    GEMM2_K(slm_gemm2s_##BM, BM, WAVES, false, true, false)      \
    GEMM2_K(slm_gemm2hs_##BM, BM, WAVES, true, true, false)      \
    GEMM2_K(slm_gemm2hsw_##BM, BM, WAVES, true, true, true)
// the QKV projection with the attention-input epilogue (fp32 and fp16 mode)
#define GEMM2R_K(NAME, H, W16)                                                                  \
    KERNEL void __launch_bounds__(1024)                                                         \
        NAME(float* y, float* part, const float* w, const float* x, int rows, int cols, int m,   \
             float* q, float* k, float* v, float* kring, float* vring, const float* cs,          \
             const float* sn, const long long* kdyn, const long long* vdyn, long long kpos,     \
             long long vpos, long long cap, int d, int ring16) {                                 \
        gemm2_body<64, 16, H, false, 1, W16>(y, part, w, x, rows, cols, m,                      \
                                        GemmEpi{q, k, v, kring, vring, cs, sn, nullptr, kdyn, vdyn, kpos, vpos, cap, d, ring16}); \
    }
GEMM2R_K(slm_gemm2r_64, false, false)
GEMM2R_K(slm_gemm2hr_64, true, false)
GEMM2R_K(slm_gemm2hrw_64, true, true)
// the linear-attention QKVG projection with the per-head L2 epilogue (fp32 and fp16 mode)
#define GEMM2N_K(NAME, H, W16)                                                                   \
    KERNEL void __launch_bounds__(1024)                                                          \
        NAME(float* y, float* part, const float* w, const float* x, int rows, int cols, int m,    \
             float* q, float* k, float* v, float* g, int d) {                                     \
        gemm2_body<64, 16, H, false, 2, W16>(                                                    \
            y, part, w, x, rows, cols, m,                                                        \
            GemmEpi{q, k, v, nullptr, nullptr, nullptr, nullptr, g, nullptr, nullptr, 0, 0, 0, d, 0}); \
    }
GEMM2N_K(slm_gemm2n_64, false, false)
GEMM2N_K(slm_gemm2hn_64, true, false)
GEMM2N_K(slm_gemm2hnw_64, true, true)
GEMM2(32, 4)
// Plain fp32 tiles for skinny prompts (the host picks by the chip's fill): 32 and 16 rows
// with two slice groups of four waves; 48 rows with four waves of three row blocks each.
KERNEL void __launch_bounds__(512) slm_gemm2k_32(float* y, float* part, const float* w,
                                                 const float* x, int rows, int cols, int m) {
    gemm2_body<32, 4, false, false, 0, false, 2>(y, part, w, x, rows, cols, m);
}
KERNEL void __launch_bounds__(512) slm_gemm2k_16(float* y, float* part, const float* w,
                                                 const float* x, int rows, int cols, int m) {
    gemm2_body<16, 4, false, false, 0, false, 2, 1>(y, part, w, x, rows, cols, m);
}
KERNEL void __launch_bounds__(256) slm_gemm2_48(float* y, float* part, const float* w,
                                                const float* x, int rows, int cols, int m) {
    gemm2_body<48, 4, false, false, 0, false, 1, 1>(y, part, w, x, rows, cols, m);
}
// the same tiles in fp16 mode (fp16 operands; ..w: fp16 weights)
KERNEL void __launch_bounds__(512) slm_gemm2hk_16(float* y, float* part, const float* w,
                                                  const float* x, int rows, int cols, int m) {
    gemm2_body<16, 4, true, false, 0, false, 2, 1>(y, part, w, x, rows, cols, m);
}
KERNEL void __launch_bounds__(512) slm_gemm2hwk_16(float* y, float* part, const float* w,
                                                   const float* x, int rows, int cols, int m) {
    gemm2_body<16, 4, true, false, 0, true, 2, 1>(y, part, w, x, rows, cols, m);
}
KERNEL void __launch_bounds__(256) slm_gemm2h_48(float* y, float* part, const float* w,
                                                 const float* x, int rows, int cols, int m) {
    gemm2_body<48, 4, true, false, 0, false, 1, 1>(y, part, w, x, rows, cols, m);
}
KERNEL void __launch_bounds__(256) slm_gemm2hw_48(float* y, float* part, const float* w,
                                                  const float* x, int rows, int cols, int m) {
    gemm2_body<48, 4, true, false, 0, true, 1, 1>(y, part, w, x, rows, cols, m);
}
GEMM2(64, 16)
GEMM2(96, 8)
GEMM2(128, 16)

// ---------------------------------------------------------------------------------------
// attention (ops.rs:31-66, 218-227; cpu.rs:352-403)
// ---------------------------------------------------------------------------------------
//
// A wave works on 16 columns; column c is query (qtile·qpt + c/group) of query head
// (kvh·group + c%group), all sharing kv head kvh (group = heads / key_heads, qpt =
// 16 / group). The query at position p sees [lo, hi) = [max(0, p-reach+1),
// max(0, p+1-gap)), stored at slots p % cap.
//
// Keys are grouped by absolute position: 16-key tiles, 64-key segments (4 tiles), 256-key
// superblocks (4 segments). A segment's partial (max m, sum l, o = Σ p·v) is an online
// softmax over its tiles in order; a tile with no visible key for a column leaves that
// column's partial unchanged. Partials fold in order: segments into a superblock (inside
// one workgroup, one wave per segment), superblocks into the result (slm_attn_combine).
// Scores use the same 16x16x4 MFMA chain over dh as linear; P·V runs four MFMAs per tile
// (MFMA r takes keys r, r+4, r+8, r+12).

// v combined with lane l ^ 16 (or l ^ 32) through register lane swaps: v_permlane16_swap
// gives every lane its row pair's even-row and odd-row values (v_permlane32_swap its half
// pair's), so a symmetric op of the two is the lane's value with its partner's — the same bits
// as op(v, shfl_xor(v, 16)) for the commutative max, + and |.
__device__ __forceinline__ float xmax16(float v) {
    auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float xmax32(float v) {
    auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float xsum16(float v) {
    auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float xsum32(float v) {
    auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ int xor16i(int v) {
    auto p = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
    return (int)(p[0] | p[1]);
}
__device__ __forceinline__ int xor32i(int v) {
    auto p = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
    return (int)(p[0] | p[1]);
}

// (M, L, O) ⊕= (mB, lB, oB); an empty partial (l = 0) changes nothing.
__device__ __forceinline__ void fold(float& M, float& L, float& O, float mB, float lB,
                                     float oB) {
    if (lB == 0.0f) return;
    if (L == 0.0f) {
        M = mB;
        L = lB;
        O = oB;
        return;
    }
    float mn = fmaxf(M, mB);
    float a = expf(M - mn), b = expf(mB - mn);
    L = L * a + lB * b;
    O = O * a + oB * b;
    M = mn;
}

struct Col {
    bool valid;
    long long lo, hi;    // visible positions [lo, hi)
    long long qidx;      // query index within the call
    int head;            // query head
};

__device__ __forceinline__ Col column(int c, long long qtile, long long pos, int m,
                                      long long reach, long long gap, int group, int qpt,
                                      int kvh) {
    Col k;
    int qi = c / group, hg = c % group;
    k.qidx = qtile * qpt + qi;
    k.head = kvh * group + hg;
    k.valid = (c < qpt * group) && (k.qidx < m);
    long long p = pos + k.qidx;
    k.lo = (reach - 1 > p) ? 0 : p - (reach - 1);
    k.hi = (gap > p + 1) ? 0 : p + 1 - gap;
    if (!k.valid) k.lo = k.hi = 0;
    return k;
}

// One 64-key segment for the wave's 16 columns. The lane keeps its column's (m, l) and
// o for dims 16dt + 4g + r. The keys and values of every tile some column sees are loaded
// before any arithmetic (one memory latency per segment), both as float4 rows; each tile
// of values then goes through this wave's LDS tile `vt` ([16 keys][16·DT + 4]) into the
// layout the P·V MFMA takes.
template <int DT>
__device__ void attn_segment(const Col& col, const f4 (&qv)[DT], const float* __restrict__ kb,
                             const float* __restrict__ vb, long long seg_lo, long long cap,
                             int dh, float scale, float& mo, float& lo, f4 (&o)[DT], float* vt) {
    constexpr int VS = 16 * DT + 4;
    int lane = threadIdx.x & 63;
    int i = lane & 15, g = lane >> 4;
    mo = NEG_INF;
    lo = 0.0f;
#pragma unroll
    for (int dt = 0; dt < DT; dt++) o[dt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    bool need[4];
    f4 kr[4][DT], vq[4][DT];
#pragma unroll
    for (int st = 0; st < 4; st++) {
        long long b0 = seg_lo + 16 * st;
        bool sees = col.valid && col.lo < b0 + 16 && col.hi > b0;
        need[st] = __ballot(sees) != 0;
        if (need[st]) {
            // key and value b0 + i, dims 16t + 4g .. +3 (the scores' A operand for keys)
            long long slot = (b0 + i) % cap;
            const float* krow = kb + slot * dh;
            const float* vrow = vb + slot * dh;
#pragma unroll
            for (int t = 0; t < DT; t++) {
                int c = 16 * t + 4 * g;
                kr[st][t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
                vq[st][t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
                if (c < dh) {
                    kr[st][t] = *(const f4*)(krow + c);
                    vq[st][t] = *(const f4*)(vrow + c);
                }
            }
        }
    }
#pragma unroll
    for (int st = 0; st < 4; st++) {
        if (!need[st]) continue;
        long long b0 = seg_lo + 16 * st;
        // scores: lane holds S[key b0 + 4g + r][column i]
        f4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < DT; t++) {
            s = mfma4(kr[st][t].x, qv[t].x, s);
            s = mfma4(kr[st][t].y, qv[t].y, s);
            s = mfma4(kr[st][t].z, qv[t].z, s);
            s = mfma4(kr[st][t].w, qv[t].w, s);
        }
        // values: A operand of P·V for MFMA r is value of key b0 + 4g + r, dim 16dt + i
#pragma unroll
        for (int t = 0; t < DT; t++) *(f4*)(vt + i * VS + 16 * t + 4 * g) = vq[st][t];
        float vr[4][DT];
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int dt = 0; dt < DT; dt++) vr[r][dt] = vt[(4 * g + r) * VS + 16 * dt + i];
        float sv[4];
        bool any = false;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            long long kp = b0 + 4 * g + r;
            bool ok = kp >= col.lo && kp < col.hi;
            sv[r] = ok ? s[r] * scale : NEG_INF;
            any = any || ok;
        }
        float mx = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
        mx = xmax16(mx);
        mx = xmax32(mx);
        int anyi = any ? 1 : 0;
        anyi = xor16i(anyi);
        anyi = xor32i(anyi);
        float mnew = fmaxf(mo, mx);
        float muse = mnew == NEG_INF ? 0.0f : mnew;
        float p[4];
#pragma unroll
        for (int r = 0; r < 4; r++) p[r] = sv[r] == NEG_INF ? 0.0f : expf(sv[r] - muse);
        float rs = ((p[0] + p[1]) + p[2]) + p[3];
        rs = xsum16(rs);
        rs = xsum32(rs);
        float alpha = expf(mo - muse);
        f4 on[DT];
#pragma unroll
        for (int dt = 0; dt < DT; dt++) on[dt] = o[dt] * alpha;
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int dt = 0; dt < DT; dt++) on[dt] = mfma4(vr[r][dt], p[r], on[dt]);
        if (anyi) {
            lo = lo * alpha + rs;
            mo = mnew;
#pragma unroll
            for (int dt = 0; dt < DT; dt++) o[dt] = on[dt];
        }
    }
}

// Superblock partials. Grid (query tiles, key heads, superblock slots); SLM_SB_SEGS waves,
// wave w takes segment SLM_SB_SEGS·sb + w, where sb = floor(first visible position /
// SLM_SB_KEYS) + blockIdx.z. Output part[z][qidx][head][2 + DP]: m, l, o.
template <int DT>
__device__ void attn_part_body(float* __restrict__ part, const float* __restrict__ q,
                               const float* __restrict__ kc, const float* __restrict__ vc,
                               const long long* __restrict__ dyn, long long pos_imm, int m,
                               long long reach, long long gap, long long cap, int heads,
                               int key_heads, int dh, float scale, int wpp,
                               float* __restrict__ y, int* __restrict__ ctr) {
    constexpr int DP = 16 * DT;
    constexpr int NT = 64 * SLM_SB_SEGS;
    extern __shared__ __attribute__((aligned(16))) float lds[];  // [wpp][16][DP + 2] folds, then [waves][16][DP + 4] values
    long long pos = dyn_or(dyn, pos_imm);
    int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int i = lane & 15, g = lane >> 4;
    int group = heads / key_heads, qpt = 16 / group;
    int kvh = blockIdx.y;
    long long first = (reach - 1 > pos) ? 0 : pos - (reach - 1);
    long long sb = first / SLM_SB_KEYS + blockIdx.z;
    Col col = column(i, blockIdx.x, pos, m, reach, gap, group, qpt, kvh);
    // this lane's share of its column's query: B[k = g][j = i] for each 16-dim block
    f4 qv[DT];
    const float* qrow = q + (col.qidx * heads + col.head) * (long long)dh;
#pragma unroll
    for (int t = 0; t < DT; t++) {
        int c = 16 * t + 4 * g;
        qv[t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        if (col.valid && c < dh) qv[t] = *(const f4*)(qrow + c);
    }
    float mo, lo;
    f4 o[DT];
    float* vt = lds + wpp * 16 * (DP + 2) + wave * 16 * (DP + 4);
    attn_segment<DT>(col, qv, kc + (long long)kvh * cap * dh, vc + (long long)kvh * cap * dh,
                     (sb * SLM_SB_SEGS + wave) * 64, cap, dh, scale, mo, lo, o, vt);
    // fold the segments in order, wpp at a time through LDS
    constexpr int PER = (16 * DP + NT - 1) / NT;  // (column, dim) pairs per thread
    float FM[PER], FL[PER], FO[PER];
#pragma unroll
    for (int u = 0; u < PER; u++) {
        FM[u] = NEG_INF;
        FL[u] = 0.0f;
        FO[u] = 0.0f;
    }
    for (int ph = 0; ph < SLM_SB_SEGS; ph += wpp) {
        if (wave >= ph && wave < ph + wpp) {
            float* L = lds + ((wave - ph) * 16 + i) * (DP + 2);
#pragma unroll
            for (int dt = 0; dt < DT; dt++)
#pragma unroll
                for (int r = 0; r < 4; r++) L[2 + 16 * dt + 4 * g + r] = o[dt][r];
            if (g == 0) {
                L[0] = mo;
                L[1] = lo;
            }
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < PER; u++) {
            int t = threadIdx.x + NT * u;
            if (t < 16 * DP) {
                int cc = t / DP, dd = t % DP;
                for (int w = 0; w < wpp; w++) {
                    const float* L = lds + (w * 16 + cc) * (DP + 2);
                    fold(FM[u], FL[u], FO[u], L[0], L[1], L[2 + dd]);
                }
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int u = 0; u < PER; u++) {
        int t = threadIdx.x + NT * u;
        if (t < 16 * DP) {
            int cc = t / DP, dd = t % DP;
            Col c2 = column(cc, blockIdx.x, pos, m, reach, gap, group, qpt, kvh);
            if (c2.valid && dd < dh) {
                float* P = part + (((long long)blockIdx.z * m + c2.qidx) * heads + c2.head) *
                                      (long long)(DP + 2);
                if (ctr) {  // written through to where every workgroup's loads see it
                    if (dd == 0) {
                        __hip_atomic_store(P, FM[u], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        __hip_atomic_store(P + 1, FL[u], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                    __hip_atomic_store(P + 2 + dd, FO[u], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                } else {
                    if (dd == 0) {
                        P[0] = FM[u];
                        P[1] = FL[u];
                    }
                    P[2 + dd] = FO[u];
                }
            }
        }
    }
    if (!ctr) return;
    // The last workgroup of this (query tile, key head) to finish combines its superblocks
    // (the expressions of slm_attn_combine). Each workgroup's partial stores have completed
    // before it counts itself in; the combining workgroup reads them with loads that see
    // memory, not a stale cache line, and puts the counter back to zero for the next launch.
    __builtin_amdgcn_s_waitcnt(0);
    __shared__ int last;
    __syncthreads();
    if (threadIdx.x == 0) {
        int* c = ctr + (long long)blockIdx.x * gridDim.y + blockIdx.y;
        int before = __hip_atomic_fetch_add(c, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = before == (int)gridDim.z - 1;
        if (last) __hip_atomic_store(c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last) return;
    // one invalidate of this workgroup's stale cache lines, then ordinary loads, eight
    // superblocks in flight at a time
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    int nsb = (int)gridDim.z;
    long long stride = (long long)m * heads * (DP + 2);
#pragma unroll
    for (int u = 0; u < PER; u++) {
        int t = threadIdx.x + NT * u;
        if (t >= 16 * DP) continue;
        int cc = t / DP, dd = t % DP;
        Col c2 = column(cc, blockIdx.x, pos, m, reach, gap, group, qpt, kvh);
        if (!c2.valid || dd >= dh) continue;
        const float* P = part + (c2.qidx * heads + c2.head) * (long long)(DP + 2);
        float M = NEG_INF;
        for (int z0 = 0; z0 < nsb; z0 += 8) {
            float lz[8], mz[8];
#pragma unroll
            for (int v = 0; v < 8; v++) {  // past the last superblock: reads the last again
                int z = min(z0 + v, nsb - 1);
                lz[v] = P[z * stride + 1];
                mz[v] = P[z * stride];
            }
#pragma unroll
            for (int v = 0; v < 8; v++)
                if (z0 + v < nsb && lz[v] > 0.0f) M = fmaxf(M, mz[v]);
        }
        float L = 0.0f, O = 0.0f;
        for (int z0 = 0; z0 < nsb; z0 += 8) {
            float lz[8], mz[8], oz[8];
#pragma unroll
            for (int v = 0; v < 8; v++) {
                const float* Q = P + min(z0 + v, nsb - 1) * stride;
                lz[v] = Q[1];
                mz[v] = Q[0];
                oz[v] = Q[2 + dd];
            }
#pragma unroll
            for (int v = 0; v < 8; v++)
                if (z0 + v < nsb && lz[v] > 0.0f) {
                    float w = expf(mz[v] - M);
                    L = L + lz[v] * w;
                    O = O + oz[v] * w;
                }
        }
        float ov = L > 0.0f ? O / L : 0.0f;
        y[(c2.qidx * heads + c2.head) * (long long)dh + dd] = slm_h16 ? r16(ov) : ov;
    }
}

#define ATTN_PART(DT)                                                                    \
    KERNEL void __launch_bounds__(64 * SLM_SB_SEGS) slm_attn_part_##DT(                               \
        float* part, const float* q, const float* kc, const float* vc,                   \
        const long long* dyn, long long pos_imm, int m, long long reach, long long gap,  \
        long long cap, int heads, int key_heads, int dh, float scale, int wpp, float* y,  \
        int* ctr) {                                                                      \
        attn_part_body<DT>(part, q, kc, vc, dyn, pos_imm, m, reach, gap, cap, heads,      \
                           key_heads, dh, scale, wpp, y, ctr);                           \
    }
ATTN_PART(1)
ATTN_PART(2)
ATTN_PART(4)
ATTN_PART(8)
ATTN_PART(16)

// Prompt attention with the keys and values of a superblock shared in LDS: a workgroup of
// 16 waves takes ATTN_QG query tiles of one key head against one superblock. The waves
// first copy the superblock's keys and values into LDS (rows of 16 chunks of 16 bytes, chunk
// c at c ^ (key & 15)) — only the 16-key tiles some query of the workgroup sees, and nothing
// at all for a superblock none sees (its partials are written empty); then wave w runs
// segment w % 4 for query tile w / 4 with the arithmetic of attn_segment (operands from LDS
// instead of registers; dims at or past dh read as zero, as there). The segments of each tile
// are folded in order into superblock partials part[z][qidx][head][2 + 16·DT], which
// slm_attn_combine then combines. Grid (query tile groups, key heads, superblock slots),
// placed XCD-aware (pq_place).
#define ATTN_QG 4

// Output dim of o[dt][r] in lane (i, g) of a prompt-attention wave. With DT = 4 the P·V MFMA
// of block dt takes dims 4i + dt (A row i), so that the four values a lane needs of one key
// are one 16-byte chunk (one LDS read per key instead of four); the accumulator then holds
// dims 4·(4g + r) + dt. Each dim's chain (keys in the same order) is unchanged. DT < 4 keeps
// dims 16dt + i, as attn_segment.
template <int DT>
__device__ __forceinline__ int pq_dim(int dt, int r, int g) {
    return DT == 4 ? 4 * (4 * g + r) + dt : 16 * dt + 4 * g + r;
}

// One 16-key tile (keys 16·st .. 16·st + 15 of the segment whose rows start at kt / vt) for
// the wave's 16 columns; b0 is its first position; koff / voff are the lane's LDS offsets
// (floats) of its key chunks (t) and value rows (r) in tile 0. FULL: dh = 16·DT (no dim
// tests). A tile that every valid column sees whole takes no per-key test (the same values:
// a valid column's keys all pass, an invalid column's none); when every column is valid too,
// every lane's state updates. A rescale by α = 1 (the running maximum unchanged in every
// lane) is skipped: o·1 = o.
template <int DT, bool FULL>
__device__ __forceinline__ void pq_tile(const Col& col, bool allvalid, const f4 (&qv)[DT],
                                        const float* kt, const float* vt, const int (&koff)[DT],
                                        const int (&voff)[4], int st, long long b0, int dh,
                                        float scale, float& mo, float& lo, f4 (&o)[DT]) {
    int lane = threadIdx.x & 63;
    int i = lane & 15, g = lane >> 4;
    bool sees = col.valid && col.lo < b0 + 16 && col.hi > b0;
    if (__ballot(sees) == 0) return;
    bool whole = __ballot(col.valid && (col.lo > b0 || col.hi < b0 + 16)) == 0;
    const float* kst = kt + 1024 * st;
    const float* vst = vt + 1024 * st;
    // scores' A operand: key 16st + i of the segment, dims 16t + 4g .. +3
    f4 kr[DT];
#pragma unroll
    for (int t = 0; t < DT; t++) {
        kr[t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        if (FULL || 16 * t + 4 * g < dh) kr[t] = *(const f4*)(kst + koff[t]);
    }
    // values: MFMA r of block dt takes value of key 16st + 4g + r, dim pq_dim's A row i
    float vr[4][DT];
    if (DT == 4) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            f4 w = f4{0.0f, 0.0f, 0.0f, 0.0f};
            if (FULL || 4 * i < dh) w = *(const f4*)(vst + voff[r]);
#pragma unroll
            for (int dt = 0; dt < DT; dt++) vr[r][dt] = w[dt];
        }
    } else {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            int kv = 16 * st + 4 * g + r;
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                int dd = 16 * dt + i;
                vr[r][dt] = (FULL || dd < dh) ? vt[4 * (16 * kv + ((dd >> 2) ^ (kv & 15))) + (dd & 3)] : 0.0f;
            }
        }
    }
    f4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < DT; t++) {
        s = mfma4(kr[t].x, qv[t].x, s);
        s = mfma4(kr[t].y, qv[t].y, s);
        s = mfma4(kr[t].z, qv[t].z, s);
        s = mfma4(kr[t].w, qv[t].w, s);
    }
    float sv[4];
    int anyi;
    if (whole) {
#pragma unroll
        for (int r = 0; r < 4; r++) sv[r] = col.valid ? s[r] * scale : NEG_INF;
        anyi = col.valid ? 1 : 0;
    } else {
        bool any = false;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            long long kp = b0 + 4 * g + r;
            bool ok = kp >= col.lo && kp < col.hi;
            sv[r] = ok ? s[r] * scale : NEG_INF;
            any = any || ok;
        }
        anyi = any ? 1 : 0;
        anyi = xor16i(anyi);
        anyi = xor32i(anyi);
    }
    float mx = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
    mx = xmax16(mx);
    mx = xmax32(mx);
    float mnew = fmaxf(mo, mx);
    float muse = mnew == NEG_INF ? 0.0f : mnew;
    float p[4];
#pragma unroll
    for (int r = 0; r < 4; r++) p[r] = sv[r] == NEG_INF ? 0.0f : expf(sv[r] - muse);
    float rs = ((p[0] + p[1]) + p[2]) + p[3];
    rs = xsum16(rs);
    rs = xsum32(rs);
    float alpha = expf(mo - muse);
    if (whole && allvalid) {  // every lane updates
        if (__ballot(alpha != 1.0f) != 0) {
#pragma unroll
            for (int dt = 0; dt < DT; dt++) o[dt] = o[dt] * alpha;
        }
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int dt = 0; dt < DT; dt++) o[dt] = mfma4(vr[r][dt], p[r], o[dt]);
        lo = lo * alpha + rs;
        mo = mnew;
        return;
    }
    f4 on[DT];
#pragma unroll
    for (int dt = 0; dt < DT; dt++) on[dt] = o[dt] * alpha;
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
        for (int dt = 0; dt < DT; dt++) on[dt] = mfma4(vr[r][dt], p[r], on[dt]);
    if (anyi) {
        lo = lo * alpha + rs;
        mo = mnew;
#pragma unroll
        for (int dt = 0; dt < DT; dt++) o[dt] = on[dt];
    }
}

// Workgroups go round-robin to the eight XCDs in launch order, each XCD with its own L2: the
// workgroups L, L + 8, L + 16, ... (one XCD) take the query tile groups of one (key head,
// superblock) in turn, so those groups read its keys and values through one L2. A tail of
// the grid that does not fill whole rounds of 8 x groups keeps the plain order. (The host
// keeps the grid under 2^31 workgroups.)
__device__ __forceinline__ void pq_place(int& gx, int& kvh, int& z) {
    unsigned G = gridDim.x, Y = gridDim.y;
    unsigned L = blockIdx.x + G * (blockIdx.y + Y * blockIdx.z);
    unsigned total = G * Y * gridDim.z, full = total / (8 * G) * (8 * G), unit;
    if (L < full) {
        unsigned s = L >> 3;
        gx = (int)(s % G);
        unit = (s / G) * 8 + (L & 7);
    } else {
        gx = (int)(L % G);
        unit = L / G;
    }
    kvh = (int)(unit % Y);
    z = (int)(unit / Y);
}

// The 16-key tiles [ta, tb) of a segment starting at position sbase that meet [LO, HI).
__device__ __forceinline__ void pq_tiles(long long sbase, long long LO, long long HI, int& ta, int& tb) {
    long long a = LO <= sbase ? 0 : (LO - sbase) >> 4;
    long long b = HI <= sbase ? 0 : (HI - sbase + 15) >> 4;
    tb = (int)(b < 4 ? b : 4);
    ta = (int)(a < tb ? a : tb);
}

// With KH the rings hold fp16 values: the copies go through registers (four halves a lane,
// widened exactly, written where the fp32 copy puts them); the rest is unchanged.
template <int DT, bool FULL, bool KH = false>
__device__ void attn_pq_run(float* __restrict__ part, const float* __restrict__ q,
                            const float* __restrict__ kc, const float* __restrict__ vc,
                            long long pos, int m, long long reach, long long gap, long long cap,
                            int heads, int key_heads, int dh, float scale) {
    constexpr int DP = 16 * DT;
    constexpr int NT = 64 * SLM_SB_SEGS * ATTN_QG;
    constexpr int NC = ATTN_QG * 16;  // columns of the workgroup
    extern __shared__ __attribute__((aligned(16))) float lds[];  // keys [256][64], values [256][64]; then the fold slots
    float* kt = lds;
    float* vt = lds + SLM_SB_KEYS * 64;
    int lane = threadIdx.x & 63;
    int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int seg = wave % SLM_SB_SEGS, qt = wave / SLM_SB_SEGS;
    int i = lane & 15, g = lane >> 4;
    int group = heads / key_heads, qpt = 16 / group;
    int gx, kvh, z;
    pq_place(gx, kvh, z);
    long long first = (reach - 1 > pos) ? 0 : pos - (reach - 1);
    long long k0 = (first / SLM_SB_KEYS + z) * SLM_SB_KEYS;  // the superblock's first position
    // every position some query of the workgroup sees lies in [LO, HI)
    long long q0 = (long long)gx * ATTN_QG * qpt;
    long long q1 = ((long long)m < q0 + ATTN_QG * qpt ? (long long)m : q0 + ATTN_QG * qpt) - 1;
    long long LO = (reach - 1 > pos + q0) ? 0 : pos + q0 - (reach - 1);
    long long HI = (gap > pos + q1 + 1) ? 0 : pos + q1 + 1 - gap;
    // a superblock no query of the workgroup sees: nothing to write (slm_attn_combine reads
    // only the superblocks each row sees)
    if (HI <= LO || HI <= k0 || LO >= k0 + SLM_SB_KEYS) return;
    Col col = column(i, (long long)gx * ATTN_QG + qt, pos, m, reach, gap, group, qpt, kvh);
    // this lane's share of its column's query: B[k = g][j = i] for each 16-dim block
    f4 qv[DT];
    const float* qrow = q + (col.qidx * heads + col.head) * (long long)dh;
#pragma unroll
    for (int t = 0; t < DT; t++) {
        int c = 16 * t + 4 * g;
        qv[t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        if (col.valid && (FULL || c < dh)) qv[t] = *(const f4*)(qrow + c);
    }
    // the copies: wave w takes segment w / 4, and of each tile it copies the four keys
    // 4·(w % 4) .. +3 (one instruction, lane L: key + L/16, chunk (L % 16) ^ (key & 15); a
    // chunk at or past dh copies the row's last one, read as zero below)
    h4 hk[KH ? 4 : 1], hv[KH ? 4 : 1];
    int cs = wave >> 2, cta, ctb;
    pq_tiles(k0 + 64 * cs, LO, HI, cta, ctb);
    {
        int nch = dh >> 2;
        unsigned cap32 = (unsigned)cap;
        unsigned base = (k0 >> 32) == 0 ? (unsigned)k0 % cap32 : (unsigned)(k0 % cap);
        bool wrap1 = cap >= SLM_SB_KEYS;  // base + key < 2·cap: one subtraction wraps it
        auto where = [&](int st, int& row) {  // the element offset of this lane's chunk of tile st
            row = 64 * cs + 16 * st + 4 * (wave & 3);
            int key = row + (lane >> 4);
            int chunk = (lane & 15) ^ (key & 15);
            if (!FULL || DT < 4) chunk = min(chunk, nch - 1);  // rows hold 16 chunks
            unsigned slot = base + (unsigned)key;
            slot = wrap1 ? (slot >= cap32 ? slot - cap32 : slot) : slot % cap32;
            return (long long)slot * dh + 4 * chunk;
        };
        if constexpr (KH) {
            const _Float16* kb = (const _Float16*)kc + (long long)kvh * cap * dh;
            const _Float16* vb = (const _Float16*)vc + (long long)kvh * cap * dh;
#pragma unroll
            for (int st = 0; st < 4; st++) {
                if (st < cta || st >= ctb) continue;
                int row;
                long long off = where(st, row);
                hk[st] = gld((const h4*)(kb + off));
                hv[st] = gld((const h4*)(vb + off));
            }
        } else {
            const float* kb = kc + (long long)kvh * cap * dh;
            const float* vb = vc + (long long)kvh * cap * dh;
            for (int st = cta; st < ctb; st++) {
                int row;
                long long off = where(st, row);
                __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(kb + off),
                                                 (__attribute__((address_space(3))) void*)(kt + 64 * row), 16, 0, 0);
                __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(vb + off),
                                                 (__attribute__((address_space(3))) void*)(vt + 64 * row), 16, 0, 0);
            }
        }
    }
    bool allvalid = __ballot(col.valid) == ~0ull;
    int koff[DT], voff[4];
#pragma unroll
    for (int t = 0; t < DT; t++) koff[t] = 64 * i + 4 * ((4 * t + g) ^ i);
#pragma unroll
    for (int r = 0; r < 4; r++) voff[r] = 64 * (4 * g + r) + 4 * (i ^ (4 * g + r));
    vm_wait<0>();
    if constexpr (KH) {  // the widened halves where the fp32 copies put their rows
#pragma unroll
        for (int st = 0; st < 4; st++) {
            if (st < cta || st >= ctb) continue;
            int row = 64 * cs + 16 * st + 4 * (wave & 3);
            *(f4*)(kt + 64 * row + 4 * lane) = wide4(hk[st]);
            *(f4*)(vt + 64 * row + 4 * lane) = wide4(hv[st]);
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    float mo = NEG_INF, lo = 0.0f;
    f4 o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; dt++) o[dt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    {
        long long sbase = k0 + 64 * seg;
        int ta, tb;
        pq_tiles(sbase, LO, HI, ta, tb);
        const float* ks = kt + seg * 64 * 64;
        const float* vs = vt + seg * 64 * 64;
#pragma unroll
        for (int st = 0; st < 4; st++) {
            if (st < ta || st >= tb) continue;
            pq_tile<DT, FULL>(col, allvalid, qv, ks, vs, koff, voff, st, sbase + 16 * st, dh,
                              scale, mo, lo, o);
        }
    }
    __syncthreads();  // every wave is done with the keys and values: their LDS holds the folds
    // fold each tile's segments in order (fold()'s expressions): wave (tile, s) takes the
    // accumulator registers r = s of the tile's four segment waves, lane for lane (lane i of
    // every one of them holds column i), with the column's (m, l) of each segment
    f4* X = (f4*)lds;                                       // [wave][r][lane]: o[0..3][r]
    float2* Y = (float2*)(lds + 4 * (SLM_SB_SEGS * ATTN_QG) * 4 * 64);  // [wave][lane]: (m, l)
#pragma unroll
    for (int r = 0; r < 4; r++) {
        f4 v = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int dt = 0; dt < DT; dt++) v[dt] = o[dt][r];
        X[(wave * 4 + r) * 64 + lane] = v;
    }
    Y[wave * 64 + lane] = float2{mo, lo};
    __syncthreads();
    // (with fewer than four segment waves a tile, each takes the registers r = s, s + SEGS, ..)
    static_assert(4 % SLM_SB_SEGS == 0, "accumulator registers over the segment waves");
#pragma unroll
    for (int r = seg; r < 4; r += SLM_SB_SEGS) {
        f4 xv[SLM_SB_SEGS];
        float2 ml[SLM_SB_SEGS];
#pragma unroll
        for (int w = 0; w < SLM_SB_SEGS; w++) {
            xv[w] = X[((qt * SLM_SB_SEGS + w) * 4 + r) * 64 + lane];
            ml[w] = Y[(qt * SLM_SB_SEGS + w) * 64 + lane];
        }
        float FM = NEG_INF, FL = 0.0f;
        f4 FO = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int w = 0; w < SLM_SB_SEGS; w++) {
            float mB = ml[w].x, lB = ml[w].y;
            if (lB == 0.0f) continue;
            if (FL == 0.0f) {
                FM = mB;
                FL = lB;
                FO = xv[w];
                continue;
            }
            float mn = fmaxf(FM, mB);
            float a = expf(FM - mn), b = expf(mB - mn);
            FL = FL * a + lB * b;
#pragma unroll
            for (int dt = 0; dt < DT; dt++) FO[dt] = FO[dt] * a + xv[w][dt] * b;
            FM = mn;
        }
        if (col.valid) {
            float* P = part + (((long long)z * m + col.qidx) * heads + col.head) * (long long)(DP + 2);
            if (g == 0 && r == 0) {
                P[0] = FM;
                P[1] = FL;
            }
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                int dd = pq_dim<DT>(dt, r, g);
                if (FULL || dd < dh) P[2 + dd] = FO[dt];
            }
        }
    }
}

#define ATTN_PQ(NAME, DT, KH)                                                            \
    KERNEL void __launch_bounds__(64 * SLM_SB_SEGS * ATTN_QG) NAME(                       \
        float* part, const float* q, const float* kc, const float* vc,                   \
        const long long* dyn, long long pos_imm, int m, long long reach, long long gap,  \
        long long cap, int heads, int key_heads, int dh, float scale) {                  \
        long long pos = dyn_or(dyn, pos_imm);                                            \
        if (dh == 16 * DT)                                                               \
            attn_pq_run<DT, true, KH>(part, q, kc, vc, pos, m, reach, gap, cap, heads,    \
                                      key_heads, dh, scale);                             \
        else                                                                             \
            attn_pq_run<DT, false, KH>(part, q, kc, vc, pos, m, reach, gap, cap, heads,   \
                                       key_heads, dh, scale);                            \
    }
ATTN_PQ(slm_attn_pq_1, 1, false)
ATTN_PQ(slm_attn_pq_2, 2, false)
ATTN_PQ(slm_attn_pq_4, 4, false)
// over fp16 rings
ATTN_PQ(slm_attn_pq16_1, 1, true)
ATTN_PQ(slm_attn_pq16_2, 2, true)
ATTN_PQ(slm_attn_pq16_4, 4, true)

// One-token attention (m = 1) on the vector ALUs, with the arithmetic of slm_attn_part_*
// element for element. A 16x16x4 f32 MFMA step is, bit for bit, fmaf over k = 0..3 in
// order (denormals kept), so a score is the fmaf chain from 0 over dims 16t + 4g + c with t,
// then c, then g outermost to innermost, and an output dim is o·α followed by the fmaf chain
// over the keys 4g + r of a 16-key tile, r outer and g inner; the tile softmax, the row-sum
// order ((p0 + p1) + p2) + p3 per four keys then (s0 + s1) + (s2 + s3), the segment fold and
// the superblock combine are the same expressions. Dims at or past dh, zero in both operands
// there, leave a chain unchanged and are skipped. Grid (key heads, superblock slots);
// SLM_SB_SEGS waves, wave w takes segment w of superblock sb. Each wave copies its segment's
// 64 keys and values into its own LDS (rows of 16 chunks of 16 bytes, chunk c at position
// c ^ (key & 15), so one chunk of sixteen keys and one row of sixteen chunks both fall on
// distinct banks), scores one key per lane and accumulates one output dim per lane.
// Output: part[z][0][head][2 + 16·DT], as slm_attn_part_*; with `ctr` the last workgroup of
// a key head combines the superblocks into y (its partials fit in LDS: the host checks).
#define ADEC_WAVE_FLOATS (2 * 64 * 64 + 1024)  // a wave's LDS: keys [64][64], values [64][64], queries
// With KH the rings hold fp16 values (fp16 mode's caches): each lane loads its four halves of
// a chunk into registers and writes them, widened exactly, where the copy would have put the
// floats; everything after the staging is the fp32 kernel's.
template <int DT, bool KH = false, bool STEP = false>
__device__ __forceinline__ bool attn_dec_body(float* __restrict__ part, const float* __restrict__ q,
                              const float* __restrict__ kc, const float* __restrict__ vc,
                              const long long* __restrict__ dyn, long long pos_imm,
                              long long reach, long long gap, long long cap, int heads,
                              int key_heads, int dh, float scale, float* __restrict__ y,
                              int* __restrict__ ctr, int bx, int by, int ny, int tid,
                                              const StepWait* sw = nullptr, int* gave = nullptr) {
    static_assert(!(STEP && KH), "a step phase reads fp32 rings");
    static_assert(DT >= 1 && DT <= 4, "one-token attention: head size at most 64");
    constexpr int DP = 16 * DT;
    extern __shared__ __attribute__((aligned(16))) float lds[];
    int lane = tid & 63;
    int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int group = heads / key_heads, kvh = bx;
    int nch = dh >> 2;  // 16-byte chunks per row
    // Ring order, for a ring of exactly ny superblocks (cap = 256·ny, not as a step phase):
    // workgroup y takes ring slots 256y .. 256y + 255, which hold the one superblock
    // sb ≡ y (mod ny) of the span's ny consecutive ones, so its copies need no position and
    // go out before the position is read; its partial goes to that superblock's place zb in
    // position order. Otherwise workgroup y takes superblock y of the span.
    const bool ring = !STEP && cap == (long long)ny * SLM_SB_KEYS;
    long long pos = 0, sb = 0, seg_lo = 0;
    int zb = by;
    auto at_pos = [&]() {
        pos = dyn_or(dyn, pos_imm);
        long long first = (reach - 1 > pos) ? 0 : pos - (reach - 1);
        long long fsb = first / SLM_SB_KEYS;
        if (ring) zb = (int)((by + ny - fsb % ny) % ny);
        sb = fsb + zb;
        seg_lo = (sb * SLM_SB_SEGS + wave) * 64;
    };
    if (!ring) at_pos();
    constexpr unsigned ES = KH ? 2u : 4u;  // bytes per ring element
    const char* kb = (const char*)kc + (long long)kvh * cap * dh * ES;
    const char* vb = (const char*)vc + (long long)kvh * cap * dh * ES;
    float* kt = lds + wave * ADEC_WAVE_FLOATS;  // keys; then p and the fold slots
    float* vt = kt + 64 * 64;                    // values
    float* qt = vt + 64 * 64;                    // the key head's queries [group][dh]
    // the copies, queries first: the group's query rows are contiguous (one token), 64
    // chunks per instruction (a lane past the end copies the last chunk into unused LDS)
    int nqc = (group * dh) >> 2;
    const float* qg = q + (long long)kvh * group * dh;
    auto copy_q = [&]() {
        for (int k = 0; k < (nqc + 63) / 64; k++) {
            int ch = min(64 * k + lane, nqc - 1);
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(qg + 4 * ch),
                                             (__attribute__((address_space(3))) void*)(qt + 256 * k), 16, 0, STEP ? 16 : 0);
        }
    };
    if (!STEP) copy_q();
    // keys, then values: instruction k covers keys 4k .. 4k+3; lane L takes key 4k + L/16 and
    // puts chunk (L % 16) ^ (key & 15) of its row at position L % 16 (a chunk at or past dh
    // copies the row's last one: it is never read). Key 4k + g is ring slot (seg_lo + 4k + g)
    // mod cap; with cap >= 64 each step of four keys wraps at most once, and a key head's
    // ring is under 4 GB, so byte offsets are 32-bit (the host checks both).
    // (the offsets are worked out again for the values: sixteen registers fewer held)
    unsigned rowb = (unsigned)dh * ES, wrapb = (unsigned)cap * rowb;
    unsigned slot = ring ? (unsigned)(by * SLM_SB_KEYS + wave * 64) + (unsigned)(lane >> 4)
                         : (unsigned)(seg_lo % cap) + (unsigned)(lane >> 4);
    if (slot >= (unsigned)cap) slot -= (unsigned)cap;  // (never in ring order)
    const unsigned roff0 = slot * rowb;
    auto off_of = [&](int k, unsigned roff) {
        int key = 4 * k + (lane >> 4);
        return roff + 4u * ES * (unsigned)min((lane & 15) ^ (key & 15), nch - 1);
    };
    h4 hk[KH ? 16 : 1], hv[KH ? 16 : 1];
    if constexpr (KH) {  // four halves per lane per instruction, into registers
        unsigned roff = roff0;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            hk[k] = __builtin_nontemporal_load((const GAS h4*)(kb + off_of(k, roff)));
            roff += 4 * rowb;
            if (roff >= wrapb) roff -= wrapb;
        }
        roff = roff0;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            hv[k] = __builtin_nontemporal_load((const GAS h4*)(vb + off_of(k, roff)));
            roff += 4 * rowb;
            if (roff >= wrapb) roff -= wrapb;
        }
    } else {
        // (non-temporal: the keys and values are read once per token, and should not push
        // this kernel's code and the partials out of L2)
        unsigned roff = roff0;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(kb + off_of(k, roff)),
                                             (__attribute__((address_space(3))) void*)(kt + 256 * k), 16, 0, 2);
            roff += 4 * rowb;
            if (roff >= wrapb) roff -= wrapb;
        }
        roff = roff0;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(vb + off_of(k, roff)),
                                             (__attribute__((address_space(3))) void*)(vt + 256 * k), 16, 0, 2);
            roff += 4 * rowb;
            if (roff >= wrapb) roff -= wrapb;
        }
    }
    if (ring) {
        asm volatile("" ::: "memory");  // (the position is read after the copies are out)
        at_pos();
    }
    if constexpr (STEP) {
        // As a step phase the copies above went out before the wait for the QKV phase: the
        // ring held everything but the newest key and value then. After the wait, the queries
        // and that one slot (copied again, device scope, over its first copy: a wave's copies
        // land in order) — in the wave whose segment holds the position.
        if (step_wait_wg(*sw, gave, tid)) return false;
        copy_q();
        long long kidx = pos - seg_lo;
        if (kidx >= 0 && kidx < 64 && (int)(kidx & 3) == (lane >> 4)) {
            int k = (int)(kidx >> 2);
            unsigned r = roff0 + (unsigned)k * 4u * rowb;
            if (r >= wrapb) r -= wrapb;
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(kb + off_of(k, r)),
                                             (__attribute__((address_space(3))) void*)(kt + 256 * k), 16, 0, 18);
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(vb + off_of(k, r)),
                                             (__attribute__((address_space(3))) void*)(vt + 256 * k), 16, 0, 18);
        }
        vm_wait<0>();
    } else {
        vm_wait<16>();  // the queries and keys are in (the values may still be on their way)
    }
    asm volatile("" ::: "memory");
    if constexpr (KH) {  // the keys, widened, where the copies put fp32 rows
#pragma unroll
        for (int k = 0; k < 16; k++) *(f4*)(kt + 256 * k + 4 * lane) = wide4(hk[k]);
    }
    // this lane's key: dims 16t + 4g .. +3 as kr[t][g], in registers before anything is
    // written over the keys (the p tile and the fold slots below take their first rows). As
    // a step phase (fewer registers: a quarter of the CU's each), the scores of every query
    // column (at most SLM_STEP_GROUP) instead, one dim tile of the key at a time: each
    // column's chain runs over t, e, g in the same order.
    int j = lane;
    f4 kr[STEP ? 1 : DT][4];
    float sc[SLM_STEP_GROUP];
    if constexpr (STEP) {
#pragma unroll
        for (int c = 0; c < SLM_STEP_GROUP; c++) sc[c] = 0.0f;
#pragma unroll
        for (int t = 0; t < DT; t++) {
            f4 kt4[4];
#pragma unroll
            for (int g = 0; g < 4; g++) kt4[g] = *(const f4*)(kt + 4 * (16 * j + ((4 * t + g) ^ (j & 15))));
#pragma unroll
            for (int c = 0; c < SLM_STEP_GROUP; c++) {
                if (c >= group) break;
                f4 qv[4];
#pragma unroll
                for (int g = 0; g < 4; g++) qv[g] = *(const f4*)(qt + c * dh + min(16 * t + 4 * g, dh - 4));
#pragma unroll
                for (int e = 0; e < 4; e++)
#pragma unroll
                    for (int g = 0; g < 4; g++)
                        if (16 * t + 4 * g < dh) sc[c] = fmaf(kt4[g][e], qv[g][e], sc[c]);
            }
        }
    } else {
#pragma unroll
        for (int t = 0; t < DT; t++)
#pragma unroll
            for (int g = 0; g < 4; g++) kr[t][g] = *(const f4*)(kt + 4 * (16 * j + ((4 * t + g) ^ (j & 15))));
    }
    long long kp = seg_lo + j;
    float* pt = kt;             // p of the current tile [16], over the keys once read
    float* fs = kt + 64;        // fold slots [group][DP + 2]
    // value reads of one output dim: key 4g + r of a tile is at row offset
    // 4·(16·(4g + r) + ((d / 4) ^ (4g + r))) + d % 4 from the tile's first row
    int d = lane, dc = d >> 2, dw = d & 3;
    int va[16];
#pragma unroll
    for (int kk = 0; kk < 16; kk++) va[kk] = 4 * (16 * kk + (dc ^ kk)) + dw;
    bool vwait = true;
    for (int c = 0; c < group; c++) {
        Col col = column(c, 0, pos, 1, reach, gap, group, 16 / group, kvh);
        float s = 0.0f;
        if constexpr (STEP) {
            s = sc[0];
#pragma unroll
            for (int q = 1; q < SLM_STEP_GROUP; q++)
                if (c == q) s = sc[q];
        } else {
#pragma unroll
            for (int t = 0; t < DT; t++) {
                f4 qv[4];  // the query's dims of tile t (the same for every lane: LDS broadcast)
#pragma unroll
                for (int g = 0; g < 4; g++) qv[g] = *(const f4*)(qt + c * dh + min(16 * t + 4 * g, dh - 4));
#pragma unroll
                for (int e = 0; e < 4; e++)
#pragma unroll
                    for (int g = 0; g < 4; g++)
                        if (16 * t + 4 * g < dh) s = fmaf(kr[t][g][e], qv[g][e], s);
            }
        }
        bool ok = kp >= col.lo && kp < col.hi;
        float sv = ok ? s * scale : NEG_INF;
        float tm = sv;  // tile maxima
        tm = fmaxf(tm, __shfl_xor(tm, 1));
        tm = fmaxf(tm, __shfl_xor(tm, 2));
        tm = fmaxf(tm, __shfl_xor(tm, 4));
        tm = fmaxf(tm, __shfl_xor(tm, 8));
        unsigned long long okm = __ballot(ok);
        if (vwait) {  // the values are in
            vm_wait<0>();
            asm volatile("" ::: "memory");
            if constexpr (KH) {
#pragma unroll
                for (int k = 0; k < 16; k++) *(f4*)(vt + 256 * k + 4 * lane) = wide4(hv[k]);
            }
            vwait = false;
        }
        // tile by tile: the running maximum and α of the MFMA path (uniform), this tile's p,
        // then one output dim per lane
        float mo = NEG_INF, lo = 0.0f, o = 0.0f;
#pragma unroll 1
        for (int st = 0; st < 4; st++) {
            float mx = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(tm), 16 * st));
            bool any = ((okm >> (16 * st)) & 0xffffull) != 0;
            float mnew = fmaxf(mo, mx);
            float muse = mnew == NEG_INF ? 0.0f : mnew;
            float alpha = expf(mo - muse);
            if (!any) continue;
            if ((j >> 4) == st) pt[j & 15] = sv == NEG_INF ? 0.0f : expf(sv - muse);
            float p[16];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                f4 pv = *(const f4*)(pt + 4 * u);
                p[4 * u] = pv.x;
                p[4 * u + 1] = pv.y;
                p[4 * u + 2] = pv.z;
                p[4 * u + 3] = pv.w;
            }
            float r0 = ((p[0] + p[1]) + p[2]) + p[3], r1 = ((p[4] + p[5]) + p[6]) + p[7];
            float r2 = ((p[8] + p[9]) + p[10]) + p[11], r3 = ((p[12] + p[13]) + p[14]) + p[15];
            float rs = (r0 + r1) + (r2 + r3);
            const float* vrow = vt + 1024 * st;
            float on = o * alpha;
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int g = 0; g < 4; g++) on = fmaf(vrow[va[4 * g + r]], p[4 * g + r], on);
            lo = lo * alpha + rs;
            mo = mnew;
            o = on;
            // the next tile's p overwrites this one's only after every lane has read it
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        }
        float* F = fs + c * (DP + 2);
        if (d < dh) F[2 + d] = o;
        if (lane == 0) {
            F[0] = mo;
            F[1] = lo;
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    __syncthreads();
    // fold the four segments in order, one (column, dim) per thread
    for (int t = tid; t < group * DP; t += 64 * SLM_SB_SEGS) {
        int cc = t / DP, dd = t % DP;
        if (dd >= dh) continue;
        float FM = NEG_INF, FL = 0.0f, FO = 0.0f;
#pragma unroll
        for (int w = 0; w < SLM_SB_SEGS; w++) {
            const float* F = lds + w * ADEC_WAVE_FLOATS + 64 + cc * (DP + 2);
            fold(FM, FL, FO, F[0], F[1], F[2 + dd]);
        }
        int head = kvh * group + cc;
        float* P = part + ((long long)zb * heads + head) * (long long)(DP + 2);
        if (ctr || STEP) {  // written through to where every workgroup's loads see it
            if (dd == 0) {
                __hip_atomic_store(P, FM, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(P + 1, FL, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            __hip_atomic_store(P + 2 + dd, FO, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            if (dd == 0) {
                P[0] = FM;
                P[1] = FL;
            }
            P[2 + dd] = FO;
        }
    }
    if (!ctr) return true;
    // the last workgroup of this key head combines the superblocks (slm_attn_combine's
    // expressions) from a copy of every partial in LDS, read in one pass
    __builtin_amdgcn_s_waitcnt(0);
    __shared__ int last;
    __syncthreads();
    if (tid == 0) {
        int* cp = ctr + bx;
        int before = __hip_atomic_fetch_add(cp, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = before == ny - 1;
        if (last) __hip_atomic_store(cp, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last) return true;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    // the key head's slots are group·(DP + 2) contiguous floats per superblock; thread f of a
    // pass takes float f mod 2^sh of slot f / 2^sh (2^sh: that count rounded up to a power of 2)
    int nsb = ny, sr = group * (DP + 2);
    int sh = 32 - __clz(sr - 1);
    int nf = nsb << sh;
    for (int b = 0; b < nf; b += 8 * 64 * SLM_SB_SEGS) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            int f = b + tid + u * 64 * SLM_SB_SEGS;
            int z = min(f >> sh, nsb - 1), e = min(f & ((1 << sh) - 1), sr - 1);
            v[u] = part[((long long)z * heads + kvh * group) * (DP + 2) + e];
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            int f = b + tid + u * 64 * SLM_SB_SEGS;
            int z = f >> sh, e = f & ((1 << sh) - 1);
            if (z < nsb && e < sr) lds[z * sr + e] = v[u];
        }
    }
    __syncthreads();
    for (int t = tid; t < group * DP; t += 64 * SLM_SB_SEGS) {
        int cc = t / DP, dd = t % DP;
        if (dd >= dh) continue;
        const float* P = lds + cc * (DP + 2);
        float M = NEG_INF;
        for (int z0 = 0; z0 < nsb; z0 += 8) {
            float lz[8], mz[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {  // past the last superblock: reads the last again
                int z = min(z0 + u, nsb - 1);
                lz[u] = P[z * sr + 1];
                mz[u] = P[z * sr];
            }
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (z0 + u < nsb && lz[u] > 0.0f) M = fmaxf(M, mz[u]);
        }
        float L = 0.0f, O = 0.0f;
        for (int z0 = 0; z0 < nsb; z0 += 8) {
            float lz[8], mz[8], oz[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const float* Q = P + min(z0 + u, nsb - 1) * sr;
                lz[u] = Q[1];
                mz[u] = Q[0];
                oz[u] = Q[2 + dd];
            }
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (z0 + u < nsb && lz[u] > 0.0f) {
                    float w = expf(mz[u] - M);
                    L = L + lz[u] * w;
                    O = O + oz[u] * w;
                }
        }
        float ov = L > 0.0f ? O / L : 0.0f;
        y[(long long)(kvh * group + cc) * dh + dd] = slm_h16 ? r16(ov) : ov;
    }
    return true;
}

#define ATTN_DEC(NAME, DT, KH)                                                           \
    KERNEL void __launch_bounds__(64 * SLM_SB_SEGS) NAME(                                 \
        float* part, const float* q, const float* kc, const float* vc,                   \
        const long long* dyn, long long pos_imm, long long reach, long long gap,         \
        long long cap, int heads, int key_heads, int dh, float scale, float* y,          \
        int* ctr) {                                                                      \
        attn_dec_body<DT, KH>(part, q, kc, vc, dyn, pos_imm, reach, gap, cap, heads,      \
                              key_heads, dh, scale, y, ctr, blockIdx.x, blockIdx.y,      \
                              gridDim.y, threadIdx.x);                                   \
    }
ATTN_DEC(slm_attn_dec_1, 1, false)
ATTN_DEC(slm_attn_dec_2, 2, false)
ATTN_DEC(slm_attn_dec_4, 4, false)
// over fp16 rings
ATTN_DEC(slm_attn_dec16_1, 1, true)
ATTN_DEC(slm_attn_dec16_2, 2, true)
ATTN_DEC(slm_attn_dec16_4, 4, true)

// y[qidx][head][dim] from the nsb superblock partials: with M the largest m of the
// superblocks that saw a key, w_z = e^(m_z − M), L = Σ l_z·w_z and O = Σ o_z·w_z (both in
// superblock order), y = O / L (0 when the query sees nothing, cpu.rs:378-382). The last
// workgroup of an attention launch that combines itself computes the same expressions.
KERNEL void __launch_bounds__(256) slm_attn_combine(float* __restrict__ y, const float* __restrict__ part, int m,
                             int heads, int dh, int dp, int nsb, const long long* dyn,
                             long long pos_imm, long long reach, long long gap) {
    // one wave per (query, head) row: lane z holds superblock z's m and l (64 at a time),
    // lane d the o values of dim d of every superblock, all loads of a batch in flight.
    // With reach > 0 only the superblocks the row's query sees are read (the others have
    // l = 0, which the sums skip; the prompt attention does not write them).
    int lane = threadIdx.x & 63;
    long long rw = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (rw >= (long long)m * heads) return;
    int zlo = 0, zhi = nsb;
    if (reach > 0) {
        long long pos = dyn_or(dyn, pos_imm), p = pos + rw / heads;
        long long lo = reach - 1 > p ? 0 : p - (reach - 1), hi = gap > p + 1 ? 0 : p + 1 - gap;
        long long fb = (reach - 1 > pos ? 0 : pos - (reach - 1)) / SLM_SB_KEYS;
        long long a = lo / SLM_SB_KEYS - fb, b = hi > lo ? (hi - 1) / SLM_SB_KEYS - fb + 1 : 0;
        zlo = (int)(a > 0 ? a : 0);
        zhi = (int)(b < nsb ? b : nsb);
        if (zhi < zlo) zhi = zlo;
    }
    const float* P = part + rw * (dp + 2);
    long long stride = (long long)m * heads * (dp + 2);
    float M = NEG_INF;
    for (int z0 = zlo; z0 < zhi; z0 += 64) {
        int z = z0 + lane;
        float mz = z < zhi ? P[z * stride] : NEG_INF, lz = z < zhi ? P[z * stride + 1] : 0.0f;
        float mm = lz > 0.0f ? mz : NEG_INF;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) mm = fmaxf(mm, __shfl_xor(mm, off));
        M = fmaxf(M, mm);
    }
    for (int d0 = 0; d0 < dh; d0 += 64) {
        int dd = d0 + lane;
        float L = 0.0f, O = 0.0f;
        for (int z0 = zlo; z0 < zhi; z0 += 64) {
            int z = z0 + lane;
            float mz = z < zhi ? P[z * stride] : NEG_INF, lz = z < zhi ? P[z * stride + 1] : 0.0f;
            float wz = lz > 0.0f ? expf(mz - M) : 0.0f;  // lane z: superblock z's weight
            int nz = min(64, zhi - z0);
            for (int u0 = 0; u0 < nz; u0 += 16) {
                float oz[16];
#pragma unroll
                for (int u = 0; u < 16; u++) {  // past the last superblock: reads the last again
                    int zz = z0 + min(u0 + u, nz - 1);
                    oz[u] = dd < dh ? P[zz * stride + 2 + dd] : 0.0f;
                }
#pragma unroll
                for (int u = 0; u < 16; u++) {
                    if (u0 + u >= nz) break;
                    float l = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lz), u0 + u));
                    float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wz), u0 + u));
                    if (l > 0.0f) {
                        L = L + l * w;
                        O = O + oz[u] * w;
                    }
                }
            }
        }
        float ov = L > 0.0f ? O / L : 0.0f;
        if (dd < dh) y[rw * dh + dd] = slm_h16 ? r16(ov) : ov;
    }
}

// ---------------------------------------------------------------------------------------
// diagnostics
// ---------------------------------------------------------------------------------------

// One 16x16x4 MFMA: lane l passes a[l], b[l] and writes D's four elements to out[4l..].
KERNEL void slm_probe_mfma(float* out, const float* a, const float* b) {
    int l = threadIdx.x & 63;
    f4 d = mfma4(a[l], b[l], f4{0.0f, 0.0f, 0.0f, 0.0f});
    for (int r = 0; r < 4; r++) out[4 * l + r] = d[r];
}

// ---------------------------------------------------------------------------------------
// fused decode kernels (one token), driven by the descriptors of fusion.h
// ---------------------------------------------------------------------------------------

// The prologue waves' own barrier: a counter in LDS that each of the `nw` waves bumps once
// per barrier, then waits for (the GEMV waves meanwhile wait for their weights, not for
// this). Only LDS is ordered by it. The wait gives up after `spin` polls (about a second at
// the default), so a mistake cannot hang the GPU.
// Returns whether the wait gave up.
__device__ __forceinline__ bool esync(int* ctr, int& target, int nw, int spin, int* fault) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    target += nw;
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    int it = 0;
    for (; it < spin; it++) {
        if (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= target) break;
    }
    bool gave_up = it >= spin;
    if (gave_up) wait_gave_up(fault, threadIdx.x & 63);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    return gave_up;
}

// `failed` records that one of this wave's waits gave up: from then on what other waves
// should have written to LDS before the barrier (the descriptor copy among it) may be
// missing, so the caller stops using it.
struct ESync {
    int* ctr;
    int target, nw, spin;
    int* fault;
    bool failed = false;
    __device__ __forceinline__ void operator()() { failed |= esync(ctr, target, nw, spin, fault); }
};

// Sum of squares of in[0..size) in the order of dot16_self, run by one wave: lane l and
// lane l + 16k keep the same running sum of elements l, l + 16, ... (sixteen loads in
// flight), then the sixteen sums are added left to right (a DPP scan along each row of
// sixteen lanes), and every lane returns the total.
__device__ float dot16_wave(const float* in, int size, int lane) {
    int l = lane & 15;
    int chunks = size / 16;
    float acc = 0.0f;
    int c = 0;
    for (; c + 16 <= chunks; c += 16) {
        float v[16];
#pragma unroll
        for (int u = 0; u < 16; u++) v[u] = in[(c + u) * 16 + l];
#pragma unroll
        for (int u = 0; u < 16; u++) acc = acc + v[u] * v[u];
    }
    for (; c < chunks; c++) {
        float v = in[c * 16 + l];
        acc = acc + v * v;
    }
    // ((-0.0 + acc_0) + acc_1) + ... + acc_15 as a scan along each row of sixteen lanes: at
    // step k lane l adds its own sum to what lane l - 1 held, so after step k lanes 0..k
    // hold their final prefix sums (lane 0 adds to the zero its missing neighbour reads,
    // which equals -0.0 + acc_0 since acc_0 is never -0.0); lane 15 ends with the total.
    float s = acc;
#pragma unroll
    for (int k = 1; k < 16; k++) {
        float prev = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x111, 0xf, 0xf, true));
        s = prev + acc;
    }
    s = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 15));
    float tail = -0.0f;
    for (int j = chunks * 16; j < size; j++) tail = tail + in[j] * in[j];
    return s + tail;
}

// The prologue's element-wise ops, one loop per kind so each compiles to its own
// straight-line code (the expressions of the per-op kernels). Every lane reads all its
// float4s of a 1024-element chunk before it writes any.
// (H: fp16 mode's roundings, the e_* expressions)
template <int KIND, bool H = false>
__device__ __forceinline__ float vp_elem(float a, float b, float f, float r) {
    if (KIND == VP_COPY) return a;
    if (KIND == VP_ADD) return e_add<H>(a, b);
    if (KIND == VP_MIX) return e_mix<H>(a, b, f);
    if (KIND == VP_SCALE) return e_scale<H>(a, f);
    if (KIND == VP_RMS) return e_rms<H>(a, r, b);  // b: the rms weight
    return e_silu<H>(a, b);                        // VP_SILU: g = a, u = b
}

template <int KIND, bool H>
__device__ __forceinline__ void vp_map4(const f4* a, const f4* b, f4* out, int n4, float f,
                                        float r, int tid, int nt) {
    for (int c0 = tid; c0 < n4; c0 += 4 * nt) {
        f4 A[4], B[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {  // past the end: reads the last float4 again
            int c = min(c0 + nt * j, n4 - 1);
            A[j] = a[c];
            if (KIND != VP_COPY && KIND != VP_SCALE) B[j] = b[c];
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            int c = c0 + nt * j;
            if (c >= n4) break;
            f4 v;
#pragma unroll
            for (int e = 0; e < 4; e++) v[e] = vp_elem<KIND, H>(A[j][e], B[j][e], f, r);
            out[c] = v;
        }
    }
}

template <int KIND, bool H>
__device__ __forceinline__ void vp_map1(const float* a, const float* b, float* out, int n,
                                        float f, float r, int tid, int nt) {
    for (int c0 = tid; c0 < n; c0 += 4 * nt) {
        float A[4], B[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            int c = min(c0 + nt * j, n - 1);
            A[j] = a[c];
            if (KIND != VP_COPY && KIND != VP_SCALE) B[j] = b[c];
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            int c = c0 + nt * j;
            if (c >= n) break;
            out[c] = vp_elem<KIND, H>(A[j], B[j], f, r);
        }
    }
}

template <int KIND, bool H>
__device__ __forceinline__ void vp_map(const float* a, const float* b, float* out, int n,
                                       bool v4, float f, float r, int tid, int nt) {
    if (v4) vp_map4<KIND, H>((const f4*)a, (const f4*)b, (f4*)out, n >> 2, f, r, tid, nt);
    else vp_map1<KIND, H>(a, b, out, n, f, r, tid, nt);
}

// slm_fold in LDS: out[c] = ((P0[c] + P1[c]) + P2[c]) + ..., parts [nsplit][n]; all the
// splits of a float4 are read before the sums.
template <bool H>
__device__ __forceinline__ void vp_fold(const float* part, float* out, int n, int nsplit,
                                        bool v4, int tid, int nt) {
    constexpr int ZMAX = 8;
    if (v4 && nsplit <= ZMAX) {
        int n4 = n >> 2;
        const f4* p4 = (const f4*)part;
        for (int c0 = tid; c0 < n4; c0 += 2 * nt) {
            f4 P[2][ZMAX];
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int z = 0; z < ZMAX; z++)
                    if (z < nsplit) P[j][z] = p4[z * n4 + min(c0 + nt * j, n4 - 1)];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                int c = c0 + nt * j;
                if (c >= n4) break;
                f4 v = P[j][0];
#pragma unroll
                for (int z = 1; z < ZMAX; z++)
                    if (z < nsplit) v = v + P[j][z];
#pragma unroll
                for (int e = 0; e < 4; e++) v[e] = h16<H>(v[e]);
                ((f4*)out)[c] = v;
            }
        }
        return;
    }
    for (int c = tid; c < n; c += nt) {
        float v = part[c];
        for (int z = 1; z < nsplit; z++) v = v + part[z * n + c];
        out[c] = h16<H>(v);
    }
}

// slm_attn_combine for one token in LDS, part [nsb][heads][dp + 2] (m, l, o per superblock
// and head) into out [heads][dh], in two passes with a barrier between them (the same
// expressions, so the same bits). First, one thread per (head, superblock z): M = the
// largest m of the head's superblocks that saw a key, w_z = e^(m_z − M), and the pair
// (w_z, l_z·w_z) into wl [heads][nsb] (w_z = −1: superblock z saw no key, it is skipped).
__device__ void vp_comb_w(const float* part, float2* wl, int heads, int dp, int nsb, int tid, int nt) {
    int sr = heads * (dp + 2);
    for (int p = tid; p < heads * nsb; p += nt) {
        int h = p / nsb, z = p - h * nsb;
        const float* P = part + h * (dp + 2);
        float M = NEG_INF;
        for (int z0 = 0; z0 < nsb; z0 += 8) {
            float2 ml[8];
#pragma unroll
            for (int u = 0; u < 8; u++) ml[u] = *(const float2*)(P + min(z0 + u, nsb - 1) * sr);
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (z0 + u < nsb && ml[u].y > 0.0f) M = fmaxf(M, ml[u].x);
        }
        float2 me = *(const float2*)(P + z * sr);
        float w = expf(me.x - M);
        wl[p] = me.y > 0.0f ? float2{w, me.y * w} : float2{-1.0f, 0.0f};
    }
}

// Then DW dims per thread: L = Σ l_z·w_z and O = Σ o_z·w_z in superblock order,
// out = O / L (0 when no superblock saw a key).
template <int DW, bool H>
__device__ void vp_comb_o(const float* part, const float2* wl, float* out, int heads, int dh,
                          int dp, int nsb, int tid, int nt) {
    int nq = dh / DW, sr = heads * (dp + 2);
    for (int q = tid; q < heads * nq; q += nt) {
        int h = q / nq, d0 = (q - h * nq) * DW;
        const float* P = part + h * (dp + 2) + 2 + d0;
        const float2* WL = wl + h * nsb;
        float L = 0.0f, O[DW];
#pragma unroll
        for (int e = 0; e < DW; e++) O[e] = 0.0f;
        for (int z0 = 0; z0 < nsb; z0 += 8) {
            float2 wz[8];
            float oz[8][DW];
#pragma unroll
            for (int u = 0; u < 8; u++) {  // past the last superblock: reads the last again
                int z = min(z0 + u, nsb - 1);
                wz[u] = WL[z];
                if (DW == 4) {
                    float2 a = *(const float2*)(P + z * sr), b = *(const float2*)(P + z * sr + 2);
                    oz[u][0] = a.x;
                    oz[u][1] = a.y;
                    oz[u][DW > 2 ? 2 : 0] = b.x;
                    oz[u][DW > 3 ? 3 : 0] = b.y;
                } else {
#pragma unroll
                    for (int e = 0; e < DW; e++) oz[u][e] = P[z * sr + e];
                }
            }
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (z0 + u < nsb && wz[u].x >= 0.0f) {
                    L = L + wz[u].y;
#pragma unroll
                    for (int e = 0; e < DW; e++) O[e] = O[e] + oz[u][e] * wz[u].x;
                }
        }
#pragma unroll
        for (int e = 0; e < DW; e++) out[h * dh + d0 + e] = h16<H>(L > 0.0f ? O[e] / L : 0.0f);
    }
}

// Whether an op runs on float4s: its length and every vector offset a multiple of four.
__device__ __forceinline__ bool vp_v4(const VpOp& o) {
    return ((o.in0 | (o.in1 >= 0 ? o.in1 : 0) | (o.out >= 0 ? o.out : 0) | (o.w >= 0 ? o.w : 0) |
             o.n) & 3) == 0;
}

__device__ __forceinline__ int uni(int x) { return __builtin_amdgcn_readfirstlane(x); }

// An op read from the descriptor in LDS, its fields made wave-uniform (they are), so its
// tests compile to scalar branches.
__device__ __forceinline__ VpOp vp_load(const VpOp& src) {
    VpOp o = src;
    o.kind = uni(o.kind);
    o.n = uni(o.n);
    o.wg0 = uni(o.wg0);
    o.out = uni(o.out);
    o.in0 = uni(o.in0);
    o.in1 = uni(o.in1);
    o.w = uni(o.w);
    o.nsb = uni(o.nsb);
    o.heads = uni(o.heads);
    o.dh = uni(o.dh);
    o.dp = uni(o.dp);
    o.sync = uni(o.sync);
    o.f = __int_as_float(uni(__float_as_int(o.f)));
    return o;
}

// One prologue operation on LDS vectors, run by the prologue waves (thread tid of nt)
// while the GEMV waves' weights stream in. Thread tid owns float4s (or, for an op that is
// not float4-aligned, elements) tid, tid + nt, ... of every vector, so an element-wise op
// that reads what an earlier op of the same kind of layout wrote needs no barrier; the
// caller puts one before an op that reads other threads' elements. rms sums the whole
// input in every wave (the same sum), so its factor needs no barrier either. `f` is the
// op's factor (the dynamic one of a VP_SCALE already read).
// The common case of vp_run, with fewer instructions on the critical path: a float4 op
// whose vectors hold at most one float4 per thread (thread tid owns float4 tid, as in
// vp_map4), so each thread reads its operands once, computes the expressions of vp_elem /
// vp_fold / rms and writes once.
template <int NSPLIT, bool H>
__device__ __forceinline__ f4 vp_fold4(const f4* p, int n4, int c) {
    f4 P[NSPLIT];
#pragma unroll
    for (int z = 0; z < NSPLIT; z++) P[z] = p[z * n4 + c];
    f4 v = P[0];
#pragma unroll
    for (int z = 1; z < NSPLIT; z++) v = v + P[z];
#pragma unroll
    for (int e = 0; e < 4; e++) v[e] = h16<H>(v[e]);
    return v;
}

// The fields of a prologue op that the float4 path reads, made wave-uniform.
struct VpFast {
    int n4, out, in0, in1, w, nsb, sync, wg0;
    float f;
};
__device__ __forceinline__ VpFast vp_fast_load(const VpOp& src) {
    VpFast o;
    o.n4 = uni(src.n) >> 2;
    o.out = uni(src.out);
    o.in0 = uni(src.in0);
    o.in1 = uni(src.in1 >= 0 ? src.in1 : src.w >= 0 ? src.w : src.in0);
    o.w = uni(src.w);
    o.nsb = uni(src.nsb);
    o.sync = uni(src.sync);
    o.wg0 = uni(src.wg0);
    o.f = __int_as_float(uni(__float_as_int(src.f)));
    return o;
}

template <int KIND, bool H>
__device__ __forceinline__ void vp_fast(const VpFast& o, float* lds, float f, int tid) {
    if (o.out < 0) return;  // a copy whose source slot is written out as it is
    int n4 = o.n4, c = tid;
    const f4* A = (const f4*)(lds + o.in0);
    const f4* B = (const f4*)(lds + o.in1);
    f4* O = (f4*)(lds + o.out);
    if (KIND == VP_RMS) {  // rms (cpu.rs:187-207): out = a·r·w, summed by the waves that own elements
        if (64 * (tid >> 6) >= n4) return;
        float dsum = dot16_wave(lds + o.in0, 4 * n4, tid & 63);
        float r = 1.0f / sqrtf(dsum / (float)(4 * n4) + o.f);
        if (c < n4) {
            f4 a = A[c], w = B[c], v;
#pragma unroll
            for (int e = 0; e < 4; e++) v[e] = e_rms<H>(a[e], r, w[e]);
            O[c] = v;
        }
        return;
    }
    if (c >= n4) return;
    if (KIND == VP_FOLD) {
        const f4* P = (const f4*)(lds + o.w);
        switch (o.nsb) {
            case 1: O[c] = vp_fold4<1, H>(P, n4, c); return;
            case 2: O[c] = vp_fold4<2, H>(P, n4, c); return;
            case 3: O[c] = vp_fold4<3, H>(P, n4, c); return;
            case 4: O[c] = vp_fold4<4, H>(P, n4, c); return;
            case 5: O[c] = vp_fold4<5, H>(P, n4, c); return;
            case 6: O[c] = vp_fold4<6, H>(P, n4, c); return;
            case 7: O[c] = vp_fold4<7, H>(P, n4, c); return;
            default: O[c] = vp_fold4<8, H>(P, n4, c); return;
        }
    }
    f4 a = A[c], b = KIND == VP_COPY || KIND == VP_SCALE ? a : B[c], v;
#pragma unroll
    for (int e = 0; e < 4; e++) v[e] = vp_elem<KIND, H>(a[e], b[e], f, 0.0f);
    O[c] = v;
}

// A prologue of compile-time kinds K... (every op on the float4 path), run by the prologue
// waves with `sync` (their barrier) before an op that reads what other threads wrote.
template <bool H, int... K>
struct VpSeq {
    template <typename Sync>
    __device__ __forceinline__ static void run(const VpOp* vp, float* lds, const float* sfac,
                                               Sync& sync, int tid, bool first) {
        int k = 0;
        (step<K>(vp, lds, sfac, sync, tid, first, k++), ...);
    }
    template <int KIND, typename Sync>
    __device__ __forceinline__ static void step(const VpOp* vp, float* lds, const float* sfac,
                                                Sync& sync, int tid, bool first, int k) {
        VpFast o = vp_fast_load(vp[k]);
        if (!first && o.wg0) return;
        if (k > 0 && (o.sync || KIND == VP_RMS)) sync();
        float f = o.f;
        if (KIND == VP_SCALE && vp[k].dyn) f = sfac[k];
        vp_fast<KIND, H>(o, lds, f, tid);
    }
};

// The prologue through its straight-line code when its signature is one of these; false
// when it is not (the caller then runs the general loop).
template <bool H, typename Sync>
__device__ __forceinline__ bool vp_seq(int sig, const VpOp* vp, float* lds, const float* sfac,
                                       Sync& sync, int tid, bool first) {
    switch (sig) {
        case SLM_SIG1(VP_RMS):
            VpSeq<H, VP_RMS>::run(vp, lds, sfac, sync, tid, first); return true;
        case SLM_SIG3(VP_FOLD, VP_ADD, VP_RMS):
            VpSeq<H, VP_FOLD, VP_ADD, VP_RMS>::run(vp, lds, sfac, sync, tid, first); return true;
        case SLM_SIG5(VP_FOLD, VP_ADD, VP_ADD, VP_ADD, VP_RMS):
            VpSeq<H, VP_FOLD, VP_ADD, VP_ADD, VP_ADD, VP_RMS>::run(vp, lds, sfac, sync, tid, first); return true;
        case SLM_SIG3(VP_ADD, VP_ADD, VP_RMS):
            VpSeq<H, VP_ADD, VP_ADD, VP_RMS>::run(vp, lds, sfac, sync, tid, first); return true;
        case SLM_SIG3(VP_FOLD, VP_ADD, VP_COPY):
            VpSeq<H, VP_FOLD, VP_ADD, VP_COPY>::run(vp, lds, sfac, sync, tid, first); return true;
        case SLM_SIG4(VP_FOLD, VP_ADD, VP_COPY, VP_RMS):
            VpSeq<H, VP_FOLD, VP_ADD, VP_COPY, VP_RMS>::run(vp, lds, sfac, sync, tid, first); return true;
        case SLM_SIG5(VP_COPY, VP_COPY, VP_COPY, VP_COPY, VP_RMS):
            VpSeq<H, VP_COPY, VP_COPY, VP_COPY, VP_COPY, VP_RMS>::run(vp, lds, sfac, sync, tid, first); return true;
        default:
            return false;
    }
}

template <bool H>
__device__ void vp_run(const VpOp& o, float* lds, float f, int tid, int nt) {
    if (o.out < 0) return;  // a copy whose source slot is written out as it is
    int n = o.n;
    const float* a = lds + o.in0;
    const float* b = lds + (o.in1 >= 0 ? o.in1 : o.w >= 0 ? o.w : o.in0);
    float* out = lds + o.out;
    bool v4 = vp_v4(o);
    switch (o.kind) {
        case VP_COPY: vp_map<VP_COPY, H>(a, b, out, n, v4, f, 0.0f, tid, nt); break;
        case VP_ADD: vp_map<VP_ADD, H>(a, b, out, n, v4, f, 0.0f, tid, nt); break;
        case VP_MIX: vp_map<VP_MIX, H>(a, b, out, n, v4, f, 0.0f, tid, nt); break;
        case VP_SCALE: vp_map<VP_SCALE, H>(a, b, out, n, v4, f, 0.0f, tid, nt); break;
        case VP_SILU: vp_map<VP_SILU, H>(a, b, out, n, v4, f, 0.0f, tid, nt); break;
        case VP_FOLD: vp_fold<H>(lds + o.w, out, n, o.nsb, v4, tid, nt); break;
        case VP_COMB:  // the second pass (the caller ran vp_comb_w and a barrier)
            if (o.dh % 4 == 0) vp_comb_o<4, H>(lds + o.w, (const float2*)(lds + o.in1), out, o.heads, o.dh, o.dp, o.nsb, tid, nt);
            else vp_comb_o<1, H>(lds + o.w, (const float2*)(lds + o.in1), out, o.heads, o.dh, o.dp, o.nsb, tid, nt);
            break;
        case VP_RMS: {  // rms (cpu.rs:187-207) of one group: out = a·r·w
            // (only the waves that own elements of the group sum it, each the same sum)
            if (64 * (tid >> 6) >= (v4 ? n >> 2 : n)) break;
            float dsum = dot16_wave(a, n, tid & 63);
            float r = 1.0f / sqrtf(dsum / (float)n + o.f);
            vp_map<VP_RMS, H>(a, b, out, n, v4, f, r, tid, nt);
            break;
        }
        default: break;
    }
}

struct FgUnit {
    int seg, tile, split;
};

// n / d through m = ceil(2^32 / d) (the planner's FgSeg::mtiles, mhalf): the high word of n·m,
// exact while n·d < 2^32 (indices here stay far below); d = 1 gives n.
__device__ __forceinline__ int mdiv(int n, int d, unsigned m) {
    return d == 1 ? n : (int)__umulhi((unsigned)n, m);
}

__device__ __forceinline__ FgUnit fg_unit(const FgDesc& d, int u) {
    int k = 0;
    for (int q = 1; q < d.nseg; q++)
        if (u >= d.seg[q].unit_first) k = q;
    const FgSeg& s = d.seg[k];
    int local = u - s.unit_first;
    int split = mdiv(local, s.tiles, s.mtiles);
    return FgUnit{k, local - split * s.tiles, split};
}

// Row of lane row i (0..15) of tile t of a matrix of `rows` rows in tiles of rpt rows (16, 12,
// 8 or 4; lane rows past rpt hold none: `rows` is returned, one past the last). In the first
// pair_rows rows lane rows i and i + rpt/2 hold a (row, row + half) pair.
__device__ __forceinline__ long long fg_row_of(int rpt, int pair_rows, int half, unsigned mhalf, int rows,
                                               int t, int i) {
    if (i >= rpt) return rows;
    int hp = rpt >> 1;
    if (t * rpt < pair_rows) {
        bool second = i >= hp;
        int P = t * hp + (second ? i - hp : i);
        int q = mdiv(P, half, mhalf);
        return (long long)q * 2 * half + (P - q * half) + (second ? half : 0);
    }
    return (long long)t * rpt + i;
}
__device__ __forceinline__ long long fg_row(const FgSeg& s, int t, int i) {
    return fg_row_of(s.rpt, s.pair_rows, s.half, s.mhalf, s.rows, t, i);
}

// Sixteen zero bytes: what a lane past the end of a weight matrix loads.
__device__ __attribute__((aligned(16))) float slm_zero16[4];

// Where one GEMV lane's weights of unit u come from, worked out once per unit: the
// lane's row start (or the zero page), the first 16-column block of its slice and how
// many of the slice's four blocks lie inside the matrix (0: the slice is past the end).
struct FgLane {
    const float* base;
    int kb0, nkb;
};

// Descriptor dwords [base, base + 128) of the kernel argument, one per lane in two VGPRs: the
// whole region costs one memory round trip (each dependent scalar load of a cold scalar cache
// costs one), and a field is then a readlane with an index known at compile time.
struct KDw {
    int v0, v1;
    __device__ __forceinline__ int operator[](int q) const {
        return __builtin_amdgcn_readlane(q < 64 ? v0 : v1, q & 63);
    }
    __device__ __forceinline__ long long q64(int q) const {
        return (long long)(unsigned)(*this)[q] | ((long long)(*this)[q + 1] << 32);
    }
};
__device__ __forceinline__ KDw kdw_load(const int* k, int base, int lane) {
    return KDw{gld(k + base + lane), gld(k + base + 64 + lane)};
}

// fg_lane from the descriptor's dwords in registers (KDw: the header at dword 0, the segments
// at the dword of FgDesc::seg), for the first round, before the descriptor is in LDS.
template <bool W16>
__device__ __forceinline__ FgLane fg_lane_k(const KDw& hd, const KDw& sd, int u, int wave, int i, int g) {
    constexpr int SW = (int)(sizeof(FgSeg) / 4);
    constexpr int HU = (int)(offsetof(FgDesc, units) / 4), HC = (int)(offsetof(FgDesc, cols) / 4);
    constexpr int HN = (int)(offsetof(FgDesc, nsl) / 4), HS = (int)(offsetof(FgDesc, nseg) / 4);
    constexpr int SF = (int)(offsetof(FgSeg, unit_first) / 4), ST = (int)(offsetof(FgSeg, tiles) / 4);
    constexpr int SWT = (int)(offsetof(FgSeg, w) / 4), SR = (int)(offsetof(FgSeg, rows) / 4);
    constexpr int SP = (int)(offsetof(FgSeg, pair_rows) / 4), SH = (int)(offsetof(FgSeg, half) / 4);
    constexpr int SRT = (int)(offsetof(FgSeg, rpt) / 4);
    constexpr int SMT = (int)(offsetof(FgSeg, mtiles) / 4), SMH = (int)(offsetof(FgSeg, mhalf) / 4);
    static_assert(sizeof(FgSeg) % 4 == 0 && SLM_SEG_MAX * sizeof(FgSeg) <= 512, "segment table layout");
    FgLane p{slm_zero16, 0, 0};
    if (u >= hd[HU]) return p;
    int nseg = hd[HS], k = 0;
#pragma unroll
    for (int q = 1; q < SLM_SEG_MAX; q++)
        if (q < nseg && u >= sd[q * SW + SF]) k = q;
    int local = u - sd[k * SW + SF], tiles = sd[k * SW + ST];
    int split = mdiv(local, tiles, (unsigned)sd[k * SW + SMT]), tile = local - split * tiles;
    int sl = split * SLM_SPLIT + wave;
    int cols = hd[HC];
    int kblocks = (cols + 15) >> 4;
    if (sl >= hd[HN]) return p;
    p.kb0 = sl * SLM_KS;
    p.nkb = min(SLM_KS, kblocks - p.kb0);
    int rows = sd[k * SW + SR];
    long long row = fg_row_of(sd[k * SW + SRT], sd[k * SW + SP], sd[k * SW + SH], (unsigned)sd[k * SW + SMH], rows,
                              tile, i);
    if (row < rows) {
        const float* w = (const float*)sd.q64(k * SW + SWT);
        if constexpr (W16) p.base = (const float*)((const _Float16*)w + row * cols + 4 * g);
        else p.base = w + row * cols + 4 * g;
    }
    return p;
}

// (W16: the matrices hold fp16 weights; `base` then addresses halves)
template <bool W16>
__device__ __forceinline__ FgLane fg_lane(const FgDesc& d, int u, int wave, int i, int g) {
    FgLane p{slm_zero16, 0, 0};
    if (u >= d.units) return p;
    FgUnit un = fg_unit(d, u);
    const FgSeg& s = d.seg[un.seg];
    int sl = un.split * SLM_SPLIT + wave;
    int kblocks = (d.cols + 15) >> 4;
    if (sl >= d.nsl) return p;
    p.kb0 = sl * SLM_KS;
    p.nkb = min(SLM_KS, kblocks - p.kb0);
    long long row = fg_row(s, un.tile, i);
    if (row < s.rows) {
        if constexpr (W16) p.base = (const float*)((const _Float16*)s.w + row * d.cols + 4 * g);
        else p.base = s.w + row * d.cols + 4 * g;
    }
    return p;
}

// The weights of one unit's slice for this lane: four float4s. Lanes past the matrix load
// zeros from slm_zero16, so the loads are always four and their results are used as they
// arrive, without a select that would wait for them.
// (W16: four halves per block, widened exactly; the zero page reads as zeros either way)
template <bool W16>
__device__ __forceinline__ void fg_load(const FgLane& p, f4 (&wa)[SLM_KS]) {
    bool ok = p.base != slm_zero16;
#pragma unroll
    for (int q = 0; q < SLM_KS; q++) {
        if constexpr (W16) {
            const h4* src = ok && q < p.nkb ? (const h4*)((const _Float16*)p.base + (p.kb0 + q) * 16)
                                            : (const h4*)slm_zero16;
            wa[q] = wide4(gld(src));
        } else {
            const float* src = ok && q < p.nkb ? p.base + (p.kb0 + q) * 16 : slm_zero16;
            wa[q] = gld((const f4*)src);
        }
    }
}

// slm_attn_combine's expressions for head h of one token, run by one wave: every lane
// finds M (the largest m of the superblocks that saw a key) from the (m, l) pairs, lane z
// holds superblock z's weight w_z = e^(m_z − M) and l_z·w_z, lane d sums dim d in
// superblock order; x[64h + d] = O / L (0 when no superblock saw a key). nsb ≤ 64.
template <bool C, bool H>
__device__ __forceinline__ void fg_comb_wave(const float* part, float* x, int heads, int dp,
                                             int nsb, int h, int lane, float* gout) {
    int sr = heads * (dp + 2);
    const float* P = part + h * (dp + 2);
    // M: lane z holds superblock z's (m, l); the largest m with l > 0 across the wave (a
    // maximum, so its order does not matter: NaNs drop out, and -inf starts it as a pass over
    // the superblocks in order does)
    float2 me = lane < nsb ? *(const float2*)(P + lane * sr) : float2{NEG_INF, 0.0f};
    float M = me.y > 0.0f ? me.x : NEG_INF;
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) M = fmaxf(M, __shfl_xor(M, d));
    M = fmaxf(NEG_INF, M);
    float wz = -1.0f, lwz = 0.0f;
    if (lane < nsb) {
        float w = expf(me.x - M);
        if (me.y > 0.0f) {
            wz = w;
            lwz = me.y * w;
        }
    }
    float L = 0.0f, O = 0.0f;
    for (int z0 = 0; z0 < nsb; z0 += 8) {
        float oz[8];
#pragma unroll
        for (int u = 0; u < 8; u++) oz[u] = P[min(z0 + u, nsb - 1) * sr + 2 + lane];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            if (z0 + u >= nsb) break;
            float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wz), z0 + u));
            float lw = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lwz), z0 + u));
            if (w >= 0.0f) {
                L = L + lw;
                O = O + oz[u] * w;
            }
        }
    }
    float v = h16<H>(L > 0.0f ? O / L : 0.0f);
    x[64 * h + lane] = v;
    if (gout) stc<C>(gout + 64 * h + lane, v);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the wave's LDS writes are done
}

// The canonical chain of the lane's slice; lanes of row 0 of B hold the token.
template <bool H>
__device__ __forceinline__ void fg_chain(const FgLane& p, int i, int g, const f4 (&wa)[SLM_KS],
                                         const float* xin, float* out) {
    if (p.nkb <= 0) return;
    f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int q = 0; q < SLM_KS; q++) {
        if (q < p.nkb) {
            f4 xb = {0.0f, 0.0f, 0.0f, 0.0f};
            if (i == 0) xb = *(const f4*)(xin + (p.kb0 + q) * 16 + 4 * g);
            if constexpr (H) {
                acc = block16h(wa[q], xb, acc);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) acc = mfma4(wa[q][e], xb[e], acc);
            }
        }
    }
    if (i == 0) {
#pragma unroll
        for (int r = 0; r < 4; r++) out[4 * g + r] = acc[r];
    }
}

// The greedy pick's order on (value, row): a larger value first, then a smaller row — the
// first maximum of sample.rs:48-53 (b = 0, then b = i whenever x[i] > x[b]). −0 and +0 are
// equal; a NaN never wins, except at row 0, where it wins outright (nothing compares greater
// than the NaN that b starts on). Key 0: no row.
__device__ __forceinline__ unsigned long long pick_key(float v, int row) {
    if (v != v) return row == 0 ? ~0ull : 0ull;
    unsigned u = __float_as_uint(v == 0.0f ? 0.0f : v);
    unsigned k = (u >> 31) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)k << 32) | (unsigned long long)(0xFFFFFFFFu - (unsigned)row);
}

// The end of a fused GEMV with the greedy pick (EPI_PICK), run by the epilogue wave of every
// workgroup: its rows' largest key goes into the launch's 64-bit atomic maximum, and the last
// workgroup to count itself in writes the pick out and clears the key and the counter for
// the next launch. (The release of the count orders the maximum before it; the acquire of
// the last count sees every workgroup's.)
__device__ void fg_pick_finish(const FgSeg& g, unsigned long long best, int lane, int nwg) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        unsigned lo = __shfl_xor((unsigned)best, off), hi = __shfl_xor((unsigned)(best >> 32), off);
        unsigned long long o = ((unsigned long long)hi << 32) | lo;
        best = o > best ? o : best;
    }
    if (lane != 0) return;
    unsigned long long* key = (unsigned long long*)g.o3;
    int* ctr = (int*)g.o3 + 2;
    if (best) __hip_atomic_fetch_max(key, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    int before = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (before != nwg - 1) return;
    unsigned long long k = __hip_atomic_load(key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    long long r = k ? (long long)(0xFFFFFFFFu - (unsigned)(k & 0xFFFFFFFFull)) : 0;
    gst((long long*)g.o1, r);
    if (g.o2) gst((unsigned*)g.o2 + (g.dyn ? gld(g.dyn) : g.imm), (unsigned)r);
    __hip_atomic_store(key, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The fused GEMV, fp32 (slm_fg), fp16 mode (slm_fgh) and fp16 mode with fp16 weights
// (slm_fghw): one body, fg_run, whose descriptor is the kernel's only argument.
#include "fg_body.inc"
#define FG_KERNEL(NAME, H, W)                                                                   \
    KERNEL void __launch_bounds__(1024) NAME(const FgDesc dk) {                                 \
        fg_run<H, W, false>(dk, (const int*)(const void*)__builtin_amdgcn_kernarg_segment_ptr(), \
                            blockIdx.x, gridDim.x, StepWait{nullptr, 0, 0, nullptr},            \
                            threadIdx.x);                                                       \
    }
FG_KERNEL(slm_fg, false, false)
FG_KERNEL(slm_fgh, true, false)
FG_KERNEL(slm_fghw, true, true)

// The splits of a linear added in order: y[c] = ((P0[c] + P1[c]) + P2[c]) + ...
KERNEL void slm_fold(float* __restrict__ y, const float* __restrict__ part, long long n, int nsplit) {
    bool h = slm_h16;  // (the linear's output: rounded in fp16 mode)
    GRID_LOOP(c, n) {
        float v = part[c];
        for (int z = 1; z < nsplit; z++) v = v + part[z * n + c];
        y[c] = h ? r16(v) : v;
    }
}

// A prompt row chain: workgroup r runs the ops on token row r, each op over the row with
// the expression of its own kernel (slm_copy / slm_columns, slm_add / slm_add_row,
// slm_mix, slm_silu_mul, slm_rope, slm_store, slm_rms / slm_l2norm, slm_fold). Between two
// ops a barrier orders LDS only: a later op reads what an earlier one made from LDS, never
// from global memory (the planner sees to it), so no global write has to land first.
// With `vec` the ops move float4s, each thread issuing all loads of a batch of four before
// it uses any.
__device__ __forceinline__ float row_in(const float* lds, int off, const RowIn& s, long long r,
                                        int i) {
    return off >= 0 ? lds[off + i] : s.g[r * s.stride + i];
}
__device__ __forceinline__ void row_put(float* lds, const RowOp& o, float* yr, int i, float v) {
    if (o.out >= 0) lds[o.out + i] = v;
    if (yr) yr[i] = v;
}
__device__ __forceinline__ f4 row_in4(const float* lds, int off, const RowIn& s, long long r,
                                      int i) {  // i: a multiple of 4
    return off >= 0 ? *(const f4*)(lds + off + i) : *(const f4*)(s.g + r * s.stride + i);
}
__device__ __forceinline__ void row_put4(float* lds, const RowOp& o, float* yr, int i, f4 v) {
    if (o.out >= 0) *(f4*)(lds + o.out + i) = v;
    if (yr) *(f4*)(yr + i) = v;
}
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
// (h: fp16 mode's roundings, the e_* expressions)
template <int KIND>
__device__ __forceinline__ float row_ew(float a, float b, float f, bool h) {
    if (KIND == R_COPY) return a;
    if (KIND == R_ADD) return h ? e_add<true>(a, b) : e_add<false>(a, b);
    if (KIND == R_MIX) return h ? e_mix<true>(a, b, f) : e_mix<false>(a, b, f);
    return h ? e_silu<true>(a, b) : e_silu<false>(a, b);  // R_SILU: a = gate, b = up
}
// out = f(a, b) element by element
template <int KIND>
__device__ __forceinline__ void row_elementwise(const RowOp& o, float* lds, float* yr, long long r,
                                                int tid, bool h) {
    int n = o.n;
    bool two = KIND != R_COPY;
    if (o.vec) {
        for (int b0 = 0; b0 < n; b0 += 4 * 1024) {
            f4 av[4], bv[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                int i = b0 + 4 * (tid + 256 * u);
                if (i < n) {
                    av[u] = row_in4(lds, o.la, o.a, r, i);
                    if (two) bv[u] = row_in4(lds, o.lb, o.b, r, i);
                }
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                int i = b0 + 4 * (tid + 256 * u);
                if (i < n) {
                    f4 v;
#pragma unroll
                    for (int e = 0; e < 4; e++) v[e] = row_ew<KIND>(av[u][e], two ? bv[u][e] : 0.0f, o.f0, h);
                    row_put4(lds, o, yr, i, v);
                }
            }
        }
        return;
    }
    for (int i = tid; i < n; i += 256)
        row_put(lds, o, yr, i, row_ew<KIND>(row_in(lds, o.la, o.a, r, i),
                                              two ? row_in(lds, o.lb, o.b, r, i) : 0.0f, o.f0, h));
}
// An op read from the descriptor in LDS, its fields made wave-uniform (they are).
__device__ __forceinline__ const float* uni_ptr(const float* p) {
    unsigned long long v = (unsigned long long)p;
    unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)v), hi = __builtin_amdgcn_readfirstlane((unsigned)(v >> 32));
    return (const float*)(((unsigned long long)hi << 32) | lo);
}
__device__ __forceinline__ long long uni_ll(long long x) {
    unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)x), hi = __builtin_amdgcn_readfirstlane((unsigned)((unsigned long long)x >> 32));
    return (long long)(((unsigned long long)hi << 32) | lo);
}
__device__ __forceinline__ RowOp row_load(const RowOp& src) {
    RowOp o = src;
    o.kind = uni(o.kind); o.n = uni(o.n);
    o.la = uni(o.la); o.lb = uni(o.lb); o.lc = uni(o.lc); o.ld = uni(o.ld);
    o.out = uni(o.out); o.tmp = uni(o.tmp); o.i0 = uni(o.i0); o.i1 = uni(o.i1); o.vec = uni(o.vec);
    o.h16 = uni(o.h16);
    o.f0 = __int_as_float(uni(__float_as_int(o.f0)));
    o.a.g = uni_ptr(o.a.g); o.b.g = uni_ptr(o.b.g); o.c.g = uni_ptr(o.c.g); o.d.g = uni_ptr(o.d.g);
    o.a.stride = uni_ll(o.a.stride); o.b.stride = uni_ll(o.b.stride);
    o.c.stride = uni_ll(o.c.stride); o.d.stride = uni_ll(o.d.stride);
    o.y = (float*)uni_ptr(o.y); o.ystride = uni_ll(o.ystride);
    o.q0 = uni_ll(o.q0); o.q1 = uni_ll(o.q1);
    o.dyn = (const long long*)uni_ptr((const float*)o.dyn);
    return o;
}
KERNEL void __launch_bounds__(256) slm_rows(const RowDesc dk) {
    // The header, the prefetch table and the first op come into registers with one dword per
    // lane (one memory round trip, no LDS hop), so the operand prefetches — and, when the chain
    // starts with a fold of split partials, those partials — are issued at once; the whole
    // descriptor goes to LDS for the ops meanwhile (one wide load per thread).
    __shared__ RowDesc d;
    constexpr int ND4 = (int)(sizeof(RowDesc) / 16), PF0 = (int)(offsetof(RowDesc, pf) / 4);
    constexpr int PFW = (int)(sizeof(RowPf) / 4), O0 = (int)(offsetof(RowDesc, op) / 4);
    static_assert(sizeof(RowDesc) % 16 == 0 && ND4 <= 256, "descriptor copy: a float4 per thread");
    static_assert(O0 + (int)(sizeof(RowOp) / 4) <= 128, "the first op in the registers' dwords");
    extern __shared__ __attribute__((aligned(16))) float lds[];
    long long r = blockIdx.x;
    int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    KDw hd = kdw_load((const int*)(const void*)__builtin_amdgcn_kernarg_segment_ptr(), 0, lane);
    f4 dv = {0.0f, 0.0f, 0.0f, 0.0f};
    if (tid < ND4) dv = ((const f4*)(const void*)__builtin_amdgcn_kernarg_segment_ptr())[tid];
    int nops = hd[0], npf = hd[1];
    bool h16r = hd[2] != 0;  // fp16 mode: every op's output rounded (RowDesc::r16)
#pragma unroll
    for (int e = 0; e < SLM_ROW_PF; e++) {
        if (e >= npf) break;
        const float* src = (const float*)hd.q64(PF0 + PFW * e) + r * hd.q64(PF0 + PFW * e + 2);
        int n4 = hd[PF0 + PFW * e + 4] >> 2, plds = hd[PF0 + PFW * e + 5];
        for (int j = wave; 64 * j < n4; j += 4) {
            int c = 64 * j + lane;
            if (c < n4)
                __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(src + 4 * c),
                                                 (__attribute__((address_space(3))) void*)(lds + plds + 256 * j),
                                                 16, 0, 0);
        }
    }
    // a first op that folds at most 8 split partials of a row of at most 1024 floats (float4s):
    // this thread's partials, in registers
    constexpr int FOLD_PRE = 8;
    constexpr int OK = O0 + (int)(offsetof(RowOp, kind) / 4), ON = O0 + (int)(offsetof(RowOp, n) / 4);
    constexpr int OI0 = O0 + (int)(offsetof(RowOp, i0) / 4), OV = O0 + (int)(offsetof(RowOp, vec) / 4);
    constexpr int OAG = O0 + (int)(offsetof(RowOp, a) / 4), OQ0 = O0 + (int)(offsetof(RowOp, q0) / 4);
    static_assert(offsetof(RowIn, g) == 0 && offsetof(RowIn, stride) == 8, "RowIn layout");
    f4 fpre[FOLD_PRE];
    bool early = nops > 0 && hd[OK] == R_FOLD && hd[OV] && hd[ON] <= 1024 && hd[OI0] <= FOLD_PRE;
    if (early) {
        int nf = hd[ON], nz = hd[OI0], i = 4 * tid;
        const float* pp = (const float*)hd.q64(OAG) + r * hd.q64(OAG + 2) + i;
        long long q0 = hd.q64(OQ0);
#pragma unroll
        for (int z = 0; z < FOLD_PRE; z++)
            if (z < nz && i < nf) fpre[z] = *(const f4*)(pp + z * q0);
    }
    if (tid < ND4) ((f4*)&d)[tid] = dv;
    vm_wait<0>();
    __syncthreads();
    for (int k = 0; k < nops; k++) {
        const RowOp o = row_load(d.op[k]);
        int kind = o.kind, n = o.n;
        float* yr = o.y ? o.y + r * o.ystride : nullptr;
        if (kind == R_COPY) {
            row_elementwise<R_COPY>(o, lds, yr, r, tid, h16r);
        } else if (kind == R_ADD) {
            row_elementwise<R_ADD>(o, lds, yr, r, tid, h16r);
        } else if (kind == R_MIX) {
            row_elementwise<R_MIX>(o, lds, yr, r, tid, h16r);
        } else if (kind == R_SILU) {
            row_elementwise<R_SILU>(o, lds, yr, r, tid, h16r);
        } else if (kind == R_ROPE) {
            int heads = o.i0, dh = o.i1, half = dh / 2;
            if (o.vec) {  // four consecutive i of one head per thread
                int q4 = half >> 2;
                for (int t = tid; t < heads * q4; t += 256) {
                    int h = t / q4, i = 4 * (t % q4), at = h * dh;
                    f4 c = row_in4(lds, o.lc, o.c, r, i), sn = row_in4(lds, o.ld, o.d, r, i);
                    f4 a = row_in4(lds, o.la, o.a, r, at + i), b = row_in4(lds, o.la, o.a, r, at + half + i);
                    f4 v0, v1;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        v0[e] = h16r ? e_rope_l<true>(a[e], b[e], c[e], sn[e]) : e_rope_l<false>(a[e], b[e], c[e], sn[e]);
                        v1[e] = h16r ? e_rope_r<true>(a[e], b[e], c[e], sn[e]) : e_rope_r<false>(a[e], b[e], c[e], sn[e]);
                    }
                    row_put4(lds, o, yr, at + i, v0);
                    row_put4(lds, o, yr, at + half + i, v1);
                }
            } else {
                for (int t = tid; t < heads * half; t += 256) {
                    int h = t / half, i = t % half, at = h * dh;
                    float c = row_in(lds, o.lc, o.c, r, i), sn = row_in(lds, o.ld, o.d, r, i);
                    float a = row_in(lds, o.la, o.a, r, at + i), b = row_in(lds, o.la, o.a, r, at + half + i);
                    row_put(lds, o, yr, at + i, h16r ? e_rope_l<true>(a, b, c, sn) : e_rope_l<false>(a, b, c, sn));
                    row_put(lds, o, yr, at + half + i, h16r ? e_rope_r<true>(a, b, c, sn) : e_rope_r<false>(a, b, c, sn));
                }
            }
        } else if (kind == R_STORE) {
            int heads = o.i0, dh = o.i1;
            long long pos = dyn_or(o.dyn, o.q1);
            long long slot = (pos + r) % o.q0;
            if (o.h16) {  // an fp16 ring: each value rounded to nearest even
                _Float16* ring = (_Float16*)o.y;
                for (int t = tid; t < heads * dh; t += 256) {
                    int h = t / dh, e = t % dh;
                    ring[((long long)h * o.q0 + slot) * dh + e] = (_Float16)row_in(lds, o.la, o.a, r, t);
                }
            } else if (o.vec) {
                int d4 = dh >> 2;
                for (int t = tid; t < heads * d4; t += 256) {
                    int h = t / d4, e = 4 * (t % d4);
                    *(f4*)(o.y + ((long long)h * o.q0 + slot) * dh + e) = row_in4(lds, o.la, o.a, r, h * dh + e);
                }
            } else {
                for (int t = tid; t < heads * dh; t += 256) {
                    int h = t / dh, e = t % dh;
                    o.y[((long long)h * o.q0 + slot) * dh + e] = row_in(lds, o.la, o.a, r, t);
                }
            }
        } else if (kind == R_RMS || kind == R_L2NORM) {
            int size = o.i0, groups = n / size;
            int src = o.la;
            if (src < 0) {  // the row goes to LDS first, where the sums read it
                if (o.vec) {
                    for (int b0 = 0; b0 < n; b0 += 4 * 1024) {
                        f4 av[4];
#pragma unroll
                        for (int u = 0; u < 4; u++) {
                            int i = b0 + 4 * (tid + 256 * u);
                            if (i < n) av[u] = *(const f4*)(o.a.g + r * o.a.stride + i);
                        }
#pragma unroll
                        for (int u = 0; u < 4; u++) {
                            int i = b0 + 4 * (tid + 256 * u);
                            if (i < n) *(f4*)(lds + o.tmp + i) = av[u];
                        }
                    }
                } else {
                    for (int i = tid; i < n; i += 256) lds[o.tmp + i] = o.a.g[r * o.a.stride + i];
                }
                lds_barrier();
                src = o.tmp;
            }
            for (int grp = wave; grp < groups; grp += 4) {  // one wave per group
                const float* in = lds + src + grp * size;
                float dd = dot16_wave(in, size, lane);
                float rr = kind == R_RMS ? 1.0f / sqrtf(dd / (float)size + o.f0)
                                         : 1.0f / fmaxf(sqrtf(dd), 1e-12f);
                if (o.vec) {
                    for (int j = 4 * lane; j < size; j += 256) {
                        f4 v = *(const f4*)(in + j), w, out;
                        if (kind == R_RMS) w = row_in4(lds, o.lb, o.b, 0, j);
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            out[e] = kind == R_RMS ? (h16r ? e_rms<true>(v[e], rr, w[e]) : v[e] * rr * w[e])
                                                   : (h16r ? r16(v[e] * rr) : v[e] * rr);
                        row_put4(lds, o, yr, grp * size + j, out);
                    }
                } else {
                    for (int j = lane; j < size; j += 64) {
                        float v = kind == R_RMS ? (h16r ? e_rms<true>(in[j], rr, row_in(lds, o.lb, o.b, 0, j))
                                                        : in[j] * rr * row_in(lds, o.lb, o.b, 0, j))
                                                : (h16r ? r16(in[j] * rr) : in[j] * rr);
                        row_put(lds, o, yr, grp * size + j, v);
                    }
                }
            }
        } else if (kind == R_FOLD) {
            if (k == 0 && early) {  // the partials are in registers
                int i = 4 * tid;
                if (i < n) {
                    f4 v = fpre[0];
#pragma unroll
                    for (int z = 1; z < FOLD_PRE; z++)
                        if (z < o.i0)
#pragma unroll
                            for (int e = 0; e < 4; e++) v[e] = v[e] + fpre[z][e];
                    if (h16r)
#pragma unroll
                        for (int e = 0; e < 4; e++) v[e] = r16(v[e]);
                    row_put4(lds, o, yr, i, v);
                }
            } else if (o.vec) {
                for (int b0 = 0; b0 < n; b0 += 4 * 256) {
                    int i = b0 + 4 * tid;
                    if (i >= n) continue;
                    const float* pp = o.a.g + r * o.a.stride + i;
                    f4 v = *(const f4*)pp;
                    for (int z0 = 1; z0 < o.i0; z0 += 4) {  // four partials in flight
                        f4 w[4];
#pragma unroll
                        for (int u = 0; u < 4; u++)
                            if (z0 + u < o.i0) w[u] = *(const f4*)(pp + (z0 + u) * o.q0);
#pragma unroll
                        for (int u = 0; u < 4; u++)
                            if (z0 + u < o.i0)
#pragma unroll
                                for (int e = 0; e < 4; e++) v[e] = v[e] + w[u][e];
                    }
                    if (h16r)
#pragma unroll
                        for (int e = 0; e < 4; e++) v[e] = r16(v[e]);
                    row_put4(lds, o, yr, i, v);
                }
            } else {
                for (int i = tid; i < n; i += 256) {
                    const float* pp = o.a.g + r * o.a.stride + i;
                    float v = pp[0];
                    for (int z = 1; z < o.i0; z++) v = v + pp[z * o.q0];
                    row_put(lds, o, yr, i, h16r ? r16(v) : v);
                }
            }
        }
        lds_barrier();
    }
}

// One token of gated linear attention per head, one workgroup per head (the m = 1 case of
// gla_body, same expressions). When `l2`, q and k are first l2-normalised per head
// (model.rs:465-467, the expressions of slm_l2norm); when `fuse`, the head RMSNorm and the
// SiLU gate of model.rs:483-484 follow, in the expressions of slm_rms and slm_silu_mul.
template <int RPL, bool STEP = false>
__device__ __forceinline__ bool gla1_body(const GlaDesc& g, int h, int tid, int nt,
                                          const StepWait* sw = nullptr, int* gave = nullptr) {
    extern __shared__ __attribute__((aligned(16))) float lds[];  // [dh + 4] rms, [dh] q, [dh] k, 4 norms
    int dh = g.dh;
    int b = tid >> 4, j = tid & 15;
    bool live = b < dh;
    float* Sh = g.s + (long long)h * dh * dh;
    long long at = (long long)h * dh;
    // A launch of its own loads the step's q, k, v and decay first and the state (dh x dh a
    // head) after them, so that the state streams in while the norms run: its barriers only
    // order LDS (lds_bar), so none of them waits for the state or for a store. As a step
    // phase, the state, from earlier steps, is read before the wait for the phase that made
    // q, k, v and the decay, and those after it. (nt ≥ dh: one element of q and k a thread.)
    // (every lane loads, from a clamped index where it has nothing to load, and drops the
    // value after: the loads are then a fixed sequence, so the wait for q and k does not wait
    // for the state behind them)
    float q0 = 0.0f, k0 = 0.0f, vb = 0.0f, draw = 0.0f, bias = g.bias[h];
    int tq = min(tid, dh - 1), bq = min(b, dh - 1);
    // (and, when fused, the gate and the head norm's weight, used last)
    float gt = 0.0f, hnw = g.fuse ? g.hn[bq] : 0.0f;
    if (!STEP) {
        q0 = gld(g.q + at + tq);
        k0 = gld(g.k + at + tq);
        vb = gld(g.v + at + bq);
        draw = gld(g.decay + h);
        if (g.fuse) gt = gld(g.gate + at + bq);
        asm volatile("" : : : "memory");  // (issued before the state's loads)
    }
    // The state: where dh = 64 (RPL = 4, 1024 threads), thread t loads elements t, t + 1024, ...
    // (whole rows a wave, one memory line per 32 lanes) and the values reach their lanes
    // through LDS (row a at a·65: lanes of one column read distinct banks); otherwise each
    // lane loads its own rows of its column.
    constexpr bool ST64 = RPL == 4;
    bool staged = ST64 && dh == 64 && nt == 1024;
    float* ls = lds + 4 * dh + 16;
    float st[RPL];
    if (staged) {
#pragma unroll
        for (int q = 0; q < RPL; q++) st[q] = Sh[tid + q * 1024];
    } else {
#pragma unroll
        for (int rr = 0; rr < RPL; rr++) {
            int a = min(j * RPL + rr, dh - 1);
            st[rr] = Sh[(long long)a * dh + bq];
        }
    }
    if (STEP) {
        if (step_wait_wg(*sw, gave, tid)) return false;
        q0 = ldc<STEP>(g.q + at + tq);
        k0 = ldc<STEP>(g.k + at + tq);
        vb = ldc<STEP>(g.v + at + bq);
        draw = ldc<STEP>(g.decay + h);
        if (g.fuse) gt = ldc<STEP>(g.gate + at + bq);
    }
    if (!live) vb = 0.0f;
    if (!staged) {
#pragma unroll
        for (int rr = 0; rr < RPL; rr++)
            if (!live || j * RPL + rr >= dh) st[rr] = 0.0f;
    }
    auto bar = [] {
        if (STEP) __syncthreads();
        else lds_bar();
    };
    float* lq = lds + dh + 4;
    float* lk = lq + dh;
    float* nr = lk + dh;
    if (tid < dh) {
        lq[tid] = q0;
        lk[tid] = k0;
    }
    bar();
    if (g.l2) {
        if (tid < 32) {
            float d = dot16_self(tid < 16 ? lq : lk, dh, tid & 15);
            if ((tid & 15) == 0) nr[tid >> 4] = 1.0f / fmaxf(sqrtf(d), 1e-12f);
        }
        bar();
        float rq = nr[0], rk = nr[1];
        float aq = 0.0f, ak = 0.0f;
        int c = tid;
        if (c < dh) {
            aq = lq[c] * rq;
            ak = lk[c] * rk;
            if (g.r16) {
                aq = r16(aq);
                ak = r16(ak);
            }
            stc<STEP>(g.qn + at + c, aq);
            stc<STEP>(g.kn + at + c, ak);
        }
        bar();
        if (c < dh) {
            lq[c] = aq;
            lk[c] = ak;
        }
        bar();
    }
    if (staged) {  // (every lane of dh = 64 is live, with all its rows)
#pragma unroll
        for (int q = 0; q < RPL; q++) {
            int e = tid + q * 1024;
            ls[(e >> 6) * 65 + (e & 63)] = st[q];
        }
        bar();
#pragma unroll
        for (int rr = 0; rr < RPL; rr++) st[rr] = ls[(j * RPL + rr) * 65 + b];
    }
    bool hm = g.r16 != 0;
    float dc = hm ? gla_decay<true>(draw, bias) : gla_decay<false>(draw, bias);
    float part = !live ? 0.0f : hm ? gla_rows<RPL, true>(st, lk, lq, dc, vb, j, dh) : gla_rows<RPL, false>(st, lk, lq, dc, vb, j, dh);
    float t2 = gla_colsum(part);
    if (hm) t2 = r16(t2);
    if (staged) {  // back through LDS (each lane's own slots), then whole rows a wave
#pragma unroll
        for (int rr = 0; rr < RPL; rr++) ls[(j * RPL + rr) * 65 + b] = st[rr];
    } else {
#pragma unroll
        for (int rr = 0; rr < RPL; rr++) {
            int a = j * RPL + rr;
            if (live && a < dh) Sh[(long long)a * dh + b] = st[rr];
        }
    }
    if (live && j == 0) stc<STEP>(g.y + at + b, t2);
    if (g.fuse && live && j == 0) lds[b] = t2;
    bar();
    if (staged) {
#pragma unroll
        for (int q = 0; q < RPL; q++) {
            int e = tid + q * 1024;
            Sh[e] = ls[(e >> 6) * 65 + (e & 63)];
        }
    }
    if (!g.fuse) return true;
    if (tid < 16) {
        float d = dot16_self(lds, dh, tid);
        if (tid == 0) lds[dh] = 1.0f / sqrtf(d / (float)dh + g.eps);
    }
    bar();
    if (live && j == 0) {
        float y2 = hm ? e_rms<true>(lds[b], lds[dh], hnw) : lds[b] * lds[dh] * hnw;
        stc<STEP>(g.y2 + at + b, y2);
        stc<STEP>(g.out + at + b, hm ? e_silu<true>(gt, y2) : y2 * gt / (1.0f + expf(-gt)));
    }
    return true;
}

#define GLA1(R)                                                                   \
    KERNEL void __launch_bounds__(1024) slm_gla1_##R(const GlaDesc g) { gla1_body<R>(g, blockIdx.x, threadIdx.x, blockDim.x); }
GLA1(1)
GLA1(2)
GLA1(4)

// ---------------------------------------------------------------------------------------
// one one-token step in one launch
// ---------------------------------------------------------------------------------------

// Every workgroup runs the step's phases in order: the kernels the planner made for the step
// (fused GEMVs, one-token attentions that leave their superblock partials to the next fused
// GEMV, one-token GLAs), each as the workgroups of its own grid would have run it, waiting
// before it until every workgroup is done with the previous phase (StepWait). Workgroups past
// a phase's grid pass it at once. A wait that gives up ends the workgroup (the others' waits
// then give up in turn), so a mistake cannot hang the GPU. The launch needs every workgroup
// resident at once: 256 workgroups of 1024 threads, one per compute unit. One kernel per head
// size class (V: the attention's 16-dim tiles and the GLA's rows per lane, 1, 2 or 4), so
// that each holds only the code its phases run.
// The kernel argument, read again where it is used: nothing of it stays in registers across
// a phase (the fused GEMV needs nearly every scalar register).
__device__ __forceinline__ const StepArgs* step_args() {
    const StepArgs* p = (const StepArgs*)(const void*)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(p));
    return p;
}
template <int V>
__device__ __forceinline__ void step_run() {
    __shared__ int gave;
    for (int p = 0;; p++) {
        // The thread and workgroup indices, taken afresh each phase: the compiler cannot
        // lift what a phase works out from them out of the loop, where it would hold
        // registers through every other phase.
        int tid = threadIdx.x, bid = blockIdx.x;
        asm volatile("" : "+v"(tid), "+s"(bid));
        int lane = tid & 63, wave = tid >> 6;
        const StepArgs& a = *step_args();
        if (p >= a.nph) break;
        const StepPh* ph = (const StepPh*)a.prog;
        int kind = uni(ph[p].kind), grid = uni(ph[p].grid), gx = uni(ph[p].gx);
        const char* arg = a.prog + uni(ph[p].arg);
        StepWait sw{p > 0 ? a.flags : nullptr, a.epoch + (unsigned)p, a.spin, a.fault};
        if (bid < grid) {
            if (kind == PH_FG) {
                if (!fg_run<false, false, true>(*(const FgDesc*)arg, (const int*)arg, bid, grid, sw, tid)) return;
            } else if (kind == PH_ADEC) {
                // one (key head, superblock) a workgroup on waves 0..3, as the kernel; it waits
                // for the previous phase once its old keys and values are on their way
                const AdecArgs& A = *(const AdecArgs*)arg;
                if (wave < SLM_SB_SEGS) {
                    if (!attn_dec_body<V, false, true>(A.part, A.q, A.kc, A.vc, A.dyn, A.pos_imm, A.reach,
                                                       A.gap, A.cap, (int)A.heads, (int)A.key_heads,
                                                       (int)A.dh, A.scale, nullptr, nullptr, bid % gx,
                                                       bid / gx, grid / gx, tid, &sw, &gave))
                        return;
                } else {  // the body's barriers: the wait's, then its own
                    lds_bar();
                    if (gave) return;
                    __syncthreads();
                }
            } else {
                if (!gla1_body<V, true>(*(const GlaDesc*)arg, bid, tid, SLM_STEP_THREADS, &sw, &gave)) return;
            }
        }
        // this workgroup's stores are complete before its flag moves
        __builtin_amdgcn_s_waitcnt(0);
        __builtin_amdgcn_s_setprio(0);  // (a fused GEMV's prologue waves raised theirs)
        __syncthreads();
        if (tid == 0) {
            const StepArgs& e = *step_args();
            __hip_atomic_store(e.flags + bid, e.epoch + (unsigned)p + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}
KERNEL void __launch_bounds__(SLM_STEP_THREADS) slm_step_1(const StepArgs) { step_run<1>(); }
KERNEL void __launch_bounds__(SLM_STEP_THREADS) slm_step_2(const StepArgs) { step_run<2>(); }
KERNEL void __launch_bounds__(SLM_STEP_THREADS) slm_step_4(const StepArgs) { step_run<4>(); }
