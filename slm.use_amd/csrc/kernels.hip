// gfx950 (CDNA4) kernels for the token loop of SLM.use: one code object, loaded by the
// host runtime with hipModuleLoadData. Compiled with -ffp-contract=off so that every
// expression rounds exactly as written wherever it is inlined.
//
// Each operation computes every output element in an order that does not depend on how
// many tokens a call carries (m = 1 decode or an m = 256 prompt chunk), so a prompt read
// in chunks leaves bit-identical state to one read token by token:
//   - linear: one fixed MFMA chain per output (v_mfma_f32_16x16x4f32 over 16-column
//     blocks, columns split into 256-wide slices whose partial sums are added in order);
//     the m <= 16 kernel and the m > 16 kernel run the same chain;
//   - attend: keys are grouped by absolute position into 16-key tiles, 64-key segments
//     and 512-key superblocks; a segment is an online softmax over its tiles, segments
//     fold into superblocks in order and superblocks into the result in order;
//   - gla: one kernel for every m, tokens in order;
//   - rms / l2norm: the 16-accumulator dot of the reference CPU backend (src/cpu.rs:9-21),
//     so these two are bit-identical to it;
//   - the rest is element-wise.

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef float f4 __attribute__((ext_vector_type(4)));

#define KERNEL extern "C" __global__

#define GRID_LOOP(i, n)                                                              \
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < (n);    \
         i += (long long)gridDim.x * blockDim.x)

static constexpr float NEG_INF = -__builtin_inff();

__device__ __forceinline__ long long dyn_or(const long long* dyn, long long imm) {
    return dyn ? dyn[0] : imm;
}

__device__ __forceinline__ f4 mfma4(float a, float b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
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

KERNEL void slm_add(float* __restrict__ y, const float* __restrict__ a,
                    const float* __restrict__ b, long long n) {
    GRID_LOOP(i, n) y[i] = a[i] + b[i];
}

KERNEL void slm_add_row(float* __restrict__ y, const float* __restrict__ x,
                        const float* __restrict__ row, long long n, long long d) {
    GRID_LOOP(i, n) y[i] = x[i] + row[i % d];
}

KERNEL void slm_mix(float* __restrict__ y, const float* __restrict__ a,
                    const float* __restrict__ b, long long n, float t) {
    GRID_LOOP(i, n) y[i] = a[i] + t * (b[i] - a[i]);
}

// y = silu(g)·u = u·g / (1 + e^-g), cpu.rs:209-215.
KERNEL void slm_silu_mul(float* __restrict__ y, const float* __restrict__ g,
                         const float* __restrict__ u, long long n) {
    GRID_LOOP(i, n) {
        float v = g[i];
        y[i] = u[i] * v / (1.0f + expf(-v));
    }
}

// y[i] = f[i]·x[i] with rows of d; one factor `f0` when `f` is null.
KERNEL void slm_scale_rows(float* __restrict__ y, const float* __restrict__ x,
                           const float* __restrict__ f, float f0, long long n, long long d) {
    GRID_LOOP(i, n) y[i] = x[i] * (f ? f[i / d] : f0);
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
        y[at + i] = a * c - b * s;
        y[at + half + i] = a * s + b * c;
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
    for (int c = 0; c < chunks; c++) {
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
    for (int j = l; j < size; j += 16) out[j] = MODE == 0 ? in[j] * r * w[j] : in[j] * r;
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
// Four lanes per state column (head h, column b); lane j owns rows j·RPL .. j·RPL+RPL-1
// of S[h][:, b] in registers. Tokens run in order: d = 1/(1 + e^(decay + bias)),
// S[a][b] = d·S[a][b] + k[a]·v[b], y[b] = Σ_a q[a]·S[a][b], where each lane sums its rows
// in order and the four partial sums are added as (P0 + P1) + (P2 + P3).
template <int RPL>
__device__ void gla_body(float* __restrict__ y, float* __restrict__ S,
                         const float* __restrict__ q, const float* __restrict__ k,
                         const float* __restrict__ v, const float* __restrict__ decay,
                         const float* __restrict__ bias, int m, int heads, int dh) {
    long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    long long col = t >> 2;
    int j = (int)(t & 3);
    bool live = col < (long long)heads * dh;
    int h = live ? (int)(col / dh) : 0, b = live ? (int)(col % dh) : 0;
    float* Sh = S + (long long)h * dh * dh;
    float st[RPL];
#pragma unroll
    for (int rr = 0; rr < RPL; rr++) {
        int a = j * RPL + rr;
        st[rr] = (live && a < dh) ? Sh[(long long)a * dh + b] : 0.0f;
    }
    float bh = live ? bias[h] : 0.0f;
    for (int i = 0; i < m; i++) {
        long long at = ((long long)i * heads + h) * dh;
        float dc = live ? 1.0f / (1.0f + expf(decay[(long long)i * heads + h] + bh)) : 0.0f;
        float vb = live ? v[at + b] : 0.0f;
        float part = 0.0f;
#pragma unroll
        for (int rr = 0; rr < RPL; rr++) {
            int a = j * RPL + rr;
            if (live && a < dh) {
                st[rr] = dc * st[rr] + k[at + a] * vb;
                part = part + q[at + a] * st[rr];
            }
        }
        float t1 = part + __shfl_xor(part, 1);
        float t2 = t1 + __shfl_xor(t1, 2);
        if (live && j == 0) y[at + b] = t2;
    }
#pragma unroll
    for (int rr = 0; rr < RPL; rr++) {
        int a = j * RPL + rr;
        if (live && a < dh) Sh[(long long)a * dh + b] = st[rr];
    }
}

#define GLA(R)                                                                          \
    KERNEL void __launch_bounds__(256)                                                  \
        slm_gla_##R(float* y, float* S, const float* q, const float* k, const float* v, \
                    const float* decay, const float* bias, int m, int heads, int dh) {  \
        gla_body<R>(y, S, q, k, v, decay, bias, m, heads, dh);                          \
    }
GLA(1)
GLA(2)
GLA(4)
GLA(8)
GLA(16)
GLA(32)
GLA(64)

// ---------------------------------------------------------------------------------------
// linear: y[i][r] = Σ_c w[r][c]·x[i][c] (ops.rs:116-126)
// ---------------------------------------------------------------------------------------
//
// The canonical chain, shared by both kernels below. For v_mfma_f32_16x16x4f32 lane l
// holds A[l%16][l/16], B[l/16][l%16] and D[4(l/16)+r][l%16] in element r. Rows of w are
// A's rows, tokens are B's columns. Columns go in blocks of 16: lane group g = l/16 loads
// the four columns 16kb+4g .. 16kb+4g+3 of its row (of w) and of its token (of x), and
// MFMA e (e = 0..3) takes element e of both, so MFMA e of block kb sums the columns
// {16kb + 4g + e : g = 0..3}. Blocks are chained in order within a slice of 16 blocks
// (256 columns) starting from zero, and the slice sums are added in order:
// y = ((P0 + P1) + P2) + ...   Columns past `cols` load as zero.

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

// m <= 16: one workgroup per 16 rows, one wave per slice (waves take slices w, w+W, ...),
// slice partials meet in LDS and one pass adds them in order. A wave loads its whole
// slice (16 rows x 256 columns of w, and the tokens' columns) before the chain starts, so
// one memory latency covers it.
template <bool VEC>
__device__ void linear_small_body(float* __restrict__ y, const float* __restrict__ w,
                                  const float* __restrict__ x, int rows, int cols, int m) {
    extern __shared__ float part[];  // [slices][16 rows][16 tokens]
    int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    int i = lane & 15, g = lane >> 4;
    long long r0 = (long long)blockIdx.x * 16;
    int kblocks = (cols + 15) >> 4, nsl = (kblocks + 15) >> 4;
    for (int s = wave; s < nsl; s += waves) {
        int nkb = min(16, kblocks - s * 16);
        f4 wa[16], xb[16];
#pragma unroll
        for (int u = 0; u < 16; u++) {
            long long c = (long long)(s * 16 + u) * 16 + g * 4;
            wa[u] = f4{0.0f, 0.0f, 0.0f, 0.0f};
            xb[u] = f4{0.0f, 0.0f, 0.0f, 0.0f};
            if (u < nkb) {
                wa[u] = ld4<VEC>(w, r0 + i, rows, cols, c);
                xb[u] = ld4<VEC>(x, i, m, cols, c);
            }
        }
        f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int u = 0; u < 16; u++) {
            if (u < nkb) {
                acc = mfma4(wa[u].x, xb[u].x, acc);
                acc = mfma4(wa[u].y, xb[u].y, acc);
                acc = mfma4(wa[u].z, xb[u].z, acc);
                acc = mfma4(wa[u].w, xb[u].w, acc);
            }
        }
        float* p = part + s * 256;
#pragma unroll
        for (int r = 0; r < 4; r++) p[(4 * g + r) * 16 + i] = acc[r];
    }
    __syncthreads();
    for (int t = threadIdx.x; t < 256; t += blockDim.x) {
        int rr = t >> 4, tt = t & 15;
        float tot = part[t];
        for (int s = 1; s < nsl; s++) tot = tot + part[s * 256 + t];
        if (r0 + rr < rows && tt < m) y[(long long)tt * rows + r0 + rr] = tot;
    }
}

KERNEL void __launch_bounds__(512) slm_linear_small_v(float* y, const float* w, const float* x,
                                                      int rows, int cols, int m) {
    linear_small_body<true>(y, w, x, rows, cols, m);
}
KERNEL void __launch_bounds__(512) slm_linear_small_s(float* y, const float* w, const float* x,
                                                      int rows, int cols, int m) {
    linear_small_body<false>(y, w, x, rows, cols, m);
}

// m > 16: a 64-row × 64-token tile per workgroup, 32 × 32 per wave (2 × 2 MFMA tiles).
template <bool VEC>
__device__ void linear_big_body(float* __restrict__ y, const float* __restrict__ w,
                                const float* __restrict__ x, int rows, int cols, int m) {
    int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int i = lane & 15, g = lane >> 4;
    long long rb = (long long)blockIdx.x * 64 + (wave & 1) * 32;
    long long tb = (long long)blockIdx.y * 64 + (wave >> 1) * 32;
    int kblocks = (cols + 15) >> 4, nsl = (kblocks + 15) >> 4;
    f4 tot[2][2];
    for (int s = 0; s < nsl; s++) {
        f4 acc[2][2];
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int v = 0; v < 2; v++) acc[u][v] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        int kb1 = min(s * 16 + 16, kblocks);
        for (int kb = s * 16; kb < kb1; kb++) {
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
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int v = 0; v < 2; v++) tot[u][v] = s == 0 ? acc[u][v] : tot[u][v] + acc[u][v];
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

// ---------------------------------------------------------------------------------------
// attention (ops.rs:31-66, 218-227; cpu.rs:352-403)
// ---------------------------------------------------------------------------------------
//
// A wave works on 16 columns; column c is query (qtile·qpt + c/group) of query head
// (kvh·group + c%group), all sharing kv head kvh (group = heads / key_heads, qpt =
// 16 / group). The query at position p sees [lo, hi) = [max(0, p-reach+1),
// max(0, p+1-gap)), stored at slots p % cap.
//
// Keys are grouped by absolute position: 16-key tiles, 64-key segments (4 tiles), 512-key
// superblocks (8 segments). A segment's partial (max m, sum l, o = Σ p·v) is an online
// softmax over its tiles in order; a tile with no visible key for a column leaves that
// column's partial unchanged. Partials fold in order: segments into a superblock (inside
// one workgroup, one wave per segment), superblocks into the result (slm_attn_combine).
// Scores use the same 16x16x4 MFMA chain over dh as linear; P·V runs four MFMAs per tile
// (MFMA r takes keys r, r+4, r+8, r+12).

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
// before any arithmetic (one memory latency per segment).
template <int DT>
__device__ void attn_segment(const Col& col, const f4 (&qv)[DT], const float* __restrict__ kb,
                             const float* __restrict__ vb, long long seg_lo, long long cap,
                             int dh, float scale, float& mo, float& lo, f4 (&o)[DT]) {
    int lane = threadIdx.x & 63;
    int i = lane & 15, g = lane >> 4;
    mo = NEG_INF;
    lo = 0.0f;
#pragma unroll
    for (int dt = 0; dt < DT; dt++) o[dt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    bool need[4];
    f4 kr[4][DT];
    float vr[4][4][DT];
#pragma unroll
    for (int st = 0; st < 4; st++) {
        long long b0 = seg_lo + 16 * st;
        bool sees = col.valid && col.lo < b0 + 16 && col.hi > b0;
        need[st] = __ballot(sees) != 0;
        if (need[st]) {
            // A operand of the scores: key b0 + i, dims 16t + 4g .. +3
            const float* krow = kb + ((b0 + i) % cap) * dh;
#pragma unroll
            for (int t = 0; t < DT; t++) {
                int c = 16 * t + 4 * g;
                kr[st][t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
                if (c < dh) kr[st][t] = *(const f4*)(krow + c);
            }
            // A operand of P·V for MFMA r: value of key b0 + 4g + r, dim 16dt + i
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float* vrow = vb + ((b0 + 4 * g + r) % cap) * dh;
#pragma unroll
                for (int dt = 0; dt < DT; dt++) {
                    int dim = 16 * dt + i;
                    vr[st][r][dt] = dim < dh ? vrow[dim] : 0.0f;
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
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        int anyi = any ? 1 : 0;
        anyi |= __shfl_xor(anyi, 16);
        anyi |= __shfl_xor(anyi, 32);
        float mnew = fmaxf(mo, mx);
        float muse = mnew == NEG_INF ? 0.0f : mnew;
        float p[4];
#pragma unroll
        for (int r = 0; r < 4; r++) p[r] = sv[r] == NEG_INF ? 0.0f : expf(sv[r] - muse);
        float rs = ((p[0] + p[1]) + p[2]) + p[3];
        rs = rs + __shfl_xor(rs, 16);
        rs = rs + __shfl_xor(rs, 32);
        float alpha = expf(mo - muse);
        f4 on[DT];
#pragma unroll
        for (int dt = 0; dt < DT; dt++) on[dt] = o[dt] * alpha;
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int dt = 0; dt < DT; dt++) on[dt] = mfma4(vr[st][r][dt], p[r], on[dt]);
        if (anyi) {
            lo = lo * alpha + rs;
            mo = mnew;
#pragma unroll
            for (int dt = 0; dt < DT; dt++) o[dt] = on[dt];
        }
    }
}

// Superblock partials. Grid (query tiles, key heads, superblock slots); 8 waves, wave w
// takes segment 8·sb + w, where sb = floor(first visible position / 512) + blockIdx.z.
// Output part[z][qidx][head][2 + DP]: m, l, o.
template <int DT>
__device__ void attn_part_body(float* __restrict__ part, const float* __restrict__ q,
                               const float* __restrict__ kc, const float* __restrict__ vc,
                               const long long* __restrict__ dyn, long long pos_imm, int m,
                               long long reach, long long gap, long long cap, int heads,
                               int key_heads, int dh, float scale, int wpp) {
    constexpr int DP = 16 * DT;
    extern __shared__ float lds[];  // [wpp][16][DP + 2]
    long long pos = dyn_or(dyn, pos_imm);
    int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int i = lane & 15, g = lane >> 4;
    int group = heads / key_heads, qpt = 16 / group;
    int kvh = blockIdx.y;
    long long first = (reach - 1 > pos) ? 0 : pos - (reach - 1);
    long long sb = first / 512 + blockIdx.z;
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
    attn_segment<DT>(col, qv, kc + (long long)kvh * cap * dh, vc + (long long)kvh * cap * dh,
                     (sb * 8 + wave) * 64, cap, dh, scale, mo, lo, o);
    // fold the 8 segments in order, wpp at a time through LDS
    constexpr int PER = (16 * DP + 511) / 512;  // (column, dim) pairs per thread
    float FM[PER], FL[PER], FO[PER];
#pragma unroll
    for (int u = 0; u < PER; u++) {
        FM[u] = NEG_INF;
        FL[u] = 0.0f;
        FO[u] = 0.0f;
    }
    for (int ph = 0; ph < 8; ph += wpp) {
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
            int t = threadIdx.x + 512 * u;
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
        int t = threadIdx.x + 512 * u;
        if (t < 16 * DP) {
            int cc = t / DP, dd = t % DP;
            Col c2 = column(cc, blockIdx.x, pos, m, reach, gap, group, qpt, kvh);
            if (c2.valid && dd < dh) {
                float* P = part + (((long long)blockIdx.z * m + c2.qidx) * heads + c2.head) *
                                      (long long)(DP + 2);
                if (dd == 0) {
                    P[0] = FM[u];
                    P[1] = FL[u];
                }
                P[2 + dd] = FO[u];
            }
        }
    }
}

#define ATTN_PART(DT)                                                                    \
    KERNEL void __launch_bounds__(512) slm_attn_part_##DT(                               \
        float* part, const float* q, const float* kc, const float* vc,                   \
        const long long* dyn, long long pos_imm, int m, long long reach, long long gap,  \
        long long cap, int heads, int key_heads, int dh, float scale, int wpp) {         \
        attn_part_body<DT>(part, q, kc, vc, dyn, pos_imm, m, reach, gap, cap, heads,      \
                           key_heads, dh, scale, wpp);                                   \
    }
ATTN_PART(1)
ATTN_PART(2)
ATTN_PART(4)
ATTN_PART(8)
ATTN_PART(16)

// y[qidx][head][dim] = O / L after folding the nsb superblock partials in order (0 when
// the query sees nothing, cpu.rs:378-382).
KERNEL void slm_attn_combine(float* __restrict__ y, const float* __restrict__ part, int m,
                             int heads, int dh, int dp, int nsb) {
    long long n = (long long)m * heads * dh;
    GRID_LOOP(t, n) {
        long long row = t / dh;
        int dd = (int)(t % dh);
        float M = NEG_INF, L = 0.0f, O = 0.0f;
        for (int z = 0; z < nsb; z++) {
            const float* P = part + ((long long)z * m * heads + row) * (dp + 2);
            fold(M, L, O, P[0], P[1], P[2 + dd]);
        }
        y[t] = L > 0.0f ? O / L : 0.0f;
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
