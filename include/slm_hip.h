/* slm_hip.h — the C ABI of the MI355X (gfx950) backend for SLM.use's token loop.
 *
 * One entry point per method of the reference's operator trait `Ops` (src/ops.rs:68-228).
 * The reference's model (src/model.rs) drives that trait; a Rust `impl Ops for Hip`
 * binds these functions one to one, the way src/cuda.rs binds its CUDA kernels, so
 * model.rs, the loop-count logic, the sampler, the CLI and the server run unchanged
 * above it.
 *
 * Conventions, all from src/ops.rs:1-9 and the trait signatures:
 *   - Every buffer is flat fp32 in device memory, allocated by slm_hip_alloc/upload.
 *   - An `At { buf, offset }` view (ops.rs:13-17) is passed as `buf + offset`.
 *   - Outputs never alias inputs, except the in/out state of gla (`s`) and store
 *     (`cache`), as the trait's `&mut` signatures guarantee.
 *   - Sizes are element counts. The caller sizes every output; the library checks each
 *     pointer range against its own allocation table and returns SLM_E_BOUNDS, touching
 *     nothing, when a range falls outside one live allocation.
 *   - Work is queued on one stream per context; slm_hip_read waits for it (ops.rs:88).
 *   - Every function returns SLM_OK (0) or a negative SLM_E_* code; the message is kept
 *     in the context (slm_hip_last_error), as src/cuda.rs:138 names the failing op.
 *   - One context is used from one thread at a time (src/serve.rs:1-3).
 */
#ifndef SLM_HIP_H
#define SLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    SLM_OK = 0,
    SLM_NO_DEVICE = 1,        /* slm_hip_open only: no usable GPU; not an error (cuda.rs:72-83) */
    SLM_E_INVALID = -1,       /* bad argument (null pointer, zero size where one is needed) */
    SLM_E_HIP = -2,           /* the HIP runtime failed */
    SLM_E_UNSUPPORTED = -3,   /* a shape the kernels do not handle, e.g. head size > 256 */
    SLM_E_MEMORY = -4,        /* device allocation failed */
    SLM_E_BOUNDS = -5         /* a pointer range is outside every live allocation */
};

typedef struct slm_hip slm_hip;

/* src/ops.rs:34-46. `reach` may be SIZE_MAX (global layers, model.rs:530). */
typedef struct slm_attn {
    size_t pos, m, reach, gap, cap, heads, key_heads, dh;
    float scale;
} slm_attn;

/* ---- context: replaces Cuda::probe (src/cuda.rs:72-120) and Ops::name (ops.rs:71) ---- */

/* Opens `device`, loads the embedded gfx950 code object with hipModuleLoadData. Returns
 * SLM_NO_DEVICE (and *out = NULL) on a machine without a usable GPU. */
int slm_hip_open(int device, slm_hip** out);
void slm_hip_close(slm_hip* ctx);
/* The last error message of this context ("" if none). NULL ctx: the last open failure. */
const char* slm_hip_last_error(const slm_hip* ctx);
/* Ops::name (ops.rs:71): writes e.g. "hip (AMD Instinct MI355X, gfx950)" into out[n]. */
int slm_hip_name(slm_hip* ctx, char* out, size_t n);

/* ---- buffers: Ops::zeros / zeros_cache / upload / upload_cache / read / flush
 *      (ops.rs:72-91; cuda.rs:152-169) ---- */

/* A zeroed buffer of max(n, 1) floats (ops.rs:72, cuda.rs:152-154). */
int slm_hip_alloc(slm_hip* ctx, size_t n, float** out);
/* A zeroed buffer of max(n, 1) fp16 values, for the weights of fp16 mode (mlx.rs:62 uploads
 * in the backend's dtype; no counterpart in the f32 trait). The pointer is typed float* like
 * every buffer but addresses halves: slm_hip_upload into it (at its start) rounds n floats to
 * fp16, to nearest even; slm_hip_read from it widens them back; slm_hip_linear takes it as
 * weights in fp16 mode only (SLM_E_UNSUPPORTED otherwise), with the bits of fp16 mode on the
 * same weights in fp32 (the fp16 chain rounds them to the same halves) and half the bytes.
 * No other operation takes it. Freed with slm_hip_free. */
int slm_hip_alloc_half(slm_hip* ctx, size_t n, float** out);
/* Ops::zeros_cache (ops.rs:73-76): a zeroed [heads][cap][dh] cache. In fp16 mode, where the
 * fp16 attention kernels take it (head size at most 64 and a multiple of 8, at least 64 slots),
 * the cache holds fp16 values, as the reference's MLX backend keeps every cache in its dtype
 * (mlx.rs:57-59): slm_hip_store rounds what it writes to fp16 (nearest even), slm_hip_attend
 * reads the halves widened exactly, slm_hip_upload into it rounds and slm_hip_read widens;
 * half the bytes of an fp32 ring. Otherwise an fp32 buffer, as slm_hip_alloc. */
int slm_hip_alloc_cache(slm_hip* ctx, size_t heads, size_t cap, size_t dh, float** out);
/* Doubles a cache (model.rs:383-398's relayout, on the device): head h's cap·dh values of src
 * ([heads][cap][dh]) to the start of its 2·cap·dh in dst ([heads][2·cap][dh], from
 * slm_hip_alloc_cache, zero past them). Both fp32 or both fp16. No counterpart in the trait:
 * what a `grow_cache` trait method with model.rs's host round trip as its default would call
 * (INTEGRATION.md). */
int slm_hip_grow_cache(slm_hip* ctx, float* dst, const float* src, size_t heads, size_t cap, size_t dh);
int slm_hip_free(slm_hip* ctx, float* buf);
/* Copies n host floats into dst (Ops::upload, ops.rs:77). */
int slm_hip_upload(slm_hip* ctx, float* dst, const float* src, size_t n);
/* Waits for pending work and copies n floats to the host (Ops::read, ops.rs:88-89). When the
 * same range was read right after the previous replay of the one-token step graph just
 * replayed, and nothing was queued since, the backend has already queued a copy of it into
 * mapped host memory behind the step (read-ahead) and the read only waits for that copy's flag
 * (the usual copy after a second, or if anything else came between). */
int slm_hip_read(slm_hip* ctx, float* host, const float* dev, size_t n);
/* Reads served by the read-ahead copy since the context opened. */
int slm_hip_read_ahead_stats(slm_hip* ctx, uint64_t* reads);
/* Ops::flush (ops.rs:90-91): called once at the end of every advance with every buffer
 * that outlives it. With step graphs on it ends the step (see slm_hip_set_graphs). */
int slm_hip_flush(slm_hip* ctx, const float* const* keep, size_t nkeep);

/* ---- the operations (ops.rs:93-227; cpu.rs:66-403 define the arithmetic) ---- */

/* y[i] = w[ids[i]], rows of d (ops.rs:93-94). `ids` is host memory. */
int slm_hip_gather(slm_hip* ctx, float* y, const float* w, const uint32_t* ids, size_t m,
                   size_t d);
/* One row of w at an index held in device memory (id[0], a long long below `rows`): the
 * gather of ops.rs:93-94 for one token whose id a device-side pick wrote, so greedy decode
 * steps follow each other with no host round trip (replaces the host ids of slm_hip_gather
 * in that loop, main.rs:219-222). */
int slm_hip_gather_dev(slm_hip* ctx, float* y, const float* w, const long long* id, size_t rows,
                       size_t d);
/* Greedy pick on the device: the index of the first maximum of x[0..n) under sample.rs:48-53
 * (b = 0, b = i whenever x[i] > x[b]: NaNs never win; a NaN at 0 keeps 0), written to tok[0]
 * and, when ids is not null, to ids[slot] (ids holds ids_cap uint32). Replaces the logits
 * read-back and host scan of main.rs:219 and sample.rs:33-50 in the greedy loop. */
int slm_hip_argmax(slm_hip* ctx, long long* tok, uint32_t* ids, size_t ids_cap, size_t slot,
                   const float* x, size_t n);
/* y = x (ops.rs:95). */
int slm_hip_copy(slm_hip* ctx, float* y, const float* x, size_t n);
/* y[0] = first, y[i] = x[i-1], rows of d (ops.rs:96-104). */
int slm_hip_shift(slm_hip* ctx, float* y, const float* first, const float* x, size_t m,
                  size_t d);
/* y[i] = x[i][off .. off+len], rows of `stride` (ops.rs:105-115). */
int slm_hip_columns(slm_hip* ctx, float* y, const float* x, size_t m, size_t stride,
                    size_t off, size_t len);
/* y[i] = w·x[i], w of rows × cols (ops.rs:116-126). */
int slm_hip_linear(slm_hip* ctx, float* y, const float* w, size_t rows, size_t cols,
                   const float* x, size_t m);
/* y = a + b (ops.rs:127). */
int slm_hip_add(slm_hip* ctx, float* y, const float* a, const float* b, size_t n);
/* y[i] = x[i] + row (ops.rs:128-136). */
int slm_hip_add_row(slm_hip* ctx, float* y, const float* x, const float* row, size_t m,
                    size_t d);
/* y[i] = f[i]·x[i], m = number of factors; `f` is host memory (ops.rs:137-138). */
int slm_hip_scale_rows(slm_hip* ctx, float* y, const float* x, const float* f, size_t m,
                       size_t d);
/* y = a + t·(b − a) (ops.rs:139-147). */
int slm_hip_mix(slm_hip* ctx, float* y, const float* a, const float* b, size_t n, float t);
/* RMSNorm over `groups` runs of `size`, shared weight w (ops.rs:148-158). */
int slm_hip_rms(slm_hip* ctx, float* y, const float* x, const float* w, size_t groups,
                size_t size, float eps);
/* y = silu(g)·u (ops.rs:159-166). */
int slm_hip_silu_mul(slm_hip* ctx, float* y, const float* g, const float* u, size_t n);
/* [m][half] cos/sin tables for positions pos.. (ops.rs:167-177). The first call of
 * every advance (model.rs:566); with step graphs on it begins the step. */
int slm_hip_rope_table(slm_hip* ctx, float* cos, float* sin, const float* inv, size_t pos,
                       size_t m, size_t half);
/* Half-split rotary embedding (ops.rs:178-188). */
int slm_hip_rope(slm_hip* ctx, float* y, const float* x, const float* cos, const float* sin,
                 size_t m, size_t heads, size_t dh);
/* L2-normalises `heads` runs of dh (ops.rs:189-190). */
int slm_hip_l2norm(slm_hip* ctx, float* y, const float* x, size_t heads, size_t dh);
/* Gated linear attention over m tokens in order, state s in/out (ops.rs:191-205). */
int slm_hip_gla(slm_hip* ctx, float* y, float* s, const float* q, const float* k,
                const float* v, const float* decay, const float* bias, size_t m,
                size_t heads, size_t dh);
/* Writes m [heads][dh] rows into ring slots (pos+i) % cap of cache [heads][cap][dh]
 * (ops.rs:206-217); into an fp16 cache (slm_hip_alloc_cache in fp16 mode) rounded to fp16. */
int slm_hip_store(slm_hip* ctx, float* cache, const float* src, size_t pos, size_t m,
                  size_t cap, size_t heads, size_t dh);
/* Softmax attention of m queries over the ring (ops.rs:218-227). `scores` is the trait's
 * scratch; this backend keeps its own workspace and ignores it (it may be NULL). `k` and
 * `v` are [key_heads][cap][dh], both fp32 or both fp16 caches (slm_hip_alloc_cache); fp16
 * values are widened exactly, so the result is that of fp32 rings holding the same values. */
int slm_hip_attend(slm_hip* ctx, float* y, float* scores, const float* q, const float* k,
                   const float* v, const slm_attn* a);
/* slm_hip_attend without allocation. No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under their own HIP graph capture of the context's
 * stream, serving loops, harnesses that forbid hipMalloc). The superblock partials go to a
 * fixed array of 16 MiB per GPU (static device memory, held until the process ends) instead of
 * the context's workspace, and the call issues kernel launches only — no hipMalloc, hipFree,
 * copy, fill or event. Results are bitwise those of slm_hip_attend. SLM_E_UNSUPPORTED when the
 * partials, nsb · m · heads · (dp + 2) · 4 bytes (nsb: the 256-key superblocks the queries
 * span; dp: 16 · 2^⌈log2 ⌈dh / 16⌉⌉), exceed 16 MiB, or when called inside a recorded step. Every call on one GPU shares that GPU's array: calls that overlap on
 * one GPU (two streams or contexts at once) race. */
int slm_hip_attend_noalloc(slm_hip* ctx, float* y, float* scores, const float* q, const float* k,
                           const float* v, const slm_attn* a);

/* ---- steps (no trait counterpart; backend settings like cuda.rs's one stream) ----
 * With step graphs or fusion on (both are by default), the operations of one advance —
 * from rope_table to flush — are recorded instead of launched. At flush the planner
 * lowers the step (fusing one-token runs when fusion is on); with graphs on, flush
 * replays a cached hipGraph when the step matches a recorded one (same operations,
 * buffers and sizes; positions, ids and factors may differ) and captures a new one
 * otherwise, and with graphs off it launches the planned kernels directly. A read, free
 * or upload inside a step runs what was recorded so far and finishes the step eagerly.
 * Results are identical in every mode: the same arithmetic runs. */
int slm_hip_set_graphs(slm_hip* ctx, int on);
/* One-launch steps (off by default; no trait counterpart, a backend setting): with graphs on,
 * a one-token step whose planned kernels are all fp32 fused GEMVs, one-token attentions that
 * leave their superblock partials to the next fused GEMV and one-token GLAs runs as ONE
 * launch of 256 workgroups (one per compute unit) that runs those kernels' work as phases in
 * order, each phase waiting for every workgroup to finish the one before (flags in device
 * memory, polled; values handed between phases by device-scope loads and stores); other
 * steps replay a graph. A phase's weights, and an attention phase's older keys and values,
 * are issued before its wait. Same kernels' arithmetic, so the same bits. Needs 256 compute
 * units free for the launch. Off by default: on the MI355X it measured slower than the
 * step graph (a86 at R = 4: 1625 against 1850 tok/s). */
int slm_hip_set_step_kernel(slm_hip* ctx, int on);
/* One-launch steps run and programs built since the context opened, and whether the device
 * can run them (1) or every step goes through a graph (0). */
int slm_hip_step_stats(slm_hip* ctx, uint64_t* launches, uint64_t* programs, int* available);
/* Prompt lanes (1 to 4; no trait counterpart, a backend setting): consecutive prompt steps
 * (advances of more than one token, ended by a flush) run on up to n streams at once, so
 * that chunk c + 1 starts while chunk c still runs. What a step writes and its flush does not
 * keep is dead once the step is over (ops.rs:90-91): on lanes other than the first the step
 * writes it into copies of the lane's own, and a lane waits for another only before its first
 * kernel that may touch a kept buffer (a ring, a state, a cache) that the other used last.
 * Anything else on the context (a read, an upload, a free, a one-token step) first waits for
 * every lane. A step that reads scratch before writing it, frees or grows a buffer, or holds
 * a one-token attention or a device pick runs on the context's stream as before. Results
 * are identical for any n: the same kernels run on the same values. */
int slm_hip_set_prompt_lanes(slm_hip* ctx, int n);
/* The prompt lanes in use. */
int slm_hip_get_prompt_lanes(slm_hip* ctx, int* n);
/* Prompt steps run on a lane, and those that could not, since the context opened. */
int slm_hip_prompt_lane_stats(slm_hip* ctx, uint64_t* steps, uint64_t* fallbacks);
/* fp16 mode (off by default), the analogue of the reference's --fp16 (mlx.rs:19-23,
 * main.rs:421-423, where it selects Float16 for every MLX buffer): from this call on, every
 * buffer holds fp16 values, as mlx.rs's Float16 arrays do. An upload rounds to fp16 (to
 * nearest even; mlx.rs:61-63), and every operation rounds what it writes — activations,
 * GLA states, norms' outputs, attention outputs — at mlx.rs's rounding points (a product or
 * sum of two arrays, a scalar factor turned into the dtype, RMSNorm's fp32 quotient before
 * its weight, mlx.rs:178-185; rope angles in fp32, mlx.rs:203-208); reductions (a linear's
 * chain, a norm's dot, attention's softmax, the GLA's column sums) sum in fp32. Linears round
 * both operands to fp16 at fp16 MFMAs; a linear then needs a multiple of 64 columns and
 * 16-byte aligned weights and input (else SLM_E_UNSUPPORTED). Caches from
 * slm_hip_alloc_cache hold halves. Set it before the model uploads its weights, as the
 * reference fixes the dtype when it creates the backend (mlx.rs:19-23): weights uploaded
 * before keep their fp32 values, which the linears then round themselves. The first linear
 * that reads a weight buffer keeps an fp16 copy of it (half the weight bytes, the same bits),
 * dropped when the buffer is freed, uploaded into or written by an operation. */
int slm_hip_set_fp16(slm_hip* ctx, int on);
/* Whether fp16 mode is on. */
int slm_hip_get_fp16(slm_hip* ctx, int* on);
/* The fp16 weight copies of fp16 mode (on by default; no trait counterpart, a measurement and
 * test switch): off, fp16-mode linears read the fp32 weights and round them themselves (the
 * same bits, twice the bytes), and the copies are freed. */
int slm_hip_set_half_shadows(slm_hip* ctx, int on);
/* Fusion (on by default): the planner lowers a recorded one-token step into fused
 * kernels (prologue vector ops + GEMV + epilogue) that compute the same values with the
 * same arithmetic as the per-op kernels. Off: one launch per operation. */
int slm_hip_set_fusion(slm_hip* ctx, int on);
/* Rows per tile of the fused one-token GEMV (no trait counterpart; a test and measurement
 * switch): 0 (the default) lets the planner choose 16, 12, 8 or 4 per linear (smaller tiles spread
 * a short matrix over more compute units); 16, 12, 8 or 4 forces that size wherever the linear's
 * row pairs allow it. Results are the same bits at every size. */
int slm_hip_set_tile_rows(slm_hip* ctx, int rows);
/* Counters for tests and benchmarks: graphs launched, graphs captured, eager steps. */
int slm_hip_graph_stats(slm_hip* ctx, uint64_t* launched, uint64_t* captured,
                        uint64_t* eager);
/* Operations recorded and kernel launches planned for the last step that was lowered. */
int slm_hip_last_plan(slm_hip* ctx, uint64_t* ops, uint64_t* kernels);

/* Kernel statistics (no counterpart in the reference; a measurement aid). While timing is
 * on, every launch made outside a graph is bracketed by HIP events on the backend's stream;
 * slm_hip_kernel_stat returns, for the kernel `name` (e.g. "slm_fg"), the launches, their
 * summed duration in microseconds and the algorithmic bytes they move (weights, inputs and
 * outputs). slm_hip_set_timing resets the statistics. */
int slm_hip_set_timing(slm_hip* ctx, int on);
int slm_hip_kernel_stat(slm_hip* ctx, const char* name, long long* launches, double* us,
                        double* bytes);

/* ---- diagnostics (no trait counterpart) ----
 * One v_mfma_f32_16x16x4f32 on one wave: lane l supplies a[l] and b[l] (device, 64 floats
 * each) and writes the four result elements it holds to out[4l .. 4l+3] (256 floats).
 * Tests use it to pin the lane layout the kernels assume. */
int slm_hip_probe_mfma(slm_hip* ctx, float* out, const float* a, const float* b);
/* Bounded waits (no trait counterpart; a safety net). Fused kernels synchronise some of their
 * waves through polls of LDS that give up after `polls` tries instead of waiting forever; a
 * wait that gives up sets a fault word, and the next slm_hip_read or slm_hip_flush returns
 * SLM_E_HIP (the results of the work since the previous check are not valid). The default is
 * 2^24 polls; 0 makes every such wait give up at once (tests use it to exercise the error
 * path: every kernel still runs to its end). Applies to steps recorded from this call on. */
int slm_hip_set_spin_limit(slm_hip* ctx, long long polls);
/* The context's hipStream_t, so a caller can time its work with HIP events. */
int slm_hip_stream(slm_hip* ctx, void** out);
/* Device memory (no trait counterpart; a diagnostic): the device's free and total bytes
 * (hipMemGetInfo) and the bytes this context holds from the device — its pool slabs, its
 * direct allocations and its internal buffers. */
int slm_hip_mem_info(slm_hip* ctx, size_t* free_bytes, size_t* total_bytes, size_t* held_bytes);

#ifdef __cplusplus
}
#endif

#endif /* SLM_HIP_H */
