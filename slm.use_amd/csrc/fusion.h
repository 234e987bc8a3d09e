// Descriptors of the fused decode kernels, shared by the host planner (runtime.cpp) and
// the device code (kernels.hip): plain C layouts of fixed-width fields, passed by value
// as the single kernel argument.
//
// A fused GEMV (slm_fg) runs, for one token (m = 1), in a workgroup of two kinds of waves:
//   - GEMV waves, one per 64-column slice of a split: each issues the weight loads of its
//     first unit at once, then runs the canonical MFMA chain of its slice for every unit
//     of the workgroup, the loads of the next unit in flight while one unit computes;
//   - prologue/epilogue waves: they load every global vector the kernel reads into LDS,
//     run the prologue (the step's element-wise ops, rms, the
//     fold of a split linear's partials, rope-table rows, the embedding row) that makes
//     the GEMV input, then, per unit, add the slice partials in order and run the
//     epilogue (residual add, rope + ring store, SiLU of the gate/amp pair).
// A unit is one tile (16, 12, 8 or 4 rows) of one split of one weight matrix; units go
// round-robin over the grid. Every value is computed with the same expression, in the same order, as the
// per-op kernels, so fused and unfused runs give the same bits.
#ifndef SLM_FUSION_H
#define SLM_FUSION_H

#include <stdint.h>

#define SLM_VP_MAX 12
#define SLM_SEG_MAX 3
#define SLM_PF_MAX 12
#define SLM_KS 4               // 16-column blocks per canonical slice (64 columns)
#define SLM_SPLIT 12           // slices per canonical split (768 columns)
#define SLM_FG_EPI_WAVES 4     // prologue/epilogue waves of slm_fg
#define SLM_SB_SEGS 4          // 64-key attention segments per superblock
#define SLM_SB_KEYS (64 * SLM_SB_SEGS)
#define SLM_GLA_T 32           // tokens per LDS stage of the prompt GLA kernel
#define SLM_GLA_COLS 16        // state columns per workgroup of the prompt GLA kernel (16 lanes each)
#define SLM_FG_MISC (32 + 4 * SLM_PF_MAX)  // LDS floats of slm_fg's scalars and prefetch table
#define SLM_SIG_OPS 7          // prologue ops a signature can name
// The signature of a prologue of kinds k0, k1, ...: what FgDesc.sig holds.
#define SLM_SIG1(a) (1 | ((a) << 4))
#define SLM_SIG2(a, b) (2 | ((a) << 4) | ((b) << 8))
#define SLM_SIG3(a, b, c) (3 | ((a) << 4) | ((b) << 8) | ((c) << 12))
#define SLM_SIG4(a, b, c, e) (4 | ((a) << 4) | ((b) << 8) | ((c) << 12) | ((e) << 16))
#define SLM_SIG5(a, b, c, e, f) (5 | ((a) << 4) | ((b) << 8) | ((c) << 12) | ((e) << 16) | ((f) << 20))

enum {
    VP_COPY = 1,    // out = in0
    VP_ADD,         // out = in0 + in1 (also add_row with one row)
    VP_MIX,         // out = in0 + f·(in1 − in0)
    VP_SCALE,       // out = in0 · factor (dyn[0] as f32 bits, else f)
    VP_RMS,         // out = rms(in0) · lds[w], eps f
    VP_SILU,        // out = in1 · in0 / (1 + e^−in0)   (silu_mul with g = in0, u = in1)
    VP_FOLD,        // out = ((P0 + P1) + P2) + ...: the splits of a linear, lds[w] [nsb][n]
    VP_COMB,        // out[head][dim] = the weight-max combine of one-token attention's nsb
                    // superblock partials, lds[w] [nsb][heads][dp + 2]
};

enum {
    EPI_PLAIN = 0,  // y (or the split's partial)
    EPI_RESID = 1,  // y; o1 = res + y                       (add after the linear)
    EPI_ROPE = 2,   // y = [q|k|v]; o1 = rope(q), o2 = rope(k), o3[ring] = o2, o4[ring] = v
    EPI_SILU = 3,   // y = [gate|amp]; o1 = amp · gate / (1 + e^−gate)
    EPI_PICK = 4,   // y; the greedy pick of y (the first maximum, sample.rs:48-53) to
                    // ((long long*)o1)[0] and ((unsigned*)o2)[slot] (o2 may be null; slot:
                    // dyn[0], else imm); o3: [0] the 64-bit key of the running maximum,
                    // [2] the count of finished workgroups (both zero between launches)
};

// A global vector copied into LDS by the prologue waves: src + dyn[0]·stride (when dyn).
// n is a multiple of 4 and the source 16-byte aligned.
typedef struct {
    const float* src;
    const long long* dyn;
    int32_t n, lds, stride, first4;  // first4: running count of float4s before this one
} PfOp;

typedef struct {
    int32_t kind, n, wg0;   // length; wg0: only workgroup 0 runs it (a side effect)
    int32_t out, in0, in1;  // LDS float offsets
    int32_t w;              // LDS offset of the rms weight / combine / fold partials (-1: `part`)
    int32_t heads, dh, dp, nsb;
    int32_t sync;           // 1: reads an element another thread's op produced (a barrier first)
    float* gout;            // global output, written by workgroup 0 (null: none)
    const float* part;      // combine partials in global memory (when w < 0)
    const long long* dyn;   // VP_SCALE factor on the device
    float f;
    float pad2;
} VpOp;

// One weight matrix of a fused GEMV. Its rows are grouped into tiles of rpt rows (16, 12, 8
// or 4; a tile fills rows 0..rpt-1 of the 16-row MFMA operand, the other rows are zeros): the
// first pair_rows rows (a multiple of 16) in tiles of rpt/2 (row, row + half) pairs, pair P
// at row (P / half)·2·half + P % half (the rope halves of a head, or the gate and amp rows of
// a SiLU pair), the rest in consecutive rows. Each row's chain is the same whatever the
// tile, so rpt only moves work between workgroups.
typedef struct {
    const float* w;         // weights [rows][cols]
    float* y;               // the linear's output
    float* part;            // nsplit > 1: the split partials [nsplit][rows]
    int32_t rows, tiles, nsplit, units, unit_first;
    int32_t pair_rows, half;
    int32_t epi, rpt, ring16;  // ring16 (ROPE): the rings hold fp16 values
    int32_t d, dh;          // ROPE: part width, head size
    int32_t cs_lds, sn_lds; // ROPE: LDS offsets of the cos / sin row
    // ceil(2^32 / tiles) and ceil(2^32 / half) (0 where the divisor is 0 or 1): the kernel's
    // n / d is the high word of n · m, exact while n · d < 2^32
    uint32_t mtiles, mhalf;
    float* o1;
    float* o2;
    float* o3;
    float* o4;
    const float* res;       // RESID: the residual
    long long cap;          // ring slots (ROPE)
    const long long* dyn;   // ring position of the k store (ROPE), else imm
    long long imm;
    const long long* dyn2;  // ring position of the v store (ROPE), else imm2
    long long imm2;
} FgSeg;

typedef struct __attribute__((aligned(16))) {
    int32_t npf, nvp, cols, nsl;    // nsl: canonical slices of `cols`
    int32_t W, xin, nseg, units;    // W: GEMV waves (slices per split); xin: LDS offset of x
    int32_t lds_vp, fold_off, pf4, f16;  // pf4: float4s the prologue loads; f16: fp16 mode MFMAs
    // cw ≥ 0: x is one-token attention's output, combined by the GEMV waves themselves:
    // wave w (one 64-column slice) combines head w (64 dims) from the superblock partials
    // in lds[cw] [cnsb][W][cdp + 2], and workgroup 0 writes the result to cgout
    int32_t cw, cdp, cnsb, spin;    // spin: polls a bounded wait makes before it gives up
    // sig: the prologue's op kinds when every op is a float4 op of at most one float4 per
    // prologue thread (4 bits each from bit 4, the count in bits 0..3; 0: run the general
    // loop); nsf: VP_SCALE ops whose factor lives on the device
    int32_t sig, nsf, pad0, pad1;
    float* cgout;
    int* fault;                     // a wait that gives up ORs 1 in here (host memory)
    PfOp pf[SLM_PF_MAX];
    VpOp vp[SLM_VP_MAX];
    FgSeg seg[SLM_SEG_MAX];
} FgDesc;

// Gated linear attention for one token with the ops around it in an L block
// (model.rs:463-484): optionally q, k = l2norm(q_raw), l2norm(k_raw) first; then
// y = gla(...); when fused further y2 = rms(y, head_norm) and out = silu(gate)·y2.
typedef struct {
    float* s;
    const float* q;
    const float* k;
    const float* v;
    const float* decay;
    const float* bias;
    float* y;        // the gla output
    float* y2;       // rms output
    float* out;      // silu_mul output
    const float* hn; // head_norm weight
    const float* gate;
    float* qn;       // l2: the normalised q and k, written out
    float* kn;
    int32_t heads, dh, fuse, l2;
    float eps;
    int32_t r16;     // fp16 mode: every value written rounded to fp16
} GlaDesc;

// A one-token step in one launch (slm_step): the kernels the planner made for the step, in
// order, as phases of a program that every workgroup of a 256-workgroup launch runs through.
// Workgroup w stores epoch + p + 1 into flags[w] when it is done with phase p; phase p
// begins with a wait until every flag has reached epoch + p. What a phase reads that another
// phase of the same launch wrote is read and written past the caches that are not shared by
// the whole device (device-scope loads and stores), so a phase sees the last one's results
// without the cache write-back and invalidation a kernel boundary brings.
enum {
    PH_FG = 1,    // a fused GEMV: FgDesc (slm_fg)
    PH_ADEC = 2,  // one-token attention writing its superblock partials: AdecArgs (slm_attn_dec_*)
    PH_GLA1 = 3,  // one-token gated linear attention: GlaDesc (slm_gla1_*)
};
#define SLM_STEP_WG 256       // workgroups of a step launch
#define SLM_STEP_THREADS 1024 // threads of each
#define SLM_STEP_GROUP 4      // query heads per key head a step's attention phase takes
typedef struct {
    int32_t kind, var;  // var: the attention's dim tiles (0: 1, 1: 2, 2: 4) or the GLA's rows per lane
    int32_t grid, gx;   // workgroups that run the phase; the attention's key heads (its grid's x)
    int32_t arg, pad;   // byte offset of the phase's argument block from the program's start
} StepPh;
typedef struct {
    const char* prog;   // [nph] StepPh, then the argument blocks (16-byte aligned)
    unsigned* flags;    // [SLM_STEP_WG]
    int* fault;         // a wait that gives up ORs 1 in here (host memory)
    unsigned epoch;
    int32_t nph, spin, pad;
} StepArgs;
// The one-token attention's arguments as a launch record packs them: one 8-byte slot each.
typedef struct {
    float* part;
    const float* q;
    const float* kc;
    const float* vc;
    const long long* dyn;
    long long pos_imm, reach, gap, cap;
    long long heads, key_heads, dh;  // (ints in the low half of their slots)
    float scale, pad0;
    float* y;
    int* ctr;
} AdecArgs;

// A prompt row chain (m > 1 tokens): consecutive row-local element-wise ops between two
// GEMMs run as one launch, one workgroup per token row. Each op's operands come from the
// LDS copy of an earlier op's output row or from global memory (row r at g + r·stride;
// stride 0: one vector for every row); its output row goes to LDS (when a later op reads
// it) and to global memory (unless a later op of the chain overwrites the same rows).
// Every element is computed with the expression of the per-op kernel.
#define SLM_ROW_OPS 10
#define SLM_ROW_PF 8
enum {
    R_COPY = 1,  // out = a                                   (copy, columns)
    R_ADD,       // out = a + b                               (add, add_row with b.stride 0)
    R_MIX,       // out = a + f0·(b − a)
    R_SILU,      // out = b · a / (1 + e^−a)                  (silu_mul, a = gate)
    R_ROPE,      // i0 heads of i1 dims: half-split rotation of a by cos c, sin d
    R_STORE,     // ring y [i0 heads][q0 slots][i1] at slot (pos + r) mod q0 ← a (h16: fp16 ring)
    R_RMS,       // groups of i0: a · (1/sqrt(dot/i0 + f0)) · b   (b: weights, stride 0)
    R_L2NORM,    // groups of i0: a · (1/max(sqrt(dot), 1e-12))
    R_FOLD,      // out = ((a + a[q0]) + a[2·q0]) + ...: i0 split partials, q0 apart
};
typedef struct {
    const float* g;  // global base (row r at g + r·stride), when the LDS offset is -1
    int64_t stride;
} RowIn;
typedef struct {
    int32_t kind, n;                 // n: elements per row of the output
    int32_t la, lb, lc, ld;          // LDS offsets of operands a..d, or -1 (global)
    int32_t out, tmp;                // LDS offset of the output row (-1: none); norms: a staging row
    int32_t i0, i1;
    float f0;
    int32_t vec;                     // every operand, output and row length in float4s
    int32_t h16, pad;                // R_STORE: the ring holds fp16 values
    RowIn a, b, c, d;
    float* y;                        // global output (row r at y + r·ystride), or null
    int64_t ystride;
    int64_t q0, q1;                  // store: ring slots, position; fold: partial stride
    const long long* dyn;            // store: the position on the device (or null: q1)
} RowOp;
typedef struct {  // a global operand row copied into LDS before the first op
    const float* g;  // row r at g + r·stride
    int64_t stride;
    int32_t n, lds;  // floats (a multiple of 4, 16-byte aligned rows), LDS offset
} RowPf;
typedef struct {
    int32_t nops, npf, r16, pad2;    // r16: fp16 mode (each op's output rounded to fp16)
    RowPf pf[SLM_ROW_PF];
    RowOp op[SLM_ROW_OPS];
} RowDesc;

#endif
