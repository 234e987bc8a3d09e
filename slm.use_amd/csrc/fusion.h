// Descriptors of the fused decode kernels, shared by the host planner (runtime.cpp) and
// the device code (kernels.hip): plain C layouts of fixed-width fields, passed by value
// as the single kernel argument.
//
// A fused GEMV (slm_fg) runs, for one token (m = 1):
//   1. a prologue of small vector operations (the step's element-wise ops, rms, the
//      attention combine, rope-table rows, the embedding row) that produce the GEMV's
//      input: every workgroup computes them into LDS, workgroup 0 also writes them out;
//   2. one to three weight matrices applied to that input (the canonical MFMA chain);
//   3. an epilogue on each matrix's outputs (rope + ring store, l2norm, SiLU of the
//      gate/amp pair, residual add).
// Every value is computed with the same expression, in the same order, as the per-op
// kernels, so fused and unfused runs give the same bits.
#ifndef SLM_FUSION_H
#define SLM_FUSION_H

#include <stdint.h>

#define SLM_VP_MAX 10
#define SLM_SEG_MAX 3
#define SLM_PF_MAX 12
#define SLM_PF_PER_THREAD 12   // prefetched floats per thread (flat over all PfOps)
#define SLM_KS 4               // 16-column blocks per canonical slice (64 columns)
#define SLM_FG_SLICES 3        // most slices one wave of slm_fg holds

enum {
    VP_COPY = 1,    // out = in0
    VP_ADD,         // out = in0 + in1 (also add_row with one row)
    VP_MIX,         // out = in0 + f·(in1 − in0)
    VP_SCALE,       // out = in0 · factor (dyn[0] as f32 bits, else f)
    VP_RMS,         // out = rms(in0) · lds[w], eps f
    VP_COMBINE,     // out = attention combine of the partials (lds[w], or `part`), heads × dh
    VP_SILU,        // out = in1 · in0 / (1 + e^−in0)   (silu_mul with g = in0, u = in1)
};

enum {
    EPI_PLAIN = 0,  // y
    EPI_RESID = 1,  // y; o1 = residual + y                    (add after the linear)
    EPI_ROPE = 2,   // y = [q|k|v]; o1 = rope(q), o2 = rope(k), o3[ring] = o2, o4[ring] = v
    EPI_L2 = 3,     // y = [q|k|v|g]; o1 = l2norm(q), o2 = l2norm(k)
    EPI_SILU = 4,   // y = [gate|amp]; o1 = amp · gate / (1 + e^−gate)
};

// A global vector copied into LDS before anything else runs, so the kernel waits for
// memory once: src + dyn[0]·stride (when dyn) + the workgroup's first row (when wgrow).
typedef struct {
    const float* src;
    const long long* dyn;
    int32_t n, lds, stride, wgrow;
    int32_t limit, pad;     // wgrow: rows past `limit` are not read
} PfOp;

typedef struct {
    int32_t kind, n, wg0;   // length; wg0: only workgroup 0 runs it (a side effect)
    int32_t out, in0, in1;  // LDS float offsets
    int32_t w;              // LDS offset of the rms weight / combine partials (-1: `part`)
    int32_t heads, dh, dp, nsb;
    int32_t pad;
    float* gout;            // global output, written by workgroup 0 (null: none)
    const float* part;      // combine partials in global memory (when w < 0)
    const long long* dyn;   // VP_SCALE factor on the device
    float f;
    float pad2;
} VpOp;

typedef struct {
    const float* w;         // weights [rows][cols]
    float* y;               // the linear's output
    int32_t rows, tiles;    // tiles = ceil(rows / 16)
    int32_t T;              // tiles per workgroup
    int32_t wgs;            // workgroups of this segment
    int32_t wg_first;       // index of its first workgroup
    int32_t epi;
    int32_t d, dh, hid;     // part width, head size, hidden width (SiLU pairs)
    int32_t res_lds;        // RESID: LDS offset of this workgroup's residual rows
    int32_t cs_lds, sn_lds; // ROPE: LDS offsets of the cos / sin row
    float* o1;
    float* o2;
    float* o3;
    float* o4;
    long long cap;          // ring slots (ROPE)
    const long long* dyn;   // ring position of the k store (ROPE), else imm
    long long imm;
    const long long* dyn2;  // ring position of the v store (ROPE), else imm2
    long long imm2;
} FgSeg;

typedef struct {
    int32_t npf, nvp, cols, nsl;  // nsl: canonical slices of `cols`
    int32_t Wt, xin, nseg, lds_vp;  // Wt: waves per tile; xin: LDS offset of the input (-1: x)
    int32_t fold_off, epi_off, pad0, pad1;
    const float* x;
    PfOp pf[SLM_PF_MAX];
    VpOp vp[SLM_VP_MAX];
    FgSeg seg[SLM_SEG_MAX];
} FgDesc;

// Gated linear attention for one token with the head RMSNorm and SiLU gate that follow it
// in an L block (model.rs:471-484): y = gla(...); y2 = rms(y, head_norm); out = silu(gate)·y2.
typedef struct {
    float* s;
    const float* q;
    const float* k;
    const float* v;
    const float* decay;
    const float* bias;
    float* y;        // the gla output when not fused further
    float* y2;       // rms output
    float* out;      // silu_mul output
    const float* hn; // head_norm weight
    const float* gate;
    int32_t heads, dh, fuse;
    float eps;
} GlaDesc;

#endif
