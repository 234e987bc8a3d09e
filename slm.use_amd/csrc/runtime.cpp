// Host runtime of the MI355X backend: the C ABI of include/slm_hip.h.
//
// One context = one device, one stream (default priority), the gfx950 code object loaded
// with hipModuleLoadData, a table of live allocations that every operation checks its
// pointer ranges against before anything is queued, a workspace for attention partials,
// and the step-graph cache.
//
// Every entry point validates its arguments and turns the call into an `Op`. Outside a
// step an Op is lowered to its kernels and launched at once. Inside a step (rope_table
// .. flush, with graphs on) Ops are recorded; at flush the planner lowers the whole step —
// fusing runs of one-token ops into the fused kernels of fusion.h — and the launches are
// captured into a hipGraph, which later steps with the same ops replay. Positions, token
// ids and factors live in a per-step block of device memory that is refreshed before
// each replay, so a step's ops compare equal from one token to the next.

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <climits>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <set>
#include <string>
#include <vector>

#include <emmintrin.h>

#include "fusion.h"
#include "scratch.h"
#include "slm_hip.h"

extern "C" const unsigned char slm_code_object[];
extern "C" const size_t slm_code_object_size;

namespace {

std::string g_open_error;

constexpr int MAX_ARGS = 24;
constexpr size_t BLOB = 2048;             // bytes of kernel arguments per launch
constexpr size_t DYN_CAP = 1 << 20;       // bytes of per-step dynamic values
constexpr size_t STAGE_CAP = 4 << 20;     // bytes of eager staging
constexpr size_t BOUNCE_CAP = 4 << 20;    // pinned bounce buffer for reads
constexpr int MAX_LANES = 4;              // prompt lanes (streams) a context may use
constexpr size_t MIRROR_CAP = 512 << 10;  // bytes a read-ahead copy may take
constexpr size_t MAX_GRAPHS = 8;
constexpr int VP_LEN_MAX = 4096;          // longest vector a fused prologue holds
constexpr int64_t COMB_PART_MAX = 16384;  // attention partials (floats) a fused prologue combines
constexpr int LDS_MAX = 163840;            // gfx950: 160 KB of LDS per workgroup
constexpr int FG_GRID_MAX = 256;           // workgroups of a fused GEMV: one per compute unit
constexpr int64_t ATTN_CTR_MAX = 65536;   // (query tile, key head) pairs one attention launch combines itself
constexpr int ATTN_LDS_MAX = LDS_MAX;
constexpr int ATTN_QG_HOST = 4;   // query tiles per workgroup of the prompt attention (ATTN_QG)
constexpr int ATTN_DEC_LDS = SLM_SB_SEGS * (2 * 64 * 64 + 1024) * 4;  // one-token attention: 256 keys and values, queries
constexpr int GEMM_STAGES_HOST = 2;          // slices in flight in slm_gemm2 (GEMM_STAGES)
constexpr int64_t CU_COUNT = 256;           // MI355X compute units

enum OpKind : uint32_t {
    OP_GATHER = 1, OP_COPY, OP_SHIFT, OP_COLUMNS, OP_LINEAR, OP_ADD, OP_ADD_ROW, OP_SCALE_ROWS,
    OP_MIX, OP_RMS, OP_SILU_MUL, OP_ROPE_TABLE, OP_ROPE, OP_L2NORM, OP_GLA, OP_STORE, OP_ATTEND,
    OP_ARGMAX, OP_GROW
};

// One operation, by value. p[] are device pointers (outputs first), n[] sizes, f[]
// scalars, dyn the device copy of its per-step values (position, ids, factors) or null.
struct Op {
    uint32_t kind, pad;
    const float* p[8];
    int64_t n[10];
    float f[2];
    const void* dyn;
};

// One kernel launch: the function, its grid, and its arguments by value. Scalar-argument
// kernels use 8-byte slots (values little-endian in the low bytes); descriptor kernels
// take one struct, `bytes` long.
struct Rec {
    hipFunction_t f;
    uint32_t gx, gy, gz, bx, shmem, nargs, bytes;
    double abytes = 0.0;  // algorithmic bytes the launch moves (for the kernel statistics)
    alignas(16) unsigned char blob[BLOB];
};

struct KStat {  // per kernel, from HIP events around each eager launch (timing mode)
    long long launches = 0;
    double ms = 0.0, bytes = 0.0;
};
struct Timed {
    hipEvent_t a, b;
    hipFunction_t f;
    double abytes;
};

struct Graph {
    std::vector<Op> ops;
    size_t ndyn = 0;
    hipGraphExec_t exec = nullptr;
    // or, for a one-launch step (slm_step_*): its program in device memory
    char* prog = nullptr;
    int nph = 0, step_var = 0;
    uint32_t step_shmem = 0;
    double step_abytes = 0.0;
    uint64_t used = 0;
    uint64_t id = 0;
    const float* mir_src = nullptr;  // what the host read right after the last replay (mirrored)
    size_t mir_n = 0;
};

struct Table {  // resident cos/sin rows for one inv_freq buffer
    bool h16 = false;  // built in fp16 mode: the rows hold fp16 values
    std::vector<float> inv;
    float* cos = nullptr;
    float* sin = nullptr;
    size_t rows = 0;
};

struct Kernels {
    hipFunction_t to_half;                   // fp32 -> fp16 weight shadows
    hipFunction_t to_host;                   // read-ahead copies into mapped host memory
    hipFunction_t store16, grow, grow16;     // fp16 rings; cache growth
    hipFunction_t attn_dec16[3], attn_pq16[3];  // attention over fp16 rings
    hipFunction_t copy, add, add_row, mix, silu_mul, scale_rows, shift, columns, gather,
        store, rope, rope_table, rms, l2norm, rms_wave, l2norm_wave, fill, combine, probe, fg, fold,
        gemm, gemm2_32, gemm2_64, gemm2_96, gemm2_128, gemm2h_32, gemm2h_64, gemm2h_96, gemm2h_128,
        lin_small_h, fgh;
    // fp16 mode over fp16 weights (allocated with slm_hip_alloc_half)
    hipFunction_t lin_small_hw, fghw, gemm2hw[4], gemm2hsw[4], gemm2hrw, gemm2hnw;
    hipFunction_t lin_small[2], lin_big[2];  // [vec]
    hipFunction_t gla[5], gla1[3];           // rows per lane 1, 2, 4, .. (16 lanes per column)
    hipFunction_t glah[5];                   // the prompt GLA in fp16 mode
    hipFunction_t attn[5];                   // dim tiles 1, 2, 4, 8, 16
    hipFunction_t attn_dec[3];               // one-token attention, dim tiles 1, 2, 4
    hipFunction_t argmax;                    // greedy pick on the device
    hipFunction_t gemm2s[4], gemm2hs[4];     // prompt GEMM with the SiLU pair epilogue, BM 32..128
    hipFunction_t gemm2r, gemm2hr;           // prompt QKV GEMM with the rope + ring-store epilogue
    hipFunction_t gemm2n, gemm2hn;           // prompt QKVG GEMM with the per-head L2 epilogue
    hipFunction_t rows;                      // prompt row chains
    hipFunction_t attn_pq[3];                // prompt attention, superblock shared in LDS
    hipFunction_t gemm2k_32, gemm2k_16;      // 32- and 16-row tiles, two slice groups (fp32)
    hipFunction_t gemm2_48;                  // 48-row tiles, four waves of three row blocks
    hipFunction_t gemm2hk_16, gemm2hwk_16, gemm2h_48, gemm2hw_48;  // the same in fp16 mode
    hipFunction_t step[3];                   // one-launch one-token steps, head size classes 16, 32, 64
};

}  // namespace

struct slm_hip {
    int device = 0;
    hipStream_t stream = nullptr;
    hipModule_t mod = nullptr;
    Kernels k{};
    std::string err;
    char name[256] = {0};
    std::map<uintptr_t, size_t> allocs;  // live allocations: start -> bytes
    // The memory behind slm_hip_alloc: blocks up to POOL_BLOCK_MAX bytes come out of slabs of
    // POOL_SLAB bytes (hipMalloc itself takes 0.02-0.3 ms for 1-13 MB here, which a model
    // growing its outputs inside a prompt would otherwise pay) and go back to a free list of
    // their rounded size; larger ones are allocated directly.
    std::vector<void*> slabs;
    char* slab_cur = nullptr;
    size_t slab_left = 0;
    std::map<size_t, std::vector<void*>> pool_free;  // rounded bytes -> free blocks
    std::map<uintptr_t, size_t> pooled;              // live pooled blocks: start -> rounded bytes
    std::map<uintptr_t, size_t> halves;  // the fp16 ones among them: start -> elements
    // fp16 mode's weight shadows: the fp32 weights a linear read, as the fp16 values fp16 mode
    // rounds them to (converted once on the device), so the linear streams half the bytes
    // with the same bits. Keyed by the fp32 pointer; dropped when anything writes, uploads
    // into or frees that range.
    struct Shadow {
        void* h;   // n halves
        size_t n;  // floats of the fp32 range [key, key + 4n)
    };
    std::map<uintptr_t, Shadow> shadows;
    bool shadows_on = true;
    float* ws = nullptr;                 // attention partials
    size_t ws_bytes = 0;
    int* attn_ctr = nullptr;             // [ATTN_CTR_MAX] finished superblocks per (query tile, key head)
    float* scratch = nullptr;            // this device's fixed scratch (scratch.hip), SLM_NOALLOC_SCRATCH_BYTES
    float* pick = nullptr;               // [16] the fused greedy pick's key and counter (zero between launches)
    float* part = nullptr;               // split partials of fused one-token linears (two halves)
    size_t part_bytes = 0;
    float* gpart = nullptr;              // split partials of prompt GEMMs
    size_t gpart_bytes = 0;
    std::vector<void*> retired;          // replaced internal buffers (launched work or cached
                                         // graphs may still use them): freed at close
    std::vector<void*> free_after_step;  // buffers freed while a step was recorded
    struct Deferred {
        hipEvent_t done;                 // recorded after the step that last used them
        std::vector<void*> bufs;
    };
    std::vector<Deferred> deferred;      // ... freed once their event has completed
    unsigned char* stage_host = nullptr; // eager staging: pinned ring copied into a device ring
    unsigned char* stage_dev = nullptr;
    size_t stage_head = 0;
    unsigned char* dyn_pin[2] = {nullptr, nullptr};  // step values: two pinned uploads
    hipEvent_t dyn_ev[2] = {nullptr, nullptr};
    int dyn_flip = 0;
    unsigned char* dyn_dev = nullptr;
    float* bounce = nullptr;
    hipEvent_t read_ev[2] = {nullptr, nullptr};  // the bounce buffer's halves (large reads)
    // Read-ahead of a one-token step's output: when the host read a range right after a
    // replay of a step graph, later replays of that graph copy the range into mapped host
    // memory behind the step (slm_to_host), and a read of it waits for the copy's flag instead
    // of a copy of its own.
    float* mir_host = nullptr;           // MIRROR_CAP bytes, then the flag (mapped, pinned)
    float* mir_dev = nullptr;            // ... its device address
    unsigned long long* mir_ctr = nullptr;  // slm_to_host's workgroup counter (device)
    unsigned long long mir_total = 0, mir_seq = 0;
    bool mir_armed = false;              // a copy of (mir_src, mir_n) queued, nothing since
    const float* mir_src = nullptr;
    size_t mir_n = 0;
    uint64_t last_graph = 0;             // id of the graph just replayed, nothing since
    uint64_t next_graph_id = 0;
    uint64_t n_mirror_reads = 0;
    std::map<uintptr_t, Table> tables;
    bool graphs_on = true, fusion_on = true, plan_trace = false;
    bool fp16 = false;                   // fp16 mode (slm_hip_set_fp16)
    int* h16_dev = nullptr;              // the code object's mode word slm_h16 (device)
    int fg_rpt = 0;                      // fused GEMV rows per tile: 0 = the planner's choice
    bool timing = false, capturing = false;
    std::vector<Timed> timed;             // launches whose events are not read yet
    std::vector<hipEvent_t> ev_pool;
    std::map<hipFunction_t, std::string> fname;
    std::map<std::string, KStat> kstats;
    int* fault_host = nullptr;           // bounded waits that gave up OR 1 in here (pinned, mapped)
    int* fault_dev = nullptr;            // ... its device address
    int spin = 1 << 24;                  // polls a bounded wait makes before it gives up
    bool recording = false, tainted = false;
    std::vector<Op> ops;                 // the step being recorded
    std::vector<unsigned char> dyn;
    std::vector<Graph> cache;
    uint64_t clock = 0, n_launched = 0, n_captured = 0, n_eager = 0;
    uint64_t last_ops = 0, last_kernels = 0;  // of the last step the planner lowered
    // One-launch steps: a one-token step whose kernels can all be phases of slm_step_* (fused
    // GEMVs, one-token attentions whose partials the next fused GEMV combines, one-token GLAs)
    // runs as one launch of SLM_STEP_WG workgroups over a program of those kernels' arguments,
    // each phase waiting on the flags the workgroups raise as they finish the one before.
    bool step_on = false;                // slm_hip_set_step_kernel (measured slower than graphs)
    bool step_ok = false;                // the device has a compute unit for every workgroup
    unsigned* step_flags = nullptr;      // [SLM_STEP_WG] (device)
    unsigned step_epoch = 0;             // flags reach epoch + phases by the end of a launch
    int step_static_lds = 0;             // bytes of static LDS of the step kernels
    uint64_t n_step = 0, n_step_plans = 0;

    // Prompt lanes: consecutive prompt steps run on up to MAX_LANES streams at once, each
    // lane writing the step's scratch (what the step writes and its flush does not keep:
    // dead once the step is over, ops.rs:90-91) into copies of its own, and waiting for the
    // other lanes only where a kept buffer (ring, state, cache) was last used by them.
    struct Lane {
        hipStream_t stream = nullptr;    // lane 0 is the context's stream and buffers
        float* ws = nullptr;
        size_t ws_bytes = 0;
        float* gpart = nullptr;
        size_t gpart_bytes = 0;
        float* part = nullptr;
        size_t part_bytes = 0;
        unsigned char* dyn_dev = nullptr;
        unsigned char* dyn_pin[2] = {nullptr, nullptr};
        hipEvent_t dyn_ev[2] = {nullptr, nullptr};
        int dyn_flip = 0;
        std::map<uintptr_t, std::pair<void*, size_t>> copies;  // allocation -> (copy, bytes)
        bool used = false;               // work queued since the lanes were entered
    };
    struct Touch {
        int lane;
        hipEvent_t ev;                   // recorded after that lane's last use of the buffer
    };
    std::vector<Lane> lanes;             // [0, nlanes); lanes[0] unused (the context's own)
    int nlanes = 1, next_lane = 0;
    bool lanes_active = false;           // lanes entered: the context's stream not joined yet
    bool lane_launching = false;         // launch_now queues on lane_stream
    hipStream_t lane_stream = nullptr;
    std::vector<uintptr_t> keep;         // allocations the flush being run names
    bool keep_valid = false;
    std::map<uintptr_t, Touch> touch;    // kept allocation -> its last lane use
    std::map<hipEvent_t, int> ev_refs;   // touch entries per event
    std::vector<hipEvent_t> lane_ev_pool;
    std::set<uintptr_t> l0_written;      // scratch lane 0 wrote in place since entering
    std::set<uintptr_t> ln_read;         // allocations other lanes read in place since entering
    uint64_t n_lane_steps = 0, n_lane_fallbacks = 0;
};

namespace {

int fail(slm_hip* c, int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (c) c->err = buf;
    return code;
}

#define HIPC(c, call)                                                                \
    do {                                                                             \
        hipError_t e_ = (call);                                                      \
        if (e_ != hipSuccess)                                                        \
            return fail(c, SLM_E_HIP, "%s: %s", #call, hipGetErrorString(e_));      \
    } while (0)

#define TRY(expr)                \
    do {                         \
        int rc_ = (expr);        \
        if (rc_) return rc_;     \
    } while (0)

// Is [p, p + bytes) inside one live allocation?
// Is [p, p + bytes) inside one live fp32 allocation? An fp16 allocation (slm_hip_alloc_half)
// holds halves, not floats: only upload, read and linear take it, at its start, and they
// check it before this.
bool inside(const slm_hip* c, const void* p, size_t bytes) {
    uintptr_t a = (uintptr_t)p;
    auto it = c->allocs.upper_bound(a);
    if (it == c->allocs.begin()) return false;
    --it;
    return a >= it->first && a - it->first + bytes <= it->second && !c->halves.count(it->first);
}

// Bytes from p to the end of its allocation (0 if p is in none).
size_t room(const slm_hip* c, const void* p) {
    uintptr_t a = (uintptr_t)p;
    auto it = c->allocs.upper_bound(a);
    if (it == c->allocs.begin()) return 0;
    --it;
    if (a < it->first || a >= it->first + it->second) return 0;
    return it->first + it->second - a;
}

// fp32 -> fp16, rounding to nearest even (IEEE 754 binary16: overflow to infinity,
// subnormals kept, NaNs stay NaNs with their sign) — the rounding of v_cvt_f16_f32.
uint16_t f16_of(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));  // NaN
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // rounds to or past 2^16: inf
    if (a < 0x38800000u) {  // below 2^-14: a subnormal half (or zero)
        if (a < 0x33000000u) return sign;  // at most half the smallest subnormal: ±0
        uint32_t mant = (a & 0x7fffffu) | 0x800000u;
        int shift = 126 - (int)(a >> 23);  // 14..24: bits dropped beyond the 13 of a normal
        uint32_t q = mant >> shift, rem = mant & ((1u << shift) - 1), halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (q & 1))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = (a - 0x38000000u) >> 13, rem = a & 0x1fffu;  // rebias 127 -> 15
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1))) q++;   // (a carry into the exponent is right)
    return (uint16_t)(sign | q);
}

float f32_of(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu, u;
    if (e == 0x1f) {
        u = sign | 0x7f800000u | (m << 13);
    } else if (e) {
        u = sign | ((e + 112) << 23) | (m << 13);
    } else if (!m) {
        u = sign;
    } else {  // subnormal: normalise
        int k = 0;
        while (!(m & 0x400u)) {
            m <<= 1;
            k++;
        }
        u = sign | ((uint32_t)(113 - k) << 23) | ((m & 0x3ffu) << 13);
    }
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// fp16 mode's rounding of a host value (to nearest even), as an fp32 value.
float round16(float f) { return f32_of(f16_of(f)); }

// The fp16 allocation that starts at p: its element count (0 if p starts none).
size_t half_count(const slm_hip* c, const void* p) {
    auto it = c->halves.find((uintptr_t)p);
    return it == c->halves.end() ? 0 : it->second;
}

#define NEED(c, op, p, n)                                                            \
    do {                                                                             \
        if ((n) > 0 && !inside(c, p, (size_t)(n) * 4))                               \
            return fail(c, SLM_E_BOUNDS, "%s: %s [%p, %zu floats) is outside every " \
                        "live allocation", op, #p, (const void*)(p), (size_t)(n));   \
    } while (0)

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }
bool fits_int(size_t v) { return v <= (size_t)INT_MAX; }

// ---------------------------------------------------------------------------------------
// launch records
// ---------------------------------------------------------------------------------------

template <typename T>
void put(Rec& r, T v) {
    static_assert(sizeof(T) <= 8, "argument too large");
    uint64_t s = 0;
    std::memcpy(&s, &v, sizeof(T));
    std::memcpy(r.blob + 8 * r.nargs++, &s, 8);
}

void pack(Rec&) {}
template <typename T, typename... A>
void pack(Rec& r, T v, A... rest) {
    put(r, v);
    pack(r, rest...);
}

Rec rec(hipFunction_t f, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t bx, uint32_t shmem) {
    Rec r;
    r.f = f;
    r.gx = gx;
    r.gy = gy;
    r.gz = gz;
    r.bx = bx;
    r.shmem = shmem;
    r.nargs = 0;
    r.bytes = 0;
    return r;
}

template <typename... A>
Rec mk(hipFunction_t f, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t bx, uint32_t shmem,
       A... args) {
    static_assert(sizeof...(A) <= MAX_ARGS, "more kernel arguments than a launch record holds");
    Rec r = rec(f, gx, gy, gz, bx, shmem);
    std::memset(r.blob, 0, 8 * MAX_ARGS);
    pack(r, args...);
    return r;
}

template <typename D>
Rec mk_desc(hipFunction_t f, uint32_t gx, uint32_t bx, uint32_t shmem, const D& d) {
    static_assert(sizeof(D) <= BLOB, "descriptor too large");
    Rec r = rec(f, gx, 1, 1, bx, shmem);
    std::memcpy(r.blob, &d, sizeof(D));
    r.bytes = sizeof(D);
    return r;
}

hipEvent_t pool_event(slm_hip* c) {
    if (!c->ev_pool.empty()) {
        hipEvent_t e = c->ev_pool.back();
        c->ev_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

// ---- prompt lanes: ordering ----

hipEvent_t lane_event(slm_hip* c) {
    if (!c->lane_ev_pool.empty()) {
        hipEvent_t e = c->lane_ev_pool.back();
        c->lane_ev_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) return nullptr;
    return e;
}

void ev_unref(slm_hip* c, hipEvent_t e) {
    auto it = c->ev_refs.find(e);
    if (it == c->ev_refs.end() || --it->second > 0) return;
    c->ev_refs.erase(it);
    c->lane_ev_pool.push_back(e);  // (a wait already queued on it keeps what it waited for)
}

// Orders the context's stream after all the lanes' work, so that whatever the host queues or
// waits for on it next comes after every prompt step, and leaves the lanes.
void leave_lanes(slm_hip* c) {
    if (!c->lanes_active) return;
    c->lanes_active = false;
    for (int l = 1; l < c->nlanes; l++) {
        auto& L = c->lanes[l];
        if (!L.used) continue;
        L.used = false;
        hipEvent_t e = lane_event(c);
        if (!e || hipEventRecord(e, L.stream) != hipSuccess ||
            hipStreamWaitEvent(c->stream, e, 0) != hipSuccess)
            hipStreamSynchronize(L.stream);  // no event: the host waits for the lane instead
        if (e) c->lane_ev_pool.push_back(e);
    }
    for (auto& t : c->touch) ev_unref(c, t.second.ev);
    c->touch.clear();
    c->l0_written.clear();
    c->ln_read.clear();
}

// The context's stream, for work that is not a lane's: joined with the lanes first.
hipStream_t mstream(slm_hip* c) {
    c->mir_armed = false;  // work queued after the read-ahead copy: reads go the usual way
    c->last_graph = 0;
    leave_lanes(c);
    return c->stream;
}

// Reads the events of the timed launches into the per-kernel statistics.
int collect_timing(slm_hip* c) {
    if (c->timed.empty()) return SLM_OK;
    HIPC(c, hipStreamSynchronize(mstream(c)));
    for (auto& t : c->timed) {
        float ms = 0.0f;
        HIPC(c, hipEventElapsedTime(&ms, t.a, t.b));
        KStat& k = c->kstats[c->fname[t.f]];
        k.launches++;
        k.ms += ms;
        k.bytes += t.abytes;
        c->ev_pool.push_back(t.a);
        c->ev_pool.push_back(t.b);
    }
    c->timed.clear();
    return SLM_OK;
}

// The attention counters and the fused pick's key and counter are returned to zero by the
// last workgroup of each launch that uses them. After a launch that failed, or one whose
// bounded waits gave up (its workgroups may have ended early), they start from zero again.
// Never inside a capture: a fill recorded into a graph is not replayed reliably.
void reset_counters(slm_hip* c) {
    if (c->capturing) return;
    hipMemsetAsync(c->attn_ctr, 0, ATTN_CTR_MAX * sizeof(int), mstream(c));
    hipMemsetAsync(c->pick, 0, 16 * sizeof(float), mstream(c));
}

int launch_now(slm_hip* c, const Rec& r) {
    void* ptrs[MAX_ARGS];
    if (r.bytes) {
        ptrs[0] = (void*)r.blob;
    } else {
        for (uint32_t i = 0; i < r.nargs; i++) ptrs[i] = (void*)(r.blob + 8 * i);
    }
    bool timed = c->timing && !c->capturing && !c->lane_launching;
    if (!timed) {
        hipStream_t s = c->lane_launching ? c->lane_stream : mstream(c);
        hipError_t e = hipModuleLaunchKernel(r.f, r.gx, r.gy, r.gz, r.bx, 1, 1, r.shmem, s,
                                             ptrs, nullptr);
        if (e != hipSuccess) {
            reset_counters(c);
            return fail(c, SLM_E_HIP, "hipModuleLaunchKernel: %s", hipGetErrorString(e));
        }
        return SLM_OK;
    }
    // The start and stop events of hipExtModuleLaunchKernel take the dispatch's own begin and
    // end timestamps, so the duration is the kernel's alone (what a kernel trace reports),
    // without the launch gap an event recorded around the call would add. Its grid is given
    // in work-items, a 32-bit count.
    uint64_t items = (uint64_t)r.gx * r.bx;
    if (items > UINT32_MAX)
        return fail(c, SLM_E_UNSUPPORTED, "timed launch of %llu work-items along x",
                    (unsigned long long)items);
    Timed t{pool_event(c), pool_event(c), r.f, r.abytes};
    if (!t.a || !t.b) return fail(c, SLM_E_HIP, "hipEventCreate failed");
    hipError_t e = hipExtModuleLaunchKernel(r.f, (uint32_t)items, r.gy, r.gz, r.bx, 1, 1, r.shmem,
                                            mstream(c), ptrs, nullptr, t.a, t.b, 0);
    if (e != hipSuccess) {
        c->ev_pool.push_back(t.a);
        c->ev_pool.push_back(t.b);
        reset_counters(c);
        return fail(c, SLM_E_HIP, "hipExtModuleLaunchKernel: %s", hipGetErrorString(e));
    }
    c->timed.push_back(t);
    if (c->timed.size() >= 4096) TRY(collect_timing(c));
    return SLM_OK;
}

uint32_t blocks_for(size_t n, size_t per = 256, size_t cap = 4096) {
    size_t b = (n + per - 1) / per;
    return (uint32_t)std::max<size_t>(1, std::min(b, cap));
}

int pow2_index(size_t need, int maxi) {  // smallest i with 2^i >= need
    int i = 0;
    while (i < maxi && ((size_t)1 << i) < need) i++;
    return i;
}

void dev_free(slm_hip* c, void* p);

void drop_graphs(slm_hip* c) {
    if (c->cache.empty()) return;
    hipStreamSynchronize(mstream(c));
    for (auto& g : c->cache) {
        if (g.exec) hipGraphExecDestroy(g.exec);
        if (g.prog) dev_free(c, g.prog);
    }
    c->cache.clear();
}

// ---------------------------------------------------------------------------------------
// per-op lowering (the unfused kernels)
// ---------------------------------------------------------------------------------------

// The pipelined prompt GEMM's row tile: the one that leaves the busiest CU the least work —
// rows per tile times the workgroups a CU runs (32-row tiles of four waves go two to a CU,
// the others one) — the larger tile on a tie.
int gemm2_bm(int64_t rows, int64_t m, int64_t ns) {
    int bm = 32;
    int64_t best = -1;
    for (int t : {32, 64, 96, 128}) {
        int64_t wgs = ((rows + t - 1) / t) * ((m + 63) / 64) * ns;
        int64_t per_cu = t == 32 ? 2 : 1;
        int64_t rounds = (wgs + per_cu * CU_COUNT - 1) / (per_cu * CU_COUNT);
        int64_t sharing = std::min<int64_t>(per_cu, (wgs + CU_COUNT - 1) / CU_COUNT);
        int64_t cost = rounds * t * sharing;
        if (best < 0 || cost <= best) best = cost, bm = t;
    }
    return bm;
}

uint32_t gemm2_threads(int bm) { return bm == 32 ? 256 : bm == 96 ? 512 : 1024; }

// The plain fp32 GEMM's tile rows (16 and 32: two slice groups, 48: four waves of three row
// blocks; 64, 96, 128 as gemm2_bm): the fewest rounds of one workgroup per CU, each round
// costing its tile rows (the per-SIMD MFMA work) plus a fixed 16 (launch, first copies,
// epilogue).
int gemm2_bm_plain(int64_t rows, int64_t m, int64_t ns) {
    int bm = 64;
    int64_t best = -1;
    for (int t : {16, 32, 48, 64, 96, 128}) {
        int64_t wgs = ((rows + t - 1) / t) * ((m + 63) / 64) * ns;
        int64_t rounds = (wgs + CU_COUNT - 1) / CU_COUNT;
        int64_t cost = rounds * (t + 16);
        if (best < 0 || cost < best) best = cost, bm = t;
    }
    return bm;
}

// A linear (p0 y, p1 w, p2 x; n0 rows, n1 cols, n2 m). With `fold_ns`, a split GEMM's
// partials are left in c->gpart for the caller to add (*fold_ns: the split count, 1 when
// the GEMM wrote y itself).
int lower_linear(slm_hip* c, const Op& o, std::vector<Rec>& out, int64_t* fold_ns) {
    const Kernels& k = c->k;
    const float* const* p = o.p;
    const int64_t* n = o.n;
    if (fold_ns) *fold_ns = 1;
    int64_t rows = n[0], cols = n[1], m = n[2];
    if (cols == 0) {
        out.push_back(mk(k.fill, blocks_for(m * rows), 1, 1, 256, 0, p[0],
                         (long long)(m * rows), 0.0f));
        return SLM_OK;
    }
    int vec = (cols % 4 == 0 && aligned16(p[1]) && aligned16(p[2])) ? 1 : 0;
    int64_t kblocks = (cols + 15) / 16, nsl = (kblocks + SLM_KS - 1) / SLM_KS;
    double ab = 4.0 * (double)(rows * cols + m * cols + m * rows);
    bool h = n[3] != 0;  // fp16 mode: 64-column multiples, aligned (checked when recorded)
    bool w16 = n[4] != 0;  // fp16 weights (fp16 mode)
    if (w16) ab = 2.0 * (double)(rows * cols) + 4.0 * (double)(m * cols + m * rows);
    if (h && m <= 16 && nsl <= 64) {
        uint32_t waves = (uint32_t)std::min<int64_t>(nsl, 8);
        out.push_back(mk(w16 ? k.lin_small_hw : k.lin_small_h, (uint32_t)((rows + 15) / 16), 1, 1, 64 * waves,
                         (uint32_t)(nsl * 1024), p[0], p[1], p[2], (int)rows, (int)cols, (int)m));
        out.back().abytes = ab;
        return SLM_OK;
    }
    if (h && (m <= 16 || !vec || cols % 64))
        return fail(c, SLM_E_UNSUPPORTED, "linear: fp16 mode has no kernel for %lld x %lld x %lld",
                    (long long)rows, (long long)cols, (long long)m);
    if (m <= 16 && nsl <= 64) {
        uint32_t waves = (uint32_t)std::min<int64_t>(nsl, 8);
        out.push_back(mk(k.lin_small[vec], (uint32_t)((rows + 15) / 16), 1, 1, 64 * waves,
                         (uint32_t)(nsl * 1024), p[0], p[1], p[2], (int)rows, (int)cols,
                         (int)m));
        out.back().abytes = ab;
    } else if (vec) {  // the LDS-staged GEMM, one workgroup column per split
        int64_t ns = (nsl + SLM_SPLIT - 1) / SLM_SPLIT;
        if (ns > 1 && (int64_t)c->gpart_bytes < ns * m * rows * 4)
            return fail(c, SLM_E_INVALID, "linear: no room for %lld split partials", (long long)ns);
        if (cols % 64 == 0) {
            // the tile rows by the chip's fill (in fp16 mode 32-row tiles run as 48: the slice
            // groups of 32 rows are fp32 only)
            int bm = gemm2_bm_plain(rows, m, ns);
            if (bm == 32 && h) bm = 48;
            uint32_t shmem = (uint32_t)(GEMM_STAGES_HOST * (bm * (w16 ? 32 : 64) + 64 * 64) * 4);
            uint32_t threads = bm == 48 ? 256 : gemm2_threads(bm);
            hipFunction_t f;
            if (bm == 48) f = w16 ? k.gemm2hw_48 : h ? k.gemm2h_48 : k.gemm2_48;
            else if (w16) f = k.gemm2hw[bm == 64 ? 1 : bm == 96 ? 2 : 3];
            else if (h) f = bm == 64 ? k.gemm2h_64 : bm == 96 ? k.gemm2h_96 : k.gemm2h_128;
            else f = bm == 64 ? k.gemm2_64 : bm == 96 ? k.gemm2_96 : k.gemm2_128;
            if (bm <= 32) {  // two slice groups: twice the MFMA chains per SIMD
                f = bm == 16 ? (w16 ? k.gemm2hwk_16 : h ? k.gemm2hk_16 : k.gemm2k_16) : k.gemm2k_32;
                shmem *= 2;
                threads = 512;
            }
            out.push_back(mk(f, (uint32_t)((rows + bm - 1) / bm), (uint32_t)((m + 63) / 64),
                             (uint32_t)ns, threads, shmem, p[0], c->gpart,
                             p[1], p[2], (int)rows, (int)cols, (int)m));
        } else {
            out.push_back(mk(k.gemm, (uint32_t)((rows + 63) / 64), (uint32_t)((m + 63) / 64),
                             (uint32_t)ns, 256, 0, p[0], c->gpart, p[1], p[2], (int)rows,
                             (int)cols, (int)m));
        }
        if (fold_ns) *fold_ns = ns;  // the caller adds the partials
        else if (ns > 1)
            out.push_back(mk(k.fold, blocks_for(m * rows), 1, 1, 256, 0, p[0],
                             (const float*)c->gpart, (long long)(m * rows), (int)ns));
    } else {
        out.push_back(mk(k.lin_big[vec], (uint32_t)((rows + 63) / 64),
                         (uint32_t)((m + 63) / 64), 1, 256, 0, p[0], p[1], p[2],
                         (int)rows, (int)cols, (int)m));
    }
    return SLM_OK;
}

// One-token attention on the vector-ALU kernel (the same arithmetic as the MFMA kernels; its
// ring offsets step four slots at a time and are 32-bit).
// Rings the fp16 attention kernels take (the one-token kernel and the shared-superblock prompt
// kernel): head size at most 64 and a multiple of 8, at least 64 slots, a key head's ring
// under 4 GB.
bool half_ring_ok(size_t heads, size_t dh, size_t cap) {
    return heads > 0 && dh > 0 && dh <= 64 && dh % 8 == 0 && cap >= 64 && cap * dh * 4 < ((size_t)1 << 32);
}

bool attn_dec_ok(const Op& o) {
    const int64_t* n = o.n;
    return n[1] == 1 && n[7] <= 64 && n[4] >= 64 && n[4] * n[7] * 4 < ((int64_t)1 << 32);
}

int64_t attn_dp(int64_t dh) { return (int64_t)16 << pow2_index((dh + 15) / 16, 4); }

// The superblock partials of a one-token attention, [nsb][heads][dp + 2] floats at c->ws.
int64_t attn_dec_part_floats(const Op& o) { return o.n[8] * o.n[5] * (attn_dp(o.n[7]) + 2); }

// Where an attention op's superblock partials go: the workspace, or (p4 set: the
// allocation-free entry point) the buffer it names, and then no launch uses the counters.
float* attn_part(slm_hip* c, const Op& o) { return o.p[4] ? (float*)o.p[4] : c->ws; }

// With `defer` the kernel only writes its superblock partials (a later fused prologue, or
// slm_attn_combine, combines them); otherwise it combines them itself when every partial
// of a key head fits in its LDS (and the op may use the counters), else slm_attn_combine
// runs after it.
int lower_attn_dec(slm_hip* c, const Op& o, std::vector<Rec>& out, bool defer) {
    const Kernels& k = c->k;
    const float* const* p = o.p;
    const int64_t* n = o.n;
    int64_t heads = n[5], kh = n[6], dh = n[7], nsb = n[8];
    int dti = pow2_index((dh + 15) / 16, 4);
    int64_t dp = attn_dp(dh);
    float* part = attn_part(c, o);
    bool self = !defer && !o.p[4] && kh <= ATTN_CTR_MAX &&
                nsb * (heads / kh) * (dp + 2) <= ATTN_DEC_LDS / 4;
    out.push_back(mk(n[9] ? k.attn_dec16[dti] : k.attn_dec[dti], (uint32_t)kh, (uint32_t)nsb, 1, 64 * SLM_SB_SEGS,
                     (uint32_t)ATTN_DEC_LDS, part, p[1], p[2], p[3], (const long long*)o.dyn,
                     (long long)n[0], (long long)n[2], (long long)n[3], (long long)n[4], (int)heads,
                     (int)kh, (int)dh, o.f[0], self ? p[0] : (float*)nullptr,
                     self ? c->attn_ctr : (int*)nullptr));
    if (!self && !defer)
        out.push_back(mk(k.combine, (uint32_t)((heads + 3) / 4), 1, 1, 256, 0, p[0], (const float*)part,
                         1, (int)heads, (int)dh, (int)dp, (int)nsb, (const long long*)nullptr,
                         (long long)0, (long long)0, (long long)0));
    return SLM_OK;
}

int lower_one(slm_hip* c, const Op& o, std::vector<Rec>& out) {
    const Kernels& k = c->k;
    const float* const* p = o.p;
    const int64_t* n = o.n;
    switch (o.kind) {
        case OP_ARGMAX:  // p0 tok (long long), p1 x, p2 ids (uint32); n0 n, n1 slot, n2 ids cap; dyn slot
            out.push_back(mk(k.argmax, 1, 1, 1, 1024, 0, p[1], (long long)n[0], (long long*)p[0],
                             (unsigned*)p[2], (const long long*)o.dyn, (long long)n[1]));
            return SLM_OK;
        case OP_GATHER:  // p0 y, p1 w; n0 m, n1 d; dyn ids
            out.push_back(mk(k.gather, blocks_for(n[0] * n[1]), 1, 1, 256, 0, p[0], p[1],
                             (const long long*)o.dyn, (long long)(n[0] * n[1]), (long long)n[1]));
            return SLM_OK;
        case OP_COPY:
            out.push_back(mk(k.copy, blocks_for(n[0]), 1, 1, 256, 0, p[0], p[1], (long long)n[0]));
            return SLM_OK;
        case OP_SHIFT:  // p0 y, p1 first, p2 x; n0 m, n1 d
            out.push_back(mk(k.shift, blocks_for(n[0] * n[1]), 1, 1, 256, 0, p[0], p[1], p[2],
                             (long long)(n[0] * n[1]), (long long)n[1]));
            return SLM_OK;
        case OP_COLUMNS:  // p0 y, p1 x; n0 m, n1 stride, n2 off, n3 len
            out.push_back(mk(k.columns, blocks_for(n[0] * n[3]), 1, 1, 256, 0, p[0], p[1],
                             (long long)(n[0] * n[3]), (long long)n[1], (long long)n[2],
                             (long long)n[3]));
            return SLM_OK;
        case OP_LINEAR:
            return lower_linear(c, o, out, nullptr);
        case OP_ADD:
            out.push_back(mk(k.add, blocks_for(n[0]), 1, 1, 256, 0, p[0], p[1], p[2], (long long)n[0]));
            return SLM_OK;
        case OP_ADD_ROW:  // p0 y, p1 x, p2 row; n0 m, n1 d
            out.push_back(mk(k.add_row, blocks_for(n[0] * n[1]), 1, 1, 256, 0, p[0], p[1], p[2],
                             (long long)(n[0] * n[1]), (long long)n[1]));
            return SLM_OK;
        case OP_SCALE_ROWS:  // p0 y, p1 x; n0 m, n1 d; dyn factors or f0
            out.push_back(mk(k.scale_rows, blocks_for(n[0] * n[1]), 1, 1, 256, 0, p[0], p[1],
                             (const float*)o.dyn, o.f[0], (long long)(n[0] * n[1]), (long long)n[1]));
            return SLM_OK;
        case OP_MIX:
            out.push_back(mk(k.mix, blocks_for(n[0]), 1, 1, 256, 0, p[0], p[1], p[2], (long long)n[0],
                             o.f[0]));
            return SLM_OK;
        case OP_RMS:
        case OP_L2NORM: {  // p0 y, p1 x, p2 w; n0 groups, n1 size; f0 eps
            int64_t groups = n[0], size = n[1];
            bool wide = size >= 256 && size <= 4096 && size % 4 == 0 && aligned16(p[0]) &&
                        aligned16(p[1]) && (o.kind != OP_RMS || aligned16(p[2]));
            if (wide) {  // one wave per group
                uint32_t blocks = (uint32_t)((groups + 3) / 4), shmem = (uint32_t)(4 * size * 4);
                if (o.kind == OP_RMS)
                    out.push_back(mk(k.rms_wave, blocks, 1, 1, 256, shmem, p[0], p[1], p[2],
                                     (int)groups, (int)size, o.f[0]));
                else
                    out.push_back(mk(k.l2norm_wave, blocks, 1, 1, 256, shmem, p[0], p[1],
                                     (int)groups, (int)size));
                return SLM_OK;
            }
            int64_t stride = size | 1;
            // up to 16 groups per workgroup, fewer when that leaves the chip half idle
            int64_t G = std::min<int64_t>(16, std::max<int64_t>(1, 16384 / stride));
            G = std::max<int64_t>(1, std::min<int64_t>(G, groups / 512));
            uint32_t blocks = (uint32_t)((groups + G - 1) / G);
            uint32_t shmem = (uint32_t)(G * stride * 4);
            if (o.kind == OP_RMS)
                out.push_back(mk(k.rms, blocks, 1, 1, 256, shmem, p[0], p[1], p[2], (int)groups,
                                 (int)size, o.f[0], (int)G));
            else
                out.push_back(mk(k.l2norm, blocks, 1, 1, 256, shmem, p[0], p[1], (int)groups,
                                 (int)size, (int)G));
            return SLM_OK;
        }
        case OP_SILU_MUL:
            out.push_back(mk(k.silu_mul, blocks_for(n[0]), 1, 1, 256, 0, p[0], p[1], p[2],
                             (long long)n[0]));
            return SLM_OK;
        case OP_ROPE_TABLE:  // p0 cos, p1 sin, p2 table cos, p3 table sin; n0 m, n1 half, n2 pos
            out.push_back(mk(k.rope_table, blocks_for(n[0] * n[1]), 1, 1, 256, 0, p[0], p[1], p[2],
                             p[3], (const long long*)o.dyn, (long long)n[2],
                             (long long)(n[0] * n[1]), (long long)n[1]));
            return SLM_OK;
        case OP_ROPE:  // p0 y, p1 x, p2 cos, p3 sin; n0 m, n1 heads, n2 dh
            out.push_back(mk(k.rope, blocks_for(n[0] * n[1] * n[2] / 2), 1, 1, 256, 0, p[0], p[1],
                             p[2], p[3], (long long)n[0], (long long)n[1], (long long)n[2]));
            return SLM_OK;
        case OP_GLA: {  // p0 y, p1 s, p2 q, p3 k, p4 v, p5 decay, p6 bias; n0 m, n1 heads, n2 dh
            // sixteen lanes per state column, SLM_GLA_COLS columns per workgroup
            int i = pow2_index((n[2] + 15) / 16, 4);
            uint32_t shmem = (uint32_t)(2 * SLM_GLA_T * (2 * n[2] + SLM_GLA_COLS + 1) * 4);  // two token groups
            int vec = (n[2] % 4 == 0 && aligned16(p[2]) && aligned16(p[3]) && aligned16(p[4])) ? 4 : 1;
            out.push_back(mk(c->fp16 ? k.glah[i] : k.gla[i], (uint32_t)n[1], (uint32_t)((n[2] + SLM_GLA_COLS - 1) / SLM_GLA_COLS), 1,
                             16 * SLM_GLA_COLS, shmem,
                             p[0], p[1], p[2], p[3], p[4], p[5], p[6], (int)n[0], (int)n[1],
                             (int)n[2], vec));
            return SLM_OK;
        }
        case OP_STORE:  // p0 cache, p1 src; n0 m, n1 cap, n2 heads, n3 dh, n4 pos, n5 fp16 ring
            out.push_back(mk(n[5] ? k.store16 : k.store, blocks_for(n[0] * n[2] * n[3]), 1, 1, 256, 0, p[0], p[1],
                             (const long long*)o.dyn, (long long)n[4], (long long)(n[0] * n[2] * n[3]),
                             (long long)n[1], (long long)n[2], (long long)n[3]));
            return SLM_OK;
        case OP_GROW:  // p0 new cache, p1 old; n0 heads, n1 old cap, n2 dh, n3 fp16
            out.push_back(mk(n[3] ? k.grow16 : k.grow, blocks_for(n[0] * n[1] * n[2]), 1, 1, 256, 0,
                             p[0], p[1], (long long)n[0], (long long)(n[1] * n[2])));
            return SLM_OK;
        case OP_ATTEND: {
            // p0 y, p1 q, p2 k, p3 v; n0 pos, n1 m, n2 reach, n3 gap, n4 cap, n5 heads,
            // n6 key_heads, n7 dh, n8 nsb, n9 fp16 rings; f0 scale
            int64_t m = n[1], heads = n[5], kh = n[6], dh = n[7], nsb = n[8];
            int dti = pow2_index((dh + 15) / 16, 4);
            int64_t dp = (int64_t)16 << dti;
            if (attn_dec_ok(o)) return lower_attn_dec(c, o, out, false);
            float* part = attn_part(c, o);
            int64_t qpt = 16 / (heads / kh);
            int64_t groups = ((m + qpt - 1) / qpt + ATTN_QG_HOST - 1) / ATTN_QG_HOST;
            if (m > 1 && dh <= 64 && groups * kh * nsb <= (int64_t)INT_MAX) {
                // a superblock's keys and values shared in LDS by four query tiles
                // (then every row's superblocks are combined by a kernel of their own: many
                // rows, each a wave, rather than one workgroup per tile group at the end)
                out.push_back(mk(n[9] ? k.attn_pq16[dti] : k.attn_pq[dti], (uint32_t)groups, (uint32_t)kh, (uint32_t)nsb,
                                 64 * SLM_SB_SEGS * ATTN_QG_HOST, (uint32_t)(2 * SLM_SB_KEYS * 64 * 4),
                                 part, p[1], p[2], p[3], (const long long*)o.dyn, (long long)n[0],
                                 (int)m, (long long)n[2], (long long)n[3], (long long)n[4],
                                 (int)heads, (int)kh, (int)dh, o.f[0]));
                out.push_back(mk(k.combine, (uint32_t)((m * heads + 3) / 4), 1, 1, 256, 0, p[0],
                                 (const float*)part, (int)m, (int)heads, (int)dh, (int)dp, (int)nsb,
                                 (const long long*)o.dyn, (long long)n[0], (long long)n[2],
                                 (long long)n[3]));
                return SLM_OK;
            }
            if (n[9]) return fail(c, SLM_E_UNSUPPORTED, "attend: fp16 rings of this shape");
            // LDS: wpp segment partials being folded, then each wave's tile of values
            auto shm = [&](int64_t w) { return (w * 16 * (dp + 2) + SLM_SB_SEGS * 16 * (dp + 4)) * 4; };
            int64_t wpp = SLM_SB_SEGS;
            while (wpp > 1 && shm(wpp) > ATTN_LDS_MAX) wpp /= 2;
            int64_t qtiles = (m + qpt - 1) / qpt;
            // the last workgroup of each (query tile, key head) combines the superblocks itself
            // when its counter fits; otherwise slm_attn_combine runs after
            bool self = m == 1 && !o.p[4] && qtiles * kh <= ATTN_CTR_MAX;
            out.push_back(mk(k.attn[dti], (uint32_t)qtiles, (uint32_t)kh, (uint32_t)nsb,
                             64 * SLM_SB_SEGS, (uint32_t)shm(wpp), part, p[1], p[2], p[3],
                             (const long long*)o.dyn, (long long)n[0], (int)m, (long long)n[2],
                             (long long)n[3], (long long)n[4], (int)heads, (int)kh, (int)dh, o.f[0],
                             (int)wpp, self ? p[0] : (float*)nullptr, self ? c->attn_ctr : (int*)nullptr));
            if (!self)
                out.push_back(mk(k.combine, (uint32_t)((m * heads + 3) / 4), 1, 1, 256, 0, p[0],
                                 (const float*)part, (int)m, (int)heads, (int)dh, (int)dp, (int)nsb,
                                 (const long long*)nullptr, (long long)0, (long long)0, (long long)0));
            return SLM_OK;
        }
    }
    return fail(c, SLM_E_INVALID, "unknown op %u", o.kind);
}

// ---------------------------------------------------------------------------------------
// the fusion planner (one-token steps)
// ---------------------------------------------------------------------------------------

struct Range {
    uintptr_t a, b;  // [a, b) bytes
    bool wg0 = false;  // written by workgroup 0 alone, in program order (a prologue output)
};
Range rng(const float* p, int64_t n) { return Range{(uintptr_t)p, (uintptr_t)(p + n)}; }
Range rng0(const float* p, int64_t n) { return Range{(uintptr_t)p, (uintptr_t)(p + n), true}; }
bool overlap(const Range& x, const Range& y) { return x.a < y.b && y.a < x.b; }

// An element-wise one-token op as prologue material: what it reads and writes.
enum { SRC_COPY = 1, SRC_ADD, SRC_MIX, SRC_SCALE, SRC_GATHER, SRC_RMS, SRC_ROPE_TABLE, SRC_SILU,
       SRC_FOLD, SRC_COMB };
struct VpSrc {
    int kind = 0;
    int n = 0;
    int nsplit = 0;  // SRC_FOLD: partials [nsplit][n] at in[0]; SRC_COMB: superblocks
    int heads = 0, dh = 0, dp = 0;  // SRC_COMB: partials [nsplit][heads][dp + 2] at in[0]
    const float* in[2] = {nullptr, nullptr};
    const float* out[2] = {nullptr, nullptr};
    const Op* op = nullptr;
};

// Can this op run inside a fused prologue? (one token, one row, a short vector)
bool vp_of(const Op& o, VpSrc* v) {
    const int64_t* n = o.n;
    v->op = &o;
    switch (o.kind) {
        case OP_COPY:
            v->kind = SRC_COPY; v->n = (int)n[0]; v->in[0] = o.p[1]; v->out[0] = o.p[0];
            break;
        case OP_ADD:
            v->kind = SRC_ADD; v->n = (int)n[0]; v->in[0] = o.p[1]; v->in[1] = o.p[2]; v->out[0] = o.p[0];
            break;
        case OP_ADD_ROW:
            if (n[0] != 1) return false;
            v->kind = SRC_ADD; v->n = (int)n[1]; v->in[0] = o.p[1]; v->in[1] = o.p[2]; v->out[0] = o.p[0];
            break;
        case OP_MIX:
            v->kind = SRC_MIX; v->n = (int)n[0]; v->in[0] = o.p[1]; v->in[1] = o.p[2]; v->out[0] = o.p[0];
            break;
        case OP_SCALE_ROWS:
            if (n[0] != 1) return false;
            v->kind = SRC_SCALE; v->n = (int)n[1]; v->in[0] = o.p[1]; v->out[0] = o.p[0];
            break;
        case OP_GATHER:
            if (n[0] != 1) return false;
            v->kind = SRC_GATHER; v->n = (int)n[1]; v->out[0] = o.p[0];
            break;
        case OP_RMS:
            if (n[0] != 1) return false;
            v->kind = SRC_RMS; v->n = (int)n[1]; v->in[0] = o.p[1]; v->out[0] = o.p[0];
            break;
        case OP_ROPE_TABLE:
            if (n[0] != 1) return false;
            v->kind = SRC_ROPE_TABLE; v->n = (int)n[1]; v->out[0] = o.p[0]; v->out[1] = o.p[1];
            break;
        case OP_SILU_MUL:
            v->kind = SRC_SILU; v->n = (int)n[0]; v->in[0] = o.p[1]; v->in[1] = o.p[2]; v->out[0] = o.p[0];
            break;
        case OP_COLUMNS:
            if (n[0] != 1) return false;
            v->kind = SRC_COPY; v->n = (int)n[3]; v->in[0] = o.p[1] + n[2]; v->out[0] = o.p[0];
            break;
        default:
            return false;
    }
    return v->n > 0 && v->n <= VP_LEN_MAX && v->n % 4 == 0;
}


// A ring's elements in floats of storage (fp16 rings take half).
int64_t ring_floats(int64_t n, int64_t h16) { return h16 ? (n + 1) / 2 : n; }

// A linear's weights in floats of storage (fp16 weights take half).
int64_t wfloats(const Op& o) { return o.n[4] ? (o.n[0] * o.n[1] + 1) / 2 : o.n[0] * o.n[1]; }

// What an op reads and writes, in bytes of device memory (ring and state updates count as
// both). The embedding table and the rope tables are only ever read.
void op_ranges(const Op& o, std::vector<Range>& rd, std::vector<Range>& wr) {
    const float* const* p = o.p;
    const int64_t* n = o.n;
    switch (o.kind) {
        case OP_GATHER: wr.push_back(rng(p[0], n[0] * n[1])); rd.push_back(rng(p[1], 1)); break;
        case OP_ARGMAX:
            wr.push_back(rng(p[0], 2));
            if (p[2]) wr.push_back(rng(p[2], n[2]));
            rd.push_back(rng(p[1], n[0]));
            break;
        case OP_COPY: wr.push_back(rng(p[0], n[0])); rd.push_back(rng(p[1], n[0])); break;
        case OP_SHIFT:
            wr.push_back(rng(p[0], n[0] * n[1]));
            rd.push_back(rng(p[1], n[1]));
            rd.push_back(rng(p[2], n[0] * n[1]));
            break;
        case OP_COLUMNS: wr.push_back(rng(p[0], n[0] * n[3])); rd.push_back(rng(p[1], n[0] * n[1])); break;
        case OP_LINEAR:
            wr.push_back(rng(p[0], n[2] * n[0]));
            rd.push_back(rng(p[1], wfloats(o)));
            rd.push_back(rng(p[2], n[2] * n[1]));
            break;
        case OP_ADD:
        case OP_MIX:
        case OP_SILU_MUL:
            wr.push_back(rng(p[0], n[0]));
            rd.push_back(rng(p[1], n[0]));
            rd.push_back(rng(p[2], n[0]));
            break;
        case OP_ADD_ROW:
            wr.push_back(rng(p[0], n[0] * n[1]));
            rd.push_back(rng(p[1], n[0] * n[1]));
            rd.push_back(rng(p[2], n[1]));
            break;
        case OP_SCALE_ROWS: wr.push_back(rng(p[0], n[0] * n[1])); rd.push_back(rng(p[1], n[0] * n[1])); break;
        case OP_RMS:
            wr.push_back(rng(p[0], n[0] * n[1]));
            rd.push_back(rng(p[1], n[0] * n[1]));
            rd.push_back(rng(p[2], n[1]));
            break;
        case OP_L2NORM: wr.push_back(rng(p[0], n[0] * n[1])); rd.push_back(rng(p[1], n[0] * n[1])); break;
        case OP_ROPE_TABLE: wr.push_back(rng(p[0], n[0] * n[1])); wr.push_back(rng(p[1], n[0] * n[1])); break;
        case OP_ROPE:
            wr.push_back(rng(p[0], n[0] * n[1] * n[2]));
            rd.push_back(rng(p[1], n[0] * n[1] * n[2]));
            rd.push_back(rng(p[2], n[0] * (n[2] / 2)));
            rd.push_back(rng(p[3], n[0] * (n[2] / 2)));
            break;
        case OP_GLA: {
            int64_t t = n[0] * n[1] * n[2];
            wr.push_back(rng(p[0], t));
            wr.push_back(rng(p[1], n[1] * n[2] * n[2]));
            rd.push_back(rng(p[1], n[1] * n[2] * n[2]));
            for (int q = 2; q < 5; q++) rd.push_back(rng(p[q], t));
            rd.push_back(rng(p[5], n[0] * n[1]));
            rd.push_back(rng(p[6], n[1]));
            break;
        }
        case OP_STORE:
            wr.push_back(rng(p[0], ring_floats(n[2] * n[1] * n[3], n[5])));
            rd.push_back(rng(p[0], ring_floats(n[2] * n[1] * n[3], n[5])));
            rd.push_back(rng(p[1], n[0] * n[2] * n[3]));
            break;
        case OP_GROW:
            wr.push_back(rng(p[0], ring_floats(2 * n[0] * n[1] * n[2], n[3])));
            rd.push_back(rng(p[1], ring_floats(n[0] * n[1] * n[2], n[3])));
            break;
        case OP_ATTEND:
            wr.push_back(rng(p[0], n[1] * n[5] * n[7]));
            rd.push_back(rng(p[1], n[1] * n[5] * n[7]));
            rd.push_back(rng(p[2], ring_floats(n[6] * n[4] * n[7], n[9])));
            rd.push_back(rng(p[3], ring_floats(n[6] * n[4] * n[7], n[9])));
            break;
    }
}

// Is what [r) holds after op `from - 1` never read again? True when a later op overwrites
// all of it before any op reads it; false when it is read or the step ends first (the
// caller may read it after the step).
bool dead_after(const std::vector<Op>& ops, size_t from, const Range& r) {
    std::vector<Range> rd, wr;
    for (size_t j = from; j < ops.size(); j++) {
        rd.clear();
        wr.clear();
        op_ranges(ops[j], rd, wr);
        for (auto& x : rd)
            if (overlap(x, r)) return false;
        for (auto& x : wr)
            if (x.a <= r.a && r.b <= x.b) return true;
    }
    return false;
}

// Builds one slm_fg launch: LDS slots, prefetches, prologue ops, segments.
struct FgBuild {
    FgDesc d;
    int lds = 0;  // floats of LDS handed out so far
    struct Slot {  // an LDS vector holding what global [g, g + n) holds at this point
        const float* g;
        int n, off;
    };
    std::vector<Slot> slots;     // produced by prologue ops, in order
    std::vector<int> slot_op;    // the prologue op (index into d.vp) that made each slot, -1: a prefetch
    std::vector<Range> reads, writes;
    int pf4 = 0;

    FgBuild() { std::memset(&d, 0, sizeof d); }
    int alloc(int n) {
        int off = lds;
        lds += (n + 3) & ~3;
        return off;
    }
    // LDS offset of [p, p + len) if a slot produced so far covers it; -1 none; -2 partial
    int find(const float* p, int64_t len, size_t upto) const {
        for (size_t k = std::min(upto, slots.size()); k-- > 0;) {
            const Slot& s = slots[k];
            if (p >= s.g && p + len <= s.g + s.n) return s.off + (int)(p - s.g);
            if (overlap(rng(p, len), rng(s.g, s.n))) return -2;
        }
        return -1;
    }
    // n floats from src (+ dyn[0]·stride) into LDS; n is rounded up to whole float4s, so the
    // source must be 16-byte aligned and readable that far
    bool prefetch(const float* src, int n, const long long* dyn, int stride, int* off) {
        if (d.npf >= SLM_PF_MAX || !aligned16(src) || (dyn && stride % 4)) return false;
        PfOp& p = d.pf[d.npf++];
        int n4 = (n + 3) / 4;
        p.src = src;
        p.dyn = dyn;
        p.n = 4 * n4;
        p.stride = stride;
        p.lds = alloc(4 * n4);
        p.first4 = pf4;
        pf4 += n4;
        *off = p.lds;
        return true;
    }
    // An input vector: a slot if one holds it, else a prefetch of global memory.
    bool input(const float* p, int n, int* off) {
        int r = find(p, n, slots.size());
        if (r == -2) return false;
        if (r >= 0) {
            *off = r;
            return true;
        }
        if (n % 4) return false;
        reads.push_back(rng(p, n));
        return prefetch(p, n, nullptr, 0, off);
    }
};

// Split partials of the one-token linears whose columns span several splits: two
// alternating halves of c->part, so one kernel can read the last linear's partials while
// it writes its own.
int64_t nsplit_of(int64_t cols) {
    int64_t nsl = ((cols + 15) / 16 + SLM_KS - 1) / SLM_KS;
    return (nsl + SLM_SPLIT - 1) / SLM_SPLIT;
}

// Where the planner stood between two ops it took: `out` kernels emitted so far, `next` the
// next op it takes, `low` the first op not yet inside an emitted kernel (ops it holds back
// for a later kernel: prologue ops, row chains, l2norms).
struct PlanMark {
    size_t out, next, low;
};

struct Planner {
    slm_hip* c;
    const std::vector<Op>& ops;
    std::vector<Rec>& out;
    std::vector<PlanMark>* marks = nullptr;
    std::vector<VpSrc> pend;
    int part_flip = 0;
    std::vector<VpSrc> next_pend;  // what a fused kernel leaves pending (a split's fold)
    const Op* l2q = nullptr;  // l2norm ops held back for the GLA kernel that reads them
    const Op* l2k = nullptr;

    // ---- prompt row chains (m > 1): see RowDesc ----
    struct RSlot {  // rows [g + r·stride, + n) of an op's output, held in LDS at `lds`
        const float* g;
        int64_t stride, n;
        int lds;
    };
    int64_t rrows = 0;               // the chain's token rows (0: no chain)
    size_t rstart = 0;               // index of the op the chain started at
    size_t rnext = 0;                // index of the first op after the chain
    int64_t last_m = 0;              // tokens of the last prompt linear
    RowDesc rd{};
    std::vector<const Op*> rsrc;     // the op of each chain entry (null: a split's fold)
    Rec rfold{};                     // what a chain holding only a fold launches instead
    std::vector<RSlot> rslots;
    std::vector<Range> rwr;          // every global range the chain's ops write (all rows)
    std::vector<char> rwr_slot;      // ... and whether an LDS slot holds it
    int rlds = 0;                    // LDS floats the chain uses
    static constexpr int ROW_LDS_MAX = 40000;

    static Range rows_rng(const float* g, int64_t stride, int64_t n, int64_t R) {
        return Range{(uintptr_t)g, (uintptr_t)(g + (R - 1) * stride + n)};
    }
    // Rows the op states itself (0: it is a flat vector, split by the chain's rows).
    static int64_t op_rows(const Op& o) {
        switch (o.kind) {
            case OP_COLUMNS: case OP_ROPE: case OP_STORE: case OP_ADD_ROW: return o.n[0];
            default: return 0;
        }
    }
    // The op as a row op over R rows (operands unresolved); false if it is not row-local.
    static bool row_lower(const Op& o, int64_t R, RowOp* ro, Range* foot) {
        const float* const* p = o.p;
        const int64_t* n = o.n;
        std::memset(ro, 0, sizeof *ro);
        ro->la = ro->lb = ro->lc = ro->ld = ro->out = ro->tmp = -1;
        auto flat = [&](int64_t total, int64_t* len) {
            if (total <= 0 || total % R) return false;
            *len = total / R;
            return true;
        };
        int64_t len = 0;
        switch (o.kind) {
            case OP_COPY:
                if (!flat(n[0], &len)) return false;
                ro->kind = R_COPY; ro->a = {p[1], len};
                break;
            case OP_COLUMNS:  // n0 m, n1 stride, n2 off, n3 len
                if (n[0] != R) return false;
                len = n[3];
                ro->kind = R_COPY; ro->a = {p[1] + n[2], n[1]};
                break;
            case OP_ADD:
                if (!flat(n[0], &len)) return false;
                ro->kind = R_ADD; ro->a = {p[1], len}; ro->b = {p[2], len};
                break;
            case OP_ADD_ROW:  // n0 m, n1 d
                if (n[0] != R) return false;
                len = n[1];
                ro->kind = R_ADD; ro->a = {p[1], len}; ro->b = {p[2], 0};
                break;
            case OP_MIX:
                if (!flat(n[0], &len)) return false;
                ro->kind = R_MIX; ro->a = {p[1], len}; ro->b = {p[2], len}; ro->f0 = o.f[0];
                break;
            case OP_SILU_MUL:
                if (!flat(n[0], &len)) return false;
                ro->kind = R_SILU; ro->a = {p[1], len}; ro->b = {p[2], len};
                break;
            case OP_ROPE:  // n0 m, n1 heads, n2 dh
                if (n[0] != R || n[2] % 2) return false;
                len = n[1] * n[2];
                ro->kind = R_ROPE; ro->a = {p[1], len}; ro->c = {p[2], n[2] / 2}; ro->d = {p[3], n[2] / 2};
                ro->i0 = (int32_t)n[1]; ro->i1 = (int32_t)n[2];
                break;
            case OP_STORE:  // p0 cache, p1 src; n0 m, n1 cap, n2 heads, n3 dh, n4 pos
                if (n[0] != R) return false;
                len = n[2] * n[3];
                ro->kind = R_STORE; ro->a = {p[1], len};
                ro->i0 = (int32_t)n[2]; ro->i1 = (int32_t)n[3]; ro->q0 = n[1]; ro->q1 = n[4];
                ro->h16 = (int32_t)n[5];
                ro->dyn = (const long long*)o.dyn;
                ro->n = (int32_t)len;
                ro->y = (float*)p[0];
                *foot = rng(p[0], ring_floats(n[2] * n[1] * n[3], n[5]));
                return true;
            case OP_RMS:
            case OP_L2NORM:  // n0 groups, n1 size; f0 eps
                if (n[0] % R || n[1] <= 0) return false;
                len = n[0] / R * n[1];
                ro->kind = o.kind == OP_RMS ? R_RMS : R_L2NORM;
                ro->a = {p[1], len};
                if (o.kind == OP_RMS) ro->b = {p[2], 0};
                ro->i0 = (int32_t)n[1]; ro->f0 = o.f[0];
                break;
            default:
                return false;
        }
        if (len <= 0 || len > 16384) return false;
        ro->n = (int32_t)len;
        ro->y = (float*)p[0];
        ro->ystride = len;
        *foot = rows_rng(p[0], len, len, R);
        return true;
    }
    // Where operand `in` (n floats a row) comes from: an LDS slot, global memory (-1), or
    // nowhere safe (false: an earlier op of the chain wrote part of it).
    bool row_src(const RowIn& in, int64_t n, int* lds) {
        Range f = rows_rng(in.g, in.stride, n, rrows);
        for (size_t q = rslots.size(); q-- > 0;) {
            const RSlot& sl = rslots[q];
            if (!overlap(f, rows_rng(sl.g, sl.stride, sl.n, rrows))) continue;
            if (in.stride == sl.stride && in.g >= sl.g && in.g + n <= sl.g + sl.n) {
                *lds = sl.lds + (int)(in.g - sl.g);
                return true;
            }
            return false;
        }
        for (size_t q = 0; q < rwr.size(); q++)
            if (!rwr_slot[q] && overlap(f, rwr[q])) return false;
        *lds = -1;
        return true;
    }
    // Appends op `src` (or a fold when null) to the chain; false when it cannot join.
    // Hazards between workgroups (rows) are ruled out: a global range the chain reads may
    // be written later in the chain only with the same row mapping (each row by its own
    // workgroup, after that workgroup read it); what an op reads that an earlier op wrote
    // comes from that op's LDS row; an output may overwrite an earlier one only exactly.
    struct GRead {
        const float* g;
        int64_t stride, len;
        Range f;
    };
    std::vector<GRead> rreads;
    bool row_add(const Op* src, RowOp ro, Range foot) {
        if (rd.nops >= SLM_ROW_OPS) return false;
        int n = ro.n;
        bool store = ro.kind == R_STORE, norm = ro.kind == R_RMS || ro.kind == R_L2NORM;
        struct Operand { RowIn* in; int* l; int64_t len; };
        Operand opd[4] = {{&ro.a, &ro.la, (int64_t)n},
                          {&ro.b, &ro.lb, norm ? (int64_t)ro.i0 : (int64_t)n},
                          {&ro.c, &ro.lc, (int64_t)ro.i1 / 2},
                          {&ro.d, &ro.ld, (int64_t)ro.i1 / 2}};
        std::vector<GRead> reads;
        for (auto& q : opd) {
            if (!q.in->g) continue;
            if (ro.kind == R_FOLD && q.in == &ro.a) {  // the partials of the GEMM before
                reads.push_back({ro.a.g, ro.a.stride, n,
                                 Range{(uintptr_t)ro.a.g, (uintptr_t)(ro.a.g + ro.i0 * ro.q0)}});
                continue;
            }
            if (!row_src(*q.in, q.len, q.l)) return false;
            if (*q.l < 0) reads.push_back({q.in->g, q.in->stride, q.len, rows_rng(q.in->g, q.in->stride, q.len, rrows)});
        }
        auto rowwise = [&](const GRead& x) {
            return !store && x.g == ro.y && x.stride == ro.ystride && x.len == n;
        };
        for (auto& x : reads)
            if (overlap(x.f, foot) && !rowwise(x)) return false;
        for (auto& x : rreads)
            if (overlap(x.f, foot) && !rowwise(x)) return false;
        int elide = -1;
        for (size_t q = 0; q < rwr.size(); q++) {
            if (!overlap(rwr[q], foot)) continue;
            const RowOp& e = rd.op[q];
            if (store || e.kind == R_STORE || e.y != ro.y || e.ystride != ro.ystride || e.n != ro.n ||
                elide >= 0)
                return false;
            elide = (int)q;
        }
        // float4 moves: every row length, offset and stride a multiple of 4, every global
        // base 16-byte aligned
        bool vec = n % 4 == 0 && (ro.kind != R_ROPE || ro.i1 % 8 == 0) &&
                   (ro.kind != R_STORE || ro.i1 % 4 == 0) && (!norm || ro.i0 % 4 == 0) &&
                   (!ro.y || (aligned16(ro.y) && ro.ystride % 4 == 0)) &&
                   (ro.kind != R_FOLD || ro.q0 % 4 == 0);
        for (auto& q : opd) {
            if (!q.in->g) continue;
            if (*q.l >= 0) vec = vec && *q.l % 4 == 0;
            else vec = vec && aligned16(q.in->g) && q.in->stride % 4 == 0;
        }
        ro.vec = vec ? 1 : 0;
        // global operand rows go to LDS before the first op when they fit the table: an
        // entry that already holds the rows serves again
        int pf_need = 0;
        std::vector<std::pair<int, int>> pf_new;  // (operand, entry) of new entries
        struct PfUse { int q, entry; int64_t off; };
        std::vector<PfUse> pf_use;
        for (int q = 0; q < 4; q++) {
            Operand& x = opd[q];
            if (!x.in->g || *x.l >= 0 || (ro.kind == R_FOLD && q == 0)) continue;
            if (x.len % 4 || !aligned16(x.in->g) || x.in->stride % 4) continue;
            int hit = -1;
            int64_t off = 0;
            for (int e = 0; e < rd.npf; e++) {
                const RowPf& p = rd.pf[e];
                if (p.stride == x.in->stride && x.in->g >= p.g && x.in->g + x.len <= p.g + p.n) {
                    hit = e;
                    off = x.in->g - p.g;
                    break;
                }
            }
            if (hit < 0) {
                if (rd.npf + (int)pf_new.size() >= SLM_ROW_PF) continue;
                hit = rd.npf + (int)pf_new.size();
                pf_new.push_back({q, hit});
                pf_need += (int)((x.len + 255) / 256 * 256);
            }
            pf_use.push_back({q, hit, off});
        }
        int need = store ? 0 : (n + 3) & ~3;
        bool a_pf = false;
        for (auto& u : pf_use) a_pf |= u.q == 0;
        int tmp = norm && ro.la < 0 && !a_pf ? (n + 3) & ~3 : 0;
        if (rlds + need + tmp + pf_need > ROW_LDS_MAX) return false;
        for (auto& pn : pf_new) {  // a new entry: the operand's rows, in whole 64-float4 runs
            Operand& x = opd[pn.first];
            RowPf& p = rd.pf[pn.second];
            p.g = x.in->g;
            p.stride = x.in->stride;
            p.n = (int32_t)x.len;
            p.lds = rlds;
            rlds += (int)((x.len + 255) / 256 * 256);
        }
        rd.npf += (int)pf_new.size();
        for (auto& u : pf_use) {
            *opd[u.q].l = rd.pf[u.entry].lds + (int)u.off;
            if (u.off % 4) ro.vec = 0;
        }
        // what the chain now reads from LDS it read at the start: the ranges stay recorded
        // as read, so later writes into them are held to the same rows
        if (tmp) {
            ro.tmp = rlds;
            rlds += tmp;
        }
        if (!store) {
            ro.out = rlds;
            rlds += need;
        }
        if (elide >= 0) rd.op[elide].y = nullptr;
        for (auto& x : reads) rreads.push_back(x);
        rd.op[rd.nops++] = ro;
        rsrc.push_back(src);
        rwr.push_back(foot);
        rwr_slot.push_back(!store);
        if (!store) rslots.push_back({ro.y, ro.ystride, (int64_t)n, ro.out});
        return true;
    }
    void row_reset() {
        rrows = 0;
        std::memset(&rd, 0, sizeof rd);
        rsrc.clear();
        rslots.clear();
        rwr.clear();
        rwr_slot.clear();
        rreads.clear();
        rlds = 0;
    }
    int row_flush() {
        if (!rrows) return SLM_OK;
        if (rd.nops == 1) {  // alone: its own kernel
            if (rsrc[0]) TRY(lower_one(c, *rsrc[0], out));
            else out.push_back(rfold);
        } else if (rd.nops > 1) {
            // the last op of each global range writes it, unless no later op reads it (the
            // chain's own readers take the LDS row)
            for (int q = 0; q < rd.nops; q++)
                if (rd.op[q].y && rd.op[q].kind != R_STORE && dead_after(ops, rnext, rwr[q]))
                    rd.op[q].y = nullptr;
            rd.r16 = c->fp16 ? 1 : 0;
            Rec r = mk_desc(c->k.rows, (uint32_t)rrows, 256, (uint32_t)(rlds * 4), rd);
            out.push_back(r);
        }
        row_reset();
        return SLM_OK;
    }
    // Tries op o as the chain's next op (starting a chain if there is none).
    bool row_try(const Op& o) {
        int64_t R = op_rows(o);
        if (!rrows) {
            if (!R) R = last_m;
            if (R < 2) return false;
            RowOp ro;
            Range foot;
            if (!row_lower(o, R, &ro, &foot)) return false;
            rrows = R;
            rstart = (size_t)(&o - ops.data());
            if (row_add(&o, ro, foot)) return true;
            row_reset();
            return false;
        }
        if (R && R != rrows) return false;
        RowOp ro;
        Range foot;
        if (!row_lower(o, rrows, &ro, &foot)) return false;
        return row_add(&o, ro, foot);
    }

    // Why a one-token linear runs unfused: printed when SLM_HIP_PLAN_TRACE is set.
    size_t nofuse(size_t i, const char* why) {
        if (c->plan_trace) fprintf(stderr, "slm plan: linear op %zu runs alone: %s\n", i, why);
        return 0;
    }

    int flush_l2() {
        if (l2q) TRY(lower_one(c, *l2q, out));
        if (l2k) TRY(lower_one(c, *l2k, out));
        l2q = l2k = nullptr;
        return SLM_OK;
    }

    int flush_pending() {
        for (auto& v : pend) {
            if (v.kind == SRC_FOLD) {
                out.push_back(mk(c->k.fold, blocks_for(v.n), 1, 1, 256, 0, v.out[0], v.in[0],
                                 (long long)v.n, v.nsplit));
            } else if (v.kind == SRC_COMB) {
                out.push_back(mk(c->k.combine, (uint32_t)((v.heads + 3) / 4), 1, 1, 256, 0, v.out[0],
                                 v.in[0], 1, v.heads, v.dh, v.dp, v.nsplit, (const long long*)nullptr,
                                 (long long)0, (long long)0, (long long)0));
            } else {
                TRY(lower_one(c, *v.op, out));
            }
        }
        pend.clear();
        return SLM_OK;
    }

    // Adds one prologue op; false when it cannot be fused.
    bool add_vp(FgBuild& b, const VpSrc& v, bool side) {
        const Op& so = *v.op;
        if (b.d.nvp >= SLM_VP_MAX) return false;
        int k = b.d.nvp;
        VpOp& o = b.d.vp[k];
        std::memset(&o, 0, sizeof o);
        o.n = v.n;
        o.in1 = -1;
        o.w = -1;
        o.wg0 = side ? 1 : 0;
        o.out = -1;
        auto emit_slot = [&](const float* g, int off) {
            b.slots.push_back({g, v.n, off});
            b.slot_op.push_back(k);
        };
        switch (v.kind) {
            case SRC_GATHER: {  // the row is prefetched straight into its slot
                int off;
                if (!b.prefetch(so.p[1], v.n, (const long long*)so.dyn, v.n, &off)) return false;
                b.reads.push_back(rng(so.p[1], 1));  // the embedding table is only read
                o.kind = VP_COPY;
                o.in0 = off;
                o.gout = (float*)v.out[0];
                b.d.nvp++;
                emit_slot(v.out[0], off);
                b.writes.push_back(rng0(v.out[0], v.n));
                return true;
            }
            case SRC_ROPE_TABLE: {  // two rows of the resident tables at the step's position
                int oc, os;
                if (b.d.nvp + 2 > SLM_VP_MAX) return false;
                if (!b.prefetch(so.p[2], v.n, (const long long*)so.dyn, v.n, &oc)) return false;
                if (!b.prefetch(so.p[3], v.n, (const long long*)so.dyn, v.n, &os)) return false;
                o.kind = VP_COPY;
                o.in0 = oc;
                o.gout = (float*)v.out[0];
                emit_slot(v.out[0], oc);
                b.d.nvp++;
                VpOp& o2 = b.d.vp[b.d.nvp];
                std::memset(&o2, 0, sizeof o2);
                o2.kind = VP_COPY;
                o2.n = v.n;
                o2.in0 = os;
                o2.in1 = -1;
                o2.w = -1;
                o2.out = -1;
                o2.wg0 = o.wg0;
                o2.gout = (float*)v.out[1];
                b.slots.push_back({v.out[1], v.n, os});
                b.slot_op.push_back(b.d.nvp);
                b.d.nvp++;
                b.writes.push_back(rng0(v.out[0], v.n));
                b.writes.push_back(rng0(v.out[1], v.n));
                return true;
            }
            case SRC_FOLD: {
                o.kind = VP_FOLD;
                o.nsb = v.nsplit;
                b.reads.push_back(rng(v.in[0], (int64_t)v.nsplit * v.n));
                if (!b.prefetch(v.in[0], v.nsplit * v.n, nullptr, 0, &o.w)) return false;
                break;
            }
            case SRC_COMB: {  // the attention partials, combined in LDS
                int np = v.nsplit * v.heads * (v.dp + 2);
                o.kind = VP_COMB;
                o.nsb = v.nsplit;
                o.heads = v.heads;
                o.dh = v.dh;
                o.dp = v.dp;
                b.reads.push_back(rng(v.in[0], np));
                if (!b.prefetch(v.in[0], np, nullptr, 0, &o.w)) return false;
                o.in0 = o.w;
                o.in1 = b.alloc(2 * v.heads * v.nsplit);  // the superblock weights
                break;
            }
            default: {
                o.kind = v.kind == SRC_COPY ? VP_COPY : v.kind == SRC_ADD ? VP_ADD : v.kind == SRC_MIX ? VP_MIX
                       : v.kind == SRC_SCALE ? VP_SCALE : v.kind == SRC_RMS ? VP_RMS : VP_SILU;
                if (!b.input(v.in[0], v.n, &o.in0)) return false;
                if (v.in[1] && !b.input(v.in[1], v.n, &o.in1)) return false;
                if (v.kind == SRC_RMS) {
                    b.reads.push_back(rng(so.p[2], v.n));
                    if (!b.prefetch(so.p[2], v.n, nullptr, 0, &o.w)) return false;
                    o.f = so.f[0];
                } else if (v.kind == SRC_SCALE) {
                    o.dyn = (const long long*)so.dyn;
                    o.f = so.f[0];
                } else if (v.kind == SRC_MIX) {
                    o.f = so.f[0];
                }
            }
        }
        // an input that starts inside another op's output (not at its start) holds elements
        // other threads wrote: a barrier comes first
        for (int in : {o.in0, o.in1}) {
            if (in < 0) continue;
            for (size_t q = 0; q < b.slots.size(); q++)
                if (b.slot_op[q] >= 0 && in > b.slots[q].off && in < b.slots[q].off + b.slots[q].n)
                    o.sync = 1;
        }
        o.out = b.alloc(v.n);
        o.gout = (float*)v.out[0];
        b.writes.push_back(rng0(v.out[0], v.n));
        emit_slot(v.out[0], o.out);
        b.d.nvp++;
        return true;
    }

    static void seg_init(FgSeg& s, const Op& L) {
        s.w = L.p[1];
        s.y = (float*)L.p[0];
        s.rows = (int32_t)L.n[0];
        s.rpt = 16;
        s.tiles = (int32_t)((L.n[0] + 15) / 16);
        s.nsplit = 1;
        s.epi = EPI_PLAIN;
    }

    // Rows per tile of a one-matrix fused GEMV: 16, 12, 8 or 4, whichever gives the least
    // estimated time per workgroup — rounds of two units (a load latency each, ≈1 us) plus
    // the weight bytes of the busiest workgroup at ≈24 KB/us (a compute unit's share of HBM
    // when every one streams); a smaller tile must gain a tenth. Smaller tiles spread a short
    // matrix (768 rows: 48 tiles of 16) over more compute units; the MFMA rows past the tile
    // are zeros. `forced` (slm_hip_set_tile_rows) picks one where the pairs allow it.
    static int choose_rpt(const FgSeg& s, int64_t cols, double wbytes, int forced) {
        int64_t split_cols = std::min<int64_t>(cols, (int64_t)SLM_SPLIT * SLM_KS * 16);
        int best = 16;
        double best_t = 0.0;
        for (int rpt : {16, 12, 8, 4}) {
            if (s.pair_rows % rpt) continue;
            int64_t units = (s.rows + rpt - 1) / rpt * s.nsplit;
            int64_t grid = std::min<int64_t>(units, FG_GRID_MAX);
            int64_t per = (units + grid - 1) / grid;
            double t = (double)((per + 1) / 2) + (double)per * rpt * split_cols * wbytes / 24e3;
            if (forced ? rpt == forced : (rpt == 16 || t < 0.9 * best_t)) {
                best = rpt;
                best_t = t;
            }
        }
        return best;
    }

    // Tries to fuse pend + ops[i] (a one-token linear) + what follows. Returns the number of
    // ops of `ops` consumed from i (0: no fusion).
    size_t try_fg(size_t i) {
        const Op& L = ops[i];
        int64_t rows = L.n[0], cols = L.n[1];
        if (L.n[2] != 1 || cols % 16 || cols > VP_LEN_MAX || !aligned16(L.p[1]) || rows < 1 ||
            rows > (int64_t)1 << 26)
            return nofuse(i, "shape");
        const float* x = L.p[2];
        FgBuild b;
        for (auto& v : pend)
            if (!add_vp(b, v, false)) return nofuse(i, "a pending op does not fit the prologue");
        size_t nproduced = b.slots.size();  // slots the linear may read
        int64_t nsplit = nsplit_of(cols);
        size_t used = 1;
        FgSeg seg[SLM_SEG_MAX];
        std::memset(seg, 0, sizeof seg);
        int nseg = 1;
        auto is = [&](size_t j, uint32_t kind) { return j < ops.size() && ops[j].kind == kind; };
        const float* y = L.p[0];
        FgSeg& s0 = seg[0];
        seg_init(s0, L);
        const float *cs = nullptr, *sn = nullptr;
        const Op *hold_q = nullptr, *hold_k = nullptr;
        if (nsplit > 1) {
            // the partials go out; the fold waits for the next kernel's prologue
            if ((int64_t)c->part_bytes < 2 * nsplit * rows * 4) return nofuse(i, "no room for split partials");
            s0.nsplit = (int32_t)nsplit;
            s0.part = c->part + (size_t)part_flip * (c->part_bytes / 8);
        }
        // S block: rope q, rope k, store k, store v (model.rs:430-438)
        if (nsplit == 1 && is(i + 1, OP_ROPE) && is(i + 2, OP_ROPE) && is(i + 3, OP_STORE) &&
            is(i + 4, OP_STORE)) {
            const Op &rq = ops[i + 1], &rk = ops[i + 2], &sk = ops[i + 3], &sv = ops[i + 4];
            int64_t heads = rq.n[1], dh = rq.n[2], dd = heads * dh;
            bool ok = rq.n[0] == 1 && rk.n[0] == 1 && rk.n[1] == heads && rk.n[2] == dh &&
                      rows == 3 * dd && rq.p[1] == y && rk.p[1] == y + dd && rq.p[2] == rk.p[2] &&
                      rq.p[3] == rk.p[3] && sk.n[0] == 1 && sv.n[0] == 1 && sk.p[1] == rk.p[0] &&
                      sv.p[1] == y + 2 * dd && sk.n[1] == sv.n[1] && sk.n[2] == heads &&
                      sv.n[2] == heads && sk.n[3] == dh && sv.n[3] == dh && dh % 2 == 0 &&
                      dd % 16 == 0 && sk.n[5] == sv.n[5];
            if (ok) {
                used = 5;
                s0.epi = EPI_ROPE;
                s0.pair_rows = (int32_t)(2 * dd);
                s0.half = (int32_t)(dh / 2);
                s0.d = (int32_t)dd;
                s0.dh = (int32_t)dh;
                s0.o1 = (float*)rq.p[0];
                s0.o2 = (float*)rk.p[0];
                s0.o3 = (float*)sk.p[0];
                s0.o4 = (float*)sv.p[0];
                cs = rq.p[2];
                sn = rq.p[3];
                s0.cap = sk.n[1];
                s0.ring16 = (int32_t)sk.n[5];
                s0.dyn = (const long long*)sk.dyn;
                s0.imm = sk.n[4];
                s0.dyn2 = (const long long*)sv.dyn;
                s0.imm2 = sv.n[4];
            }
        }
        // L block: the two l2norms wait for the GLA kernel; the decay linear on the same
        // input joins as a second matrix (model.rs:463-470)
        if (s0.epi == EPI_PLAIN && nsplit == 1 && is(i + 1, OP_L2NORM) && is(i + 2, OP_L2NORM) &&
            is(i + 3, OP_LINEAR)) {
            const Op &lq = ops[i + 1], &lk = ops[i + 2], &D = ops[i + 3];
            int64_t heads = lq.n[0], dh = lq.n[1], dd = heads * dh;
            bool ok = lk.n[0] == heads && lk.n[1] == dh && rows == 4 * dd && lq.p[1] == y &&
                      lk.p[1] == y + dd && D.n[2] == 1 && D.p[2] == x && D.n[1] == cols &&
                      aligned16(D.p[1]) && D.n[3] == L.n[3] && D.n[4] == L.n[4];
            // the l2norm outputs are untouched until the GLA kernel writes them
            ok = ok && !overlap(rng(lq.p[0], dd), rng(D.p[0], D.n[0])) &&
                 !overlap(rng(lk.p[0], dd), rng(D.p[0], D.n[0])) &&
                 !overlap(rng(lq.p[0], dd), rng(y, rows)) && !overlap(rng(lk.p[0], dd), rng(y, rows)) &&
                 !overlap(rng(lq.p[0], dd), rng(x, cols)) && !overlap(rng(lk.p[0], dd), rng(x, cols)) &&
                 !overlap(rng(D.p[0], D.n[0]), rng(y, rows));
            if (ok) {
                seg_init(seg[1], D);
                nseg = 2;
                used = 4;
                hold_q = &lq;
                hold_k = &lk;
            }
        }
        // MLP up: SiLU of the gate half times the amp half (model.rs:552-555)
        if (s0.epi == EPI_PLAIN && nseg == 1 && nsplit == 1 && is(i + 1, OP_SILU_MUL)) {
            const Op& sm = ops[i + 1];
            int64_t hid = rows / 2;
            if (rows % 16 == 0 && sm.n[0] == hid && sm.p[1] == y && sm.p[2] == y + hid &&
                !overlap(rng(sm.p[0], hid), rng(y, rows))) {
                used = 2;
                s0.epi = EPI_SILU;
                s0.pair_rows = (int32_t)rows;
                s0.half = (int32_t)hid;
                s0.o1 = (float*)sm.p[0];
            }
        }
        // residual add after the linear (model.rs:547, 557)
        if (s0.epi == EPI_PLAIN && nseg == 1 && nsplit == 1 && is(i + 1, OP_ADD) &&
            ops[i + 1].n[0] == rows && (ops[i + 1].p[1] == y || ops[i + 1].p[2] == y)) {
            const Op& a = ops[i + 1];
            const float* r = a.p[1] == y ? a.p[2] : a.p[1];
            if (!overlap(rng(r, rows), rng(y, rows)) && b.find(r, rows, b.slots.size()) == -1) {
                used = 2;
                s0.epi = EPI_RESID;
                s0.o1 = (float*)a.p[0];
                s0.res = r;
                b.reads.push_back(rng(r, rows));
            }
        }
        // the greedy pick of the logits (model twin's device-pick decode): each workgroup's
        // first maximum goes into a 64-bit atomic maximum, and the last workgroup to finish
        // writes the pick (sample.rs:48-53, the rule of slm_argmax)
        if (s0.epi == EPI_PLAIN && nseg == 1 && nsplit == 1 && is(i + 1, OP_ARGMAX) &&
            ops[i + 1].p[1] == y && ops[i + 1].n[0] == rows && rows <= INT32_MAX) {
            const Op& a = ops[i + 1];
            used = 2;
            s0.epi = EPI_PICK;
            s0.o1 = (float*)a.p[0];
            s0.o2 = (float*)a.p[2];
            s0.o3 = c->pick;
            s0.dyn = (const long long*)a.dyn;
            s0.imm = a.n[1];
        }
        int64_t nsl = (cols / 16 + SLM_KS - 1) / SLM_KS;
        int W = (int)std::min<int64_t>(nsl, SLM_SPLIT);
        if (nseg == 1) {
            s0.rpt = choose_rpt(s0, cols, L.n[4] ? 2.0 : 4.0, c->fg_rpt);
            s0.tiles = (s0.rows + s0.rpt - 1) / s0.rpt;
        }
        // what the segments read and write
        int units = 0;
        for (int k = 0; k < nseg; k++) {
            FgSeg& s = seg[k];
            s.units = s.tiles * s.nsplit;
            s.unit_first = units;
            units += s.units;
            b.reads.push_back(rng(s.w, L.n[4] ? ((int64_t)s.rows * cols + 1) / 2 : (int64_t)s.rows * cols));
            if (s.nsplit > 1) {
                b.writes.push_back(rng(s.part, (int64_t)s.nsplit * s.rows));
                continue;
            }
            b.writes.push_back(rng(s.y, s.rows));
            switch (s.epi) {
                case EPI_RESID: b.writes.push_back(rng(s.o1, s.rows)); break;
                case EPI_SILU: b.writes.push_back(rng(s.o1, s.half)); break;
                case EPI_PICK: {
                    const Op& a = ops[i + 1];
                    b.writes.push_back(rng(a.p[0], 2));
                    if (a.p[2]) b.writes.push_back(rng(a.p[2], a.n[2]));
                    break;
                }
                case EPI_ROPE: {
                    int64_t heads = s.d / s.dh;
                    b.writes.push_back(rng(s.o1, s.d));
                    b.writes.push_back(rng(s.o2, s.d));
                    b.writes.push_back(rng(s.o3, ring_floats(heads * s.cap * s.dh, s.ring16)));
                    b.writes.push_back(rng(s.o4, ring_floats(heads * s.cap * s.dh, s.ring16)));
                    break;
                }
            }
        }
        // the GEMV input and the epilogue inputs
        std::vector<int> want;
        int xin = b.find(x, cols, nproduced);
        if (xin == -2) return nofuse(i, "input partly produced by the prologue");
        if (xin >= 0) {
            want.push_back(xin);
        } else {
            b.reads.push_back(rng(x, cols));
            if (!b.prefetch(x, (int)cols, nullptr, 0, &xin)) return nofuse(i, "input cannot be prefetched");
        }
        if (s0.epi == EPI_ROPE) {
            int half = s0.dh / 2;
            int r1 = b.find(cs, half, nproduced), r2 = b.find(sn, half, nproduced);
            if (r1 == -2 || r2 == -2) return nofuse(i, "rope table partly produced by the prologue");
            if (r1 < 0) {
                if (half % 4) return nofuse(i, "rope table rows not whole float4s");
                b.reads.push_back(rng(cs, half));
                if (!b.prefetch(cs, half, nullptr, 0, &r1)) return nofuse(i, "rope table cannot be prefetched");
            } else {
                want.push_back(r1);
            }
            if (r2 < 0) {
                if (half % 4) return nofuse(i, "rope table rows not whole float4s");
                b.reads.push_back(rng(sn, half));
                if (!b.prefetch(sn, half, nullptr, 0, &r2)) return nofuse(i, "rope table cannot be prefetched");
            } else {
                want.push_back(r2);
            }
            s0.cs_lds = r1;
            s0.sn_lds = r2;
        }
        // element-wise ops right after the group that neither read its results nor touch
        // what it reads run in workgroup 0 (e.g. the copy s <- x after the inject linear,
        // model.rs:580-581)
        for (size_t j = i + used; j < ops.size() && nsplit == 1; j++) {
            VpSrc v;
            if (!vp_of(ops[j], &v) || (v.kind != SRC_COPY && v.kind != SRC_ADD && v.kind != SRC_MIX))
                break;
            // (prologue outputs are in LDS slots by then, and workgroup 0 writes its own
            // outputs in order; what every workgroup writes is out of reach)
            bool clash = false;
            for (int q = 0; q < 2; q++) {
                if (v.in[q])
                    for (auto& w : b.writes) clash |= !w.wg0 && overlap(rng(v.in[q], v.n), w);
                if (v.out[q]) {
                    for (auto& w : b.writes) clash |= !w.wg0 && overlap(rng(v.out[q], v.n), w);
                    for (auto& r : b.reads) clash |= overlap(rng(v.out[q], v.n), r);
                }
            }
            if (clash) break;
            FgBuild save = b;
            if (!add_vp(b, v, true)) {
                b = save;
                break;
            }
            used++;
        }
        // prologue ops every workgroup needs: those the GEMV input and the epilogue read
        std::vector<bool> need(b.d.nvp, false);
        for (size_t k = b.slots.size(); k-- > 0;) {
            const auto& sl = b.slots[k];
            int opk = b.slot_op[k];
            bool hit = false;
            for (int w : want) hit |= w >= sl.off && w < sl.off + sl.n;
            if (!hit || opk < 0 || need[opk]) continue;
            need[opk] = true;
            const VpOp& o = b.d.vp[opk];
            want.push_back(o.in0);
            if (o.in1 >= 0) want.push_back(o.in1);
            // the slot's op may read slots made earlier: resolve them on later passes
            k = b.slots.size();
        }
        for (int k = 0; k < b.d.nvp; k++) b.d.vp[k].wg0 = need[k] ? 0 : 1;
        // prologue outputs that no later op reads are not written out (their LDS copies
        // still serve this kernel); a side op that writes nothing else is dropped from
        // workgroup 0's work
        {
            std::vector<Range> kept;
            for (auto& w : b.writes)
                if (!w.wg0) kept.push_back(w);
            for (int k = 0; k < b.d.nvp; k++) {
                VpOp& o = b.d.vp[k];
                if (!o.gout) continue;
                if (dead_after(ops, i + used, rng(o.gout, o.n)))
                    o.gout = nullptr;
                else
                    kept.push_back(rng0(o.gout, o.n));
            }
            b.writes.swap(kept);
        }
        // hazards: no global write of this kernel may meet a global read or another write
        for (auto& w : b.writes)
            for (auto& r : b.reads)
                if (overlap(w, r)) {
                    if (c->plan_trace) {
                        fprintf(stderr, "slm plan: write [%#zx, %#zx) meets read [%#zx, %#zx)\n",
                                (size_t)w.a, (size_t)w.b, (size_t)r.a, (size_t)r.b);
                        for (auto& v : pend)
                            fprintf(stderr, "  pending kind %d n %d in %p %p out %p\n", v.kind, v.n,
                                    (const void*)v.in[0], (const void*)v.in[1], (const void*)v.out[0]);
                        for (size_t j = i; j < i + used; j++)
                            fprintf(stderr, "  op %zu kind %u p %p %p %p\n", j, ops[j].kind,
                                    (const void*)ops[j].p[0], (const void*)ops[j].p[1], (const void*)ops[j].p[2]);
                    }
                    return nofuse(i, "a write meets a read");
                }
        // (prologue outputs may meet each other: workgroup 0 writes them one after another)
        for (size_t a = 0; a < b.writes.size(); a++)
            for (size_t q = a + 1; q < b.writes.size(); q++)
                if (overlap(b.writes[a], b.writes[q]) && !(b.writes[a].wg0 && b.writes[q].wg0))
                    return nofuse(i, "two writes meet");
        FgDesc& d = b.d;
        d.cw = -1;
        if (nsplit == 1 && d.nvp == 1 && d.vp[0].kind == VP_COMB && d.vp[0].dh == 64 &&
            (int64_t)d.vp[0].heads * 64 == cols && d.vp[0].nsb <= 64 && xin == d.vp[0].out &&
            std::count(want.begin(), want.end(), xin) == 1) {
            // the attention output is only the GEMV's input: wave w combines head w itself
            d.cw = d.vp[0].w;
            d.cdp = d.vp[0].dp;
            d.cnsb = d.vp[0].nsb;
            d.cgout = d.vp[0].gout;
            d.nvp = 0;
        }
        d.cols = (int32_t)cols;
        d.nsl = (int32_t)nsl;
        d.W = W;
        d.xin = xin;
        d.nseg = nseg;
        d.units = units;
        d.pf4 = b.pf4;
        d.f16 = (int32_t)L.n[3];
        d.spin = c->spin;
        d.fault = c->fault_dev;
        // the prologue's signature: every op a float4 op of at most one float4 per prologue
        // thread (the straight-line code of the fused kernel), else 0 (its general loop)
        d.sig = d.nvp > 0 && d.nvp <= SLM_SIG_OPS ? d.nvp : 0;
        d.nsf = 0;
        for (int k = 0; k < d.nvp; k++) {
            const VpOp& o = d.vp[k];
            if (o.kind == VP_SCALE && o.dyn) d.nsf++;
            bool v4 = ((o.in0 | (o.in1 >= 0 ? o.in1 : 0) | (o.out >= 0 ? o.out : 0) |
                        (o.w >= 0 ? o.w : 0) | o.n) & 3) == 0;
            bool fast = v4 && o.n / 4 <= 64 * SLM_FG_EPI_WAVES && o.kind != VP_COMB &&
                        (o.kind != VP_FOLD || o.nsb <= 8);
            if (!fast) d.sig = 0;
            if (d.sig && k < SLM_SIG_OPS) d.sig |= o.kind << (4 * (k + 1));
        }
        d.lds_vp = (b.lds + 3) & ~3;
        d.fold_off = d.lds_vp + SLM_FG_MISC;
        int total = d.fold_off + 4 * W * 16;
        if (total * 4 > LDS_MAX) return nofuse(i, "LDS");
        auto magic = [](int32_t v) { return v > 1 ? (uint32_t)(((1ull << 32) + (uint64_t)v - 1) / (uint64_t)v) : 0u; };
        for (int k = 0; k < nseg; k++) {
            d.seg[k] = seg[k];
            d.seg[k].mtiles = magic(seg[k].tiles);
            d.seg[k].mhalf = magic(seg[k].half);
        }
        int threads = 64 * (W + SLM_FG_EPI_WAVES);
        uint32_t grid = (uint32_t)std::min(units, FG_GRID_MAX);
        hipFunction_t fk = L.n[4] ? c->k.fghw : d.f16 ? c->k.fgh : c->k.fg;
        out.push_back(mk_desc(fk, grid, (uint32_t)threads, (uint32_t)(total * 4), d));
        double ab = 16.0 * d.pf4;  // prologue vectors, then weights and outputs
        double wb = L.n[4] ? 2.0 : 4.0;  // bytes per weight
        for (int k = 0; k < nseg; k++) ab += wb * (double)seg[k].rows * cols + 4.0 * seg[k].rows;
        out.back().abytes = ab;
        if (nsplit > 1) {
            part_flip ^= 1;
            VpSrc f;
            f.kind = SRC_FOLD;
            f.n = (int)rows;
            f.nsplit = (int)nsplit;
            f.in[0] = s0.part;
            f.out[0] = y;
            f.op = &L;
            next_pend.push_back(f);
        }
        if (hold_q) {
            l2q = hold_q;
            l2k = hold_k;
        }
        return used;
    }

    // [l2norm q, l2norm k] + gla (one token) + rms(head_norm) + silu_mul(gate):
    // model.rs:465-484
    size_t try_gla(size_t i) {
        const Op& g = ops[i];
        if (g.n[0] != 1) return 0;
        int64_t heads = g.n[1], dh = g.n[2];
        if (dh * 16 > 1024) return 0;  // a head per workgroup, sixteen lanes per column
        GlaDesc d;
        std::memset(&d, 0, sizeof d);
        d.r16 = c->fp16 ? 1 : 0;
        d.y = (float*)g.p[0];
        d.s = (float*)g.p[1];
        d.q = g.p[2];
        d.k = g.p[3];
        d.v = g.p[4];
        d.decay = g.p[5];
        d.bias = g.p[6];
        d.heads = (int32_t)heads;
        d.dh = (int32_t)dh;
        int64_t n = heads * dh;
        if (l2q && l2q->p[0] == g.p[2] && l2k->p[0] == g.p[3] && l2q->n[0] == heads &&
            l2q->n[1] == dh && l2k->n[0] == heads && l2k->n[1] == dh) {
            // each workgroup normalises its own head before it reads q and k; the raw
            // vectors are not written, and the normalised ones (possibly in place of the
            // raw ones) meet nothing else the kernel reads or writes
            std::vector<Range> wr = {rng(g.p[0], n), rng(g.p[1], heads * dh * dh)};
            if (i + 2 < ops.size() && ops[i + 1].kind == OP_RMS && ops[i + 2].kind == OP_SILU_MUL) {
                wr.push_back(rng(ops[i + 1].p[0], n));
                wr.push_back(rng(ops[i + 2].p[0], n));
            }
            std::vector<Range> rd = {rng(g.p[4], n), rng(g.p[5], heads), rng(g.p[6], heads)};
            Range rq = rng(l2q->p[1], n), rk = rng(l2k->p[1], n);
            Range nq = rng(l2q->p[0], n), nk = rng(l2k->p[0], n);
            bool ok = !overlap(nq, nk) && !overlap(rq, nk) && !overlap(rk, nq);
            for (auto& w : wr) ok = ok && !overlap(w, rq) && !overlap(w, rk) && !overlap(w, nq) && !overlap(w, nk);
            for (auto& r : rd) ok = ok && !overlap(r, nq) && !overlap(r, nk);
            if (ok) {
                d.l2 = 1;
                d.q = l2q->p[1];
                d.k = l2k->p[1];
                d.qn = (float*)l2q->p[0];
                d.kn = (float*)l2k->p[0];
                l2q = l2k = nullptr;
            }
        }
        if (l2q) return 0;  // held l2norms this kernel cannot take: run them first
        size_t used = 1;
        if (i + 2 < ops.size() && ops[i + 1].kind == OP_RMS && ops[i + 2].kind == OP_SILU_MUL) {
            const Op &r = ops[i + 1], &sm = ops[i + 2];
            bool ok = r.n[0] == heads && r.n[1] == dh && r.p[1] == g.p[0] && sm.n[0] == n &&
                      sm.p[2] == r.p[0];
            // the gate is read while y, y2 and the output are written by other workgroups
            ok = ok && !overlap(rng(sm.p[1], n), rng(g.p[0], n)) &&
                 !overlap(rng(sm.p[1], n), rng(r.p[0], n)) && !overlap(rng(sm.p[1], n), rng(sm.p[0], n)) &&
                 !overlap(rng(r.p[0], n), rng(g.p[0], n));
            if (d.l2)
                ok = ok && !overlap(rng(sm.p[1], n), rng(d.qn, n)) && !overlap(rng(sm.p[1], n), rng(d.kn, n)) &&
                     !overlap(rng(r.p[0], n), rng(d.qn, n)) && !overlap(rng(r.p[0], n), rng(d.kn, n)) &&
                     !overlap(rng(sm.p[0], n), rng(d.qn, n)) && !overlap(rng(sm.p[0], n), rng(d.kn, n));
            if (ok) {
                d.fuse = 1;
                d.y2 = (float*)r.p[0];
                d.hn = r.p[2];
                d.eps = r.f[0];
                d.gate = sm.p[1];
                d.out = (float*)sm.p[0];
                used = 3;
            }
        }
        int ri = pow2_index((dh + 15) / 16, 2);
        // (dh = 64: the state staged in LDS, 64 rows of 65)
        size_t stage = dh == 64 ? 64 * 65 : 0;
        out.push_back(mk_desc(c->k.gla1[ri], (uint32_t)heads, (uint32_t)((dh * 16 + 63) / 64 * 64),
                              (uint32_t)((4 * dh + 16 + stage) * 4), d));
        return used;
    }

    // The prompt MLP's up projection (model.rs:552-555): up = linear(n) [m][2h], gate and amp
    // its column halves, y = silu_mul(gate, amp). When up, gate and amp are read by nothing
    // after, one GEMM writes y from paired gate/amp row tiles (slm_gemm2s_*).
    size_t try_gemm_silu(size_t i) {
        const Op& L = ops[i];
        if (i + 3 >= ops.size()) return 0;
        const Op &cg = ops[i + 1], &ca = ops[i + 2], &sm = ops[i + 3];
        int64_t rows = L.n[0], cols = L.n[1], m = L.n[2], h = rows / 2;
        if (m <= 16 || rows % 2 || cols % 64 || cols / 64 > SLM_SPLIT || !aligned16(L.p[1]) ||
            !aligned16(L.p[2]))
            return 0;
        if (cg.kind != OP_COLUMNS || ca.kind != OP_COLUMNS || sm.kind != OP_SILU_MUL) return 0;
        if (cg.p[1] != L.p[0] || ca.p[1] != L.p[0] || cg.n[0] != m || ca.n[0] != m || cg.n[1] != rows ||
            ca.n[1] != rows || cg.n[2] != 0 || ca.n[2] != h || cg.n[3] != h || ca.n[3] != h)
            return 0;
        if (sm.p[1] != cg.p[0] || sm.p[2] != ca.p[0] || sm.n[0] != m * h) return 0;
        if (!dead_after(ops, i + 4, rng(L.p[0], m * rows)) || !dead_after(ops, i + 4, rng(cg.p[0], m * h)) ||
            !dead_after(ops, i + 4, rng(ca.p[0], m * h)))
            return 0;
        Range ry = rng(sm.p[0], m * h);
        if (overlap(ry, rng(L.p[1], wfloats(L))) || overlap(ry, rng(L.p[2], m * cols))) return 0;
        int bm = gemm2_bm(rows, m, 1);
        int q = bm == 32 ? 0 : bm == 64 ? 1 : bm == 96 ? 2 : 3;
        uint32_t shmem = (uint32_t)(GEMM_STAGES_HOST * (bm * (L.n[4] ? 32 : 64) + 64 * 64) * 4);
        hipFunction_t gf = L.n[4] ? c->k.gemm2hsw[q] : L.n[3] ? c->k.gemm2hs[q] : c->k.gemm2s[q];
        out.push_back(mk(gf, (uint32_t)((h + bm / 2 - 1) / (bm / 2)),
                         (uint32_t)((m + 63) / 64), 1, gemm2_threads(bm), shmem, sm.p[0], c->gpart,
                         L.p[1], L.p[2], (int)rows, (int)cols, (int)m));
        out.back().abytes = 4.0 * (double)(rows * cols + m * cols + m * h);
        last_m = m;
        return 4;
    }

    // The prompt attention input (model.rs:417-432): mix = linear(n) [m][3d]; q = rope(mix
    // columns 0..d), k = rope(columns d..2d), v = columns 2d..3d; k and v into the rings.
    // With 64-dim heads each 64-row tile of the GEMM is one head of q, k or v, so one GEMM
    // (slm_gemm2r_64) writes mix, q, k, v and both rings; only the column scratch that the
    // chain passes through is left unwritten, so it must be read by nothing after.
    size_t try_gemm_rope(size_t i) {
        if (i + 7 >= ops.size()) return 0;
        const Op &L = ops[i], &c1 = ops[i + 1], &r1 = ops[i + 2], &c2 = ops[i + 3], &r2 = ops[i + 4],
                 &c3 = ops[i + 5], &s1 = ops[i + 6], &s2 = ops[i + 7];
        if (c1.kind != OP_COLUMNS || r1.kind != OP_ROPE || c2.kind != OP_COLUMNS || r2.kind != OP_ROPE ||
            c3.kind != OP_COLUMNS || s1.kind != OP_STORE || s2.kind != OP_STORE)
            return 0;
        int64_t rows = L.n[0], cols = L.n[1], m = L.n[2], d = rows / 3;
        if (m <= 16 || rows % 3 || d % 64 || cols % 64 || cols / 64 > SLM_SPLIT || !aligned16(L.p[1]) ||
            !aligned16(L.p[2]))
            return 0;
        const float* mix = L.p[0];
        const float* cy = c1.p[0];  // the column scratch
        auto col_ok = [&](const Op& c, int64_t off, const float* y) {
            return c.p[0] == y && c.p[1] == mix && c.n[0] == m && c.n[1] == rows && c.n[2] == off &&
                   c.n[3] == d;
        };
        if (!col_ok(c1, 0, cy) || !col_ok(c2, d, cy) || !col_ok(c3, 2 * d, c3.p[0])) return 0;
        auto rope_ok = [&](const Op& r) {
            return r.p[1] == cy && r.n[0] == m && r.n[2] == 64 && r.n[1] * 64 == d && r.p[2] == r1.p[2] &&
                   r.p[3] == r1.p[3];
        };
        if (!rope_ok(r1) || !rope_ok(r2)) return 0;
        const float *q = r1.p[0], *k = r2.p[0], *v = c3.p[0];
        auto store_ok = [&](const Op& st, const float* src) {
            return st.p[1] == src && st.n[0] == m && st.n[1] == s1.n[1] && st.n[2] * 64 == d &&
                   st.n[3] == 64 && st.n[5] == s1.n[5];
        };
        if (!store_ok(s1, k) || !store_ok(s2, v) || s1.p[0] == s2.p[0]) return 0;
        int64_t cap = s1.n[1];
        // what the chain writes, what it reads: pairwise apart, so the order of the writes
        // does not matter
        std::vector<Range> wr = {rng(mix, m * rows), rng(cy, m * d), rng(q, m * d), rng(k, m * d),
                                 rng(v, m * d), rng(s1.p[0], ring_floats(d * cap, s1.n[5])),
                                 rng(s2.p[0], ring_floats(d * cap, s1.n[5]))};
        std::vector<Range> rd = {rng(L.p[1], wfloats(L)), rng(L.p[2], m * cols), rng(r1.p[2], m * 32),
                                 rng(r1.p[3], m * 32)};
        for (size_t a = 0; a < wr.size(); a++) {
            for (size_t b = a + 1; b < wr.size(); b++)
                if (overlap(wr[a], wr[b])) return 0;
            for (auto& x : rd)
                if (overlap(wr[a], x)) return 0;
        }
        if (!dead_after(ops, i + 8, rng(cy, m * d))) return 0;
        uint32_t shmem = (uint32_t)(GEMM_STAGES_HOST * (64 * (L.n[4] ? 32 : 64) + 64 * 64) * 4);
        hipFunction_t gf = L.n[4] ? c->k.gemm2hrw : L.n[3] ? c->k.gemm2hr : c->k.gemm2r;
        out.push_back(mk(gf, (uint32_t)(rows / 64), (uint32_t)((m + 63) / 64),
                         1, gemm2_threads(64), shmem, (float*)mix, c->gpart, L.p[1], L.p[2], (int)rows,
                         (int)cols, (int)m, (float*)q, (float*)k, (float*)v, (float*)s1.p[0],
                         (float*)s2.p[0], r1.p[2], r1.p[3], (const long long*)s1.dyn, (const long long*)s2.dyn,
                         (long long)s1.n[4], (long long)s2.n[4], (long long)cap, (int)d, (int)s1.n[5]));
        out.back().abytes = 4.0 * (double)(rows * cols + m * cols + m * rows + 3 * m * d + 2 * m * d + 2 * m * 32);
        last_m = m;
        return 8;
    }

    // The prompt linear-attention input (model.rs:434-440): mix = linear(n) [m][4d]; q and k
    // = l2norm(mix columns 0..d, d..2d) per 64-dim head, v and the gate the columns 2d..3d,
    // 3d..4d. One GEMM (slm_gemm2n_64) writes mix, q, k, v and the gate; the column scratch
    // the chain passes through is left unwritten, so it must be read by nothing after.
    size_t try_gemm_l2(size_t i) {
        if (i + 6 >= ops.size()) return 0;
        const Op &L = ops[i], &c1 = ops[i + 1], &n1 = ops[i + 2], &c2 = ops[i + 3], &n2 = ops[i + 4],
                 &c3 = ops[i + 5], &c4 = ops[i + 6];
        if (c1.kind != OP_COLUMNS || n1.kind != OP_L2NORM || c2.kind != OP_COLUMNS ||
            n2.kind != OP_L2NORM || c3.kind != OP_COLUMNS || c4.kind != OP_COLUMNS)
            return 0;
        int64_t rows = L.n[0], cols = L.n[1], m = L.n[2], d = rows / 4;
        if (m <= 16 || rows % 4 || d % 64 || cols % 64 || cols / 64 > SLM_SPLIT || !aligned16(L.p[1]) ||
            !aligned16(L.p[2]))
            return 0;
        const float* mix = L.p[0];
        const float* cy = c1.p[0];
        auto col_ok = [&](const Op& c, int64_t off, const float* y) {
            return c.p[0] == y && c.p[1] == mix && c.n[0] == m && c.n[1] == rows && c.n[2] == off &&
                   c.n[3] == d;
        };
        if (!col_ok(c1, 0, cy) || !col_ok(c2, d, cy) || !col_ok(c3, 2 * d, c3.p[0]) ||
            !col_ok(c4, 3 * d, c4.p[0]))
            return 0;
        auto norm_ok = [&](const Op& o) { return o.p[1] == cy && o.n[1] == 64 && o.n[0] * 64 == m * d; };
        if (!norm_ok(n1) || !norm_ok(n2)) return 0;
        const float *q = n1.p[0], *k = n2.p[0], *v = c3.p[0], *g = c4.p[0];
        std::vector<Range> wr = {rng(mix, m * rows), rng(cy, m * d), rng(q, m * d), rng(k, m * d),
                                 rng(v, m * d), rng(g, m * d)};
        std::vector<Range> rd = {rng(L.p[1], wfloats(L)), rng(L.p[2], m * cols)};
        for (size_t a = 0; a < wr.size(); a++) {
            for (size_t b = a + 1; b < wr.size(); b++)
                if (overlap(wr[a], wr[b])) return 0;
            for (auto& x : rd)
                if (overlap(wr[a], x)) return 0;
        }
        if (!dead_after(ops, i + 7, rng(cy, m * d))) return 0;
        uint32_t shmem = (uint32_t)(GEMM_STAGES_HOST * (64 * (L.n[4] ? 32 : 64) + 64 * 64) * 4);
        hipFunction_t gf = L.n[4] ? c->k.gemm2hnw : L.n[3] ? c->k.gemm2hn : c->k.gemm2n;
        out.push_back(mk(gf, (uint32_t)(rows / 64), (uint32_t)((m + 63) / 64),
                         1, gemm2_threads(64), shmem, (float*)mix, c->gpart, L.p[1], L.p[2], (int)rows,
                         (int)cols, (int)m, (float*)q, (float*)k, (float*)v, (float*)g, (int)d));
        out.back().abytes = 4.0 * (double)(rows * cols + m * cols + m * rows + 4 * m * d);
        last_m = m;
        return 7;
    }

    void mark(size_t i) {
        if (!marks) return;
        size_t low = i;
        auto at = [&](const Op* o) { low = std::min(low, (size_t)(o - ops.data())); };
        for (auto& v : pend)
            if (v.op) at(v.op);
        if (l2q) at(l2q);
        if (l2k) at(l2k);
        if (rrows) {
            low = std::min(low, rstart);
            for (const Op* o : rsrc)
                if (o) at(o);
        }
        marks->push_back({out.size(), i, low});
    }

    int run(bool fuse) {
        size_t i = 0;
        while (i < ops.size()) {
            mark(i);
            const Op& o = ops[i];
            VpSrc v;
            // one-token attention: its partials wait for the next fused prologue to combine
            if (fuse && o.kind == OP_ATTEND && attn_dec_ok(o) && !l2q && pend.size() < SLM_VP_MAX &&
                o.n[5] * o.n[7] <= VP_LEN_MAX && (o.n[5] * o.n[7]) % 4 == 0 &&
                attn_dec_part_floats(o) <= COMB_PART_MAX && aligned16(c->ws) &&
                (int64_t)c->ws_bytes >= 4 * ((attn_dec_part_floats(o) + 3) & ~(int64_t)3)) {
                TRY(row_flush());
                TRY(flush_pending());
                TRY(lower_attn_dec(c, o, out, true));
                v.kind = SRC_COMB;
                v.n = (int)(o.n[5] * o.n[7]);
                v.nsplit = (int)o.n[8];
                v.heads = (int)o.n[5];
                v.dh = (int)o.n[7];
                v.dp = (int)attn_dp(o.n[7]);
                v.in[0] = c->ws;
                v.out[0] = o.p[0];
                v.op = &o;
                pend.push_back(v);
                i++;
                continue;
            }
            if (fuse && pend.size() < SLM_VP_MAX && vp_of(o, &v)) {
                TRY(row_flush());
                // a held l2norm's output may not be touched before the GLA kernel
                bool clash = false;
                for (const Op* h : {l2q, l2k})
                    if (h)
                        for (int q = 0; q < 2; q++) {
                            if (v.in[q]) clash |= overlap(rng(v.in[q], v.n), rng(h->p[0], h->n[0] * h->n[1]));
                            if (v.out[q]) clash |= overlap(rng(v.out[q], v.n), rng(h->p[0], h->n[0] * h->n[1])) ||
                                                   overlap(rng(v.out[q], v.n), rng(h->p[1], h->n[0] * h->n[1]));
                        }
                if (clash) TRY(flush_l2());
                pend.push_back(v);
                i++;
                continue;
            }
            if (o.kind == OP_LINEAR && o.n[2] == 1) last_m = 0;
            if (fuse && o.kind == OP_LINEAR && o.n[2] == 1 && !l2q) {
                next_pend.clear();
                size_t used = try_fg(i);
                if (used) {
                    // the prologue took every pending op; a split linear leaves its fold
                    pend.swap(next_pend);
                    next_pend.clear();
                    i += used;
                    continue;
                }
            }
            // prompt rows: element-wise ops join a row chain; a split GEMM's fold starts one
            if (fuse && pend.empty() && !l2q && o.kind != OP_LINEAR && row_try(o)) {
                rnext = ++i;
                continue;
            }
            TRY(row_flush());
            TRY(flush_pending());
            if (fuse && o.kind == OP_LINEAR && o.n[2] > 1 && !l2q) {
                if (size_t used = try_gemm_silu(i)) {
                    i += used;
                    continue;
                }
                if (size_t used = try_gemm_rope(i)) {
                    i += used;
                    continue;
                }
                if (size_t used = try_gemm_l2(i)) {
                    i += used;
                    continue;
                }
                int64_t ns = 1, rows = o.n[0], m = o.n[2];
                TRY(lower_linear(c, o, out, &ns));
                last_m = m;
                if (ns > 1) {
                    rfold = mk(c->k.fold, blocks_for(m * rows), 1, 1, 256, 0, o.p[0],
                               (const float*)c->gpart, (long long)(m * rows), (int)ns);
                    RowOp ro;
                    std::memset(&ro, 0, sizeof ro);
                    ro.kind = R_FOLD;
                    ro.la = ro.lb = ro.lc = ro.ld = ro.out = ro.tmp = -1;
                    ro.n = (int32_t)rows;
                    ro.a = {c->gpart, rows};
                    ro.i0 = (int32_t)ns;
                    ro.q0 = m * rows;
                    ro.y = (float*)o.p[0];
                    ro.ystride = rows;
                    rrows = m;
                    rstart = i;
                    rnext = i + 1;
                    if (rows > 16384 || !row_add(nullptr, ro, rows_rng(o.p[0], rows, rows, m))) {
                        row_reset();
                        out.push_back(rfold);
                    }
                }
                i++;
                continue;
            }
            if (fuse && o.kind == OP_GLA) {
                size_t used = try_gla(i);
                if (used) {
                    i += used;
                    continue;
                }
            }
            TRY(flush_l2());
            TRY(lower_one(c, o, out));
            i++;
        }
        TRY(row_flush());
        TRY(flush_pending());
        TRY(flush_l2());
        if (marks) marks->push_back({out.size(), ops.size(), ops.size()});
        return SLM_OK;
    }
};

int plan(slm_hip* c, const std::vector<Op>& ops, std::vector<Rec>& out, bool fuse,
         std::vector<PlanMark>* marks = nullptr) {
    Planner p{c, ops, out, marks, {}};
    size_t before = out.size();
    TRY(p.run(fuse));
    if (c->plan_trace) {
        fprintf(stderr, "slm plan: %zu ops ->", ops.size());
        for (size_t k = before; k < out.size(); k++) {
            const char* nm = "?";
            const Kernels& K = c->k;
            if (out[k].f == K.fg || out[k].f == K.fgh) {
                const FgDesc* d = (const FgDesc*)out[k].blob;
                fprintf(stderr, " fg[%dx%d vp", d->seg[0].rows, d->cols);
                for (int q = 0; q < d->nvp; q++)
                    fprintf(stderr, "%s%d:%d%s", q ? "," : "", d->vp[q].kind, d->vp[q].n, d->vp[q].gout ? "w" : "");
                fprintf(stderr, " pf%d]", d->npf);
                continue;
            }
            if (out[k].f == K.rows) {
                const RowDesc* d = (const RowDesc*)out[k].blob;
                fprintf(stderr, " rows[");
                for (int q = 0; q < d->nops; q++)
                    fprintf(stderr, "%s%d:%d%s", q ? "," : "", d->op[q].kind, d->op[q].n, d->op[q].y ? "w" : "");
                fprintf(stderr, " pf%d]", d->npf);
                continue;
            }
            auto it = c->fname.find(out[k].f);
            if (it != c->fname.end()) nm = it->second.c_str() + (it->second.rfind("slm_", 0) == 0 ? 4 : 0);
            fprintf(stderr, " %s", nm);
        }
        fprintf(stderr, "\n");
    }
    c->last_ops = ops.size();
    c->last_kernels = out.size() - before;
    return SLM_OK;
}

// ---------------------------------------------------------------------------------------
// dynamic values, recording, graphs
// ---------------------------------------------------------------------------------------

// The step's dynamic values into `dev` on stream s, through one of two pinned buffers (the
// other may still be in flight).
int upload_dyn_on(slm_hip* c, unsigned char* dev, unsigned char* const* pin, const hipEvent_t* ev,
                  int* flip, hipStream_t s) {
    if (c->dyn.empty()) return SLM_OK;
    int k = *flip ^= 1;
    HIPC(c, hipEventSynchronize(ev[k]));
    std::memcpy(pin[k], c->dyn.data(), c->dyn.size());
    HIPC(c, hipMemcpyAsync(dev, pin[k], c->dyn.size(), hipMemcpyHostToDevice, s));
    HIPC(c, hipEventRecord(ev[k], s));
    return SLM_OK;
}

int upload_dyn(slm_hip* c) {
    if (c->dyn.empty()) return SLM_OK;
    return upload_dyn_on(c, c->dyn_dev, c->dyn_pin, c->dyn_ev, &c->dyn_flip, mstream(c));
}

int launch_all(slm_hip* c, const std::vector<Rec>& recs) {
    for (auto& r : recs) TRY(launch_now(c, r));
    return SLM_OK;
}

// Leaves recording for the rest of this step: what was recorded runs now.
int taint(slm_hip* c) {
    if (!c->recording || c->tainted) return SLM_OK;
    c->tainted = true;
    c->n_eager++;
    TRY(upload_dyn(c));
    std::vector<Rec> recs;
    TRY(plan(c, c->ops, recs, c->fusion_on));
    c->ops.clear();
    return launch_all(c, recs);
}

bool recording(const slm_hip* c) { return c->recording && !c->tainted; }

// A fused kernel's bounded wait that gave up leaves a bit in the fault word: the step it
// belonged to did not compute what it should have. Reported (once) as SLM_E_HIP.
int check_fault(slm_hip* c) {
    int v = __atomic_load_n(c->fault_host, __ATOMIC_ACQUIRE);
    if (!v) return SLM_OK;
    __atomic_store_n(c->fault_host, 0, __ATOMIC_RELEASE);
    reset_counters(c);
    return fail(c, SLM_E_HIP, "a fused kernel's bounded wait gave up (fault word %#x): the results "
                "of the work since the last check are not valid", v);
}

void drop_shadows(slm_hip* c, uintptr_t a, uintptr_t b);

// Queues an op: recorded inside a step, lowered and launched otherwise. What it writes
// loses its fp16 shadow.
int submit(slm_hip* c, const Op& o) {
    if (!c->shadows.empty()) {
        std::vector<Range> rd, wr;
        op_ranges(o, rd, wr);
        for (const Range& r : wr) drop_shadows(c, r.a, r.b);
    }
    if (recording(c)) {
        c->ops.push_back(o);
        return SLM_OK;
    }
    std::vector<Rec> recs;
    TRY(lower_one(c, o, recs));
    return launch_all(c, recs);
}

Op op(uint32_t kind) {
    Op o;
    std::memset(&o, 0, sizeof o);
    o.kind = kind;
    return o;
}

// Dynamic values (positions, token ids, factors): returns a device pointer to a copy of
// `bytes` bytes of `src`, valid for kernels queued after it on the stream.
int stage(slm_hip* c, const void* src, size_t bytes, const void** out) {
    size_t need = (bytes + 7) & ~(size_t)7;
    if (recording(c)) {
        size_t off = c->dyn.size();
        if (off + need <= DYN_CAP) {
            c->dyn.resize(off + need);
            std::memcpy(c->dyn.data() + off, src, bytes);
            *out = c->dyn_dev + off;
            return SLM_OK;
        }
        TRY(taint(c));
    }
    if (need > STAGE_CAP) return fail(c, SLM_E_UNSUPPORTED, "stage: %zu bytes at once", bytes);
    if (c->stage_head + need > STAGE_CAP) {
        HIPC(c, hipStreamSynchronize(mstream(c)));
        c->stage_head = 0;
    }
    std::memcpy(c->stage_host + c->stage_head, src, bytes);
    HIPC(c, hipMemcpyAsync(c->stage_dev + c->stage_head, c->stage_host + c->stage_head, need,
                           hipMemcpyHostToDevice, mstream(c)));
    *out = c->stage_dev + c->stage_head;
    c->stage_head += need;
    return SLM_OK;
}

// A position: staged inside a step (so the op is the same every token), immediate outside.
int stage_pos(slm_hip* c, size_t pos, Op& o, int slot) {
    long long p = (long long)pos;
    if (recording(c)) {
        TRY(stage(c, &p, 8, &o.dyn));
        o.n[slot] = 0;
    } else {
        o.dyn = nullptr;
        o.n[slot] = p;
    }
    return SLM_OK;
}

constexpr size_t POOL_SLAB = (size_t)128 << 20, POOL_BLOCK_MAX = (size_t)32 << 20;

// Gives the slabs none of whose blocks is in use back to the device (their blocks leave the
// free lists; the slab being carved stays). Free blocks are kept by their exact size, so
// alloc/free cycles over changing sizes leave free slabs behind: they go back when an
// allocation would otherwise fail. Returns the bytes released.
size_t reclaim_slabs(slm_hip* c) {
    size_t freed = 0;
    for (size_t i = 0; i + 1 < c->slabs.size();) {
        uintptr_t a = (uintptr_t)c->slabs[i], b = a + POOL_SLAB;
        auto lo = c->pooled.lower_bound(a);
        if (lo != c->pooled.end() && lo->first < b) {
            i++;
            continue;
        }
        for (auto& f : c->pool_free) {
            auto& v = f.second;
            v.erase(std::remove_if(v.begin(), v.end(),
                                   [&](void* p) { return (uintptr_t)p >= a && (uintptr_t)p < b; }),
                    v.end());
        }
        hipFree(c->slabs[i]);
        c->slabs.erase(c->slabs.begin() + (long)i);
        freed += POOL_SLAB;
    }
    return freed;
}

hipError_t dev_alloc(slm_hip* c, size_t bytes, void** out) {
    size_t rb = (bytes + 255) & ~(size_t)255;
    if (rb > POOL_BLOCK_MAX) {
        hipError_t e = hipMalloc(out, bytes);
        if (e != hipSuccess && reclaim_slabs(c)) e = hipMalloc(out, bytes);
        return e;
    }
    auto f = c->pool_free.find(rb);
    if (f != c->pool_free.end() && !f->second.empty()) {
        *out = f->second.back();
        f->second.pop_back();
    } else {
        if (c->slab_left < rb) {  // (the last slab's tail stays unused)
            void* sl = nullptr;
            hipError_t e = hipMalloc(&sl, POOL_SLAB);
            if (e != hipSuccess && reclaim_slabs(c)) e = hipMalloc(&sl, POOL_SLAB);
            if (e != hipSuccess) return hipMalloc(out, bytes);
            c->slabs.push_back(sl);
            c->slab_cur = (char*)sl;
            c->slab_left = POOL_SLAB;
        }
        *out = c->slab_cur;
        c->slab_cur += rb;
        c->slab_left -= rb;
    }
    c->pooled[(uintptr_t)*out] = rb;
    return hipSuccess;
}

// Gives back a dev_alloc block (no work may still use it).
void dev_free(slm_hip* c, void* p) {
    auto it = c->pooled.find((uintptr_t)p);
    if (it == c->pooled.end()) {
        hipFree(p);
        return;
    }
    c->pool_free[it->second].push_back(p);
    c->pooled.erase(it);
}

// An internal buffer grows into a new allocation; the old one is kept until close, since
// launched work and cached graphs may still use it (each for sizes it was big enough for),
// so growing waits for nothing. A step being recorded keeps recording: its ops name these
// buffers only when the step is planned, after every growth it asks for; an op lowered at
// once lowers with its own partials' consumer (they share the buffer it saw).
int internal_realloc(slm_hip* c, void** p, size_t bytes) {
    void* np = nullptr;
    HIPC(c, dev_alloc(c, bytes, &np));
    if (*p) c->retired.push_back(*p);
    *p = np;
    return SLM_OK;
}

// Drops the fp16 shadows of fp32 ranges that overlap [a, b). Inside a step being recorded
// the ops recorded so far may read a shadow, so it is freed after the step has run;
// otherwise once the work queued so far is done.
void drop_shadows(slm_hip* c, uintptr_t a, uintptr_t b) {
    bool synced = false;
    for (auto it = c->shadows.begin(); it != c->shadows.end();) {
        uintptr_t k0 = it->first, k1 = k0 + it->second.n * 4;
        if (!(k0 < b && a < k1)) {
            ++it;
            continue;
        }
        if (c->recording) {
            c->free_after_step.push_back(it->second.h);
        } else {
            if (!synced) hipStreamSynchronize(mstream(c));
            synced = true;
            dev_free(c, it->second.h);
        }
        it = c->shadows.erase(it);
    }
}

// fp16 mode: the fp16 shadow of the n fp32 weights at w, made on first use by a conversion
// queued now (ahead of the step being recorded, whose ops run later on the same stream), or
// null when the weights are written inside the step being recorded before this linear reads
// them, or when the copy cannot be allocated (the linear then reads the fp32 weights and
// rounds them itself: the same bits).
int shadow_of(slm_hip* c, const float* w, size_t n, const float** out) {
    *out = nullptr;
    auto it = c->shadows.find((uintptr_t)w);
    if (it != c->shadows.end() && it->second.n >= n) {
        *out = (const float*)it->second.h;
        return SLM_OK;
    }
    if (recording(c)) {
        std::vector<Range> rd, wr;
        Range r = rng(w, (int64_t)n);
        for (const Op& o : c->ops) {
            rd.clear();
            wr.clear();
            op_ranges(o, rd, wr);
            for (const Range& x : wr)
                if (overlap(x, r)) return SLM_OK;
        }
    }
    if (it != c->shadows.end()) drop_shadows(c, (uintptr_t)w, (uintptr_t)w + 1);  // too short
    void* h = nullptr;
    if (dev_alloc(c, n * 2, &h) != hipSuccess) {  // no room for a copy: the fp32 weights serve
        (void)hipGetLastError();
        return SLM_OK;
    }
    int rc = launch_now(c, mk(c->k.to_half, blocks_for(n), 1, 1, 256, 0, h, w, (long long)n));
    if (rc) {
        hipStreamSynchronize(mstream(c));
        dev_free(c, h);
        return rc;
    }
    c->shadows[(uintptr_t)w] = slm_hip::Shadow{h, n};
    *out = (const float*)h;
    return SLM_OK;
}

int need_part(slm_hip* c, size_t bytes) {
    bytes += 64;  // fused prologues read whole float4s past an odd-sized end
    if (bytes <= c->part_bytes) return SLM_OK;
    size_t nb = std::max(bytes, c->part_bytes * 2);
    TRY(internal_realloc(c, (void**)&c->part, nb));
    c->part_bytes = nb;
    return SLM_OK;
}

int need_gpart(slm_hip* c, size_t bytes) {
    if (bytes <= c->gpart_bytes) return SLM_OK;
    size_t nb = std::max(bytes, c->gpart_bytes * 2);
    TRY(internal_realloc(c, (void**)&c->gpart, nb));
    c->gpart_bytes = nb;
    return SLM_OK;
}

int need_ws(slm_hip* c, size_t bytes) {
    bytes += 64;  // fused prologues read whole float4s past an odd-sized end
    if (bytes <= c->ws_bytes) return SLM_OK;
    size_t nb = std::max(bytes, c->ws_bytes * 2);
    TRY(internal_realloc(c, (void**)&c->ws, nb));
    c->ws_bytes = nb;
    return SLM_OK;
}

// ---- prompt lanes: running a step on one ----

// The live allocation holding address a: its start and size (false: none does).
bool alloc_at(const slm_hip* c, uintptr_t a, uintptr_t* base, size_t* bytes) {
    auto it = c->allocs.upper_bound(a);
    if (it == c->allocs.begin()) return false;
    --it;
    if (a >= it->first + it->second) return false;
    *base = it->first;
    *bytes = it->second;
    return true;
}

// A lane's own internal buffer of at least `bytes` (the one it replaces may still be read by
// the lane's queued work: retired, freed at close).
bool lane_buf(slm_hip* c, float** p, size_t* have, size_t bytes) {
    if (bytes <= *have) return true;
    void* np = nullptr;
    if (dev_alloc(c, bytes, &np) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    if (*p) c->retired.push_back(*p);
    *p = (float*)np;
    *have = bytes;
    return true;
}

// Orders the lanes after everything queued on the context's stream so far and enters them.
int enter_lanes(slm_hip* c) {
    if (c->lanes_active) return SLM_OK;
    hipEvent_t e = lane_event(c);
    if (!e) return fail(c, SLM_E_HIP, "lanes: hipEventCreate failed");
    hipError_t err = hipEventRecord(e, c->stream);
    for (int l = 1; l < c->nlanes && err == hipSuccess; l++)
        err = hipStreamWaitEvent(c->lanes[l].stream, e, 0);
    c->lane_ev_pool.push_back(e);
    if (err != hipSuccess) {
        for (int l = 1; l < c->nlanes; l++) hipStreamSynchronize(c->lanes[l].stream);
        return fail(c, SLM_E_HIP, "lanes: %s", hipGetErrorString(err));
    }
    c->lanes_active = true;
    c->next_lane = 0;
    return SLM_OK;
}

int lane_fallback(slm_hip* c) {
    c->n_lane_fallbacks++;
    return SLM_OK;
}

// Runs the recorded prompt step on the next lane (*handled set), or leaves it to the caller
// with nothing queued (*handled clear) when a lane cannot take it: the step reads scratch
// before writing it, frees or grows a buffer, holds a one-token attention or pick (the
// context's own counters), or touches in place what another lane of this session wrote or
// read without an event. On a lane other than 0 the step's scratch allocations are renamed
// to the lane's copies (same sizes, same offsets) and its dynamic values, attention and
// split partials go to the lane's buffers. Before the first kernel that may touch a kept
// allocation the lane waits for the event after another lane's last use of it; after the
// last kernel that may touch it the lane records one. The kernels' footprints come from the
// planner's marks: a kernel emitted before the planner took op i holds no op from i on; every
// op before a mark's `low` is inside a kernel emitted before that mark.
int run_lane_step(slm_hip* c, int* handled) {
    *handled = 0;
    if (c->nlanes < 2 || !c->keep_valid || c->timing || c->capturing) return SLM_OK;
    if (!c->free_after_step.empty()) return lane_fallback(c);
    const int lane = c->lanes_active ? c->next_lane : 0;
    const std::vector<Op>& ops = c->ops;
    struct Use {
        size_t first = SIZE_MAX, last = 0, bytes = 0;
        bool written = false, read_first = false;
    };
    std::map<uintptr_t, Use> use;
    const uintptr_t dyn_a = (uintptr_t)c->dyn_dev, dyn_b = dyn_a + DYN_CAP;
    auto note = [&](const Range& r, size_t i, bool w) {
        uintptr_t b;
        size_t n;
        if (r.a >= r.b || !alloc_at(c, r.a, &b, &n)) return;  // internal: tables, fp16 copies
        Use& u = use[b];
        u.bytes = n;
        if (u.first == SIZE_MAX) {
            u.first = i;
            u.read_first = !w;
        }
        u.last = i;
        u.written |= w;
    };
    std::vector<Range> rd, wr;
    for (size_t i = 0; i < ops.size(); i++) {
        const Op& o = ops[i];
        if (o.kind == OP_ARGMAX || o.kind == OP_GROW || (o.kind == OP_ATTEND && o.n[1] == 1))
            return lane_fallback(c);
        if (o.dyn && ((uintptr_t)o.dyn < dyn_a || (uintptr_t)o.dyn >= dyn_b)) return lane_fallback(c);
        rd.clear();
        wr.clear();
        op_ranges(o, rd, wr);
        for (const Range& r : rd) note(r, i, false);
        for (const Range& r : wr) note(r, i, true);
    }
    std::set<uintptr_t> kept(c->keep.begin(), c->keep.end());
    std::vector<uintptr_t> scratch, deps, ronly;
    for (auto& [b, u] : use) {
        bool k = kept.count(b) != 0;
        if (k)
            deps.push_back(b);
        else if (!u.written)
            ronly.push_back(b);
        else if (u.read_first || c->halves.count(b))
            return lane_fallback(c);
        else
            scratch.push_back(b);
        // written in place (kept, or scratch on lane 0) while another lane may read it
        if ((k || lane == 0) && u.written && c->ln_read.count(b)) return lane_fallback(c);
        // in place on a lane other than 0 while lane 0's scratch write may be in flight
        if (lane != 0 && (k || !u.written) && c->l0_written.count(b)) return lane_fallback(c);
    }

    slm_hip::Lane* L = lane ? &c->lanes[lane] : nullptr;
    std::vector<Op> tops;
    if (L) {
        std::map<uintptr_t, uintptr_t> to;  // allocation -> the lane's copy
        for (uintptr_t b : scratch) {
            auto& cp = L->copies[b];
            size_t n = use[b].bytes;
            if (!cp.first || cp.second != n) {
                void* np = nullptr;
                if (dev_alloc(c, n, &np) != hipSuccess) {
                    (void)hipGetLastError();
                    return lane_fallback(c);
                }
                if (cp.first) c->retired.push_back(cp.first);
                cp = {np, n};
            }
            to[b] = (uintptr_t)cp.first;
        }
        if (!lane_buf(c, &L->ws, &L->ws_bytes, c->ws_bytes) ||
            !lane_buf(c, &L->gpart, &L->gpart_bytes, c->gpart_bytes) ||
            !lane_buf(c, &L->part, &L->part_bytes, c->part_bytes))
            return lane_fallback(c);
        tops = ops;
        for (Op& o : tops) {
            for (int q = 0; q < 8; q++) {
                uintptr_t a = (uintptr_t)o.p[q], b;
                size_t n;
                if (!a || !alloc_at(c, a, &b, &n)) continue;
                auto it = to.find(b);
                if (it != to.end()) o.p[q] = (const float*)(it->second + (a - b));
            }
            if (o.dyn) o.dyn = L->dyn_dev + ((uintptr_t)o.dyn - dyn_a);
        }
    }

    std::vector<Rec> recs;
    std::vector<PlanMark> marks;
    int rc;
    if (L) {  // plan with the lane's partial buffers in the context's place
        std::swap(c->ws, L->ws);
        std::swap(c->ws_bytes, L->ws_bytes);
        std::swap(c->gpart, L->gpart);
        std::swap(c->gpart_bytes, L->gpart_bytes);
        std::swap(c->part, L->part);
        std::swap(c->part_bytes, L->part_bytes);
        rc = plan(c, tops, recs, c->fusion_on, &marks);
        std::swap(c->ws, L->ws);
        std::swap(c->ws_bytes, L->ws_bytes);
        std::swap(c->gpart, L->gpart);
        std::swap(c->gpart_bytes, L->gpart_bytes);
        std::swap(c->part, L->part);
        std::swap(c->part_bytes, L->part_bytes);
    } else {
        rc = plan(c, ops, recs, c->fusion_on, &marks);
    }
    TRY(rc);
    if (marks.empty()) return lane_fallback(c);

    // where each kept allocation's waits and events go
    std::vector<std::vector<uintptr_t>> wait_at(recs.size() + 1), rec_at(recs.size() + 1);
    for (uintptr_t b : deps) {
        const Use& u = use[b];
        size_t t = 0;
        while (t + 1 < marks.size() && marks[t + 1].next <= u.first) t++;
        size_t w = marks[t].out;
        t = 0;
        while (t + 1 < marks.size() && marks[t].low <= u.last) t++;
        size_t r = marks[t].out;
        if (w >= r) continue;  // no kernel of this step touches it
        wait_at[w].push_back(b);
        rec_at[r].push_back(b);
    }

    TRY(enter_lanes(c));
    *handled = 1;
    hipStream_t S = L ? L->stream : c->stream;
    if (L)
        TRY(upload_dyn_on(c, L->dyn_dev, L->dyn_pin, L->dyn_ev, &L->dyn_flip, S));
    else
        TRY(upload_dyn_on(c, c->dyn_dev, c->dyn_pin, c->dyn_ev, &c->dyn_flip, S));
    if (L) L->used = true;
    c->lane_launching = true;
    c->lane_stream = S;
    std::set<hipEvent_t> waited;
    for (size_t k = 0; k <= recs.size() && !rc; k++) {
        if (!rec_at[k].empty()) {
            hipEvent_t e = lane_event(c);
            hipError_t err = e ? hipEventRecord(e, S) : hipErrorOutOfMemory;
            if (err != hipSuccess) {
                if (e) c->lane_ev_pool.push_back(e);
                rc = fail(c, SLM_E_HIP, "lanes: event: %s", hipGetErrorString(err));
                break;
            }
            for (uintptr_t b : rec_at[k]) {
                auto it = c->touch.find(b);
                if (it != c->touch.end()) ev_unref(c, it->second.ev);
                c->touch[b] = {lane, e};
                c->ev_refs[e]++;
            }
        }
        if (k == recs.size()) break;
        for (uintptr_t b : wait_at[k]) {
            auto it = c->touch.find(b);
            if (it == c->touch.end() || it->second.lane == lane) continue;
            if (!waited.insert(it->second.ev).second) continue;
            hipError_t err = hipStreamWaitEvent(S, it->second.ev, 0);
            if (err != hipSuccess) {
                rc = fail(c, SLM_E_HIP, "lanes: wait: %s", hipGetErrorString(err));
                break;
            }
        }
        if (!rc) rc = launch_now(c, recs[k]);
    }
    c->lane_launching = false;
    if (rc) {  // what was queued is joined; the kept buffers' contents are the caller's problem
        leave_lanes(c);
        return rc;
    }
    for (uintptr_t b : scratch)
        if (lane == 0) c->l0_written.insert(b);
    for (uintptr_t b : ronly)
        if (lane != 0) c->ln_read.insert(b);
    c->next_lane = (lane + 1) % c->nlanes;
    c->n_lane_steps++;
    c->last_ops = ops.size();
    return SLM_OK;
}

int finish_step_run(slm_hip* c);

// Frees deferred buffers whose step has run (all of them, after a wait, with `wait`).
void free_deferred(slm_hip* c, bool wait) {
    for (size_t i = 0; i < c->deferred.size();) {
        auto& d = c->deferred[i];
        bool done = wait ? hipEventSynchronize(d.done) == hipSuccess : hipEventQuery(d.done) == hipSuccess;
        if (!done && !wait) {
            i++;
            continue;
        }
        for (void* p : d.bufs) {
            c->halves.erase((uintptr_t)p);
            dev_free(c, p);
        }
        hipEventDestroy(d.done);
        c->deferred.erase(c->deferred.begin() + (long)i);
    }
}

// Runs the recorded step. What was freed while it was recorded is freed once the step's
// kernels have run (an event after them; the host does not wait). A cached graph that names
// such a buffer is kept: it runs again only for an identical op list, whose ops the bounds
// checks have already found inside live allocations.
int finish_step(slm_hip* c) {
    int rc = finish_step_run(c);
    if (!c->free_after_step.empty()) {
        {
            slm_hip::Deferred d{nullptr, std::move(c->free_after_step)};
            c->free_after_step.clear();
            hipError_t e = hipEventCreateWithFlags(&d.done, hipEventDisableTiming);
            if (e == hipSuccess) e = hipEventRecord(d.done, mstream(c));
            if (e != hipSuccess) {  // no event: wait here instead
                if (d.done) hipEventDestroy(d.done);
                hipStreamSynchronize(mstream(c));
                for (void* p : d.bufs) {
                    c->halves.erase((uintptr_t)p);
                    dev_free(c, p);
                }
                if (!rc) rc = fail(c, SLM_E_HIP, "free after step: %s", hipGetErrorString(e));
            } else {
                c->deferred.push_back(std::move(d));
            }
        }
    }
    if (!c->deferred.empty()) free_deferred(c, false);
    return rc;
}

// After a step graph's launch: queue the read-ahead copy the graph has learned (the range the
// host read right after its last replay, if still inside a live allocation) and note the
// graph, so that a read of a new range right after it can be learned.
int after_graph(slm_hip* c, Graph& g) {
    if (!g.id) g.id = ++c->next_graph_id;
    bool armed = false;
    if (g.mir_src && c->mir_host && !inside(c, g.mir_src, g.mir_n * 4)) g.mir_src = nullptr;
    if (g.mir_src && c->mir_host) {
        size_t n = g.mir_n;
        uint32_t nwg = (uint32_t)std::min<size_t>((n / 4 + 255) / 256, 64);
        if (nwg == 0) nwg = 1;
        unsigned long long base = c->mir_total, seq = c->mir_seq + 1;
        Rec r = mk(c->k.to_host, nwg, 1, 1, 256, 0, c->mir_dev, g.mir_src, (long long)n, c->mir_ctr,
                   (unsigned long long)(base + nwg - 1),
                   (unsigned long long*)((char*)c->mir_dev + MIRROR_CAP), seq);
        TRY(launch_now(c, r));
        c->mir_total = base + nwg;
        c->mir_seq = seq;
        armed = true;
    }
    c->mir_armed = armed;  // (set after the launches: their mstream calls clear it)
    c->mir_src = g.mir_src;
    c->mir_n = g.mir_n;
    c->last_graph = g.id;
    return SLM_OK;
}

// The host read (dev, n) right after a replay of graph `id`: later replays copy that range
// ahead (a read of anything else makes the graph forget it).
int learn_read(slm_hip* c, uint64_t id, const float* dev, size_t n) {
    for (auto& g : c->cache) {
        if (g.id != id) continue;
        bool ok = n > 0 && n * 4 <= MIRROR_CAP && aligned16(dev);
        g.mir_src = ok ? dev : nullptr;
        g.mir_n = ok ? n : 0;
        if (ok && !c->mir_host) {
            void* h = nullptr;
            HIPC(c, hipHostMalloc(&h, MIRROR_CAP + 64, hipHostMallocMapped));
            std::memset(h, 0, MIRROR_CAP + 64);
            c->mir_host = (float*)h;
            HIPC(c, hipHostGetDevicePointer((void**)&c->mir_dev, h, 0));
            HIPC(c, hipMalloc((void**)&c->mir_ctr, 64));
            HIPC(c, hipMemset(c->mir_ctr, 0, 64));
            c->mir_total = 0;
            c->mir_seq = 0;
        }
        break;
    }
    return SLM_OK;
}

// The program of a one-launch step (slm_step_*) for a planned one-token step, into g: a
// phase per launch record, each launch's arguments copied as they are. Leaves g.prog null
// when some launch cannot be a phase: a kernel other than the fp32 fused GEMV, the one-token
// attention that leaves its partials to the next fused GEMV (no counters) and the one-token
// GLA; fp16 rings; head size classes that differ; more workgroups or LDS than a step has.
int build_step(slm_hip* c, const std::vector<Rec>& recs, Graph& g) {
    static_assert(sizeof(AdecArgs) == 15 * 8, "the attention's argument slots");
    static_assert(sizeof(StepPh) == 24, "phase table layout");
    g.prog = nullptr;
    if (!c->step_on || !c->step_ok || recs.empty()) return SLM_OK;
    const Kernels& k = c->k;
    std::vector<StepPh> ph;
    std::vector<std::pair<const unsigned char*, size_t>> args;
    int var = -1;
    uint32_t lds = 0;
    double ab = 0.0;
    auto same_var = [&](int v) {
        if (var >= 0 && var != v) return false;
        var = v;
        return true;
    };
    for (const Rec& r : recs) {
        StepPh p{};
        p.gx = (int32_t)r.gx;
        p.grid = (int32_t)(r.gx * r.gy * r.gz);
        if (r.gy != 1 && r.f != k.attn_dec[0] && r.f != k.attn_dec[1] && r.f != k.attn_dec[2]) return SLM_OK;
        if (p.grid < 1 || p.grid > SLM_STEP_WG || r.bx > SLM_STEP_THREADS || r.gz != 1) return SLM_OK;
        if (r.f == k.fg) {
            FgDesc d;
            if (r.bytes != sizeof d) return SLM_OK;
            std::memcpy(&d, r.blob, sizeof d);
            if (d.f16) return SLM_OK;
            for (int q = 0; q < d.nseg; q++)
                if (d.seg[q].ring16) return SLM_OK;
            if (64 * (d.W + SLM_FG_EPI_WAVES) != (int)r.bx) return SLM_OK;
            p.kind = PH_FG;
        } else if (r.f == k.attn_dec[0] || r.f == k.attn_dec[1] || r.f == k.attn_dec[2]) {
            if (r.bytes || r.nargs != 15 || r.bx != 64 * SLM_SB_SEGS) return SLM_OK;
            AdecArgs a;
            std::memcpy(&a, r.blob, sizeof a);
            if (a.ctr || a.y) return SLM_OK;  // (it combines itself: not a phase)
            if (a.key_heads < 1 || a.heads % a.key_heads || a.heads / a.key_heads > SLM_STEP_GROUP) return SLM_OK;
            p.kind = PH_ADEC;
            if (!same_var(r.f == k.attn_dec[0] ? 0 : r.f == k.attn_dec[1] ? 1 : 2)) return SLM_OK;
        } else if (r.f == k.gla1[0] || r.f == k.gla1[1] || r.f == k.gla1[2]) {
            if (r.bytes != sizeof(GlaDesc)) return SLM_OK;
            p.kind = PH_GLA1;
            if (!same_var(r.f == k.gla1[0] ? 0 : r.f == k.gla1[1] ? 1 : 2)) return SLM_OK;
        } else {
            return SLM_OK;
        }
        lds = std::max(lds, r.shmem);
        ab += r.abytes;
        ph.push_back(p);
        args.push_back({r.blob, r.bytes ? (size_t)r.bytes : (size_t)8 * r.nargs});
    }
    if (var < 0) var = 0;  // (GEMVs only: any of the kernels)
    if ((int)lds + c->step_static_lds > LDS_MAX) return SLM_OK;
    int nb = 0;
    if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k.step[var], SLM_STEP_THREADS, lds) != hipSuccess ||
        nb < 1)
        return SLM_OK;
    // [phase table][argument blocks, 16-byte aligned]
    size_t at = (ph.size() * sizeof(StepPh) + 15) & ~(size_t)15;
    for (size_t i = 0; i < ph.size(); i++) {
        ph[i].arg = (int32_t)at;
        at = (at + args[i].second + 15) & ~(size_t)15;
    }
    if (at > (size_t)INT_MAX) return SLM_OK;
    // (a fused GEMV reads its segment table as 128 dwords, past the descriptor's end: zeros
    // after the last block keep those reads inside the buffer)
    at += 512;
    std::vector<unsigned char> host(at, 0);
    std::memcpy(host.data(), ph.data(), ph.size() * sizeof(StepPh));
    for (size_t i = 0; i < ph.size(); i++) std::memcpy(host.data() + ph[i].arg, args[i].first, args[i].second);
    void* dev = nullptr;
    hipError_t e = dev_alloc(c, at, &dev);
    if (e != hipSuccess) return fail(c, SLM_E_MEMORY, "step program of %zu bytes: %s", at, hipGetErrorString(e));
    e = hipMemcpyAsync(dev, host.data(), at, hipMemcpyHostToDevice, mstream(c));
    if (e == hipSuccess) e = hipStreamSynchronize(mstream(c));
    if (e != hipSuccess) {
        dev_free(c, dev);
        return fail(c, SLM_E_HIP, "step program upload: %s", hipGetErrorString(e));
    }
    g.prog = (char*)dev;
    g.nph = (int)ph.size();
    g.step_var = var;
    g.step_shmem = lds;
    g.step_abytes = ab;
    c->n_step_plans++;
    return SLM_OK;
}

int launch_step(slm_hip* c, const Graph& g) {
    StepArgs a{};
    a.prog = g.prog;
    a.flags = c->step_flags;
    a.fault = c->fault_dev;
    a.epoch = c->step_epoch;
    a.nph = g.nph;
    // (a poll of the flags takes a memory round trip: a sixteenth of the LDS polls' limit
    // gives up after about as long)
    a.spin = c->spin > 0 ? std::max(1, c->spin >> 4) : 0;
    Rec r = mk_desc(c->k.step[g.step_var], SLM_STEP_WG, SLM_STEP_THREADS, g.step_shmem, a);
    r.abytes = g.step_abytes;
    TRY(launch_now(c, r));
    c->step_epoch += (unsigned)g.nph;
    c->n_step++;
    return SLM_OK;
}

// Captures the recorded step into a graph, or finds one that matches it; with graphs
// off, plans the step and launches it directly.
int finish_step_run(slm_hip* c) {
    c->recording = false;
    if (c->tainted) {
        c->tainted = false;
        return SLM_OK;
    }
    // Multi-token steps (prompt chunks) run planned but uncaptured: their kernels are long
    // enough that replaying a graph saves nothing measurable, while capturing one (for each
    // new buffer arrangement a chunk brings) costs about a millisecond.
    bool multi = false;
    for (const Op& o : c->ops)
        if (o.kind == OP_LINEAR && o.n[2] > 1) { multi = true; break; }
    if (multi) {
        int handled = 0;
        TRY(run_lane_step(c, &handled));
        if (handled) return SLM_OK;
    }
    TRY(upload_dyn(c));
    // with graphs on, a one-token step runs as one launch where its kernels allow, else as a graph
    bool step = !multi && c->graphs_on && c->step_on && c->step_ok;
    if (!c->graphs_on || multi) {
        std::vector<Rec> recs;
        TRY(plan(c, c->ops, recs, c->fusion_on));
        return launch_all(c, recs);
    }
    c->clock++;
    for (auto& g : c->cache) {
        if (g.ops.size() == c->ops.size() && g.ndyn == c->dyn.size() &&
            std::memcmp(g.ops.data(), c->ops.data(), c->ops.size() * sizeof(Op)) == 0) {
            g.used = c->clock;
            if (g.prog) TRY(launch_step(c, g));
            else HIPC(c, hipGraphLaunch(g.exec, mstream(c)));
            c->n_launched++;
            return after_graph(c, g);
        }
    }
    if (c->plan_trace) {  // what sets this step apart from a cached one of the same length
        for (auto& g : c->cache) {
            if (g.ops.size() != c->ops.size()) continue;
            for (size_t i = 0; i < g.ops.size(); i++) {
                const Op &a = g.ops[i], &b = c->ops[i];
                if (std::memcmp(&a, &b, sizeof(Op)) == 0) continue;
                int pi = -1, ni = -1;
                for (int q = 0; q < 8 && pi < 0; q++) if (a.p[q] != b.p[q]) pi = q;
                for (int q = 0; q < 10 && ni < 0; q++) if (a.n[q] != b.n[q]) ni = q;
                fprintf(stderr, "slm graph miss: op %zu kind %u differs (p[%d] n[%d]: %lld vs %lld, dyn %s)\n",
                        i, b.kind, pi, ni, ni >= 0 ? (long long)a.n[ni] : 0LL, ni >= 0 ? (long long)b.n[ni] : 0LL,
                        a.dyn != b.dyn ? "differs" : "same");
                break;
            }
            if (g.ndyn != c->dyn.size()) fprintf(stderr, "slm graph miss: dyn bytes %zu vs %zu\n", g.ndyn, c->dyn.size());
        }
    }
    std::vector<Rec> recs;
    TRY(plan(c, c->ops, recs, c->fusion_on));
    if (c->cache.size() >= MAX_GRAPHS) {
        auto old = std::min_element(c->cache.begin(), c->cache.end(),
                                    [](const Graph& a, const Graph& b) { return a.used < b.used; });
        HIPC(c, hipStreamSynchronize(mstream(c)));
        if (old->exec) hipGraphExecDestroy(old->exec);
        if (old->prog) dev_free(c, old->prog);
        c->cache.erase(old);
    }
    Graph g;
    g.ops = c->ops;
    g.ndyn = c->dyn.size();
    g.used = c->clock;
    if (step) {
        TRY(build_step(c, recs, g));
        if (g.prog) {
            c->cache.push_back(std::move(g));
            Graph& n = c->cache.back();
            TRY(launch_step(c, n));
            c->n_launched++;
            return after_graph(c, n);
        }
    }
    hipGraph_t graph = nullptr;
    HIPC(c, hipStreamBeginCapture(mstream(c), hipStreamCaptureModeThreadLocal));
    c->capturing = true;
    for (auto& r : recs) {
        int rc = launch_now(c, r);
        if (rc) {
            c->capturing = false;
            hipStreamEndCapture(mstream(c), &graph);
            if (graph) hipGraphDestroy(graph);
            return rc;
        }
    }
    c->capturing = false;
    HIPC(c, hipStreamEndCapture(mstream(c), &graph));
    hipError_t e = hipGraphInstantiate(&g.exec, graph, nullptr, nullptr, 0);
    hipGraphDestroy(graph);
    if (e != hipSuccess) return fail(c, SLM_E_HIP, "hipGraphInstantiate: %s", hipGetErrorString(e));
    HIPC(c, hipGraphLaunch(g.exec, mstream(c)));
    c->n_captured++;
    c->n_launched++;
    c->cache.push_back(std::move(g));
    return after_graph(c, c->cache.back());
}

int get_fn(slm_hip* c, hipFunction_t* f, const char* name) {
    hipError_t e = hipModuleGetFunction(f, c->mod, name);
    if (e != hipSuccess) return fail(c, SLM_E_HIP, "kernel %s: %s", name, hipGetErrorString(e));
    return SLM_OK;
}

int load_kernels(slm_hip* c) {
    Kernels& k = c->k;
    struct {
        hipFunction_t* f;
        const char* n;
    } fns[] = {{&k.copy, "slm_copy"},           {&k.add, "slm_add"},
               {&k.add_row, "slm_add_row"},     {&k.mix, "slm_mix"},
               {&k.silu_mul, "slm_silu_mul"},   {&k.scale_rows, "slm_scale_rows"},
               {&k.shift, "slm_shift"},         {&k.columns, "slm_columns"},
               {&k.gather, "slm_gather"},       {&k.store, "slm_store"},
               {&k.rope, "slm_rope"},           {&k.rope_table, "slm_rope_table"},
               {&k.rms, "slm_rms"},             {&k.l2norm, "slm_l2norm"},
               {&k.rms_wave, "slm_rms_wave"},   {&k.l2norm_wave, "slm_l2norm_wave"},
               {&k.fill, "slm_fill"},           {&k.combine, "slm_attn_combine"},
               {&k.to_half, "slm_to_half"},     {&k.store16, "slm_store16"},
               {&k.to_host, "slm_to_host"},
               {&k.grow, "slm_grow"},           {&k.grow16, "slm_grow16"},
               {&k.attn_dec16[0], "slm_attn_dec16_1"}, {&k.attn_dec16[1], "slm_attn_dec16_2"},
               {&k.attn_dec16[2], "slm_attn_dec16_4"}, {&k.attn_pq16[0], "slm_attn_pq16_1"},
               {&k.attn_pq16[1], "slm_attn_pq16_2"},   {&k.attn_pq16[2], "slm_attn_pq16_4"},
               {&k.probe, "slm_probe_mfma"},    {&k.fg, "slm_fg"},
               {&k.fold, "slm_fold"},           {&k.gemm, "slm_gemm"},
               {&k.gemm2_32, "slm_gemm2_32"},   {&k.gemm2_64, "slm_gemm2_64"},
               {&k.gemm2k_32, "slm_gemm2k_32"}, {&k.gemm2k_16, "slm_gemm2k_16"},
               {&k.gemm2_48, "slm_gemm2_48"},   {&k.gemm2hk_16, "slm_gemm2hk_16"},
               {&k.gemm2hwk_16, "slm_gemm2hwk_16"}, {&k.gemm2h_48, "slm_gemm2h_48"},
               {&k.gemm2hw_48, "slm_gemm2hw_48"},
               {&k.gemm2_96, "slm_gemm2_96"},   {&k.gemm2_128, "slm_gemm2_128"},
               {&k.gemm2h_32, "slm_gemm2h_32"}, {&k.gemm2h_64, "slm_gemm2h_64"},
               {&k.gemm2h_96, "slm_gemm2h_96"}, {&k.gemm2h_128, "slm_gemm2h_128"},
               {&k.lin_small_h, "slm_linear_small_vh"}, {&k.fgh, "slm_fgh"},
               {&k.lin_small[0], "slm_linear_small_s"}, {&k.lin_small[1], "slm_linear_small_v"},
               {&k.lin_big[0], "slm_linear_big_s"},     {&k.lin_big[1], "slm_linear_big_v"},
               {&k.gla[0], "slm_gla_1"},   {&k.gla[1], "slm_gla_2"},   {&k.gla[2], "slm_gla_4"},
               {&k.gla[3], "slm_gla_8"},   {&k.gla[4], "slm_gla_16"},
               {&k.glah[0], "slm_glah_1"}, {&k.glah[1], "slm_glah_2"}, {&k.glah[2], "slm_glah_4"},
               {&k.glah[3], "slm_glah_8"}, {&k.glah[4], "slm_glah_16"},
               {&k.gla1[0], "slm_gla1_1"}, {&k.gla1[1], "slm_gla1_2"}, {&k.gla1[2], "slm_gla1_4"},
               {&k.attn[0], "slm_attn_part_1"}, {&k.attn[1], "slm_attn_part_2"},
               {&k.attn[2], "slm_attn_part_4"}, {&k.attn[3], "slm_attn_part_8"},
               {&k.attn[4], "slm_attn_part_16"},
               {&k.attn_dec[0], "slm_attn_dec_1"}, {&k.attn_dec[1], "slm_attn_dec_2"},
               {&k.attn_dec[2], "slm_attn_dec_4"}, {&k.rows, "slm_rows"},
               {&k.attn_pq[0], "slm_attn_pq_1"}, {&k.attn_pq[1], "slm_attn_pq_2"},
               {&k.attn_pq[2], "slm_attn_pq_4"},     {&k.argmax, "slm_argmax"},
               {&k.gemm2s[0], "slm_gemm2s_32"},   {&k.gemm2s[1], "slm_gemm2s_64"},
               {&k.gemm2s[2], "slm_gemm2s_96"},   {&k.gemm2s[3], "slm_gemm2s_128"},
               {&k.gemm2hs[0], "slm_gemm2hs_32"}, {&k.gemm2hs[1], "slm_gemm2hs_64"},
               {&k.gemm2hs[2], "slm_gemm2hs_96"}, {&k.gemm2hs[3], "slm_gemm2hs_128"},
               {&k.gemm2r, "slm_gemm2r_64"},      {&k.gemm2hr, "slm_gemm2hr_64"},
               {&k.gemm2n, "slm_gemm2n_64"},      {&k.gemm2hn, "slm_gemm2hn_64"},
               {&k.lin_small_hw, "slm_linear_small_vhw"}, {&k.fghw, "slm_fghw"},
               {&k.gemm2hw[0], "slm_gemm2hw_32"}, {&k.gemm2hw[1], "slm_gemm2hw_64"},
               {&k.gemm2hw[2], "slm_gemm2hw_96"}, {&k.gemm2hw[3], "slm_gemm2hw_128"},
               {&k.gemm2hsw[0], "slm_gemm2hsw_32"}, {&k.gemm2hsw[1], "slm_gemm2hsw_64"},
               {&k.gemm2hsw[2], "slm_gemm2hsw_96"}, {&k.gemm2hsw[3], "slm_gemm2hsw_128"},
               {&k.gemm2hrw, "slm_gemm2hrw_64"},  {&k.gemm2hnw, "slm_gemm2hnw_64"},
               {&k.step[0], "slm_step_1"},        {&k.step[1], "slm_step_2"},
               {&k.step[2], "slm_step_4"}};
    for (auto& f : fns) {
        TRY(get_fn(c, f.f, f.n));
        c->fname[*f.f] = f.n;
    }
    return SLM_OK;
}

}  // namespace

// =======================================================================================
// C ABI
// =======================================================================================

extern "C" {

int slm_hip_open(int device, slm_hip** out) {
    if (!out) return SLM_E_INVALID;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0 || device < 0 || device >= n) {
        g_open_error = "no usable AMD GPU";
        return SLM_NO_DEVICE;
    }
    slm_hip* c = new slm_hip();
    c->device = device;
    auto bail = [&](int rc) {
        g_open_error = c->err;
        slm_hip_close(c);
        return rc;
    };
#define OPEN_HIP(call)                                                                  \
    do {                                                                                \
        hipError_t e_ = (call);                                                         \
        if (e_ != hipSuccess)                                                           \
            return bail(fail(c, SLM_E_HIP, "%s: %s", #call, hipGetErrorString(e_)));   \
    } while (0)
    OPEN_HIP(hipSetDevice(device));
    hipDeviceProp_t prop;
    OPEN_HIP(hipGetDeviceProperties(&prop, device));
    snprintf(c->name, sizeof c->name, "hip (%s, %s)", prop.name[0] ? prop.name : "AMD GPU",
             prop.gcnArchName);
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return bail(fail(c, SLM_E_UNSUPPORTED, "device %d is %s; the library is built for gfx950",
                         device, prop.gcnArchName));
    OPEN_HIP(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
    OPEN_HIP(slm_scratch_address((void**)&c->scratch));  // this device current (hipSetDevice above)
    OPEN_HIP(hipModuleLoadData(&c->mod, slm_code_object));
    int rc = load_kernels(c);
    if (rc) return bail(rc);
    OPEN_HIP(hipHostMalloc((void**)&c->stage_host, STAGE_CAP, hipHostMallocDefault));
    OPEN_HIP(hipMalloc((void**)&c->stage_dev, STAGE_CAP));
    for (int i = 0; i < 2; i++) {
        OPEN_HIP(hipHostMalloc((void**)&c->dyn_pin[i], DYN_CAP, hipHostMallocDefault));
        OPEN_HIP(hipEventCreateWithFlags(&c->dyn_ev[i], hipEventDisableTiming));
    }
    OPEN_HIP(hipMalloc((void**)&c->dyn_dev, DYN_CAP));
    OPEN_HIP(hipHostMalloc((void**)&c->bounce, BOUNCE_CAP, hipHostMallocDefault));
    for (int i = 0; i < 2; i++) OPEN_HIP(hipEventCreateWithFlags(&c->read_ev[i], hipEventDisableTiming));
    OPEN_HIP(hipHostMalloc((void**)&c->fault_host, 64, hipHostMallocMapped));
    *c->fault_host = 0;
    OPEN_HIP(hipHostGetDevicePointer((void**)&c->fault_dev, c->fault_host, 0));
    c->ws_bytes = 1 << 20;
    OPEN_HIP(hipMalloc((void**)&c->ws, c->ws_bytes));
    OPEN_HIP(hipMalloc((void**)&c->attn_ctr, ATTN_CTR_MAX * sizeof(int)));
    OPEN_HIP(hipMemset(c->attn_ctr, 0, ATTN_CTR_MAX * sizeof(int)));
    OPEN_HIP(hipMalloc((void**)&c->pick, 16 * sizeof(float)));
    OPEN_HIP(hipMemset(c->pick, 0, 16 * sizeof(float)));
    {  // fp16 mode's word in the code object, zero: fp32 mode
        size_t bytes = 0;
        OPEN_HIP(hipModuleGetGlobal((hipDeviceptr_t*)&c->h16_dev, &bytes, c->mod, "slm_h16"));
        if (bytes != sizeof(int)) return bail(fail(c, SLM_E_HIP, "slm_h16: %zu bytes", bytes));
        int zero = 0;
        OPEN_HIP(hipMemcpy(c->h16_dev, &zero, sizeof zero, hipMemcpyHostToDevice));
    }
    OPEN_HIP(hipMalloc((void**)&c->step_flags, SLM_STEP_WG * sizeof(unsigned)));
    OPEN_HIP(hipMemset(c->step_flags, 0, SLM_STEP_WG * sizeof(unsigned)));
    {  // a step launch needs all its workgroups resident: one per compute unit
        int lds = 0;
        OPEN_HIP(hipFuncGetAttribute(&lds, HIP_FUNC_ATTRIBUTE_SHARED_SIZE_BYTES, c->k.step[2]));
        c->step_static_lds = lds;
        c->step_ok = prop.multiProcessorCount >= SLM_STEP_WG;
    }

    c->dyn.reserve(DYN_CAP);
    c->ops.reserve(4096);
    c->plan_trace = getenv("SLM_HIP_PLAN_TRACE") != nullptr;
    const char* env = getenv("SLM_HIP_GRAPHS");
    if (env && env[0] == '0') c->graphs_on = false;
    env = getenv("SLM_HIP_FUSION");
    if (env && env[0] == '0') c->fusion_on = false;
    // three prompt lanes by default (a 4096-token a86 prompt at R = 4 measured 155 K tok/s on
    // one, 194 K on two, 216 K on three, 198 K on four)
    env = getenv("SLM_HIP_LANES");
    int lanes = env && env[0] >= '1' && env[0] <= '0' + MAX_LANES && !env[1] ? env[0] - '0' : 3;
    if (slm_hip_set_prompt_lanes(c, lanes) != SLM_OK) return bail(SLM_E_HIP);
#undef OPEN_HIP
    *out = c;
    return SLM_OK;
}

void slm_hip_close(slm_hip* c) {
    if (!c) return;
    if (c->stream) {
        leave_lanes(c);
        hipStreamSynchronize(c->stream);
    }
    for (int l = 1; l < (int)c->lanes.size(); l++)
        if (c->lanes[l].stream) hipStreamSynchronize(c->lanes[l].stream);
    for (auto& g : c->cache)
        if (g.exec) hipGraphExecDestroy(g.exec);
    auto release = [&](void* p) {  // (pooled blocks go with their slabs)
        if (p && !c->pooled.count((uintptr_t)p)) hipFree(p);
    };
    for (auto& g : c->cache) release(g.prog);
    if (c->step_flags) hipFree(c->step_flags);
    for (auto& t : c->tables) {
        release(t.second.cos);
        release(t.second.sin);
    }
    for (auto& a : c->allocs) release((void*)a.first);
    for (auto& sh : c->shadows) release(sh.second.h);
    release(c->ws);
    if (c->attn_ctr) hipFree(c->attn_ctr);
    if (c->pick) hipFree(c->pick);
    release(c->part);
    release(c->gpart);
    for (int l = 1; l < (int)c->lanes.size(); l++) {
        auto& L = c->lanes[l];
        for (auto& cp : L.copies) release(cp.second.first);
        release(L.ws);
        release(L.gpart);
        release(L.part);
        if (L.dyn_dev) hipFree(L.dyn_dev);
        for (int i = 0; i < 2; i++) {
            if (L.dyn_pin[i]) hipHostFree(L.dyn_pin[i]);
            if (L.dyn_ev[i]) hipEventDestroy(L.dyn_ev[i]);
        }
        if (L.stream) hipStreamDestroy(L.stream);
    }
    if (c->mir_host) hipHostFree(c->mir_host);
    if (c->mir_ctr) hipFree(c->mir_ctr);
    for (auto& r : c->ev_refs) hipEventDestroy(r.first);
    for (auto e : c->lane_ev_pool) hipEventDestroy(e);
    for (void* r : c->retired) release(r);
    for (void* r : c->free_after_step) release(r);
    free_deferred(c, true);
    for (void* sl : c->slabs) hipFree(sl);
    collect_timing(c);
    for (auto e : c->ev_pool) hipEventDestroy(e);
    if (c->stage_dev) hipFree(c->stage_dev);
    if (c->dyn_dev) hipFree(c->dyn_dev);
    if (c->stage_host) hipHostFree(c->stage_host);
    if (c->bounce) hipHostFree(c->bounce);
    if (c->fault_host) hipHostFree(c->fault_host);
    for (int i = 0; i < 2; i++) {
        if (c->dyn_pin[i]) hipHostFree(c->dyn_pin[i]);
        if (c->dyn_ev[i]) hipEventDestroy(c->dyn_ev[i]);
        if (c->read_ev[i]) hipEventDestroy(c->read_ev[i]);
    }
    if (c->mod) hipModuleUnload(c->mod);
    if (c->stream) hipStreamDestroy(c->stream);
    delete c;
}

const char* slm_hip_last_error(const slm_hip* c) {
    return c ? c->err.c_str() : g_open_error.c_str();
}

int slm_hip_name(slm_hip* c, char* out, size_t n) {
    if (!c || !out || n == 0) return SLM_E_INVALID;
    snprintf(out, n, "%s", c->name);
    return SLM_OK;
}

int slm_hip_alloc(slm_hip* c, size_t n, float** out) {
    if (!c || !out) return SLM_E_INVALID;
    size_t bytes = std::max<size_t>(n, 1) * 4;
    float* p = nullptr;
    hipError_t e = dev_alloc(c, bytes, (void**)&p);
    if (e != hipSuccess) return fail(c, SLM_E_MEMORY, "alloc %zu floats: %s", n, hipGetErrorString(e));
    // zeroed on the stream now, ordered before any later use of the buffer (also before
    // the launches of a step being recorded, which run at flush)
    int rc = launch_now(c, mk(c->k.fill, blocks_for(bytes / 4), 1, 1, 256, 0, p,
                              (long long)(bytes / 4), 0.0f));
    if (rc) {
        dev_free(c, p);
        return rc;
    }
    c->allocs[(uintptr_t)p] = bytes;
    *out = p;
    return SLM_OK;
}

int slm_hip_alloc_half(slm_hip* c, size_t n, float** out) {
    if (!c || !out) return SLM_E_INVALID;
    size_t nf = (std::max<size_t>(n, 1) + 1) / 2;  // floats of storage (zeroed: +0 halves)
    TRY(slm_hip_alloc(c, nf, out));
    c->halves[(uintptr_t)*out] = std::max<size_t>(n, 1);
    return SLM_OK;
}

int slm_hip_alloc_cache(slm_hip* c, size_t heads, size_t cap, size_t dh, float** out) {
    if (!c || !out) return SLM_E_INVALID;
    if (c->fp16 && half_ring_ok(heads, dh, cap)) return slm_hip_alloc_half(c, heads * cap * dh, out);
    return slm_hip_alloc(c, heads * cap * dh, out);
}

int slm_hip_grow_cache(slm_hip* c, float* dst, const float* src, size_t heads, size_t cap, size_t dh) {
    if (!c) return SLM_E_INVALID;
    if (!heads || !cap || !dh) return SLM_OK;
    size_t hd = half_count(c, dst), hs = half_count(c, src), n = heads * cap * dh;
    if ((hd != 0) != (hs != 0))
        return fail(c, SLM_E_INVALID, "grow_cache: one fp16 cache and one fp32 cache");
    if (hd) {
        if (hd < 2 * n || hs < n)
            return fail(c, SLM_E_BOUNDS, "grow_cache: %zu x %zu x %zu into %zu halves from %zu", heads, cap, dh, hd, hs);
    } else {
        NEED(c, "grow_cache", dst, 2 * n);
        NEED(c, "grow_cache", src, n);
    }
    Op o = op(OP_GROW);
    o.p[0] = dst;
    o.p[1] = src;
    o.n[0] = (int64_t)heads;
    o.n[1] = (int64_t)cap;
    o.n[2] = (int64_t)dh;
    o.n[3] = hd ? 1 : 0;
    return submit(c, o);
}

int slm_hip_free(slm_hip* c, float* p) {
    if (!c) return SLM_E_INVALID;
    if (!p) return SLM_OK;
    auto it = c->allocs.find((uintptr_t)p);
    if (it == c->allocs.end()) return fail(c, SLM_E_BOUNDS, "free: %p was not allocated here", (void*)p);
    drop_shadows(c, (uintptr_t)p, (uintptr_t)p + it->second);
    // the prompt lanes' copies of it go with it
    std::vector<void*> copies;
    for (int l = 1; l < (int)c->lanes.size(); l++) {
        auto cp = c->lanes[l].copies.find((uintptr_t)p);
        if (cp == c->lanes[l].copies.end()) continue;
        if (cp->second.first) copies.push_back(cp->second.first);
        c->lanes[l].copies.erase(cp);
    }
    if (recording(c)) {
        // (an output growing inside a step, cuda.rs:122-127) the step keeps recording: ops
        // recorded before may still name the buffer, so it is freed once the step has run
        c->allocs.erase(it);
        c->halves.erase((uintptr_t)p);  // no later call may take it as fp16 weights
        c->free_after_step.push_back(p);
        for (void* q : copies) c->free_after_step.push_back(q);
        return SLM_OK;
    }
    TRY(taint(c));
    drop_graphs(c);
    c->allocs.erase(it);
    c->halves.erase((uintptr_t)p);
    HIPC(c, hipStreamSynchronize(mstream(c)));
    dev_free(c, p);
    for (void* q : copies) dev_free(c, q);
    return SLM_OK;
}

int slm_hip_upload(slm_hip* c, float* dst, const float* src, size_t n) {
    if (!c || (n && !src)) return SLM_E_INVALID;
    if (size_t nh = half_count(c, dst)) {  // an fp16 allocation: n values rounded to fp16
        if (n > nh) return fail(c, SLM_E_BOUNDS, "upload: %zu values into %zu halves", n, nh);
        if (n == 0) return SLM_OK;
        TRY(taint(c));
        HIPC(c, hipStreamSynchronize(mstream(c)));
        uint16_t* b = (uint16_t*)c->bounce;
        for (size_t done = 0; done < n;) {
            size_t part = std::min(n - done, BOUNCE_CAP / 2);
            for (size_t i = 0; i < part; i++) b[i] = f16_of(src[done + i]);
            HIPC(c, hipMemcpy((uint16_t*)dst + done, b, part * 2, hipMemcpyHostToDevice));
            done += part;
        }
        return SLM_OK;
    }
    NEED(c, "upload", dst, n);
    if (n == 0) return SLM_OK;
    TRY(taint(c));
    drop_shadows(c, (uintptr_t)dst, (uintptr_t)(dst + n));
    for (auto it = c->tables.begin(); it != c->tables.end();) {  // inv_freq rewritten
        if (it->first >= (uintptr_t)dst && it->first < (uintptr_t)(dst + n)) {
            drop_graphs(c);
            hipStreamSynchronize(mstream(c));
            dev_free(c, it->second.cos);
            dev_free(c, it->second.sin);
            it = c->tables.erase(it);
        } else {
            ++it;
        }
    }
    HIPC(c, hipStreamSynchronize(mstream(c)));
    if (!c->fp16) {
        HIPC(c, hipMemcpy(dst, src, n * 4, hipMemcpyHostToDevice));
        return SLM_OK;
    }
    // fp16 mode: the values rounded to fp16 as they go up (mlx.rs:61-63 uploads every buffer
    // in its dtype), through the bounce buffer
    for (size_t done = 0; done < n;) {
        size_t part = std::min(n - done, BOUNCE_CAP / 4);
        for (size_t i = 0; i < part; i++) c->bounce[i] = round16(src[done + i]);
        HIPC(c, hipMemcpy(dst + done, c->bounce, part * 4, hipMemcpyHostToDevice));
        done += part;
    }
    return SLM_OK;
}

int slm_hip_read(slm_hip* c, float* host, const float* dev, size_t n) {
    if (!c || (n && !host)) return SLM_E_INVALID;
    if (size_t nh = half_count(c, dev)) {  // an fp16 allocation: n values widened to fp32
        if (n > nh) return fail(c, SLM_E_BOUNDS, "read: %zu values from %zu halves", n, nh);
        TRY(taint(c));
        for (size_t done = 0; done < n;) {
            size_t part = std::min(n - done, BOUNCE_CAP / 2);
            HIPC(c, hipMemcpyAsync(c->bounce, (const uint16_t*)dev + done, part * 2,
                                   hipMemcpyDeviceToHost, mstream(c)));
            HIPC(c, hipStreamSynchronize(mstream(c)));
            const uint16_t* b = (const uint16_t*)c->bounce;
            for (size_t i = 0; i < part; i++) host[done + i] = f32_of(b[i]);
            done += part;
        }
        if (n == 0) HIPC(c, hipStreamSynchronize(mstream(c)));
        return check_fault(c);
    }
    NEED(c, "read", dev, n);
    // the read-ahead copy of exactly this range, queued behind the step just replayed with
    // nothing after it: wait for its flag (a second at most, then the usual way)
    if (c->mir_armed && !c->recording && dev == c->mir_src && n == c->mir_n) {
        c->mir_armed = false;
        const unsigned long long* flag = (const unsigned long long*)((char*)c->mir_host + MIRROR_CAP);
        auto t0 = std::chrono::steady_clock::now();
        bool got = false;
        for (unsigned it = 0;; it++) {
            if (__atomic_load_n(flag, __ATOMIC_ACQUIRE) >= c->mir_seq) {
                got = true;
                break;
            }
            if ((it & 1023) == 1023 && std::chrono::steady_clock::now() - t0 > std::chrono::seconds(1)) break;
            _mm_pause();
        }
        if (got) {
            std::memcpy(host, c->mir_host, n * 4);
            c->n_mirror_reads++;
            return check_fault(c);
        }
    }
    uint64_t after = c->recording ? 0 : c->last_graph;  // the graph this read follows, if any
    TRY(taint(c));
    hipStream_t s = mstream(c);
    if (n * 4 <= BOUNCE_CAP) {
        HIPC(c, hipMemcpyAsync(c->bounce, dev, n * 4, hipMemcpyDeviceToHost, s));
        HIPC(c, hipStreamSynchronize(s));
        std::memcpy(host, c->bounce, n * 4);
        if (after) TRY(learn_read(c, after, dev, n));
        return check_fault(c);
    }
    // larger: the two halves of the bounce buffer in turn, the copy of part k + 1 running
    // while the host copies part k out
    const size_t P = BOUNCE_CAP / 8;  // floats a half
    size_t parts = (n + P - 1) / P;
    auto issue = [&](size_t k) -> hipError_t {
        size_t part = std::min(n - k * P, P);
        hipError_t e = hipMemcpyAsync(c->bounce + (k & 1) * P, dev + k * P, part * 4,
                                      hipMemcpyDeviceToHost, s);
        return e == hipSuccess ? hipEventRecord(c->read_ev[k & 1], s) : e;
    };
    HIPC(c, issue(0));
    for (size_t k = 0; k < parts; k++) {
        if (k + 1 < parts) HIPC(c, issue(k + 1));
        HIPC(c, hipEventSynchronize(c->read_ev[k & 1]));
        std::memcpy(host + k * P, c->bounce + (k & 1) * P, std::min(n - k * P, P) * 4);
    }
    return check_fault(c);
}

int slm_hip_flush(slm_hip* c, const float* const* keep, size_t nkeep) {
    if (!c || (nkeep && !keep)) return SLM_E_INVALID;
    TRY(check_fault(c));  // (work already finished; the rest is reported by a later check)
    if (!c->recording) return SLM_OK;
    // what outlives the step (ops.rs:90-91): a prompt step may then run on a lane, the rest
    // of what it writes being dead once it is over
    c->keep.clear();
    for (size_t i = 0; i < nkeep; i++) {
        uintptr_t b;
        size_t n;
        if (keep[i] && alloc_at(c, (uintptr_t)keep[i], &b, &n)) c->keep.push_back(b);
    }
    c->keep_valid = true;
    int rc = finish_step(c);
    c->keep_valid = false;
    return rc;
}

int slm_hip_set_spin_limit(slm_hip* c, long long polls) {
    if (!c || polls < 0) return SLM_E_INVALID;
    TRY(taint(c));
    drop_graphs(c);  // the graphs hold the old limit in their descriptors
    c->spin = (int)std::min<long long>(polls, INT_MAX);
    return SLM_OK;
}

int slm_hip_set_graphs(slm_hip* c, int on) {
    if (!c) return SLM_E_INVALID;
    if (c->recording) TRY(finish_step(c));
    if (!on) drop_graphs(c);
    c->graphs_on = on != 0;
    return SLM_OK;
}

int slm_hip_set_step_kernel(slm_hip* c, int on) {
    if (!c) return SLM_E_INVALID;
    if (c->recording) TRY(finish_step(c));
    if (c->step_on != (on != 0)) drop_graphs(c);
    c->step_on = on != 0;
    return SLM_OK;
}

int slm_hip_step_stats(slm_hip* c, uint64_t* launches, uint64_t* programs, int* available) {
    if (!c) return SLM_E_INVALID;
    if (launches) *launches = c->n_step;
    if (programs) *programs = c->n_step_plans;
    if (available) *available = c->step_ok ? 1 : 0;
    return SLM_OK;
}

int slm_hip_set_prompt_lanes(slm_hip* c, int n) {
    if (!c || n < 1 || n > MAX_LANES) return SLM_E_INVALID;
    leave_lanes(c);
    if ((int)c->lanes.size() < n) c->lanes.resize(n);
    for (int l = 1; l < n; l++) {
        auto& L = c->lanes[l];
        if (!L.stream) HIPC(c, hipStreamCreateWithFlags(&L.stream, hipStreamNonBlocking));
        for (int i = 0; i < 2; i++) {
            if (!L.dyn_pin[i]) HIPC(c, hipHostMalloc((void**)&L.dyn_pin[i], DYN_CAP, hipHostMallocDefault));
            if (!L.dyn_ev[i]) HIPC(c, hipEventCreateWithFlags(&L.dyn_ev[i], hipEventDisableTiming));
        }
        if (!L.dyn_dev) HIPC(c, hipMalloc((void**)&L.dyn_dev, DYN_CAP));
    }
    c->nlanes = n;
    return SLM_OK;
}

int slm_hip_read_ahead_stats(slm_hip* c, uint64_t* reads) {
    if (!c || !reads) return SLM_E_INVALID;
    *reads = c->n_mirror_reads;
    return SLM_OK;
}

int slm_hip_get_prompt_lanes(slm_hip* c, int* n) {
    if (!c || !n) return SLM_E_INVALID;
    *n = c->nlanes;
    return SLM_OK;
}

int slm_hip_prompt_lane_stats(slm_hip* c, uint64_t* steps, uint64_t* fallbacks) {
    if (!c || !steps || !fallbacks) return SLM_E_INVALID;
    *steps = c->n_lane_steps;
    *fallbacks = c->n_lane_fallbacks;
    return SLM_OK;
}

int slm_hip_set_fp16(slm_hip* c, int on) {
    if (!c) return SLM_E_INVALID;
    if (c->recording) TRY(finish_step(c));
    if (c->fp16 == (on != 0)) return SLM_OK;
    // planned steps and resident rope tables belong to one mode; the kernels that run in both
    // read the mode word
    leave_lanes(c);
    drop_graphs(c);
    HIPC(c, hipStreamSynchronize(c->stream));
    for (auto& t : c->tables) {
        dev_free(c, t.second.cos);
        dev_free(c, t.second.sin);
    }
    c->tables.clear();
    int v = on != 0;
    HIPC(c, hipMemcpy(c->h16_dev, &v, sizeof v, hipMemcpyHostToDevice));
    c->fp16 = on != 0;
    return SLM_OK;
}

int slm_hip_set_tile_rows(slm_hip* c, int rows) {
    if (!c || (rows != 0 && rows != 4 && rows != 8 && rows != 12 && rows != 16)) return SLM_E_INVALID;
    if (c->recording) TRY(finish_step(c));
    if (c->fg_rpt != rows) drop_graphs(c);
    c->fg_rpt = rows;
    return SLM_OK;
}

int slm_hip_set_half_shadows(slm_hip* c, int on) {
    if (!c) return SLM_E_INVALID;
    if (c->recording) TRY(finish_step(c));
    if (c->shadows_on != (on != 0)) drop_graphs(c);
    c->shadows_on = on != 0;
    if (!c->shadows_on) drop_shadows(c, 0, UINTPTR_MAX);
    return SLM_OK;
}

int slm_hip_get_fp16(slm_hip* c, int* on) {
    if (!c || !on) return SLM_E_INVALID;
    *on = c->fp16 ? 1 : 0;
    return SLM_OK;
}

int slm_hip_set_fusion(slm_hip* c, int on) {
    if (!c) return SLM_E_INVALID;
    if (c->recording) TRY(finish_step(c));
    if (c->fusion_on != (on != 0)) drop_graphs(c);
    c->fusion_on = on != 0;
    return SLM_OK;
}

int slm_hip_graph_stats(slm_hip* c, uint64_t* launched, uint64_t* captured, uint64_t* eager) {
    if (!c) return SLM_E_INVALID;
    if (launched) *launched = c->n_launched;
    if (captured) *captured = c->n_captured;
    if (eager) *eager = c->n_eager;
    return SLM_OK;
}

int slm_hip_set_timing(slm_hip* c, int on) {
    if (!c) return SLM_E_INVALID;
    TRY(collect_timing(c));
    c->timing = on != 0;
    c->kstats.clear();
    return SLM_OK;
}

int slm_hip_kernel_stat(slm_hip* c, const char* name, long long* launches, double* us,
                        double* bytes) {
    if (!c || !name) return SLM_E_INVALID;
    TRY(collect_timing(c));
    auto it = c->kstats.find(name);
    KStat k = it == c->kstats.end() ? KStat{} : it->second;
    if (launches) *launches = k.launches;
    if (us) *us = 1e3 * k.ms;
    if (bytes) *bytes = k.bytes;
    return SLM_OK;
}

int slm_hip_last_plan(slm_hip* c, uint64_t* ops, uint64_t* kernels) {
    if (!c) return SLM_E_INVALID;
    if (ops) *ops = c->last_ops;
    if (kernels) *kernels = c->last_kernels;
    return SLM_OK;
}

// ---- element-wise operations ----

int slm_hip_copy(slm_hip* c, float* y, const float* x, size_t n) {
    if (!c) return SLM_E_INVALID;
    NEED(c, "copy", y, n);
    NEED(c, "copy", x, n);
    if (!n) return SLM_OK;
    Op o = op(OP_COPY);
    o.p[0] = y;
    o.p[1] = x;
    o.n[0] = (int64_t)n;
    return submit(c, o);
}

int slm_hip_add(slm_hip* c, float* y, const float* a, const float* b, size_t n) {
    if (!c) return SLM_E_INVALID;
    NEED(c, "add", y, n);
    NEED(c, "add", a, n);
    NEED(c, "add", b, n);
    if (!n) return SLM_OK;
    Op o = op(OP_ADD);
    o.p[0] = y;
    o.p[1] = a;
    o.p[2] = b;
    o.n[0] = (int64_t)n;
    return submit(c, o);
}

int slm_hip_add_row(slm_hip* c, float* y, const float* x, const float* row, size_t m, size_t d) {
    if (!c) return SLM_E_INVALID;
    NEED(c, "add_row", y, m * d);
    NEED(c, "add_row", x, m * d);
    NEED(c, "add_row", row, d);
    if (!m || !d) return SLM_OK;
    Op o = op(OP_ADD_ROW);
    o.p[0] = y;
    o.p[1] = x;
    o.p[2] = row;
    o.n[0] = (int64_t)m;
    o.n[1] = (int64_t)d;
    return submit(c, o);
}

int slm_hip_mix(slm_hip* c, float* y, const float* a, const float* b, size_t n, float t) {
    if (!c) return SLM_E_INVALID;
    NEED(c, "mix", y, n);
    NEED(c, "mix", a, n);
    NEED(c, "mix", b, n);
    if (!n) return SLM_OK;
    Op o = op(OP_MIX);
    o.p[0] = y;
    o.p[1] = a;
    o.p[2] = b;
    o.n[0] = (int64_t)n;
    o.f[0] = t;
    return submit(c, o);
}

int slm_hip_silu_mul(slm_hip* c, float* y, const float* g, const float* u, size_t n) {
    if (!c) return SLM_E_INVALID;
    NEED(c, "silu_mul", y, n);
    NEED(c, "silu_mul", g, n);
    NEED(c, "silu_mul", u, n);
    if (!n) return SLM_OK;
    Op o = op(OP_SILU_MUL);
    o.p[0] = y;
    o.p[1] = g;
    o.p[2] = u;
    o.n[0] = (int64_t)n;
    return submit(c, o);
}

int slm_hip_scale_rows(slm_hip* c, float* y, const float* x, const float* f, size_t m, size_t d) {
    if (!c || (m && !f)) return SLM_E_INVALID;
    NEED(c, "scale_rows", y, m * d);
    NEED(c, "scale_rows", x, m * d);
    if (!m || !d) return SLM_OK;
    Op o = op(OP_SCALE_ROWS);
    o.p[0] = y;
    o.p[1] = x;
    o.n[0] = (int64_t)m;
    o.n[1] = (int64_t)d;
    if (m == 1 && !recording(c)) {
        o.f[0] = f[0];
    } else {
        TRY(stage(c, f, m * 4, &o.dyn));
    }
    return submit(c, o);
}

int slm_hip_shift(slm_hip* c, float* y, const float* first, const float* x, size_t m, size_t d) {
    if (!c) return SLM_E_INVALID;
    if (!m) return SLM_OK;
    NEED(c, "shift", y, m * d);
    NEED(c, "shift", first, d);
    NEED(c, "shift", x, (m - 1) * d);
    if (!d) return SLM_OK;
    Op o = op(OP_SHIFT);
    o.p[0] = y;
    o.p[1] = first;
    o.p[2] = x;
    o.n[0] = (int64_t)m;
    o.n[1] = (int64_t)d;
    return submit(c, o);
}

int slm_hip_columns(slm_hip* c, float* y, const float* x, size_t m, size_t stride, size_t off,
                    size_t len) {
    if (!c) return SLM_E_INVALID;
    if (!m || !len) return SLM_OK;
    if (off + len > stride) return fail(c, SLM_E_INVALID, "columns: off + len > stride");
    NEED(c, "columns", y, m * len);
    NEED(c, "columns", x, (m - 1) * stride + off + len);
    Op o = op(OP_COLUMNS);
    o.p[0] = y;
    o.p[1] = x;
    o.n[0] = (int64_t)m;
    o.n[1] = (int64_t)stride;
    o.n[2] = (int64_t)off;
    o.n[3] = (int64_t)len;
    return submit(c, o);
}

int slm_hip_gather(slm_hip* c, float* y, const float* w, const uint32_t* ids, size_t m, size_t d) {
    if (!c || (m && !ids)) return SLM_E_INVALID;
    NEED(c, "gather", y, m * d);
    if (!m || !d) return SLM_OK;
    size_t rows = room(c, w) / 4 / d;
    std::vector<long long> v(m);
    for (size_t i = 0; i < m; i++) {
        if (ids[i] >= rows)
            return fail(c, SLM_E_BOUNDS, "gather: id %u is past the %zu rows of w", ids[i], rows);
        v[i] = ids[i];
    }
    Op o = op(OP_GATHER);
    o.p[0] = y;
    o.p[1] = w;
    o.n[0] = (int64_t)m;
    o.n[1] = (int64_t)d;
    TRY(stage(c, v.data(), m * 8, &o.dyn));
    return submit(c, o);
}

int slm_hip_gather_dev(slm_hip* c, float* y, const float* w, const long long* id, size_t rows, size_t d) {
    if (!c || !id || !rows) return SLM_E_INVALID;
    NEED(c, "gather_dev", y, d);
    NEED(c, "gather_dev", w, rows * d);
    NEED(c, "gather_dev", (const float*)id, 2);
    if (!d) return SLM_OK;
    Op o = op(OP_GATHER);
    o.p[0] = y;
    o.p[1] = w;
    o.n[0] = 1;
    o.n[1] = (int64_t)d;
    o.dyn = id;  // read on the device when the op runs (slm_argmax writes an index below rows)
    return submit(c, o);
}

int slm_hip_argmax(slm_hip* c, long long* tok, uint32_t* ids, size_t ids_cap, size_t slot,
                   const float* x, size_t n) {
    if (!c || !tok || !n || n > (size_t)INT32_MAX || (ids && slot >= ids_cap)) return SLM_E_INVALID;
    NEED(c, "argmax", x, n);
    NEED(c, "argmax", (const float*)tok, 2);
    if (ids) NEED(c, "argmax", (const float*)ids, ids_cap);
    Op o = op(OP_ARGMAX);
    o.p[0] = (float*)tok;
    o.p[1] = x;
    o.p[2] = (float*)ids;
    o.n[0] = (int64_t)n;
    o.n[2] = (int64_t)ids_cap;
    if (ids) TRY(stage_pos(c, slot, o, 1));  // the slot staged per step (graphs stay reusable)
    return submit(c, o);
}

int slm_hip_store(slm_hip* c, float* cache, const float* src, size_t pos, size_t m, size_t cap,
                  size_t heads, size_t dh) {
    if (!c) return SLM_E_INVALID;
    if (!m || !heads || !dh) return SLM_OK;
    if (!cap) return fail(c, SLM_E_INVALID, "store: cap is 0");
    size_t h16 = half_count(c, cache);  // an fp16 ring (slm_hip_alloc_cache in fp16 mode)
    if (h16) {
        if (h16 < heads * cap * dh)
            return fail(c, SLM_E_BOUNDS, "store: %zu x %zu x %zu ring in %zu halves", heads, cap, dh, h16);
    } else {
        NEED(c, "store", cache, heads * cap * dh);
    }
    NEED(c, "store", src, m * heads * dh);
    Op o = op(OP_STORE);
    o.p[0] = cache;
    o.p[1] = src;
    o.n[0] = (int64_t)m;
    o.n[1] = (int64_t)cap;
    o.n[2] = (int64_t)heads;
    o.n[3] = (int64_t)dh;
    o.n[5] = h16 ? 1 : 0;
    TRY(stage_pos(c, pos, o, 4));
    return submit(c, o);
}

int slm_hip_rope(slm_hip* c, float* y, const float* x, const float* cs, const float* sn,
                 size_t m, size_t heads, size_t dh) {
    if (!c) return SLM_E_INVALID;
    if (dh % 2) return fail(c, SLM_E_UNSUPPORTED, "rope: odd head size %zu", dh);
    NEED(c, "rope", y, m * heads * dh);
    NEED(c, "rope", x, m * heads * dh);
    NEED(c, "rope", cs, m * dh / 2);
    NEED(c, "rope", sn, m * dh / 2);
    if (!m || !heads || !dh) return SLM_OK;
    Op o = op(OP_ROPE);
    o.p[0] = y;
    o.p[1] = x;
    o.p[2] = cs;
    o.p[3] = sn;
    o.n[0] = (int64_t)m;
    o.n[1] = (int64_t)heads;
    o.n[2] = (int64_t)dh;
    return submit(c, o);
}

int slm_hip_rope_table(slm_hip* c, float* cs, float* sn, const float* inv, size_t pos, size_t m,
                       size_t half) {
    if (!c) return SLM_E_INVALID;
    NEED(c, "rope_table", cs, m * half);
    NEED(c, "rope_table", sn, m * half);
    NEED(c, "rope_table", inv, half);
    // the first call of every advance (model.rs:566) ends the previous step, makes sure the
    // resident table covers this one, then begins it
    if (c->recording) TRY(finish_step(c));
    Table& t = c->tables[(uintptr_t)inv];
    if (half && t.inv.size() != half) {  // first sight of this inv_freq buffer
        t.h16 = c->fp16;
        t.inv.assign(half, 0.0f);
        HIPC(c, hipStreamSynchronize(mstream(c)));
        HIPC(c, hipMemcpy(t.inv.data(), inv, half * 4, hipMemcpyDeviceToHost));
        t.rows = 0;
    }
    if (half && pos + m > t.rows) {
        size_t rows = std::max<size_t>({pos + m, t.rows * 2, 8192});
        // cpu.rs:228-236: angle (pos + i) as f32 times inv[j], then libm cos/sin
        std::vector<float> hc(rows * half), hs(rows * half);
        // (fp16 mode: the angles in fp32 from the fp16 inv_freq, cos and sin rounded to fp16,
        // mlx.rs:203-208)
        for (size_t p = 0; p < rows; p++) {
            float fp = (float)p;
            for (size_t j = 0; j < half; j++) {
                float a = fp * t.inv[j];
                hc[p * half + j] = t.h16 ? round16(cosf(a)) : cosf(a);
                hs[p * half + j] = t.h16 ? round16(sinf(a)) : sinf(a);
            }
        }
        TRY(internal_realloc(c, (void**)&t.cos, rows * half * 4));
        TRY(internal_realloc(c, (void**)&t.sin, rows * half * 4));
        HIPC(c, hipMemcpy(t.cos, hc.data(), rows * half * 4, hipMemcpyHostToDevice));
        HIPC(c, hipMemcpy(t.sin, hs.data(), rows * half * 4, hipMemcpyHostToDevice));
        t.rows = rows;
    }
    if (c->graphs_on || c->fusion_on) {
        c->recording = true;
        c->tainted = false;
        c->ops.clear();
        c->dyn.clear();
    }
    if (!m || !half) return SLM_OK;
    Op o = op(OP_ROPE_TABLE);
    o.p[0] = cs;
    o.p[1] = sn;
    o.p[2] = t.cos;
    o.p[3] = t.sin;
    o.n[0] = (int64_t)m;
    o.n[1] = (int64_t)half;
    TRY(stage_pos(c, pos, o, 2));
    return submit(c, o);
}

// ---- normalisation ----

static int norm_op(slm_hip* c, uint32_t kind, float* y, const float* x, const float* w,
                   size_t groups, size_t size, float eps) {
    if (!fits_int(groups) || !fits_int(size) || groups * size > (size_t)INT_MAX)
        return fail(c, SLM_E_UNSUPPORTED, "norm: %zu groups of %zu", groups, size);
    if ((size | 1) * 4 > 65536) return fail(c, SLM_E_UNSUPPORTED, "norm: size %zu is above 16383", size);
    Op o = op(kind);
    o.p[0] = y;
    o.p[1] = x;
    o.p[2] = w;
    o.n[0] = (int64_t)groups;
    o.n[1] = (int64_t)size;
    o.f[0] = eps;
    return submit(c, o);
}

int slm_hip_rms(slm_hip* c, float* y, const float* x, const float* w, size_t groups, size_t size,
                float eps) {
    if (!c) return SLM_E_INVALID;
    NEED(c, "rms", y, groups * size);
    NEED(c, "rms", x, groups * size);
    NEED(c, "rms", w, size);
    if (!groups || !size) return SLM_OK;
    return norm_op(c, OP_RMS, y, x, w, groups, size, eps);
}

int slm_hip_l2norm(slm_hip* c, float* y, const float* x, size_t heads, size_t dh) {
    if (!c) return SLM_E_INVALID;
    NEED(c, "l2norm", y, heads * dh);
    NEED(c, "l2norm", x, heads * dh);
    if (!heads || !dh) return SLM_OK;
    return norm_op(c, OP_L2NORM, y, x, nullptr, heads, dh, 0.0f);
}

// ---- linear ----

int slm_hip_linear(slm_hip* c, float* y, const float* w, size_t rows, size_t cols,
                   const float* x, size_t m) {
    if (!c) return SLM_E_INVALID;
    NEED(c, "linear", y, m * rows);
    size_t nh = half_count(c, w);
    if (nh) {  // fp16 weights: fp16 mode only (the same halves the fp16 chain rounds to)
        if (rows * cols > nh) return fail(c, SLM_E_BOUNDS, "linear: %zu x %zu weights in %zu halves", rows, cols, nh);
        if (!c->fp16)
            return fail(c, SLM_E_UNSUPPORTED, "linear: fp16 weights need fp16 mode (slm_hip_set_fp16)");
    } else {
        NEED(c, "linear", w, rows * cols);
    }
    NEED(c, "linear", x, m * cols);
    if (!m || !rows) return SLM_OK;
    if (!nh && c->fp16 && c->shadows_on && cols % 64 == 0 && aligned16(w) && aligned16(x)) {
        const float* h = nullptr;
        TRY(shadow_of(c, w, rows * cols, &h));
        if (h) {
            w = h;
            nh = rows * cols;
        }
    }
    if (!fits_int(rows) || !fits_int(cols) || !fits_int(m))
        return fail(c, SLM_E_UNSUPPORTED, "linear: %zu x %zu x %zu", rows, cols, m);
    if (m == 1 && c->fusion_on && cols <= (size_t)VP_LEN_MAX) {
        int64_t ns = nsplit_of((int64_t)cols);
        if (ns > 1) TRY(need_part(c, (size_t)(2 * ns) * rows * 4));
    }
    if (m > 16) {
        int64_t ns = nsplit_of((int64_t)cols);
        if (ns > 1) TRY(need_gpart(c, (size_t)ns * m * rows * 4));
    }
    Op o = op(OP_LINEAR);
    o.p[0] = y;
    o.p[1] = w;
    o.p[2] = x;
    o.n[0] = (int64_t)rows;
    o.n[1] = (int64_t)cols;
    o.n[2] = (int64_t)m;
    o.n[3] = c->fp16 ? 1 : 0;
    o.n[4] = nh ? 1 : 0;  // fp16 weights
    if (c->fp16 && (cols % 64 || !aligned16(w) || !aligned16(x)))
        return fail(c, SLM_E_UNSUPPORTED,
                    "linear: fp16 mode needs a multiple of 64 columns and 16-byte aligned w and x (%zu)", cols);
    return submit(c, o);
}

// ---- gated linear attention ----

int slm_hip_gla(slm_hip* c, float* y, float* s, const float* q, const float* k, const float* v,
                const float* decay, const float* bias, size_t m, size_t heads, size_t dh) {
    if (!c) return SLM_E_INVALID;
    size_t n = m * heads * dh;
    NEED(c, "gla", y, n);
    NEED(c, "gla", s, heads * dh * dh);
    NEED(c, "gla", q, n);
    NEED(c, "gla", k, n);
    NEED(c, "gla", v, n);
    NEED(c, "gla", decay, m * heads);
    NEED(c, "gla", bias, heads);
    if (!m || !heads || !dh) return SLM_OK;
    if (dh > 256) return fail(c, SLM_E_UNSUPPORTED, "gla: head size %zu is above 256", dh);
    if (!fits_int(m) || !fits_int(heads * dh * 4))
        return fail(c, SLM_E_UNSUPPORTED, "gla: %zu tokens x %zu heads", m, heads);
    Op o = op(OP_GLA);
    o.p[0] = y;
    o.p[1] = s;
    o.p[2] = q;
    o.p[3] = k;
    o.p[4] = v;
    o.p[5] = decay;
    o.p[6] = bias;
    o.n[0] = (int64_t)m;
    o.n[1] = (int64_t)heads;
    o.n[2] = (int64_t)dh;
    return submit(c, o);
}

// ---- attention ----

}  // extern "C"

namespace {

// The checks and the op of an attention call; *part_bytes: the superblock partials it needs.
int attend_op(slm_hip* c, float* y, const float* q, const float* k, const float* v,
              const slm_attn* a, Op& o, size_t* part_bytes) {
    *part_bytes = 0;
    if (!c || !a) return SLM_E_INVALID;
    size_t m = a->m, heads = a->heads, kh = a->key_heads, dh = a->dh, cap = a->cap;
    NEED(c, "attend", y, m * heads * dh);
    if (!m || !heads || !dh) return SLM_OK;
    if (dh > 256) return fail(c, SLM_E_UNSUPPORTED, "attend: head size %zu is above the 256 the kernels allow", dh);
    if (dh % 4) return fail(c, SLM_E_UNSUPPORTED, "attend: head size %zu is not a multiple of 4", dh);
    if (!kh || heads % kh) return fail(c, SLM_E_INVALID, "attend: %zu heads over %zu key heads", heads, kh);
    size_t group = heads / kh;
    if (group > 16) return fail(c, SLM_E_UNSUPPORTED, "attend: %zu query heads per key head", group);
    if (!cap || a->reach == 0) return fail(c, SLM_E_INVALID, "attend: cap or reach is 0");
    NEED(c, "attend", q, m * heads * dh);
    size_t hk = half_count(c, k), hv = half_count(c, v);  // fp16 rings
    if (hk || hv) {
        if (!hk || !hv) return fail(c, SLM_E_INVALID, "attend: one fp16 ring and one fp32 ring");
        if (hk < kh * cap * dh || hv < kh * cap * dh)
            return fail(c, SLM_E_BOUNDS, "attend: %zu x %zu x %zu rings in %zu and %zu halves", kh, cap, dh, hk, hv);
        if (!half_ring_ok(heads, dh, cap))
            return fail(c, SLM_E_UNSUPPORTED, "attend: fp16 rings need head size <= 64, a multiple of 8, "
                        "and at least 64 slots");
    } else {
        NEED(c, "attend", k, kh * cap * dh);
        NEED(c, "attend", v, kh * cap * dh);
    }
    if (!aligned16(q) || !aligned16(k) || !aligned16(v))
        return fail(c, SLM_E_UNSUPPORTED, "attend: q, k and v must be 16-byte aligned");
    if (!fits_int(m) || !fits_int(heads))
        return fail(c, SLM_E_UNSUPPORTED, "attend: %zu queries", m);
    const long long BIG = (long long)1 << 50;
    long long reach = a->reach > (size_t)BIG ? BIG : (long long)a->reach;
    long long gap = a->gap > (size_t)BIG ? BIG : (long long)a->gap;
    long long pos = (long long)a->pos;
    // superblock slots: a fixed count for a window, else the current span
    size_t nsb;
    if (reach < BIG / 2) {
        nsb = (size_t)((reach + (long long)m - 2) / SLM_SB_KEYS + 2);
    } else {
        long long first = reach - 1 > pos ? 0 : pos - (reach - 1);
        long long last = pos + (long long)m - 1 - gap;
        nsb = last >= first ? (size_t)(last / SLM_SB_KEYS - first / SLM_SB_KEYS + 1) : 1;
    }
    size_t qpt = 16 / group;
    size_t qtiles = (m + qpt - 1) / qpt;
    if (a->cap >= ((size_t)1 << 31))
        return fail(c, SLM_E_UNSUPPORTED, "attend: ring of %zu slots (at most 2^31 - 1)", a->cap);
    if (qtiles > UINT32_MAX || nsb > 65535)
        return fail(c, SLM_E_UNSUPPORTED, "attend: %zu query tiles x %zu superblocks", qtiles, nsb);
    size_t dp = (size_t)16 << pow2_index((dh + 15) / 16, 4);
    *part_bytes = nsb * m * heads * (dp + 2) * 4;
    o = op(OP_ATTEND);
    o.p[0] = y;
    o.p[1] = q;
    o.p[2] = k;
    o.p[3] = v;
    o.n[1] = (int64_t)m;
    o.n[2] = reach;
    o.n[3] = gap;
    o.n[4] = (int64_t)cap;
    o.n[5] = (int64_t)heads;
    o.n[6] = (int64_t)kh;
    o.n[7] = (int64_t)dh;
    o.n[8] = (int64_t)nsb;
    o.n[9] = hk ? 1 : 0;
    o.f[0] = c->fp16 ? round16(a->scale) : a->scale;  // (fp16 mode: the dtype's scalar, mlx.rs:344)
    if (hk && m > 1 && (int64_t)((qtiles + ATTN_QG_HOST - 1) / ATTN_QG_HOST) * (int64_t)kh * (int64_t)nsb > (int64_t)INT_MAX)
        return fail(c, SLM_E_UNSUPPORTED, "attend: fp16 rings: %zu query tiles", qtiles);
    return SLM_OK;
}

}  // namespace

extern "C" {

int slm_hip_attend(slm_hip* c, float* y, float* scores, const float* q, const float* k,
                   const float* v, const slm_attn* a) {
    (void)scores;  // the trait's scratch: this backend keeps its own workspace
    Op o;
    size_t part_bytes = 0;
    int rc = attend_op(c, y, q, k, v, a, o, &part_bytes);
    if (rc || !part_bytes) return rc;
    TRY(need_ws(c, part_bytes));
    TRY(stage_pos(c, a->pos, o, 0));
    return submit(c, o);
}

// slm_hip_attend with the superblock partials in this device's fixed scratch: kernel launches
// only, on the context's stream (no allocation, copy, fill or event), so that a caller may run
// it under its own stream capture. Not inside a recorded step (the step's plan may allocate).
int slm_hip_attend_noalloc(slm_hip* c, float* y, float* scores, const float* q, const float* k,
                           const float* v, const slm_attn* a) {
    (void)scores;
    Op o;
    size_t part_bytes = 0;
    int rc = attend_op(c, y, q, k, v, a, o, &part_bytes);
    if (rc || !part_bytes) return rc;
    if (c->recording)
        return fail(c, SLM_E_UNSUPPORTED, "attend_noalloc: called inside a recorded step (between "
                    "rope_table and flush); call it outside a step");
    if (part_bytes > SLM_NOALLOC_SCRATCH_BYTES)
        return fail(c, SLM_E_UNSUPPORTED, "attend_noalloc: %zu bytes of superblock partials exceed the "
                    "fixed scratch of %zu bytes (fewer queries per call, or slm_hip_attend)",
                    part_bytes, (size_t)SLM_NOALLOC_SCRATCH_BYTES);
    if (!c->scratch) return fail(c, SLM_E_HIP, "attend_noalloc: no device scratch");
    o.p[4] = c->scratch;
    o.n[0] = (int64_t)a->pos;  // an immediate position (outside a step: nothing is staged)
    o.dyn = nullptr;
    std::vector<Rec> recs;
    TRY(lower_one(c, o, recs));
    for (auto& r : recs) {
        void* ptrs[MAX_ARGS];
        for (uint32_t i = 0; i < r.nargs; i++) ptrs[i] = (void*)(r.blob + 8 * i);
        if (r.bytes) return fail(c, SLM_E_HIP, "attend_noalloc: unexpected descriptor launch");
        hipError_t e = hipModuleLaunchKernel(r.f, r.gx, r.gy, r.gz, r.bx, 1, 1, r.shmem, mstream(c),
                                             ptrs, nullptr);
        if (e != hipSuccess)
            return fail(c, SLM_E_HIP, "attend_noalloc: hipModuleLaunchKernel: %s", hipGetErrorString(e));
    }
    return SLM_OK;
}

// ---- diagnostics ----

int slm_hip_stream(slm_hip* c, void** out) {
    if (!c || !out) return SLM_E_INVALID;
    *out = (void*)mstream(c);
    return SLM_OK;
}

int slm_hip_mem_info(slm_hip* c, size_t* free_bytes, size_t* total_bytes, size_t* held_bytes) {
    if (!c || !free_bytes || !total_bytes || !held_bytes) return SLM_E_INVALID;
    HIPC(c, hipSetDevice(c->device));
    HIPC(c, hipMemGetInfo(free_bytes, total_bytes));
    // pool slabs, plus what went to hipMalloc directly (blocks above the pool's largest)
    size_t held = c->slabs.size() * POOL_SLAB;
    auto direct = [&](const void* p, size_t bytes) {
        if (p && !c->pooled.count((uintptr_t)p)) held += bytes;
    };
    for (auto& a : c->allocs) direct((const void*)a.first, a.second);
    for (auto& sh : c->shadows) direct(sh.second.h, sh.second.n * 2);
    direct(c->ws, c->ws_bytes);
    direct(c->part, c->part_bytes);
    direct(c->gpart, c->gpart_bytes);
    *held_bytes = held;
    return SLM_OK;
}

// Runs one 16x16x4 f32 MFMA on lane inputs a[64], b[64] (device) into out[256].
int slm_hip_probe_mfma(slm_hip* c, float* out, const float* a, const float* b) {
    if (!c) return SLM_E_INVALID;
    NEED(c, "probe", out, 256);
    NEED(c, "probe", a, 64);
    NEED(c, "probe", b, 64);
    TRY(taint(c));
    return launch_now(c, mk(c->k.probe, 1, 1, 1, 64, 0, out, a, b));
}

}  // extern "C"
