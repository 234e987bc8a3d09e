// Host runtime of the MI355X backend: the C ABI of include/slm_hip.h.
//
// One context = one device, one stream (default priority), the gfx950 code object loaded
// with hipModuleLoadData, a table of live allocations that every operation checks its
// pointer ranges against before anything is queued, a workspace for attention partials,
// and the step-graph cache. Kernels live in kernels.hip; this file only validates, sizes
// launches and queues them.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "slm_hip.h"

extern "C" const unsigned char slm_code_object[];
extern "C" const size_t slm_code_object_size;

namespace {

std::string g_open_error;

constexpr int MAX_ARGS = 16;
constexpr size_t DYN_CAP = 1 << 20;          // bytes of per-step dynamic values
constexpr size_t STAGE_CAP = 4 << 20;        // bytes of eager staging
constexpr size_t BOUNCE_CAP = 4 << 20;       // pinned bounce buffer for reads
constexpr size_t MAX_GRAPHS = 8;

// One queued kernel launch: everything hipModuleLaunchKernel needs, by value, so a step
// can be compared with a cached one byte for byte.
struct Rec {
    hipFunction_t f;
    uint32_t gx, gy, gz, bx, shmem, nargs;
    uint64_t args[MAX_ARGS];
};

struct Graph {
    std::vector<Rec> recs;
    size_t ndyn = 0;
    hipGraphExec_t exec = nullptr;
    uint64_t used = 0;
};

struct Table {  // resident cos/sin rows for one inv_freq buffer
    std::vector<float> inv;
    float* cos = nullptr;
    float* sin = nullptr;
    size_t rows = 0;
};

struct Kernels {
    hipFunction_t copy, add, add_row, mix, silu_mul, scale_rows, shift, columns, gather,
        store, rope, rope_table, rms, l2norm, fill, combine, probe;
    hipFunction_t lin_small[2], lin_big[2];  // [vec]
    hipFunction_t gla[7];                    // rows per lane 1, 2, 4, .., 64
    hipFunction_t attn[5];                   // dim tiles 1, 2, 4, 8, 16
};

}  // namespace

struct slm_hip {
    int device = 0;
    hipStream_t stream = nullptr;
    hipModule_t mod = nullptr;
    Kernels k{};
    std::string err;
    char name[256] = {0};
    // live allocations: start -> bytes
    std::map<uintptr_t, size_t> allocs;
    // attention partials
    float* ws = nullptr;
    size_t ws_bytes = 0;
    // eager staging: pinned host ring copied into a device ring
    unsigned char* stage_host = nullptr;
    unsigned char* stage_dev = nullptr;
    size_t stage_head = 0;
    // step dynamic values: host copy (this step), two pinned uploads, one device area
    unsigned char* dyn_pin[2] = {nullptr, nullptr};
    hipEvent_t dyn_ev[2] = {nullptr, nullptr};
    int dyn_flip = 0;
    unsigned char* dyn_dev = nullptr;
    float* bounce = nullptr;
    std::map<uintptr_t, Table> tables;
    // step graphs
    bool graphs_on = true;
    bool recording = false;
    bool tainted = false;
    std::vector<Rec> recs;
    std::vector<unsigned char> dyn;
    std::vector<Graph> cache;
    uint64_t clock = 0, n_launched = 0, n_captured = 0, n_eager = 0;
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

// Is [p, p + bytes) inside one live allocation?
bool inside(const slm_hip* c, const void* p, size_t bytes) {
    uintptr_t a = (uintptr_t)p;
    auto it = c->allocs.upper_bound(a);
    if (it == c->allocs.begin()) return false;
    --it;
    return a >= it->first && a - it->first + bytes <= it->second;
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

#define NEED(c, op, p, n)                                                            \
    do {                                                                             \
        if ((n) > 0 && !inside(c, p, (size_t)(n) * 4))                               \
            return fail(c, SLM_E_BOUNDS, "%s: %s [%p, %zu floats) is outside every " \
                        "live allocation", op, #p, (const void*)(p), (size_t)(n));   \
    } while (0)

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }
bool fits_int(size_t v) { return v <= (size_t)INT_MAX; }

template <typename T>
void put(Rec& r, T v) {
    static_assert(sizeof(T) <= 8, "argument too large");
    uint64_t s = 0;
    std::memcpy(&s, &v, sizeof(T));
    r.args[r.nargs++] = s;
}

void pack(Rec&) {}
template <typename T, typename... A>
void pack(Rec& r, T v, A... rest) {
    put(r, v);
    pack(r, rest...);
}

// Argument sizes per kernel, needed to hand hipModuleLaunchKernel pointers into the
// 8-byte slots: values are stored little-endian in the low bytes, so a pointer to the
// slot serves every argument type up to 8 bytes.
int launch_now(slm_hip* c, const Rec& r) {
    void* ptrs[MAX_ARGS];
    for (uint32_t i = 0; i < r.nargs; i++) ptrs[i] = (void*)&r.args[i];
    HIPC(c, hipModuleLaunchKernel(r.f, r.gx, r.gy, r.gz, r.bx, 1, 1, r.shmem, c->stream, ptrs,
                                  nullptr));
    return SLM_OK;
}

void drop_graphs(slm_hip* c) {
    if (c->cache.empty()) return;
    hipStreamSynchronize(c->stream);
    for (auto& g : c->cache)
        if (g.exec) hipGraphExecDestroy(g.exec);
    c->cache.clear();
}

int upload_dyn(slm_hip* c) {
    if (c->dyn.empty()) return SLM_OK;
    int k = c->dyn_flip ^= 1;
    HIPC(c, hipEventSynchronize(c->dyn_ev[k]));
    std::memcpy(c->dyn_pin[k], c->dyn.data(), c->dyn.size());
    HIPC(c, hipMemcpyAsync(c->dyn_dev, c->dyn_pin[k], c->dyn.size(), hipMemcpyHostToDevice,
                           c->stream));
    HIPC(c, hipEventRecord(c->dyn_ev[k], c->stream));
    return SLM_OK;
}

// Leaves recording for the rest of this step: what was recorded runs now.
int taint(slm_hip* c) {
    if (!c->recording || c->tainted) return SLM_OK;
    c->tainted = true;
    c->n_eager++;
    int rc = upload_dyn(c);
    if (rc) return rc;
    for (auto& r : c->recs)
        if ((rc = launch_now(c, r))) return rc;
    c->recs.clear();
    return SLM_OK;
}

int emit(slm_hip* c, const Rec& r) {
    if (c->recording && !c->tainted) {
        c->recs.push_back(r);
        return SLM_OK;
    }
    return launch_now(c, r);
}

template <typename... A>
int go(slm_hip* c, hipFunction_t f, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t bx,
       uint32_t shmem, A... args) {
    Rec r;
    r.f = f;
    r.gx = gx;
    r.gy = gy;
    r.gz = gz;
    r.bx = bx;
    r.shmem = shmem;
    r.nargs = 0;
    std::memset(r.args, 0, sizeof r.args);
    pack(r, args...);
    return emit(c, r);
}

uint32_t blocks_for(size_t n, size_t per = 256, size_t cap = 4096) {
    size_t b = (n + per - 1) / per;
    return (uint32_t)std::max<size_t>(1, std::min(b, cap));
}

// Dynamic values (positions, token ids, factors): returns a device pointer to a copy of
// `bytes` bytes of `src`, valid for kernels queued after it on the stream.
int stage(slm_hip* c, const void* src, size_t bytes, const void** out) {
    size_t need = (bytes + 7) & ~(size_t)7;
    if (c->recording && !c->tainted) {
        size_t off = c->dyn.size();
        if (off + need <= DYN_CAP) {
            c->dyn.resize(off + need);
            std::memcpy(c->dyn.data() + off, src, bytes);
            *out = c->dyn_dev + off;
            return SLM_OK;
        }
        int rc = taint(c);
        if (rc) return rc;
    }
    if (need > STAGE_CAP) return fail(c, SLM_E_UNSUPPORTED, "stage: %zu bytes at once", bytes);
    if (c->stage_head + need > STAGE_CAP) {
        HIPC(c, hipStreamSynchronize(c->stream));
        c->stage_head = 0;
    }
    std::memcpy(c->stage_host + c->stage_head, src, bytes);
    HIPC(c, hipMemcpyAsync(c->stage_dev + c->stage_head, c->stage_host + c->stage_head, need,
                           hipMemcpyHostToDevice, c->stream));
    *out = c->stage_dev + c->stage_head;
    c->stage_head += need;
    return SLM_OK;
}

// Reallocations of internal buffers happen between launches only: recorded work that
// may point at the old buffer runs first, and graphs that do are dropped.
int internal_realloc(slm_hip* c, void** p, size_t bytes) {
    int rc = taint(c);
    if (rc) return rc;
    drop_graphs(c);
    HIPC(c, hipStreamSynchronize(c->stream));
    if (*p) HIPC(c, hipFree(*p));
    *p = nullptr;
    HIPC(c, hipMalloc(p, bytes));
    return SLM_OK;
}

int need_ws(slm_hip* c, size_t bytes) {
    if (bytes <= c->ws_bytes) return SLM_OK;
    size_t nb = std::max(bytes, c->ws_bytes * 2);
    int rc = internal_realloc(c, (void**)&c->ws, nb);
    if (rc) return rc;
    c->ws_bytes = nb;
    return SLM_OK;
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
    } fns[] = {{&k.copy, "slm_copy"},
               {&k.add, "slm_add"},
               {&k.add_row, "slm_add_row"},
               {&k.mix, "slm_mix"},
               {&k.silu_mul, "slm_silu_mul"},
               {&k.scale_rows, "slm_scale_rows"},
               {&k.shift, "slm_shift"},
               {&k.columns, "slm_columns"},
               {&k.gather, "slm_gather"},
               {&k.store, "slm_store"},
               {&k.rope, "slm_rope"},
               {&k.rope_table, "slm_rope_table"},
               {&k.rms, "slm_rms"},
               {&k.l2norm, "slm_l2norm"},
               {&k.fill, "slm_fill"},
               {&k.combine, "slm_attn_combine"},
               {&k.probe, "slm_probe_mfma"},
               {&k.lin_small[0], "slm_linear_small_s"},
               {&k.lin_small[1], "slm_linear_small_v"},
               {&k.lin_big[0], "slm_linear_big_s"},
               {&k.lin_big[1], "slm_linear_big_v"},
               {&k.gla[0], "slm_gla_1"},
               {&k.gla[1], "slm_gla_2"},
               {&k.gla[2], "slm_gla_4"},
               {&k.gla[3], "slm_gla_8"},
               {&k.gla[4], "slm_gla_16"},
               {&k.gla[5], "slm_gla_32"},
               {&k.gla[6], "slm_gla_64"},
               {&k.attn[0], "slm_attn_part_1"},
               {&k.attn[1], "slm_attn_part_2"},
               {&k.attn[2], "slm_attn_part_4"},
               {&k.attn[3], "slm_attn_part_8"},
               {&k.attn[4], "slm_attn_part_16"}};
    for (auto& f : fns) {
        int rc = get_fn(c, f.f, f.n);
        if (rc) return rc;
    }
    return SLM_OK;
}

int fill(slm_hip* c, float* y, size_t n, float v) {
    return go(c, c->k.fill, blocks_for(n), 1, 1, 256, 0, y, (long long)n, v);
}

int pow2_index(size_t need, int maxi) {  // smallest i with 2^i >= need
    int i = 0;
    while (i < maxi && ((size_t)1 << i) < need) i++;
    return i;
}

// Captures the recorded step into a graph, or finds one that matches it.
int finish_step(slm_hip* c) {
    c->recording = false;
    if (c->tainted) {
        c->tainted = false;
        return SLM_OK;
    }
    int rc = upload_dyn(c);
    if (rc) return rc;
    c->clock++;
    for (auto& g : c->cache) {
        if (g.recs.size() == c->recs.size() && g.ndyn == c->dyn.size() &&
            std::memcmp(g.recs.data(), c->recs.data(), c->recs.size() * sizeof(Rec)) == 0) {
            g.used = c->clock;
            HIPC(c, hipGraphLaunch(g.exec, c->stream));
            c->n_launched++;
            return SLM_OK;
        }
    }
    if (c->cache.size() >= MAX_GRAPHS) {
        auto old = std::min_element(c->cache.begin(), c->cache.end(),
                                    [](const Graph& a, const Graph& b) { return a.used < b.used; });
        HIPC(c, hipStreamSynchronize(c->stream));
        hipGraphExecDestroy(old->exec);
        c->cache.erase(old);
    }
    Graph g;
    g.recs = c->recs;
    g.ndyn = c->dyn.size();
    g.used = c->clock;
    hipGraph_t graph = nullptr;
    HIPC(c, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
    for (auto& r : g.recs) {
        rc = launch_now(c, r);
        if (rc) {
            hipStreamEndCapture(c->stream, &graph);
            if (graph) hipGraphDestroy(graph);
            return rc;
        }
    }
    HIPC(c, hipStreamEndCapture(c->stream, &graph));
    hipError_t e = hipGraphInstantiate(&g.exec, graph, nullptr, nullptr, 0);
    hipGraphDestroy(graph);
    if (e != hipSuccess) return fail(c, SLM_E_HIP, "hipGraphInstantiate: %s", hipGetErrorString(e));
    HIPC(c, hipGraphLaunch(g.exec, c->stream));
    c->n_captured++;
    c->n_launched++;
    c->cache.push_back(std::move(g));
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
        return bail(fail(c, SLM_E_UNSUPPORTED, "device %d is %s; this build is for gfx950",
                         device, prop.gcnArchName));
    OPEN_HIP(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
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
    c->ws_bytes = 1 << 20;
    OPEN_HIP(hipMalloc((void**)&c->ws, c->ws_bytes));
    c->dyn.reserve(DYN_CAP);
    c->recs.reserve(4096);
    const char* env = getenv("SLM_HIP_GRAPHS");
    if (env && env[0] == '0') c->graphs_on = false;
#undef OPEN_HIP
    *out = c;
    return SLM_OK;
}

void slm_hip_close(slm_hip* c) {
    if (!c) return;
    if (c->stream) hipStreamSynchronize(c->stream);
    for (auto& g : c->cache)
        if (g.exec) hipGraphExecDestroy(g.exec);
    for (auto& t : c->tables) {
        hipFree(t.second.cos);
        hipFree(t.second.sin);
    }
    for (auto& a : c->allocs) hipFree((void*)a.first);
    if (c->ws) hipFree(c->ws);
    if (c->stage_dev) hipFree(c->stage_dev);
    if (c->dyn_dev) hipFree(c->dyn_dev);
    if (c->stage_host) hipHostFree(c->stage_host);
    if (c->bounce) hipHostFree(c->bounce);
    for (int i = 0; i < 2; i++) {
        if (c->dyn_pin[i]) hipHostFree(c->dyn_pin[i]);
        if (c->dyn_ev[i]) hipEventDestroy(c->dyn_ev[i]);
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
    hipError_t e = hipMalloc((void**)&p, bytes);
    if (e != hipSuccess) return fail(c, SLM_E_MEMORY, "alloc %zu floats: %s", n, hipGetErrorString(e));
    // zeroed on the stream now, ordered before any later use of the buffer (also before
    // the launches of a step being recorded, which run at flush)
    Rec r;
    r.f = c->k.fill;
    r.gx = blocks_for(bytes / 4);
    r.gy = r.gz = 1;
    r.bx = 256;
    r.shmem = 0;
    r.nargs = 0;
    std::memset(r.args, 0, sizeof r.args);
    pack(r, p, (long long)(bytes / 4), 0.0f);
    int rc = launch_now(c, r);
    if (rc) {
        hipFree(p);
        return rc;
    }
    c->allocs[(uintptr_t)p] = bytes;
    *out = p;
    return SLM_OK;
}

int slm_hip_free(slm_hip* c, float* p) {
    if (!c) return SLM_E_INVALID;
    if (!p) return SLM_OK;
    auto it = c->allocs.find((uintptr_t)p);
    if (it == c->allocs.end()) return fail(c, SLM_E_BOUNDS, "free: %p was not allocated here", (void*)p);
    int rc = taint(c);
    if (rc) return rc;
    drop_graphs(c);
    c->allocs.erase(it);
    HIPC(c, hipStreamSynchronize(c->stream));
    HIPC(c, hipFree(p));
    return SLM_OK;
}

int slm_hip_upload(slm_hip* c, float* dst, const float* src, size_t n) {
    if (!c || (n && !src)) return SLM_E_INVALID;
    NEED(c, "upload", dst, n);
    if (n == 0) return SLM_OK;
    int rc = taint(c);
    if (rc) return rc;
    for (auto it = c->tables.begin(); it != c->tables.end();) {  // inv_freq rewritten
        if (it->first >= (uintptr_t)dst && it->first < (uintptr_t)(dst + n)) {
            drop_graphs(c);
            hipFree(it->second.cos);
            hipFree(it->second.sin);
            it = c->tables.erase(it);
        } else {
            ++it;
        }
    }
    HIPC(c, hipStreamSynchronize(c->stream));
    HIPC(c, hipMemcpy(dst, src, n * 4, hipMemcpyHostToDevice));
    return SLM_OK;
}

int slm_hip_read(slm_hip* c, float* host, const float* dev, size_t n) {
    if (!c || (n && !host)) return SLM_E_INVALID;
    NEED(c, "read", dev, n);
    int rc = taint(c);
    if (rc) return rc;
    size_t done = 0;
    while (done < n) {
        size_t part = std::min(n - done, BOUNCE_CAP / 4);
        HIPC(c, hipMemcpyAsync(c->bounce, dev + done, part * 4, hipMemcpyDeviceToHost, c->stream));
        HIPC(c, hipStreamSynchronize(c->stream));
        std::memcpy(host + done, c->bounce, part * 4);
        done += part;
    }
    if (n == 0) HIPC(c, hipStreamSynchronize(c->stream));
    return SLM_OK;
}

int slm_hip_flush(slm_hip* c, const float* const* keep, size_t nkeep) {
    (void)keep;
    (void)nkeep;
    if (!c) return SLM_E_INVALID;
    if (c->recording) return finish_step(c);
    return SLM_OK;
}

int slm_hip_set_graphs(slm_hip* c, int on) {
    if (!c) return SLM_E_INVALID;
    if (c->recording) {
        int rc = finish_step(c);
        if (rc) return rc;
    }
    c->graphs_on = on != 0;
    return SLM_OK;
}

int slm_hip_graph_stats(slm_hip* c, uint64_t* launched, uint64_t* captured, uint64_t* eager) {
    if (!c) return SLM_E_INVALID;
    if (launched) *launched = c->n_launched;
    if (captured) *captured = c->n_captured;
    if (eager) *eager = c->n_eager;
    return SLM_OK;
}

// ---- element-wise operations ----

int slm_hip_copy(slm_hip* c, float* y, const float* x, size_t n) {
    if (!c) return SLM_E_INVALID;
    NEED(c, "copy", y, n);
    NEED(c, "copy", x, n);
    if (!n) return SLM_OK;
    return go(c, c->k.copy, blocks_for(n), 1, 1, 256, 0, y, x, (long long)n);
}

int slm_hip_add(slm_hip* c, float* y, const float* a, const float* b, size_t n) {
    if (!c) return SLM_E_INVALID;
    NEED(c, "add", y, n);
    NEED(c, "add", a, n);
    NEED(c, "add", b, n);
    if (!n) return SLM_OK;
    return go(c, c->k.add, blocks_for(n), 1, 1, 256, 0, y, a, b, (long long)n);
}

int slm_hip_add_row(slm_hip* c, float* y, const float* x, const float* row, size_t m, size_t d) {
    if (!c) return SLM_E_INVALID;
    NEED(c, "add_row", y, m * d);
    NEED(c, "add_row", x, m * d);
    NEED(c, "add_row", row, d);
    if (!m || !d) return SLM_OK;
    return go(c, c->k.add_row, blocks_for(m * d), 1, 1, 256, 0, y, x, row, (long long)(m * d),
              (long long)d);
}

int slm_hip_mix(slm_hip* c, float* y, const float* a, const float* b, size_t n, float t) {
    if (!c) return SLM_E_INVALID;
    NEED(c, "mix", y, n);
    NEED(c, "mix", a, n);
    NEED(c, "mix", b, n);
    if (!n) return SLM_OK;
    return go(c, c->k.mix, blocks_for(n), 1, 1, 256, 0, y, a, b, (long long)n, t);
}

int slm_hip_silu_mul(slm_hip* c, float* y, const float* g, const float* u, size_t n) {
    if (!c) return SLM_E_INVALID;
    NEED(c, "silu_mul", y, n);
    NEED(c, "silu_mul", g, n);
    NEED(c, "silu_mul", u, n);
    if (!n) return SLM_OK;
    return go(c, c->k.silu_mul, blocks_for(n), 1, 1, 256, 0, y, g, u, (long long)n);
}

int slm_hip_scale_rows(slm_hip* c, float* y, const float* x, const float* f, size_t m, size_t d) {
    if (!c || (m && !f)) return SLM_E_INVALID;
    NEED(c, "scale_rows", y, m * d);
    NEED(c, "scale_rows", x, m * d);
    if (!m || !d) return SLM_OK;
    const void* fd = nullptr;
    float f0 = 0.0f;
    if (m == 1 && !(c->recording && !c->tainted)) {
        f0 = f[0];
    } else {
        int rc = stage(c, f, m * 4, &fd);
        if (rc) return rc;
    }
    return go(c, c->k.scale_rows, blocks_for(m * d), 1, 1, 256, 0, y, x, (const float*)fd, f0,
              (long long)(m * d), (long long)d);
}

int slm_hip_shift(slm_hip* c, float* y, const float* first, const float* x, size_t m, size_t d) {
    if (!c) return SLM_E_INVALID;
    if (!m) return SLM_OK;
    NEED(c, "shift", y, m * d);
    NEED(c, "shift", first, d);
    NEED(c, "shift", x, (m - 1) * d);
    if (!d) return SLM_OK;
    return go(c, c->k.shift, blocks_for(m * d), 1, 1, 256, 0, y, first, x, (long long)(m * d),
              (long long)d);
}

int slm_hip_columns(slm_hip* c, float* y, const float* x, size_t m, size_t stride, size_t off,
                    size_t len) {
    if (!c) return SLM_E_INVALID;
    if (!m || !len) return SLM_OK;
    if (off + len > stride) return fail(c, SLM_E_INVALID, "columns: off + len > stride");
    NEED(c, "columns", y, m * len);
    NEED(c, "columns", x, (m - 1) * stride + off + len);
    return go(c, c->k.columns, blocks_for(m * len), 1, 1, 256, 0, y, x, (long long)(m * len),
              (long long)stride, (long long)off, (long long)len);
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
    const void* dv = nullptr;
    int rc = stage(c, v.data(), m * 8, &dv);
    if (rc) return rc;
    return go(c, c->k.gather, blocks_for(m * d), 1, 1, 256, 0, y, w, (const long long*)dv,
              (long long)(m * d), (long long)d);
}

int slm_hip_store(slm_hip* c, float* cache, const float* src, size_t pos, size_t m, size_t cap,
                  size_t heads, size_t dh) {
    if (!c) return SLM_E_INVALID;
    if (!m || !heads || !dh) return SLM_OK;
    if (!cap) return fail(c, SLM_E_INVALID, "store: cap is 0");
    NEED(c, "store", cache, heads * cap * dh);
    NEED(c, "store", src, m * heads * dh);
    const void* dp = nullptr;
    long long p = (long long)pos;
    if (c->recording && !c->tainted) {
        int rc = stage(c, &p, 8, &dp);
        if (rc) return rc;
    }
    return go(c, c->k.store, blocks_for(m * heads * dh), 1, 1, 256, 0, cache, src,
              (const long long*)dp, dp ? 0LL : p, (long long)(m * heads * dh), (long long)cap,
              (long long)heads, (long long)dh);
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
    return go(c, c->k.rope, blocks_for(m * heads * dh / 2), 1, 1, 256, 0, y, x, cs, sn,
              (long long)m, (long long)heads, (long long)dh);
}

int slm_hip_rope_table(slm_hip* c, float* cs, float* sn, const float* inv, size_t pos, size_t m,
                       size_t half) {
    if (!c) return SLM_E_INVALID;
    NEED(c, "rope_table", cs, m * half);
    NEED(c, "rope_table", sn, m * half);
    NEED(c, "rope_table", inv, half);
    // the first call of every advance (model.rs:566) begins a step
    if (c->graphs_on) {
        if (c->recording) {
            int rc = finish_step(c);
            if (rc) return rc;
        }
        c->recording = true;
        c->tainted = false;
        c->recs.clear();
        c->dyn.clear();
    }
    if (!m || !half) return SLM_OK;
    Table& t = c->tables[(uintptr_t)inv];
    if (t.inv.size() != half) {  // first sight of this inv_freq buffer
        int rc = taint(c);
        if (rc) return rc;
        t.inv.assign(half, 0.0f);
        HIPC(c, hipStreamSynchronize(c->stream));
        HIPC(c, hipMemcpy(t.inv.data(), inv, half * 4, hipMemcpyDeviceToHost));
        t.rows = 0;
    }
    if (pos + m > t.rows) {
        size_t rows = std::max<size_t>({pos + m, t.rows * 2, 8192});
        // cpu.rs:228-236: angle (pos + i) as f32 times inv[j], then libm cos/sin
        std::vector<float> hc(rows * half), hs(rows * half);
        for (size_t p = 0; p < rows; p++) {
            float fp = (float)p;
            for (size_t j = 0; j < half; j++) {
                float a = fp * t.inv[j];
                hc[p * half + j] = cosf(a);
                hs[p * half + j] = sinf(a);
            }
        }
        int rc = internal_realloc(c, (void**)&t.cos, rows * half * 4);
        if (!rc) rc = internal_realloc(c, (void**)&t.sin, rows * half * 4);
        if (rc) return rc;
        HIPC(c, hipMemcpy(t.cos, hc.data(), rows * half * 4, hipMemcpyHostToDevice));
        HIPC(c, hipMemcpy(t.sin, hs.data(), rows * half * 4, hipMemcpyHostToDevice));
        t.rows = rows;
    }
    const void* dp = nullptr;
    long long p = (long long)pos;
    if (c->recording && !c->tainted) {
        int rc = stage(c, &p, 8, &dp);
        if (rc) return rc;
    }
    return go(c, c->k.rope_table, blocks_for(m * half), 1, 1, 256, 0, cs, sn,
              (const float*)t.cos, (const float*)t.sin, (const long long*)dp, dp ? 0LL : p,
              (long long)(m * half), (long long)half);
}

// ---- normalisation ----

static int norm_launch(slm_hip* c, hipFunction_t f, float* y, const float* x, const float* w,
                size_t groups, size_t size, float eps, bool rms) {
    if (!fits_int(groups) || !fits_int(size) || groups * size > (size_t)INT_MAX)
        return fail(c, SLM_E_UNSUPPORTED, "%s: %zu groups of %zu", rms ? "rms" : "l2norm", groups, size);
    size_t stride = size | 1;
    size_t G = std::min<size_t>(16, std::max<size_t>(1, 16384 / stride));
    if (G * stride * 4 > 65536) return fail(c, SLM_E_UNSUPPORTED, "norm: size %zu is above 16383", size);
    uint32_t blocks = (uint32_t)((groups + G - 1) / G);
    uint32_t shmem = (uint32_t)(G * stride * 4);
    if (rms) return go(c, f, blocks, 1, 1, 256, shmem, y, x, w, (int)groups, (int)size, eps, (int)G);
    return go(c, f, blocks, 1, 1, 256, shmem, y, x, (int)groups, (int)size, (int)G);
}

int slm_hip_rms(slm_hip* c, float* y, const float* x, const float* w, size_t groups, size_t size,
                float eps) {
    if (!c) return SLM_E_INVALID;
    NEED(c, "rms", y, groups * size);
    NEED(c, "rms", x, groups * size);
    NEED(c, "rms", w, size);
    if (!groups || !size) return SLM_OK;
    return norm_launch(c, c->k.rms, y, x, w, groups, size, eps, true);
}

int slm_hip_l2norm(slm_hip* c, float* y, const float* x, size_t heads, size_t dh) {
    if (!c) return SLM_E_INVALID;
    NEED(c, "l2norm", y, heads * dh);
    NEED(c, "l2norm", x, heads * dh);
    if (!heads || !dh) return SLM_OK;
    return norm_launch(c, c->k.l2norm, y, x, nullptr, heads, dh, 0.0f, false);
}

// ---- linear ----

int slm_hip_linear(slm_hip* c, float* y, const float* w, size_t rows, size_t cols,
                   const float* x, size_t m) {
    if (!c) return SLM_E_INVALID;
    NEED(c, "linear", y, m * rows);
    NEED(c, "linear", w, rows * cols);
    NEED(c, "linear", x, m * cols);
    if (!m || !rows) return SLM_OK;
    if (!cols) return fill(c, y, m * rows, 0.0f);
    if (!fits_int(rows) || !fits_int(cols) || !fits_int(m))
        return fail(c, SLM_E_UNSUPPORTED, "linear: %zu x %zu x %zu", rows, cols, m);
    int vec = (cols % 4 == 0 && aligned16(w) && aligned16(x)) ? 1 : 0;
    size_t kblocks = (cols + 15) / 16, nsl = (kblocks + 15) / 16;
    if (m <= 16 && nsl <= 64) {
        uint32_t waves = (uint32_t)std::min<size_t>(nsl, 8);
        return go(c, c->k.lin_small[vec], (uint32_t)((rows + 15) / 16), 1, 1, 64 * waves,
                  (uint32_t)(nsl * 1024), y, w, x, (int)rows, (int)cols, (int)m);
    }
    return go(c, c->k.lin_big[vec], (uint32_t)((rows + 63) / 64), (uint32_t)((m + 63) / 64), 1,
              256, 0, y, w, x, (int)rows, (int)cols, (int)m);
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
    int i = pow2_index((dh + 3) / 4, 6);
    size_t threads = heads * dh * 4;
    return go(c, c->k.gla[i], (uint32_t)((threads + 255) / 256), 1, 1, 256, 0, y, s, q, k, v,
              decay, bias, (int)m, (int)heads, (int)dh);
}

// ---- attention ----

int slm_hip_attend(slm_hip* c, float* y, float* scores, const float* q, const float* k,
                   const float* v, const slm_attn* a) {
    (void)scores;  // the trait's scratch: this backend keeps its own workspace
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
    NEED(c, "attend", k, kh * cap * dh);
    NEED(c, "attend", v, kh * cap * dh);
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
        nsb = (size_t)((reach + (long long)m - 2) / 512 + 2);
    } else {
        long long first = reach - 1 > pos ? 0 : pos - (reach - 1);
        long long last = pos + (long long)m - 1 - gap;
        nsb = last >= first ? (size_t)(last / 512 - first / 512 + 1) : 1;
    }
    int dti = pow2_index((dh + 15) / 16, 4);
    size_t dp = (size_t)16 << dti;
    size_t wpp = 8;
    while (wpp > 1 && wpp * 16 * (dp + 2) * 4 > 65536) wpp /= 2;
    size_t qpt = 16 / group;
    size_t qtiles = (m + qpt - 1) / qpt;
    size_t part_floats = nsb * m * heads * (dp + 2);
    int rc = need_ws(c, part_floats * 4);
    if (rc) return rc;
    const void* dpos = nullptr;
    if (c->recording && !c->tainted) {
        rc = stage(c, &pos, 8, &dpos);
        if (rc) return rc;
    }
    if (qtiles > UINT32_MAX || nsb > 65535)
        return fail(c, SLM_E_UNSUPPORTED, "attend: %zu query tiles x %zu superblocks", qtiles, nsb);
    rc = go(c, c->k.attn[dti], (uint32_t)qtiles, (uint32_t)kh, (uint32_t)nsb, 512,
            (uint32_t)(wpp * 16 * (dp + 2) * 4), c->ws, q, k, v, (const long long*)dpos,
            dpos ? 0LL : pos, (int)m, reach, gap, (long long)cap, (int)heads, (int)kh, (int)dh,
            a->scale, (int)wpp);
    if (rc) return rc;
    return go(c, c->k.combine, blocks_for(m * heads * dh), 1, 1, 256, 0, y, (const float*)c->ws,
              (int)m, (int)heads, (int)dh, (int)dp, (int)nsb);
}

// ---- diagnostics ----

int slm_hip_stream(slm_hip* c, void** out) {
    if (!c || !out) return SLM_E_INVALID;
    *out = (void*)c->stream;
    return SLM_OK;
}

// Runs one 16x16x4 f32 MFMA on lane inputs a[64], b[64] (device) into out[256].
int slm_hip_probe_mfma(slm_hip* c, float* out, const float* a, const float* b) {
    if (!c) return SLM_E_INVALID;
    NEED(c, "probe", out, 256);
    NEED(c, "probe", a, 64);
    NEED(c, "probe", b, 64);
    return go(c, c->k.probe, 1, 1, 1, 64, 0, out, a, b);
}

}  // extern "C"
