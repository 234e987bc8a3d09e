// The model twin: src/model.rs restated in C++ over the C ABI of slm_hip.h.
//
// `Ops` below is the C++ counterpart of a Rust `impl Ops for Hip` (what src/hip.rs would
// be): a buffer is a device pointer with a length, an `At` view is pointer + offset, and
// outputs grow only, as src/cuda.rs:122-127 sizes them. `Model` then makes exactly the
// calls of src/model.rs, in the same order, with the same swaps.

#include <algorithm>
#include <cmath>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <emmintrin.h>
#include <limits>
#include <map>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "slm_model.h"

namespace {

// ---------------------------------------------------------------------------------------
// JSON (config.json and the safetensors header)
// ---------------------------------------------------------------------------------------

struct Json {
    enum Type { NUL, BOOL, NUM, STR, ARR, OBJ } type = NUL;
    double num = 0;
    bool b = false;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;
    const Json* get(const std::string& k) const {
        for (auto& kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
};

struct Parser {
    const char* p;
    const char* end;
    void ws() {
        while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) p++;
    }
    [[noreturn]] void bad(const char* what) { throw std::runtime_error(std::string("json: ") + what); }
    char peek() {
        ws();
        if (p >= end) bad("unexpected end");
        return *p;
    }
    void expect(char ch) {
        if (peek() != ch) bad("unexpected character");
        p++;
    }
    std::string string() {
        expect('"');
        std::string s;
        while (p < end && *p != '"') {
            if (*p == '\\') {
                p++;
                if (p >= end) bad("bad escape");
                char e = *p++;
                switch (e) {
                    case 'n': s += '\n'; break;
                    case 't': s += '\t'; break;
                    case 'r': s += '\r'; break;
                    case 'b': s += '\b'; break;
                    case 'f': s += '\f'; break;
                    case 'u': {
                        if (end - p < 4) bad("bad \\u");
                        unsigned v = std::stoul(std::string(p, 4), nullptr, 16);
                        p += 4;
                        if (v < 0x80) {
                            s += (char)v;
                        } else if (v < 0x800) {
                            s += (char)(0xC0 | (v >> 6));
                            s += (char)(0x80 | (v & 0x3F));
                        } else {
                            s += (char)(0xE0 | (v >> 12));
                            s += (char)(0x80 | ((v >> 6) & 0x3F));
                            s += (char)(0x80 | (v & 0x3F));
                        }
                        break;
                    }
                    default: s += e;
                }
            } else {
                s += *p++;
            }
        }
        if (p >= end) bad("unterminated string");
        p++;
        return s;
    }
    Json value() {
        Json j;
        char ch = peek();
        if (ch == '{') {
            p++;
            j.type = Json::OBJ;
            if (peek() == '}') {
                p++;
                return j;
            }
            for (;;) {
                std::string k = string();
                expect(':');
                j.obj.emplace_back(k, value());
                if (peek() == ',') {
                    p++;
                    continue;
                }
                expect('}');
                return j;
            }
        }
        if (ch == '[') {
            p++;
            j.type = Json::ARR;
            if (peek() == ']') {
                p++;
                return j;
            }
            for (;;) {
                j.arr.push_back(value());
                if (peek() == ',') {
                    p++;
                    continue;
                }
                expect(']');
                return j;
            }
        }
        if (ch == '"') {
            j.type = Json::STR;
            j.str = string();
            return j;
        }
        if (!std::strncmp(p, "true", 4) && end - p >= 4) {
            p += 4;
            j.type = Json::BOOL;
            j.b = true;
            return j;
        }
        if (!std::strncmp(p, "false", 5) && end - p >= 5) {
            p += 5;
            j.type = Json::BOOL;
            return j;
        }
        if (!std::strncmp(p, "null", 4) && end - p >= 4) {
            p += 4;
            return j;
        }
        char* e = nullptr;
        std::string tok(p, std::min<ptrdiff_t>(end - p, 64));
        j.num = std::strtod(tok.c_str(), &e);
        if (e == tok.c_str()) bad("bad value");
        p += e - tok.c_str();
        j.type = Json::NUM;
        return j;
    }
};

Json parse_json(const std::string& text) {
    Parser ps{text.data(), text.data() + text.size()};
    return ps.value();
}

std::string read_file(const std::string& path) {
    FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) throw std::runtime_error("reading " + path + ": cannot open");
    std::string s;
    char buf[1 << 16];
    size_t n;
    while ((n = std::fread(buf, 1, sizeof buf, f)) > 0) s.append(buf, n);
    std::fclose(f);
    return s;
}

// ---------------------------------------------------------------------------------------
// src/config.rs:20-105
// ---------------------------------------------------------------------------------------

struct Config {
    size_t vocab_size = 0, d_model = 0, n_heads = 0, global_kv_heads = 4;
    float global_rope_base = 0;
    uint32_t global_logn = 0, global_kshift = 0, global_emb = 0, global_far = 0;
    std::string prelude, core, coda;
    size_t window = 0, max_loops = 0, default_loops = 0;
    uint32_t loop_lora = 0, state_loops = 0;
    float damp = 1.0f, rope_base = 0, norm_eps = 0;
    size_t head_dim() const { return d_model / n_heads; }

    static Config load(const std::string& dir) {
        std::string path = dir + "/config.json";
        Json j = parse_json(read_file(path));
        Config c;
        auto num = [&](const char* k, bool required) -> const Json* {
            const Json* v = j.get(k);
            if (!v) {
                if (required) throw std::runtime_error("parsing " + path + ": missing " + k);
                return nullptr;
            }
            if (v->type != Json::NUM) throw std::runtime_error("parsing " + path + ": " + k + " is not a number");
            return v;
        };
        auto str = [&](const char* k) {
            const Json* v = j.get(k);
            if (!v || v->type != Json::STR) throw std::runtime_error("parsing " + path + ": missing " + k);
            return v->str;
        };
        auto sz = [&](const char* k, size_t dflt, bool req) {
            const Json* v = num(k, req);
            return v ? (size_t)v->num : dflt;
        };
        c.vocab_size = sz("vocab_size", 0, true);
        c.d_model = sz("d_model", 0, true);
        c.n_heads = sz("n_heads", 0, true);
        c.global_kv_heads = sz("global_kv_heads", 4, false);
        if (const Json* v = num("global_rope_base", false)) c.global_rope_base = (float)v->num;
        c.global_logn = (uint32_t)sz("global_logn", 0, false);
        c.global_kshift = (uint32_t)sz("global_kshift", 0, false);
        c.global_emb = (uint32_t)sz("global_emb", 0, false);
        c.global_far = (uint32_t)sz("global_far", 0, false);
        c.prelude = str("prelude");
        c.core = str("core");
        c.coda = str("coda");
        c.window = sz("window", 0, true);
        c.max_loops = sz("max_loops", 0, true);
        c.default_loops = sz("default_loops", 0, true);
        c.loop_lora = (uint32_t)sz("loop_lora", 0, false);
        c.state_loops = (uint32_t)sz("state_loops", 0, false);
        if (const Json* v = num("damp", false)) c.damp = (float)v->num;
        c.rope_base = (float)num("rope_base", true)->num;
        c.norm_eps = (float)num("norm_eps", true)->num;
        if (c.loop_lora != 0) throw std::runtime_error("loop_lora models are not supported");
        if (c.state_loops != 0) throw std::runtime_error("state_loops models are not supported");
        if (c.global_rope_base != 0.0f) throw std::runtime_error("global_rope_base is not supported");
        if (!c.n_heads || c.d_model % c.n_heads)
            throw std::runtime_error("d_model is not a multiple of n_heads");
        return c;
    }

    size_t loops(size_t n) const {  // config.rs:96-105 (n == 0: the default)
        if (core.empty()) return 0;
        if (n == 0) n = default_loops;
        if (n < 1 || n > max_loops)
            throw std::runtime_error("loops must be between 1 and " + std::to_string(max_loops));
        return n;
    }
};

// ---------------------------------------------------------------------------------------
// The Ops binding (the C++ counterpart of a Rust `impl Ops for Hip`)
// ---------------------------------------------------------------------------------------

struct SlmError : std::runtime_error {
    int code;
    SlmError(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

struct Buf {
    float* p = nullptr;
    size_t n = 0;
};

struct At {
    const Buf* b;
    size_t off;
};
At at(const Buf& b, size_t off) { return At{&b, off}; }

class Ops {
  public:
    explicit Ops(slm_hip* c) : c_(c) {}
    slm_hip* ctx() const { return c_; }

    void ok(int rc, const char* op) const {
        if (rc != SLM_OK)
            throw SlmError(rc, std::string(op) + ": " + slm_hip_last_error(c_));
    }
    // cuda.rs:59-61: a view must lie inside its buffer
    const float* view(At x, size_t n, const char* op) const {
        if (x.off + n > x.b->n)
            throw SlmError(SLM_E_BOUNDS, std::string(op) + ": view past the end of a buffer");
        return x.b->p + x.off;
    }
    Buf zeros(size_t n) const {  // ops.rs:72, cuda.rs:152-154
        Buf b;
        ok(slm_hip_alloc(c_, n, &b.p), "zeros");
        b.n = std::max<size_t>(n, 1);
        return b;
    }
    Buf upload(const float* data, size_t n) const {  // ops.rs:77
        Buf b = zeros(n);
        ok(slm_hip_upload(c_, b.p, data, n), "upload");
        return b;
    }
    // ops.rs:73-76 zeros_cache (a [heads][cap][dh] cache; fp16 in fp16 mode, slm_hip.h)
    Buf zeros_cache(size_t heads, size_t cap, size_t dh) const {
        Buf b;
        ok(slm_hip_alloc_cache(c_, heads, cap, dh, &b.p), "zeros_cache");
        b.n = std::max<size_t>(heads * cap * dh, 1);
        return b;
    }
    // ops.rs:79-88 upload_cache
    Buf upload_cache(const float* data, size_t heads, size_t cap, size_t dh) const {
        Buf b = zeros_cache(heads, cap, dh);
        ok(slm_hip_upload(c_, b.p, data, heads * cap * dh), "upload_cache");
        return b;
    }
    void release(Buf& b) const {
        if (b.p) slm_hip_free(c_, b.p);
        b = Buf{};
    }
    // cuda.rs:122-127: outputs grow only
    void ensure(Buf& y, size_t n) const {
        if (y.n < n) {
            release(y);
            y = zeros(n);
        }
    }
    std::vector<float> read(const Buf& b, size_t n) const {
        std::vector<float> out(n);
        read_into(b, out.data(), n);
        return out;
    }
    void read_into(const Buf& b, float* out, size_t n) const {
        if (n > b.n) throw SlmError(SLM_E_BOUNDS, "read: past the end of a buffer");
        ok(slm_hip_read(c_, out, b.p, n), "read");
    }
    void flush(const std::vector<const Buf*>& keep) const {
        std::vector<const float*> ptrs;
        for (auto* b : keep) ptrs.push_back(b->p);
        ok(slm_hip_flush(c_, ptrs.data(), ptrs.size()), "flush");
    }
    void gather(Buf& y, const Buf& w, const uint32_t* ids, size_t m, size_t d) const {
        ensure(y, m * d);
        ok(slm_hip_gather(c_, y.p, w.p, ids, m, d), "gather");
    }
    void gather_dev(Buf& y, const Buf& w, const Buf& tok, size_t rows, size_t d) const {
        ensure(y, d);
        ok(slm_hip_gather_dev(c_, y.p, w.p, (const long long*)tok.p, rows, d), "gather_dev");
    }
    void argmax(Buf& tok, Buf& ids, size_t slot, const Buf& x, size_t n) const {
        ok(slm_hip_argmax(c_, (long long*)tok.p, (uint32_t*)ids.p, ids.n, slot, x.p, n), "argmax");
    }
    void copy(Buf& y, At x, size_t n) const {
        ensure(y, n);
        ok(slm_hip_copy(c_, y.p, view(x, n, "copy"), n), "copy");
    }
    void shift(Buf& y, const Buf& first, At x, size_t m, size_t d) const {
        ensure(y, m * d);
        ok(slm_hip_shift(c_, y.p, first.p, view(x, (m - 1) * d, "shift"), m, d), "shift");
    }
    void columns(Buf& y, const Buf& x, size_t m, size_t stride, size_t off, size_t len) const {
        ensure(y, m * len);
        ok(slm_hip_columns(c_, y.p, x.p, m, stride, off, len), "columns");
    }
    void linear(Buf& y, const Buf& w, size_t rows, size_t cols, At x, size_t m) const {
        ensure(y, m * rows);
        ok(slm_hip_linear(c_, y.p, w.p, rows, cols, view(x, m * cols, "linear"), m), "linear");
    }
    void add(Buf& y, At a, At b, size_t n) const {
        ensure(y, n);
        ok(slm_hip_add(c_, y.p, view(a, n, "add"), view(b, n, "add"), n), "add");
    }
    void add_row(Buf& y, At x, At row, size_t m, size_t d) const {
        ensure(y, m * d);
        ok(slm_hip_add_row(c_, y.p, view(x, m * d, "add_row"), view(row, d, "add_row"), m, d),
           "add_row");
    }
    void scale_rows(Buf& y, At x, const std::vector<float>& f, size_t d) const {
        size_t m = f.size();
        ensure(y, m * d);
        ok(slm_hip_scale_rows(c_, y.p, view(x, m * d, "scale_rows"), f.data(), m, d), "scale_rows");
    }
    void mix(Buf& y, At a, At b, size_t n, float t) const {
        ensure(y, n);
        ok(slm_hip_mix(c_, y.p, view(a, n, "mix"), view(b, n, "mix"), n, t), "mix");
    }
    void rms(Buf& y, At x, const Buf& w, size_t groups, size_t size, float eps) const {
        ensure(y, groups * size);
        ok(slm_hip_rms(c_, y.p, view(x, groups * size, "rms"), w.p, groups, size, eps), "rms");
    }
    void silu_mul(Buf& y, At g, At u, size_t n) const {
        ensure(y, n);
        ok(slm_hip_silu_mul(c_, y.p, view(g, n, "silu_mul"), view(u, n, "silu_mul"), n), "silu_mul");
    }
    void rope_table(Buf& cs, Buf& sn, const Buf& inv, size_t pos, size_t m, size_t half) const {
        ensure(cs, m * half);
        ensure(sn, m * half);
        ok(slm_hip_rope_table(c_, cs.p, sn.p, inv.p, pos, m, half), "rope_table");
    }
    void rope(Buf& y, At x, const Buf& cs, const Buf& sn, size_t m, size_t heads, size_t dh) const {
        ensure(y, m * heads * dh);
        ok(slm_hip_rope(c_, y.p, view(x, m * heads * dh, "rope"), cs.p, sn.p, m, heads, dh), "rope");
    }
    void l2norm(Buf& y, At x, size_t heads, size_t dh) const {
        ensure(y, heads * dh);
        ok(slm_hip_l2norm(c_, y.p, view(x, heads * dh, "l2norm"), heads, dh), "l2norm");
    }
    void gla(Buf& y, Buf& s, At q, At k, At v, const Buf& decay, const Buf& bias, size_t m,
             size_t heads, size_t dh) const {
        ensure(y, m * heads * dh);
        size_t n = m * heads * dh;
        ok(slm_hip_gla(c_, y.p, s.p, view(q, n, "gla"), view(k, n, "gla"), view(v, n, "gla"),
                       decay.p, bias.p, m, heads, dh),
           "gla");
    }
    void store(Buf& cache, At src, size_t pos, size_t m, size_t cap, size_t heads, size_t dh) const {
        ok(slm_hip_store(c_, cache.p, view(src, m * heads * dh, "store"), pos, m, cap, heads, dh),
           "store");
    }
    void attend(Buf& y, Buf& scores, At q, const Buf& k, const Buf& v, const slm_attn& a) const {
        ensure(y, a.m * a.heads * a.dh);
        ok(slm_hip_attend(c_, y.p, scores.p, view(q, a.m * a.heads * a.dh, "attend"), k.p, v.p, &a),
           "attend");
    }

  private:
    slm_hip* c_;
};

// ---------------------------------------------------------------------------------------
// src/model.rs
// ---------------------------------------------------------------------------------------

constexpr size_t CHUNK = 256;           // model.rs:27
constexpr size_t MAX_SCORES = 1u << 28;  // model.rs:30

struct Mat {
    Buf w;
    size_t rows = 0, cols = 0;
};

enum Kind { WINDOW, LINEAR, GLOBAL };

struct Block {
    Kind kind = WINDOW;
    Buf norm1, norm2;
    Mat up, down;
    Mat qkv, o;                     // S (o shared by all kinds)
    Mat qkvg, decay;                // L
    Buf bias, head_norm;            // L
    Mat q, kv;                      // G
    bool has_norm_e = false;
    Buf norm_e;                     // G
};

struct State {
    Kind kind = WINDOW;
    Buf k, v;      // S ring / G cache
    Buf s;         // L
    Buf prev;      // G
    size_t cap = 0;
    Buf scores;    // G
};

struct Scratch {
    Buf n, mix, q, k, v, g, y, y2, h, t, d, shifted, prev_kv, up, gate, mid, scores, cos, sin;
};

struct Tensor {
    std::vector<size_t> shape;
    const char* data;  // little-endian f32, possibly unaligned
    size_t count;
};

}  // namespace

struct slm_model {
    Ops ops;
    Config cfg;
    std::string error;
    Mat embed;
    std::vector<Block> prelude, core, coda;
    bool looped = false;
    Mat inject, loop_embed;
    Buf norm_f, inv_freq;
    size_t global_cap0 = 1u << 13;  // model.rs:320
    bool device_grow = false;       // grow by device copies instead of model.rs's read + upload
    explicit slm_model(slm_hip* c) : ops(c) {}
};

struct slm_session {
    slm_model* model;
    size_t loops = 0, pos = 0;
    std::vector<State> prelude;
    std::vector<std::vector<State>> core;
    std::vector<State> coda;
    Scratch sc;
    Buf x, s, e0, e_proj, last, logits;
    Buf tok, ids;  // device-side greedy decode: the next token (a long long), the picks (uint32)
};

namespace {

std::string g_load_error;  // the message of the last failed slm_model_load

using Model = slm_model;
using Session = slm_session;

void free_buf(const Ops& ops, Buf& b) { ops.release(b); }

// model.rs:36-54: f32-only safetensors, read through a read-only memory map of the file: the
// header is parsed from the mapping and each tensor is uploaded straight from it (through an
// aligned copy only when its offset is not a multiple of 4 bytes), so loading neither reads
// the file into a buffer first nor keeps more than the mapping.
struct Weights {
    const char* bytes = nullptr;
    size_t size = 0;
    std::map<std::string, Tensor> tensors;

    explicit Weights(const std::string& dir) {
        std::string path = dir + "/model.safetensors";
        int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
        if (fd < 0) throw std::runtime_error("reading " + path + ": cannot open");
        struct stat st;
        if (::fstat(fd, &st) != 0 || st.st_size < 8) {
            ::close(fd);
            throw std::runtime_error(path + ": too short");
        }
        size = (size_t)st.st_size;
        void* m = ::mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
        ::close(fd);
        if (m == MAP_FAILED) throw std::runtime_error(path + ": cannot map");
        bytes = (const char*)m;
        try {
            parse(path);
        } catch (...) {
            ::munmap(m, size);
            throw;
        }
    }
    ~Weights() {
        if (bytes) ::munmap((void*)bytes, size);
    }
    Weights(const Weights&) = delete;
    Weights& operator=(const Weights&) = delete;

    void parse(const std::string& path) {
        uint64_t hl = 0;
        std::memcpy(&hl, bytes, 8);
        if (hl > size - 8) throw std::runtime_error(path + ": bad header length");
        Json h = parse_json(std::string(bytes + 8, hl));
        size_t base = 8 + hl;
        for (auto& kv : h.obj) {
            if (kv.first == "__metadata__") continue;
            const Json* dt = kv.second.get("dtype");
            const Json* sh = kv.second.get("shape");
            const Json* off = kv.second.get("data_offsets");
            if (!dt || !sh || !off || off->arr.size() != 2) throw std::runtime_error(kv.first + ": bad entry");
            if (dt->str != "F32") throw std::runtime_error(kv.first + ": expected f32 weights");
            Tensor t;
            size_t count = 1;
            for (auto& d : sh->arr) {
                t.shape.push_back((size_t)d.num);
                count *= (size_t)d.num;
            }
            size_t a = (size_t)off->arr[0].num, b = (size_t)off->arr[1].num;
            if (b < a || b > size - base || b - a != count * 4)
                throw std::runtime_error(kv.first + ": bad data offsets");
            t.data = bytes + base + a;
            t.count = count;
            tensors[kv.first] = t;
        }
    }
    Tensor take(const std::string& name) {
        auto it = tensors.find(name);
        if (it == tensors.end()) throw std::runtime_error("missing weight " + name);
        Tensor t = it->second;
        tensors.erase(it);
        return t;
    }
};

// model.rs:69-83: one tensor to the device, from the mapping. Always fp32, as model.rs
// uploads it (in fp16 mode the backend keeps fp16 shadows of the weights its linears read).
Buf upload_tensor(const Ops& ops, const Tensor& t) {
    if (((uintptr_t)t.data & 3) == 0) return ops.upload((const float*)t.data, t.count);
    std::vector<float> host(t.count);
    std::memcpy(host.data(), t.data, t.count * 4);
    return ops.upload(host.data(), t.count);
}

Mat mat(const Ops& ops, Weights& w, const std::string& name) {
    Tensor t = w.take(name);
    if (t.shape.size() != 2) throw std::runtime_error(name + ": expected a matrix");
    Mat m;
    m.w = upload_tensor(ops, t);
    m.rows = t.shape[0];
    m.cols = t.shape[1];
    return m;
}

Buf vec(const Ops& ops, Weights& w, const std::string& name) {
    return upload_tensor(ops, w.take(name));
}

// model.rs:114-153
Block load_block(const Model& M, Weights& w, const std::string& prefix, char kind) {
    const Ops& ops = M.ops;
    auto n = [&](const char* s) { return prefix + "." + s; };
    Block b;
    switch (kind) {
        case 'S':
            b.kind = WINDOW;
            b.qkv = mat(ops, w, n("mixer.qkv.weight"));
            b.o = mat(ops, w, n("mixer.o.weight"));
            break;
        case 'L':
            b.kind = LINEAR;
            b.qkvg = mat(ops, w, n("mixer.qkvg.weight"));
            b.decay = mat(ops, w, n("mixer.decay.weight"));
            b.bias = vec(ops, w, n("mixer.decay.bias"));
            b.head_norm = vec(ops, w, n("mixer.head_norm.weight"));
            b.o = mat(ops, w, n("mixer.o.weight"));
            break;
        case 'G':
            b.kind = GLOBAL;
            b.q = mat(ops, w, n("mixer.q.weight"));
            b.kv = mat(ops, w, n("mixer.kv.weight"));
            b.o = mat(ops, w, n("mixer.o.weight"));
            if (M.cfg.global_emb != 0) {
                b.has_norm_e = true;
                b.norm_e = vec(ops, w, n("mixer.norm_e.weight"));
            }
            break;
        default:
            throw std::runtime_error(std::string("unknown layer type ") + kind);
    }
    b.norm1 = vec(ops, w, n("norm1.weight"));
    b.norm2 = vec(ops, w, n("norm2.weight"));
    b.up = mat(ops, w, n("mlp.up.weight"));
    b.down = mat(ops, w, n("mlp.down.weight"));
    return b;
}

// model.rs:226-269
void load(Model& M, const std::string& dir) {
    M.cfg = Config::load(dir);
    Weights w(dir);
    auto blocks = [&](const char* name, const std::string& kinds, std::vector<Block>& out) {
        for (size_t i = 0; i < kinds.size(); i++)
            out.push_back(load_block(M, w, std::string(name) + "." + std::to_string(i), kinds[i]));
    };
    blocks("prelude", M.cfg.prelude, M.prelude);
    blocks("core", M.cfg.core, M.core);
    blocks("coda", M.cfg.coda, M.coda);
    M.looped = !M.cfg.core.empty();
    if (M.looped) {
        M.inject = mat(M.ops, w, "inject_e.weight");
        M.loop_embed = mat(M.ops, w, "loop_embed.weight");
    }
    M.embed = mat(M.ops, w, "embed.weight");
    M.norm_f = vec(M.ops, w, "norm_f.weight");
    size_t dh = M.cfg.head_dim();
    std::vector<float> inv(dh / 2);
    for (size_t i = 0; i < dh / 2; i++)
        inv[i] = 1.0f / std::pow(M.cfg.rope_base, (float)(2 * i) / (float)dh);
    M.inv_freq = M.ops.upload(inv.data(), inv.size());
}

size_t ring_cap(const Model& M) { return M.cfg.window + CHUNK; }  // model.rs:304-306

State new_state(const Model& M, const Block& b) {  // model.rs:308-331
    const Ops& ops = M.ops;
    size_t h = M.cfg.n_heads, dh = M.cfg.head_dim();
    State st;
    st.kind = b.kind;
    switch (b.kind) {
        case WINDOW:
            st.k = ops.zeros_cache(h, ring_cap(M), dh);
            st.v = ops.zeros_cache(h, ring_cap(M), dh);
            break;
        case LINEAR:
            st.s = ops.zeros(h * dh * dh);
            break;
        case GLOBAL:
            st.cap = M.global_cap0;
            st.k = ops.zeros_cache(M.cfg.global_kv_heads, st.cap, dh);
            st.v = ops.zeros_cache(M.cfg.global_kv_heads, st.cap, dh);
            st.prev = ops.zeros(M.cfg.d_model);
            st.scores = ops.zeros(1);
            break;
    }
    return st;
}

void free_state(const Ops& ops, State& st) {
    free_buf(ops, st.k);
    free_buf(ops, st.v);
    free_buf(ops, st.s);
    free_buf(ops, st.prev);
    free_buf(ops, st.scores);
}

// model.rs:333-381
Session* new_session(Model& M, size_t loops_in) {
    size_t loops = M.cfg.loops(loops_in);
    const Ops& ops = M.ops;
    size_t d = M.cfg.d_model, half = M.cfg.head_dim() / 2;
    Session* se = new Session();
    se->model = &M;
    se->loops = loops;
    try {
        for (auto& b : M.prelude) se->prelude.push_back(new_state(M, b));
        for (size_t r = 0; r < loops; r++) {
            se->core.emplace_back();
            for (auto& b : M.core) se->core.back().push_back(new_state(M, b));
        }
        for (auto& b : M.coda) se->coda.push_back(new_state(M, b));
        Scratch& sc = se->sc;
        sc.n = ops.zeros(d);
        sc.mix = ops.zeros(4 * d);
        sc.q = ops.zeros(d);
        sc.k = ops.zeros(d);
        sc.v = ops.zeros(d);
        sc.g = ops.zeros(d);
        sc.y = ops.zeros(d);
        sc.y2 = ops.zeros(d);
        sc.h = ops.zeros(d);
        sc.t = ops.zeros(d);
        sc.d = ops.zeros(M.cfg.n_heads);
        sc.shifted = ops.zeros(d);
        sc.prev_kv = ops.zeros(2 * d);
        sc.up = ops.zeros(4 * d);
        sc.gate = ops.zeros(2 * d);
        sc.mid = ops.zeros(2 * d);
        sc.scores = ops.zeros(1);
        sc.cos = ops.zeros(half);
        sc.sin = ops.zeros(half);
        se->x = ops.zeros(d);
        se->s = ops.zeros(d);
        se->e0 = ops.zeros(d);
        se->e_proj = ops.zeros(d);
        se->last = ops.zeros(d);
        se->logits = ops.zeros(M.cfg.vocab_size);
    } catch (...) {
        delete se;
        throw;
    }
    return se;
}

// A zeroed host array from calloc (large ones come as untouched zero pages).
struct HostFloats {
    float* p;
    explicit HostFloats(size_t n) : p((float*)std::calloc(n ? n : 1, sizeof(float))) {
        if (!p) throw SlmError(SLM_E_MEMORY, "out of host memory");
    }
    ~HostFloats() { std::free(p); }
    HostFloats(const HostFloats&) = delete;
    HostFloats& operator=(const HostFloats&) = delete;
};

// model.rs:383-398: doubles a global cache. By default the reference's own sequence, which a
// Rust `impl Ops for Hip` under an unchanged model.rs issues: `read` each cache (inside the
// advance: the backend runs what the step recorded so far), lay every head's `cap` rows out
// at the start of its `2·cap` rows on the host, `upload_cache` the result and drop the old
// buffer. With `device_grow` set (slm_model_set_device_grow) the same relayout runs on the
// device into a new zeroed cache, queued on the stream (slm_hip_grow_cache: the same
// contents, no host round trip).
void grow(const Model& M, Buf& k, Buf& v, size_t& cap) {
    size_t kh = M.cfg.global_kv_heads, dh = M.cfg.head_dim();
    size_t old = cap, nw = cap * 2;
    for (Buf* buf : {&k, &v}) {
        Buf nb;
        if (M.device_grow) {
            nb = M.ops.zeros_cache(kh, nw, dh);
            M.ops.ok(slm_hip_grow_cache(M.ops.ctx(), nb.p, buf->p, kh, old, dh), "grow");
        } else {
            // host buffers as Rust's vec![0f32; n] gets them (cuda.rs:161, model.rs:389):
            // zeroed pages from calloc, touched only where written or read
            HostFloats data(kh * old * dh), out(kh * nw * dh);
            M.ops.read_into(*buf, data.p, kh * old * dh);
            for (size_t h = 0; h < kh; h++)
                std::copy(data.p + h * old * dh, data.p + (h + 1) * old * dh, out.p + h * nw * dh);
            nb = M.ops.upload_cache(out.p, kh, nw, dh);
        }
        M.ops.release(*buf);
        *buf = nb;
    }
    cap = nw;
}

// model.rs:400-560
void block(const Model& M, const Block& b, State& st, Buf& x, const Buf& e0, Scratch& sc,
           size_t pos, size_t m) {
    const Ops& ops = M.ops;
    const Config& c = M.cfg;
    size_t d = c.d_model, heads = c.n_heads, dh = c.head_dim();
    float eps = c.norm_eps;
    float scale = 1.0f / std::sqrt((float)dh);
    size_t n = m * d;
    ops.rms(sc.n, at(x, 0), b.norm1, m, d, eps);
    // model.rs:417-426: one token needs no copy to split a row
    auto col = [&](Buf& y, const Buf& src, size_t stride, size_t off, size_t len) -> At {
        if (m == 1) return at(src, off);
        ops.columns(y, src, m, stride, off, len);
        return at(y, 0);
    };
    bool has_h = true;
    if (b.kind == WINDOW) {
        ops.linear(sc.mix, b.qkv.w, b.qkv.rows, d, at(sc.n, 0), m);
        At raw = col(sc.y, sc.mix, 3 * d, 0, d);
        ops.rope(sc.q, raw, sc.cos, sc.sin, m, heads, dh);
        raw = col(sc.y, sc.mix, 3 * d, d, d);
        ops.rope(sc.k, raw, sc.cos, sc.sin, m, heads, dh);
        At vals = col(sc.v, sc.mix, 3 * d, 2 * d, d);
        size_t cap = ring_cap(M);
        ops.store(st.k, at(sc.k, 0), pos, m, cap, heads, dh);
        ops.store(st.v, vals, pos, m, cap, heads, dh);
        slm_attn a{pos, m, c.window, 0, cap, heads, heads, dh, scale};
        ops.attend(sc.y, sc.scores, at(sc.q, 0), st.k, st.v, a);
        ops.linear(sc.h, b.o.w, d, d, at(sc.y, 0), m);
    } else if (b.kind == LINEAR) {
        ops.linear(sc.mix, b.qkvg.w, b.qkvg.rows, d, at(sc.n, 0), m);
        At raw = col(sc.y, sc.mix, 4 * d, 0, d);
        ops.l2norm(sc.q, raw, m * heads, dh);
        raw = col(sc.y, sc.mix, 4 * d, d, d);
        ops.l2norm(sc.k, raw, m * heads, dh);
        At vals = col(sc.v, sc.mix, 4 * d, 2 * d, d);
        At gate = col(sc.g, sc.mix, 4 * d, 3 * d, d);
        ops.linear(sc.d, b.decay.w, heads, d, at(sc.n, 0), m);
        ops.gla(sc.y, st.s, at(sc.q, 0), at(sc.k, 0), vals, sc.d, b.bias, m, heads, dh);
        ops.rms(sc.y2, at(sc.y, 0), b.head_norm, m * heads, dh, eps);
        ops.silu_mul(sc.y, gate, at(sc.y2, 0), n);
        ops.linear(sc.h, b.o.w, d, d, at(sc.y, 0), m);
    } else {
        if (b.has_norm_e) {
            ops.rms(sc.t, at(e0, 0), b.norm_e, m, d, eps);
            ops.add(sc.y, at(sc.n, 0), at(sc.t, 0), n);
            std::swap(sc.n, sc.y);
        }
        size_t kh = c.global_kv_heads, kd = c.global_kv_heads * dh;
        ops.linear(sc.q, b.q.w, d, d, at(sc.n, 0), m);
        ops.linear(sc.mix, b.kv.w, 2 * kd, d, at(sc.n, 0), m);
        if (c.global_logn != 0) {
            float lg = std::log((float)c.global_logn);
            std::vector<float> f(m);
            for (size_t i = 0; i < m; i++) f[i] = std::log1p((float)(pos + i)) / lg;
            ops.scale_rows(sc.y, at(sc.q, 0), f, d);
            std::swap(sc.q, sc.y);
        }
        while (pos + m > st.cap) grow(M, st.k, st.v, st.cap);
        At keys;
        if (c.global_kshift != 0) {
            ops.shift(sc.shifted, st.prev, at(sc.n, 0), m, d);
            ops.linear(sc.prev_kv, b.kv.w, 2 * kd, d, at(sc.shifted, 0), m);
            ops.copy(st.prev, at(sc.n, (m - 1) * d), d);
            keys = col(sc.k, sc.prev_kv, 2 * kd, 0, kd);
        } else {
            keys = col(sc.k, sc.mix, 2 * kd, 0, kd);
        }
        At vals = col(sc.v, sc.mix, 2 * kd, kd, kd);
        ops.store(st.k, keys, pos, m, st.cap, kh, dh);
        ops.store(st.v, vals, pos, m, st.cap, kh, dh);
        size_t far = c.global_far != 0 ? c.window : 0;
        if (pos + m > far) {
            slm_attn a{pos, m, std::numeric_limits<size_t>::max(), far, st.cap, heads, kh, dh, scale};
            ops.attend(sc.y, st.scores, at(sc.q, 0), st.k, st.v, a);
            ops.linear(sc.h, b.o.w, d, d, at(sc.y, 0), m);
        } else {
            has_h = false;
        }
    }
    if (has_h) {
        ops.add(sc.t, at(x, 0), at(sc.h, 0), n);
        std::swap(x, sc.t);
    }
    ops.rms(sc.n, at(x, 0), b.norm2, m, d, eps);
    size_t hidden = b.down.cols;
    ops.linear(sc.up, b.up.w, 2 * hidden, d, at(sc.n, 0), m);
    At gate = col(sc.gate, sc.up, 2 * hidden, 0, hidden);
    At amp = col(sc.mid, sc.up, 2 * hidden, hidden, hidden);
    ops.silu_mul(sc.y, gate, amp, m * hidden);
    ops.linear(sc.h, b.down.w, d, hidden, at(sc.y, 0), m);
    ops.add(sc.t, at(x, 0), at(sc.h, 0), n);
    std::swap(x, sc.t);
}

std::vector<const Buf*> kept(const Session& se) {  // model.rs:626-638
    std::vector<const Buf*> keep{&se.logits};
    auto add = [&](const State& st) {
        switch (st.kind) {
            case WINDOW: keep.push_back(&st.k); keep.push_back(&st.v); break;
            case LINEAR: keep.push_back(&st.s); break;
            case GLOBAL: keep.push_back(&st.k); keep.push_back(&st.v); keep.push_back(&st.prev); break;
        }
    };
    for (auto& st : se.prelude) add(st);
    for (auto& r : se.core)
        for (auto& st : r) add(st);
    for (auto& st : se.coda) add(st);
    return keep;
}

// model.rs:563-640
// With `pick` >= 0 (one token, greedy decode on the device) the token comes from se.tok and
// the step ends with the pick of the next one into se.tok and se.ids[pick].
void advance(Model& M, Session& se, const uint32_t* tokens, size_t m, bool want_logits,
             long pick = -1) {
    const Ops& ops = M.ops;
    size_t d = M.cfg.d_model, pos = se.pos;
    if (m == 0 || m > CHUNK) throw SlmError(SLM_E_INVALID, "advance takes 1 to 256 tokens");
    ops.rope_table(se.sc.cos, se.sc.sin, M.inv_freq, pos, m, M.cfg.head_dim() / 2);
    if (pick >= 0)
        ops.gather_dev(se.e0, M.embed.w, se.tok, M.cfg.vocab_size, d);
    else
        ops.gather(se.e0, M.embed.w, tokens, m, d);
    ops.copy(se.x, at(se.e0, 0), m * d);
    for (size_t i = 0; i < M.prelude.size(); i++)
        block(M, M.prelude[i], se.prelude[i], se.x, se.e0, se.sc, pos, m);
    if (M.looped) {
        ops.linear(se.e_proj, M.inject.w, d, d, at(se.x, 0), m);
        ops.copy(se.s, at(se.x, 0), m * d);
        for (size_t r = 0; r < se.loops; r++) {
            ops.add(se.sc.t, at(se.s, 0), at(se.e_proj, 0), m * d);
            ops.add_row(se.x, at(se.sc.t, 0), at(M.loop_embed.w, r * d), m, d);
            for (size_t i = 0; i < M.core.size(); i++)
                block(M, M.core[i], se.core[r][i], se.x, se.e0, se.sc, pos, m);
            if (M.cfg.damp == 1.0f) {
                std::swap(se.s, se.x);
            } else {
                ops.mix(se.sc.t, at(se.s, 0), at(se.x, 0), m * d, M.cfg.damp);
                std::swap(se.s, se.sc.t);
            }
        }
        std::swap(se.x, se.s);
    }
    for (size_t i = 0; i < M.coda.size(); i++)
        block(M, M.coda[i], se.coda[i], se.x, se.e0, se.sc, pos, m);
    if (want_logits) {
        ops.copy(se.last, at(se.x, (m - 1) * d), d);
        ops.rms(se.sc.n, at(se.last, 0), M.norm_f, 1, d, M.cfg.norm_eps);
        ops.linear(se.logits, M.embed.w, M.cfg.vocab_size, d, at(se.sc.n, 0), 1);
        if (pick >= 0) ops.argmax(se.tok, se.ids, (size_t)pick, se.logits, M.cfg.vocab_size);
    }
    se.pos += m;
    ops.flush(kept(se));
}

size_t chunk_at(const Model& M, size_t pos, size_t limit) {  // model.rs:647-654
    size_t chunk = std::min(limit, CHUNK);
    if (M.cfg.coda.find('G') != std::string::npos || M.cfg.prelude.find('G') != std::string::npos)
        return std::min(chunk, std::max<size_t>(MAX_SCORES / M.cfg.n_heads / (pos + 1), 1));
    return chunk;
}

void feed(Model& M, Session& se, const uint32_t* tokens, size_t n, size_t limit) {  // model.rs:658-667
    if (limit == 0) throw SlmError(SLM_E_INVALID, "feed: limit is 0");
    size_t done = 0;
    while (done < n) {
        size_t m = std::min(chunk_at(M, se.pos, limit), n - done);
        advance(M, se, tokens + done, m, done + m == n);
        done += m;
    }
}

size_t state_bytes(const Model& M, const Session& se) {  // model.rs:674-690
    const Config& c = M.cfg;
    size_t dh = c.head_dim(), n = 0;
    auto one = [&](const State& st) -> size_t {
        switch (st.kind) {
            case WINDOW: return 2 * c.n_heads * ring_cap(M) * dh;
            case LINEAR: return c.n_heads * dh * dh;
            default: return 2 * c.global_kv_heads * se.pos * dh + c.d_model;
        }
    };
    for (auto& st : se.prelude) n += one(st);
    for (auto& r : se.core)
        for (auto& st : r) n += one(st);
    for (auto& st : se.coda) n += one(st);
    return n * 4;
}

size_t params(const Model& M) {  // model.rs:275-302
    auto m = [](const Mat& x) { return x.rows * x.cols; };
    const Config& c = M.cfg;
    auto blk = [&](const Block& b) {
        size_t mixer = 0;
        if (b.kind == WINDOW) mixer = m(b.qkv) + m(b.o);
        else if (b.kind == LINEAR) mixer = m(b.qkvg) + m(b.decay) + m(b.o) + c.n_heads + c.head_dim();
        else mixer = m(b.q) + m(b.kv) + m(b.o) + (b.has_norm_e ? c.d_model : 0);
        return mixer + 2 * c.d_model + m(b.up) + m(b.down);
    };
    size_t total = 0;
    for (auto& b : M.prelude) total += blk(b);
    for (auto& b : M.core) total += blk(b);
    for (auto& b : M.coda) total += blk(b);
    total += m(M.embed) + c.d_model;
    if (M.looped) total += m(M.inject) + m(M.loop_embed);
    return total;
}

template <typename F>
int guard(slm_model* m, F f) {
    try {
        f();
        return SLM_OK;
    } catch (const SlmError& e) {
        if (m) m->error = e.what();
        return e.code;
    } catch (const std::exception& e) {
        if (m) m->error = e.what();
        return SLM_E_INVALID;
    }
}

void free_model_bufs(Model& M) {
    const Ops& ops = M.ops;
    for (auto* bl : {&M.prelude, &M.core, &M.coda})
        for (auto& b : *bl)
            for (Buf* p : {&b.norm1, &b.norm2, &b.up.w, &b.down.w, &b.qkv.w, &b.o.w, &b.qkvg.w,
                           &b.decay.w, &b.bias, &b.head_norm, &b.q.w, &b.kv.w, &b.norm_e})
                free_buf(ops, *p);
    for (Buf* p : {&M.embed.w, &M.inject.w, &M.loop_embed.w, &M.norm_f, &M.inv_freq}) free_buf(ops, *p);
}

}  // namespace

// =======================================================================================
// C ABI
// =======================================================================================

extern "C" {

int slm_model_load(slm_hip* ctx, const char* dir, slm_model** out) {
    if (!ctx || !dir || !out) return SLM_E_INVALID;
    *out = nullptr;
    slm_model* m = new slm_model(ctx);
    int rc = guard(m, [&] { load(*m, dir); });
    if (rc != SLM_OK) {
        g_load_error = m->error;
        free_model_bufs(*m);
        delete m;
        return rc;
    }
    *out = m;
    return SLM_OK;
}

void slm_model_free(slm_model* m) {
    if (!m) return;
    free_model_bufs(*m);
    delete m;
}

const char* slm_model_error(const slm_model* m) { return m ? m->error.c_str() : g_load_error.c_str(); }

size_t slm_model_params(const slm_model* m) { return m ? params(*m) : 0; }

int slm_model_set_global_cap(slm_model* m, size_t cap) {
    if (!m || cap == 0) return SLM_E_INVALID;
    m->global_cap0 = cap;
    return SLM_OK;
}

int slm_model_set_device_grow(slm_model* m, int on) {
    if (!m) return SLM_E_INVALID;
    m->device_grow = on != 0;
    return SLM_OK;
}

int slm_session_new(slm_model* m, size_t loops, slm_session** out) {
    if (!m || !out) return SLM_E_INVALID;
    *out = nullptr;
    return guard(m, [&] { *out = new_session(*m, loops); });
}

void slm_session_free(slm_session* s) {
    if (!s) return;
    const Ops& ops = s->model->ops;
    for (auto& st : s->prelude) free_state(ops, st);
    for (auto& r : s->core)
        for (auto& st : r) free_state(ops, st);
    for (auto& st : s->coda) free_state(ops, st);
    Scratch& sc = s->sc;
    for (Buf* p : {&sc.n, &sc.mix, &sc.q, &sc.k, &sc.v, &sc.g, &sc.y, &sc.y2, &sc.h, &sc.t, &sc.d,
                   &sc.shifted, &sc.prev_kv, &sc.up, &sc.gate, &sc.mid, &sc.scores, &sc.cos, &sc.sin,
                   &s->x, &s->s, &s->e0, &s->e_proj, &s->last, &s->logits, &s->tok, &s->ids})
        free_buf(ops, *p);
    delete s;
}

size_t slm_session_pos(const slm_session* s) { return s ? s->pos : 0; }
size_t slm_session_loops(const slm_session* s) { return s ? s->loops : 0; }

int slm_session_feed(slm_session* s, const uint32_t* tokens, size_t n, size_t limit) {
    if (!s || (n && !tokens)) return SLM_E_INVALID;
    return guard(s->model, [&] { feed(*s->model, *s, tokens, n, limit); });
}

int slm_session_advance(slm_session* s, const uint32_t* tokens, size_t n, int want_logits) {
    if (!s || !tokens) return SLM_E_INVALID;
    return guard(s->model, [&] { advance(*s->model, *s, tokens, n, want_logits != 0); });
}

int slm_session_step(slm_session* s, uint32_t token) {
    if (!s) return SLM_E_INVALID;
    return guard(s->model, [&] { advance(*s->model, *s, &token, 1, true); });
}

int slm_session_logits(slm_session* s, float* out) {
    if (!s || !out) return SLM_E_INVALID;
    return guard(s->model, [&] {
        std::vector<float> l = s->model->ops.read(s->logits, s->model->cfg.vocab_size);
        std::memcpy(out, l.data(), l.size() * 4);
    });
}

size_t slm_session_state_bytes(const slm_session* s) { return s ? state_bytes(*s->model, *s) : 0; }

size_t slm_session_kept_count(const slm_session* s) { return s ? kept(*s).size() : 0; }

size_t slm_session_kept_len(const slm_session* s, size_t i) {
    if (!s) return 0;
    auto k = kept(*s);
    return i < k.size() ? k[i]->n : 0;
}

int slm_session_kept_read(slm_session* s, size_t i, float* out, size_t n) {
    if (!s || !out) return SLM_E_INVALID;
    return guard(s->model, [&] {
        auto k = kept(*s);
        if (i >= k.size()) throw SlmError(SLM_E_INVALID, "kept_read: no such buffer");
        std::vector<float> v = s->model->ops.read(*k[i], std::min(n, k[i]->n));
        std::memcpy(out, v.data(), v.size() * 4);
    });
}

// sample.rs:48-53, the greedy pick: b = 0, then b = i whenever l[i] > l[b]. That is the first
// index holding the largest value under `>` (NaNs never win; a NaN at 0 keeps 0, since nothing
// compares greater than it; −0 and +0 are one value). Found in two passes that do not wait on
// each other element by element: the largest value with eight running maxima (x > m ? x : m,
// which skips NaNs), then the first index whose value equals it (== also takes −0 for +0).
// (SSE2, part of every x86-64 host: _mm_max_ps(x, m) is x > m ? x : m lane by lane, so a NaN in
// x leaves m; _mm_cmpeq_ps finds the lanes equal to the maximum.)
size_t slm_pick_greedy(const float* l, size_t n) {
    if (n == 0 || l[0] != l[0]) return 0;
    __m128 a0 = _mm_set1_ps(l[0]), a1 = a0, a2 = a0, a3 = a0;
    size_t i = 0;
    for (; i + 16 <= n; i += 16) {
        a0 = _mm_max_ps(_mm_loadu_ps(l + i), a0);
        a1 = _mm_max_ps(_mm_loadu_ps(l + i + 4), a1);
        a2 = _mm_max_ps(_mm_loadu_ps(l + i + 8), a2);
        a3 = _mm_max_ps(_mm_loadu_ps(l + i + 12), a3);
    }
    float acc[16];
    _mm_storeu_ps(acc, a0);
    _mm_storeu_ps(acc + 4, a1);
    _mm_storeu_ps(acc + 8, a2);
    _mm_storeu_ps(acc + 12, a3);
    float m = acc[0];
    for (int k = 1; k < 16; k++) m = acc[k] > m ? acc[k] : m;
    for (; i < n; i++) m = l[i] > m ? l[i] : m;
    __m128 mv = _mm_set1_ps(m);
    for (i = 0; i + 4 <= n; i += 4) {
        int hit = _mm_movemask_ps(_mm_cmpeq_ps(_mm_loadu_ps(l + i), mv));
        if (hit) return i + (size_t)__builtin_ctz((unsigned)hit);
    }
    for (; i < n; i++)
        if (l[i] == m) return i;
    return 0;
}

int slm_session_decode_greedy(slm_session* s, size_t n, uint32_t* ids) {
    if (!s || (n && !ids)) return SLM_E_INVALID;
    return guard(s->model, [&] {
        Model& M = *s->model;
        size_t V = M.cfg.vocab_size;
        std::vector<float> l(V);
        for (size_t t = 0; t < n; t++) {
            M.ops.ok(slm_hip_read(M.ops.ctx(), l.data(), s->logits.p, V), "read");
            ids[t] = (uint32_t)slm_pick_greedy(l.data(), V);
            advance(M, *s, &ids[t], 1, true);
        }
    });
}

int slm_session_decode_greedy_device(slm_session* s, size_t n, uint32_t* ids) {
    if (!s || (n && !ids)) return SLM_E_INVALID;
    return guard(s->model, [&] {
        Model& M = *s->model;
        const Ops& ops = M.ops;
        size_t V = M.cfg.vocab_size;
        if (!n) return;
        if (s->tok.n < 2) {
            ops.release(s->tok);
            s->tok = ops.zeros(2);
        }
        if (s->ids.n < n + 1) {
            ops.release(s->ids);
            s->ids = ops.zeros(n + 1);
        }
        ops.argmax(s->tok, s->ids, 0, s->logits, V);  // the first pick, from the current logits
        for (size_t t = 0; t < n; t++) advance(M, *s, nullptr, 1, true, (long)(t + 1));
        std::vector<float> got = ops.read(s->ids, n);  // uint32 ids in float-sized slots
        std::memcpy(ids, got.data(), n * 4);
    });
}

}  // extern "C"
