// ORACLE — test infrastructure only. Nothing in the product links, loads or calls this
// file; only tests/, the smoke check and bench.py's CPU-baseline leg do, and only as what
// the GPU results are compared against or as the timed CPU baseline.
//
// A CPU restatement of the reference's CPU backend and model, op for op and in the same
// arithmetic order, so that it computes what the reference computes bit for bit:
//   - ops:    src/cpu.rs:9-404 (dot with 16 accumulators, axpy, every Ops method)
//   - ranges: src/ops.rs:48-66 (Attn::base/span/range)
//   - model:  src/model.rs:26-691 (Model::load/session/grow/block/advance/feed/chunk_at)
//   - pick:   src/sample.rs:17-93 (xorshift64* Rng, repeat penalty, greedy argmax,
//             temperature / top-k / top-p)
// Rust never fuses a multiply and an add and calls glibc's expf/sinf/cosf/powf/logf/
// log1pf for f32::exp/sin/cos/powf/ln/ln_1p on linux-gnu, so this file is compiled with
// -ffp-contract=off and no fast-math, against glibc's libm.
//
// rayon's parallel loops in cpu.rs split only independent outputs (linear: outputs,
// attend: queries, gla: heads), so the results do not depend on the thread count; the
// OpenMP loops below split the same units.
//
// Parity pins (tests/): the whole model against the reference's PyTorch fixture
// tests/fixtures/tiny/expected.safetensors under the split matrix of tests/parity.rs:15-46;
// every op against float64 brute force; ring wrap against a non-ring brute force attention;
// grow against a run with a larger initial cache; pick against src/sample.rs:95-152.

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <limits>
#include <map>
#include <memory>
#include <string>
#include <utility>
#include <vector>

namespace {

using Buf = std::vector<float>;

// src/cpu.rs:9-21. Sixteen running sums over 16-wide chunks, a left-to-right tail, then
// the sums added left to right and the tail last. Rust's f32 Sum starts from -0.0.
float dot(const float* a, const float* b, size_t n) {
    float acc[16];
    for (int i = 0; i < 16; i++) acc[i] = 0.0f;
    size_t chunks = n / 16;
    for (size_t c = 0; c < chunks; c++) {
        const float* x = a + c * 16;
        const float* y = b + c * 16;
        for (int i = 0; i < 16; i++) acc[i] += x[i] * y[i];
    }
    float tail = -0.0f;
    for (size_t j = chunks * 16; j < n; j++) tail += a[j] * b[j];
    float s = -0.0f;
    for (int i = 0; i < 16; i++) s += acc[i];
    return s + tail;
}

// src/cpu.rs:23-28.
void axpy(float* y, float a, const float* x, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] += a * x[i];
}

// src/cpu.rs:34-38: outputs are resized to exactly n, keeping what was there.
void resize(Buf& y, size_t n) {
    if (y.size() != n) y.resize(n, 0.0f);
}

// A read-only position inside a buffer, src/ops.rs:13-29.
struct At {
    const Buf* buf;
    size_t offset;
    const float* ptr(size_t n) const {
        if (offset + n > buf->size()) {
            std::fprintf(stderr, "oracle: view [%zu, %zu) outside a buffer of %zu\n", offset,
                         offset + n, buf->size());
            std::abort();
        }
        return buf->data() + offset;
    }
};
At at(const Buf& b, size_t off) { return At{&b, off}; }

// src/ops.rs:31-66.
struct Attn {
    size_t pos, m, reach, gap, cap, heads, key_heads, dh;
    float scale;
    size_t base() const { return reach - 1 > pos ? 0 : pos - (reach - 1); }
    // ops.rs:62-65: p.saturating_sub(reach - 1) .. (p + 1).saturating_sub(gap)
    void range(size_t i, size_t* lo, size_t* hi) const {
        size_t p = pos + i;
        *lo = (reach - 1 > p) ? 0 : p - (reach - 1);
        *hi = (gap > p + 1) ? 0 : p + 1 - gap;
    }
};

// ---------------------------------------------------------------------------------------
// The CPU backend, src/cpu.rs:43-404.
// ---------------------------------------------------------------------------------------

void op_gather(Buf& y, const Buf& w, const uint32_t* ids, size_t m, size_t d) {
    resize(y, m * d);
    for (size_t i = 0; i < m; i++) std::memcpy(&y[i * d], &w[(size_t)ids[i] * d], d * 4);
}

void op_copy(Buf& y, At x, size_t n) {
    const float* s = x.ptr(n);
    resize(y, n);
    std::memcpy(y.data(), s, n * 4);
}

void op_shift(Buf& y, const Buf& first, At x, size_t m, size_t d) {
    const float* s = x.ptr((m - 1) * d);
    resize(y, m * d);
    std::memcpy(y.data(), first.data(), d * 4);
    std::memcpy(y.data() + d, s, (m - 1) * d * 4);
}

void op_columns(Buf& y, const Buf& x, size_t m, size_t stride, size_t off, size_t len) {
    resize(y, m * len);
    for (size_t i = 0; i < m; i++) std::memcpy(&y[i * len], &x[i * stride + off], len * 4);
}

void op_linear(Buf& y, const Buf& w, size_t rows, size_t cols, At x, size_t m) {
    const float* xs = x.ptr(m * cols);
    resize(y, m * rows);
    const float* ws = w.data();
    float* ys = y.data();
    long n = (long)(m * rows);
#pragma omp parallel for schedule(static)
    for (long t = 0; t < n; t++) {
        size_t i = (size_t)t / rows, r = (size_t)t % rows;
        ys[t] = dot(ws + r * cols, xs + i * cols, cols);
    }
}

void op_add(Buf& y, At a, At b, size_t n) {
    const float* p = a.ptr(n);
    const float* q = b.ptr(n);
    resize(y, n);
    for (size_t i = 0; i < n; i++) y[i] = p[i] + q[i];
}

void op_add_row(Buf& y, At x, At row, size_t m, size_t d) {
    const float* r = row.ptr(d);
    const float* s = x.ptr(m * d);
    resize(y, m * d);
    for (size_t i = 0; i < m; i++)
        for (size_t j = 0; j < d; j++) y[i * d + j] = s[i * d + j] + r[j];
}

void op_scale_rows(Buf& y, At x, const float* f, size_t m, size_t d) {
    const float* s = x.ptr(m * d);
    resize(y, m * d);
    for (size_t i = 0; i < m; i++)
        for (size_t j = 0; j < d; j++) y[i * d + j] = s[i * d + j] * f[i];
}

void op_mix(Buf& y, At a, At b, size_t n, float t) {
    const float* p = a.ptr(n);
    const float* q = b.ptr(n);
    resize(y, n);
    for (size_t i = 0; i < n; i++) y[i] = p[i] + t * (q[i] - p[i]);
}

void op_rms(Buf& y, At x, const Buf& w, size_t groups, size_t size, float eps) {
    const float* s = x.ptr(groups * size);
    resize(y, groups * size);
    for (size_t g = 0; g < groups; g++) {
        const float* in = s + g * size;
        float r = 1.0f / std::sqrt(dot(in, in, size) / (float)size + eps);
        for (size_t i = 0; i < size; i++) y[g * size + i] = in[i] * r * w[i];
    }
}

void op_silu_mul(Buf& y, At g, At u, size_t n) {
    const float* gs = g.ptr(n);
    const float* us = u.ptr(n);
    resize(y, n);
    for (size_t i = 0; i < n; i++) {
        float v = gs[i];
        y[i] = us[i] * v / (1.0f + std::exp(-v));
    }
}

void op_rope_table(Buf& cs, Buf& sn, const Buf& inv, size_t pos, size_t m, size_t half) {
    resize(cs, m * half);
    resize(sn, m * half);
    for (size_t i = 0; i < m; i++) {
        float p = (float)(pos + i);
        for (size_t j = 0; j < half; j++) {
            float a = p * inv[j];
            cs[i * half + j] = std::cos(a);
            sn[i * half + j] = std::sin(a);
        }
    }
}

void op_rope(Buf& y, At x, const Buf& cs, const Buf& sn, size_t m, size_t heads, size_t dh) {
    const float* s = x.ptr(m * heads * dh);
    resize(y, m * heads * dh);
    size_t half = dh / 2;
    for (size_t t = 0; t < m * heads; t++) {
        size_t row = t / heads;
        const float* c = &cs[row * half];
        const float* n = &sn[row * half];
        const float* h = s + t * dh;
        float* o = &y[t * dh];
        for (size_t i = 0; i < half; i++) {
            float a = h[i], b = h[half + i];
            o[i] = a * c[i] - b * n[i];
            o[half + i] = a * n[i] + b * c[i];
        }
    }
}

void op_l2norm(Buf& y, At x, size_t heads, size_t dh) {
    const float* s = x.ptr(heads * dh);
    resize(y, heads * dh);
    for (size_t h = 0; h < heads; h++) {
        const float* in = s + h * dh;
        float r = 1.0f / std::fmax(std::sqrt(dot(in, in, dh)), 1e-12f);
        for (size_t i = 0; i < dh; i++) y[h * dh + i] = in[i] * r;
    }
}

void op_gla(Buf& y, Buf& st, At qa, At ka, At va, const Buf& decay, const Buf& bias, size_t m,
            size_t heads, size_t dh) {
    size_t n = m * heads * dh;
    const float* q = qa.ptr(n);
    const float* k = ka.ptr(n);
    const float* v = va.ptr(n);
    resize(y, n);
    float* ys = y.data();
#pragma omp parallel for schedule(static)
    for (long hl = 0; hl < (long)heads; hl++) {
        size_t h = (size_t)hl;
        float* state = &st[h * dh * dh];
        std::vector<float> o(dh);
        for (size_t i = 0; i < m; i++) {
            size_t base = (i * heads + h) * dh;
            float d = 1.0f / (1.0f + std::exp(decay[i * heads + h] + bias[h]));
            const float* vh = v + base;
            for (size_t a = 0; a < dh; a++) {
                float kv = k[base + a];
                float* row = state + a * dh;
                for (size_t b = 0; b < dh; b++) row[b] = d * row[b] + kv * vh[b];
            }
            std::fill(o.begin(), o.end(), 0.0f);
            for (size_t a = 0; a < dh; a++) axpy(o.data(), q[base + a], state + a * dh, dh);
            std::memcpy(ys + base, o.data(), dh * 4);
        }
    }
}

void op_store(Buf& cache, At src, size_t pos, size_t m, size_t cap, size_t heads, size_t dh) {
    const float* s = src.ptr(m * heads * dh);
    for (size_t i = 0; i < m; i++) {
        size_t slot = (pos + i) % cap;
        for (size_t h = 0; h < heads; h++)
            std::memcpy(&cache[(h * cap + slot) * dh], s + (i * heads + h) * dh, dh * 4);
    }
}

void op_attend(Buf& y, At qa, const Buf& k, const Buf& v, const Attn& a) {
    size_t heads = a.heads, dh = a.dh, cap = a.cap, m = a.m;
    size_t group = heads / a.key_heads;
    const float* q = qa.ptr(m * heads * dh);
    resize(y, m * heads * dh);
    float* ys = y.data();
#pragma omp parallel for schedule(static)
    for (long il = 0; il < (long)m; il++) {
        size_t i = (size_t)il;
        size_t lo, hi;
        a.range(i, &lo, &hi);
        size_t len = hi > lo ? hi - lo : 0;
        std::vector<float> sc(len);
        for (size_t h = 0; h < heads; h++) {
            float* o = ys + (i * heads + h) * dh;
            std::fill(o, o + dh, 0.0f);
            if (len == 0) continue;
            size_t base = (h / group) * cap * dh;
            const float* qh = q + (i * heads + h) * dh;
            float mx = -std::numeric_limits<float>::infinity();
            for (size_t j = 0; j < len; j++) {
                size_t p = lo + j;
                sc[j] = dot(qh, &k[base + (p % cap) * dh], dh) * a.scale;
                mx = std::fmax(mx, sc[j]);
            }
            float sum = 0.0f;
            for (size_t j = 0; j < len; j++) {
                sc[j] = std::exp(sc[j] - mx);
                sum += sc[j];
            }
            for (size_t j = 0; j < len; j++) {
                size_t p = lo + j;
                axpy(o, sc[j] / sum, &v[base + (p % cap) * dh], dh);
            }
        }
    }
}

// ---------------------------------------------------------------------------------------
// The model, src/model.rs.
// ---------------------------------------------------------------------------------------

// Mirrors src/config.rs:20-52 (validation is done by the Python loader, config.rs:63-79).
struct Config {
    size_t vocab_size, d_model, n_heads, global_kv_heads;
    uint32_t global_logn, global_kshift, global_emb, global_far;
    std::string prelude, core, coda;
    size_t window, max_loops, default_loops;
    float damp, rope_base, norm_eps;
    size_t head_dim() const { return d_model / n_heads; }
};

constexpr size_t CHUNK = 256;          // model.rs:27
constexpr size_t MAX_SCORES = 1u << 28; // model.rs:30

struct Mat {
    Buf w;
    size_t rows = 0, cols = 0;
};

enum Kind { WINDOW, LINEAR, GLOBAL };

struct Block {
    Kind kind;
    Buf norm1, norm2;
    Mat up, down;
    Mat qkv, o;                      // S
    Mat qkvg, decay;                 // L (o shared)
    Buf bias, head_norm;             // L
    Mat q, kv;                       // G (o shared)
    bool has_norm_e = false;
    Buf norm_e;                      // G
};

struct State {
    Kind kind;
    Buf k, v;      // S ring / G cache
    Buf s;         // L
    Buf prev;      // G
    size_t cap = 0;
    Buf scores;
};

struct Scratch {
    Buf n, mix, q, k, v, g, y, y2, h, t, d, shifted, prev_kv, up, gate, mid, scores, cos, sin;
};

struct Model;

struct Session {
    Model* model;
    size_t loops = 0, pos = 0;
    std::vector<State> prelude;
    std::vector<std::vector<State>> core;
    std::vector<State> coda;
    Scratch sc;
    Buf x, s, e0, e_proj, last, logits;
};

struct Model {
    Config cfg;
    std::map<std::string, std::pair<std::vector<size_t>, Buf>> tensors;
    Mat embed;
    std::vector<Block> prelude, core, coda;
    bool looped = false;
    Mat inject, loop_embed;
    Buf norm_f, inv_freq;
    size_t global_cap0 = 1u << 13;  // model.rs:320
    std::string error;

    bool take(const std::string& name, std::pair<std::vector<size_t>, Buf>* out) {
        auto it = tensors.find(name);
        if (it == tensors.end()) {
            error = "missing weight " + name;
            return false;
        }
        *out = std::move(it->second);
        tensors.erase(it);
        return true;
    }
    bool mat(const std::string& name, Mat* m) {
        std::pair<std::vector<size_t>, Buf> t;
        if (!take(name, &t)) return false;
        if (t.first.size() != 2) {
            error = name + ": expected a matrix";
            return false;
        }
        m->rows = t.first[0];
        m->cols = t.first[1];
        m->w = std::move(t.second);
        return true;
    }
    bool vec(const std::string& name, Buf* b) {
        std::pair<std::vector<size_t>, Buf> t;
        if (!take(name, &t)) return false;
        *b = std::move(t.second);
        return true;
    }

    // model.rs:114-153
    bool load_block(const std::string& prefix, char kind, Block* b) {
        auto n = [&](const char* s) { return prefix + "." + s; };
        switch (kind) {
            case 'S':
                b->kind = WINDOW;
                if (!mat(n("mixer.qkv.weight"), &b->qkv) || !mat(n("mixer.o.weight"), &b->o))
                    return false;
                break;
            case 'L':
                b->kind = LINEAR;
                if (!mat(n("mixer.qkvg.weight"), &b->qkvg) ||
                    !mat(n("mixer.decay.weight"), &b->decay) ||
                    !vec(n("mixer.decay.bias"), &b->bias) ||
                    !vec(n("mixer.head_norm.weight"), &b->head_norm) ||
                    !mat(n("mixer.o.weight"), &b->o))
                    return false;
                break;
            case 'G':
                b->kind = GLOBAL;
                if (!mat(n("mixer.q.weight"), &b->q) || !mat(n("mixer.kv.weight"), &b->kv) ||
                    !mat(n("mixer.o.weight"), &b->o))
                    return false;
                if (cfg.global_emb != 0) {
                    b->has_norm_e = true;
                    if (!vec(n("mixer.norm_e.weight"), &b->norm_e)) return false;
                }
                break;
            default:
                error = std::string("unknown layer type ") + kind;
                return false;
        }
        return vec(n("norm1.weight"), &b->norm1) && vec(n("norm2.weight"), &b->norm2) &&
               mat(n("mlp.up.weight"), &b->up) && mat(n("mlp.down.weight"), &b->down);
    }

    // model.rs:226-269
    bool finish() {
        auto blocks = [&](const char* name, const std::string& kinds, std::vector<Block>* out) {
            for (size_t i = 0; i < kinds.size(); i++) {
                Block b;
                if (!load_block(std::string(name) + "." + std::to_string(i), kinds[i], &b))
                    return false;
                out->push_back(std::move(b));
            }
            return true;
        };
        if (!blocks("prelude", cfg.prelude, &prelude) || !blocks("core", cfg.core, &core) ||
            !blocks("coda", cfg.coda, &coda))
            return false;
        looped = !cfg.core.empty();
        if (looped) {
            if (!mat("inject_e.weight", &inject) || !mat("loop_embed.weight", &loop_embed))
                return false;
        }
        if (!mat("embed.weight", &embed) || !vec("norm_f.weight", &norm_f)) return false;
        size_t dh = cfg.head_dim();
        inv_freq.resize(dh / 2);
        for (size_t i = 0; i < dh / 2; i++)
            inv_freq[i] = 1.0f / std::pow(cfg.rope_base, (float)(2 * i) / (float)dh);
        return true;
    }

    size_t cap() const { return cfg.window + CHUNK; }  // model.rs:304-306

    State new_state(const Block& b) const {  // model.rs:308-331
        State st;
        st.kind = b.kind;
        size_t h = cfg.n_heads, dh = cfg.head_dim();
        switch (b.kind) {
            case WINDOW:
                st.k.assign(h * cap() * dh, 0.0f);
                st.v.assign(h * cap() * dh, 0.0f);
                break;
            case LINEAR:
                st.s.assign(h * dh * dh, 0.0f);
                break;
            case GLOBAL:
                st.cap = global_cap0;
                st.k.assign(cfg.global_kv_heads * st.cap * dh, 0.0f);
                st.v.assign(cfg.global_kv_heads * st.cap * dh, 0.0f);
                st.prev.assign(cfg.d_model, 0.0f);
                st.scores.assign(1, 0.0f);
                break;
        }
        return st;
    }

    // model.rs:333-381 (the CPU backend resizes scratch on use, so sizes only need to exist)
    Session* session(size_t loops) {
        Session* se = new Session();
        se->model = this;
        se->loops = loops;
        for (auto& b : prelude) se->prelude.push_back(new_state(b));
        for (size_t r = 0; r < loops; r++) {
            std::vector<State> sts;
            for (auto& b : core) sts.push_back(new_state(b));
            se->core.push_back(std::move(sts));
        }
        for (auto& b : coda) se->coda.push_back(new_state(b));
        size_t d = cfg.d_model, half = cfg.head_dim() / 2;
        Scratch& sc = se->sc;
        sc.n.assign(d, 0);
        sc.mix.assign(4 * d, 0);
        sc.q.assign(d, 0);
        sc.k.assign(d, 0);
        sc.v.assign(d, 0);
        sc.g.assign(d, 0);
        sc.y.assign(d, 0);
        sc.y2.assign(d, 0);
        sc.h.assign(d, 0);
        sc.t.assign(d, 0);
        sc.d.assign(cfg.n_heads, 0);
        sc.shifted.assign(d, 0);
        sc.prev_kv.assign(2 * d, 0);
        sc.up.assign(4 * d, 0);
        sc.gate.assign(2 * d, 0);
        sc.mid.assign(2 * d, 0);
        sc.scores.assign(1, 0);
        sc.cos.assign(half, 0);
        sc.sin.assign(half, 0);
        se->x.assign(d, 0);
        se->s.assign(d, 0);
        se->e0.assign(d, 0);
        se->e_proj.assign(d, 0);
        se->last.assign(d, 0);
        se->logits.assign(cfg.vocab_size, 0);
        return se;
    }

    // model.rs:383-398: doubles a global cache, moving every head's data.
    void grow(Buf& k, Buf& v, size_t& cap) const {
        size_t kh = cfg.global_kv_heads, dh = cfg.head_dim();
        size_t old = cap, nw = cap * 2;
        for (Buf* buf : {&k, &v}) {
            Buf out(kh * nw * dh, 0.0f);
            for (size_t h = 0; h < kh; h++)
                std::memcpy(&out[h * nw * dh], &(*buf)[h * old * dh], old * dh * 4);
            *buf = std::move(out);
        }
        cap = nw;
    }

    // model.rs:400-560
    void block(const Block& b, State& st, Buf& x, const Buf& e0, Scratch& sc, size_t pos,
               size_t m) const {
        const Config& c = cfg;
        size_t d = c.d_model, heads = c.n_heads, dh = c.head_dim();
        float eps = c.norm_eps;
        float scale = 1.0f / std::sqrt((float)dh);
        size_t n = m * d;
        op_rms(sc.n, at(x, 0), b.norm1, m, d, eps);
        // model.rs:417-426: one token needs no copy to split a row.
        auto col = [&](Buf& y, const Buf& src, size_t stride, size_t off, size_t len) -> At {
            if (m == 1) return at(src, off);
            op_columns(y, src, m, stride, off, len);
            return at(y, 0);
        };
        bool has_h = true;
        if (b.kind == WINDOW) {
            op_linear(sc.mix, b.qkv.w, b.qkv.rows, d, at(sc.n, 0), m);
            At raw = col(sc.y, sc.mix, 3 * d, 0, d);
            op_rope(sc.q, raw, sc.cos, sc.sin, m, heads, dh);
            raw = col(sc.y, sc.mix, 3 * d, d, d);
            op_rope(sc.k, raw, sc.cos, sc.sin, m, heads, dh);
            At vals = col(sc.v, sc.mix, 3 * d, 2 * d, d);
            size_t cp = cap();
            op_store(st.k, at(sc.k, 0), pos, m, cp, heads, dh);
            op_store(st.v, vals, pos, m, cp, heads, dh);
            Attn a{pos, m, c.window, 0, cp, heads, heads, dh, scale};
            op_attend(sc.y, at(sc.q, 0), st.k, st.v, a);
            op_linear(sc.h, b.o.w, d, d, at(sc.y, 0), m);
        } else if (b.kind == LINEAR) {
            op_linear(sc.mix, b.qkvg.w, b.qkvg.rows, d, at(sc.n, 0), m);
            At raw = col(sc.y, sc.mix, 4 * d, 0, d);
            op_l2norm(sc.q, raw, m * heads, dh);
            raw = col(sc.y, sc.mix, 4 * d, d, d);
            op_l2norm(sc.k, raw, m * heads, dh);
            At vals = col(sc.v, sc.mix, 4 * d, 2 * d, d);
            At gate = col(sc.g, sc.mix, 4 * d, 3 * d, d);
            op_linear(sc.d, b.decay.w, heads, d, at(sc.n, 0), m);
            op_gla(sc.y, st.s, at(sc.q, 0), at(sc.k, 0), vals, sc.d, b.bias, m, heads, dh);
            op_rms(sc.y2, at(sc.y, 0), b.head_norm, m * heads, dh, eps);
            op_silu_mul(sc.y, gate, at(sc.y2, 0), n);
            op_linear(sc.h, b.o.w, d, d, at(sc.y, 0), m);
        } else {
            if (b.has_norm_e) {
                op_rms(sc.t, at(e0, 0), b.norm_e, m, d, eps);
                op_add(sc.y, at(sc.n, 0), at(sc.t, 0), n);
                std::swap(sc.n, sc.y);
            }
            size_t kh = c.global_kv_heads, kd = c.global_kv_heads * dh;
            op_linear(sc.q, b.q.w, d, d, at(sc.n, 0), m);
            op_linear(sc.mix, b.kv.w, 2 * kd, d, at(sc.n, 0), m);
            if (c.global_logn != 0) {
                float lg = std::log((float)c.global_logn);
                std::vector<float> f(m);
                for (size_t i = 0; i < m; i++) f[i] = std::log1p((float)(pos + i)) / lg;
                op_scale_rows(sc.y, at(sc.q, 0), f.data(), m, d);
                std::swap(sc.q, sc.y);
            }
            while (pos + m > st.cap) grow(st.k, st.v, st.cap);
            At keys;
            if (c.global_kshift != 0) {
                op_shift(sc.shifted, st.prev, at(sc.n, 0), m, d);
                op_linear(sc.prev_kv, b.kv.w, 2 * kd, d, at(sc.shifted, 0), m);
                op_copy(st.prev, at(sc.n, (m - 1) * d), d);
                keys = col(sc.k, sc.prev_kv, 2 * kd, 0, kd);
            } else {
                keys = col(sc.k, sc.mix, 2 * kd, 0, kd);
            }
            At vals = col(sc.v, sc.mix, 2 * kd, kd, kd);
            op_store(st.k, keys, pos, m, st.cap, kh, dh);
            op_store(st.v, vals, pos, m, st.cap, kh, dh);
            size_t far = c.global_far != 0 ? c.window : 0;
            if (pos + m > far) {
                Attn a{pos, m, std::numeric_limits<size_t>::max(), far, st.cap, heads, kh, dh,
                       scale};
                op_attend(sc.y, at(sc.q, 0), st.k, st.v, a);
                op_linear(sc.h, b.o.w, d, d, at(sc.y, 0), m);
            } else {
                has_h = false;
            }
        }
        if (has_h) {
            op_add(sc.t, at(x, 0), at(sc.h, 0), n);
            std::swap(x, sc.t);
        }
        op_rms(sc.n, at(x, 0), b.norm2, m, d, eps);
        size_t hidden = b.down.cols;
        op_linear(sc.up, b.up.w, 2 * hidden, d, at(sc.n, 0), m);
        At gate = col(sc.gate, sc.up, 2 * hidden, 0, hidden);
        At amp = col(sc.mid, sc.up, 2 * hidden, hidden, hidden);
        op_silu_mul(sc.y, gate, amp, m * hidden);
        op_linear(sc.h, b.down.w, d, hidden, at(sc.y, 0), m);
        op_add(sc.t, at(x, 0), at(sc.h, 0), n);
        std::swap(x, sc.t);
    }

    // model.rs:563-640
    void advance(Session& se, const uint32_t* tokens, size_t m, bool want_logits) const {
        size_t d = cfg.d_model, pos = se.pos;
        op_rope_table(se.sc.cos, se.sc.sin, inv_freq, pos, m, cfg.head_dim() / 2);
        op_gather(se.e0, embed.w, tokens, m, d);
        op_copy(se.x, at(se.e0, 0), m * d);
        for (size_t i = 0; i < prelude.size(); i++)
            block(prelude[i], se.prelude[i], se.x, se.e0, se.sc, pos, m);
        if (looped) {
            op_linear(se.e_proj, inject.w, d, d, at(se.x, 0), m);
            op_copy(se.s, at(se.x, 0), m * d);
            for (size_t r = 0; r < se.loops; r++) {
                op_add(se.sc.t, at(se.s, 0), at(se.e_proj, 0), m * d);
                op_add_row(se.x, at(se.sc.t, 0), at(loop_embed.w, r * d), m, d);
                for (size_t i = 0; i < core.size(); i++)
                    block(core[i], se.core[r][i], se.x, se.e0, se.sc, pos, m);
                if (cfg.damp == 1.0f) {
                    std::swap(se.s, se.x);
                } else {
                    op_mix(se.sc.t, at(se.s, 0), at(se.x, 0), m * d, cfg.damp);
                    std::swap(se.s, se.sc.t);
                }
            }
            std::swap(se.x, se.s);
        }
        for (size_t i = 0; i < coda.size(); i++)
            block(coda[i], se.coda[i], se.x, se.e0, se.sc, pos, m);
        if (want_logits) {
            op_copy(se.last, at(se.x, (m - 1) * d), d);
            op_rms(se.sc.n, at(se.last, 0), norm_f, 1, d, cfg.norm_eps);
            op_linear(se.logits, embed.w, cfg.vocab_size, d, at(se.sc.n, 0), 1);
        }
        se.pos += m;
    }

    // model.rs:647-654
    size_t chunk_at(size_t pos, size_t limit) const {
        size_t chunk = limit < CHUNK ? limit : CHUNK;
        if (cfg.coda.find('G') != std::string::npos ||
            cfg.prelude.find('G') != std::string::npos) {
            size_t c2 = MAX_SCORES / cfg.n_heads / (pos + 1);
            if (c2 < 1) c2 = 1;
            return chunk < c2 ? chunk : c2;
        }
        return chunk;
    }

    // model.rs:658-667
    void feed(Session& se, const uint32_t* tokens, size_t n, size_t limit) const {
        size_t done = 0;
        while (done < n) {
            size_t m = chunk_at(se.pos, limit);
            if (m > n - done) m = n - done;
            advance(se, tokens + done, m, done + m == n);
            done += m;
        }
    }

    // model.rs:674-690
    size_t state_bytes(const Session& se) const {
        size_t dh = cfg.head_dim(), n = 0;
        auto one = [&](const State& st) {
            switch (st.kind) {
                case WINDOW: return 2 * cfg.n_heads * cap() * dh;
                case LINEAR: return cfg.n_heads * dh * dh;
                default: return 2 * cfg.global_kv_heads * se.pos * dh + cfg.d_model;
            }
        };
        for (auto& st : se.prelude) n += one(st);
        for (auto& r : se.core)
            for (auto& st : r) n += one(st);
        for (auto& st : se.coda) n += one(st);
        return n * 4;
    }

    // model.rs:275-302
    size_t params() const {
        auto m = [](const Mat& x) { return x.rows * x.cols; };
        const Config& c = cfg;
        size_t total = 0;
        auto block = [&](const Block& b) {
            size_t mixer = 0;
            if (b.kind == WINDOW) mixer = m(b.qkv) + m(b.o);
            else if (b.kind == LINEAR) mixer = m(b.qkvg) + m(b.decay) + m(b.o) + c.n_heads + c.head_dim();
            else mixer = m(b.q) + m(b.kv) + m(b.o) + (b.has_norm_e ? c.d_model : 0);
            return mixer + 2 * c.d_model + m(b.up) + m(b.down);
        };
        for (auto& b : prelude) total += block(b);
        for (auto& b : core) total += block(b);
        for (auto& b : coda) total += block(b);
        total += m(embed) + c.d_model;
        if (looped) total += m(inject) + m(loop_embed);
        return total;
    }
};

// Every buffer that outlives a step, in the order of model.rs:626-638 (logits first).
std::vector<const Buf*> kept(const Session& se) {
    std::vector<const Buf*> out{&se.logits};
    auto add = [&](const State& st) {
        switch (st.kind) {
            case WINDOW: out.push_back(&st.k); out.push_back(&st.v); break;
            case LINEAR: out.push_back(&st.s); break;
            case GLOBAL: out.push_back(&st.k); out.push_back(&st.v); out.push_back(&st.prev); break;
        }
    };
    for (auto& st : se.prelude) add(st);
    for (auto& r : se.core)
        for (auto& st : r) add(st);
    for (auto& st : se.coda) add(st);
    return out;
}

// src/sample.rs:17-31
struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s((seed * 0x9E3779B97F4A7C15ull) | 1) {}
    float next_f32() {
        s ^= s >> 12;
        s ^= s << 25;
        s ^= s >> 27;
        return (float)((s * 0x2545F4914F6CDD1Dull) >> 40) / (float)(1ull << 24);
    }
};

}  // namespace

// ---------------------------------------------------------------------------------------
// C ABI for the tests and the CPU baseline (ctypes).
// ---------------------------------------------------------------------------------------

extern "C" {

struct oracle_attn {
    size_t pos, m, reach, gap, cap, heads, key_heads, dh;
    float scale;
};

struct oracle_config {
    size_t vocab_size, d_model, n_heads, global_kv_heads;
    uint32_t global_logn, global_kshift, global_emb, global_far;
    const char* prelude;
    const char* core;
    const char* coda;
    size_t window, max_loops, default_loops;
    float damp, rope_base, norm_eps;
};

// ---- single ops on host arrays; outputs are sized by the caller ----
static Buf wrap(const float* p, size_t n) { return Buf(p, p + n); }

void oracle_dot(const float* a, const float* b, size_t n, float* out) { *out = dot(a, b, n); }

void oracle_linear(float* y, const float* w, size_t rows, size_t cols, const float* x, size_t m) {
    Buf yy, ww = wrap(w, rows * cols), xx = wrap(x, m * cols);
    op_linear(yy, ww, rows, cols, at(xx, 0), m);
    std::memcpy(y, yy.data(), m * rows * 4);
}
void oracle_rms(float* y, const float* x, const float* w, size_t groups, size_t size, float eps) {
    Buf yy, xx = wrap(x, groups * size), ww = wrap(w, size);
    op_rms(yy, at(xx, 0), ww, groups, size, eps);
    std::memcpy(y, yy.data(), groups * size * 4);
}
void oracle_l2norm(float* y, const float* x, size_t heads, size_t dh) {
    Buf yy, xx = wrap(x, heads * dh);
    op_l2norm(yy, at(xx, 0), heads, dh);
    std::memcpy(y, yy.data(), heads * dh * 4);
}
void oracle_silu_mul(float* y, const float* g, const float* u, size_t n) {
    Buf yy, gg = wrap(g, n), uu = wrap(u, n);
    op_silu_mul(yy, at(gg, 0), at(uu, 0), n);
    std::memcpy(y, yy.data(), n * 4);
}
void oracle_rope_table(float* cs, float* sn, const float* inv, size_t pos, size_t m, size_t half) {
    Buf c, s, ii = wrap(inv, half);
    op_rope_table(c, s, ii, pos, m, half);
    std::memcpy(cs, c.data(), m * half * 4);
    std::memcpy(sn, s.data(), m * half * 4);
}
void oracle_rope(float* y, const float* x, const float* cs, const float* sn, size_t m, size_t heads,
                 size_t dh) {
    Buf yy, xx = wrap(x, m * heads * dh), c = wrap(cs, m * dh / 2), s = wrap(sn, m * dh / 2);
    op_rope(yy, at(xx, 0), c, s, m, heads, dh);
    std::memcpy(y, yy.data(), m * heads * dh * 4);
}
void oracle_gla(float* y, float* s, const float* q, const float* k, const float* v,
                const float* decay, const float* bias, size_t m, size_t heads, size_t dh) {
    size_t n = m * heads * dh;
    Buf yy, ss = wrap(s, heads * dh * dh), qq = wrap(q, n), kk = wrap(k, n), vv = wrap(v, n),
            dd = wrap(decay, m * heads), bb = wrap(bias, heads);
    op_gla(yy, ss, at(qq, 0), at(kk, 0), at(vv, 0), dd, bb, m, heads, dh);
    std::memcpy(y, yy.data(), n * 4);
    std::memcpy(s, ss.data(), heads * dh * dh * 4);
}
void oracle_store(float* cache, const float* src, size_t pos, size_t m, size_t cap, size_t heads,
                  size_t dh) {
    Buf cc = wrap(cache, heads * cap * dh), ss = wrap(src, m * heads * dh);
    op_store(cc, at(ss, 0), pos, m, cap, heads, dh);
    std::memcpy(cache, cc.data(), heads * cap * dh * 4);
}
void oracle_attend(float* y, const float* q, const float* k, const float* v, const oracle_attn* a,
                   size_t kv_len) {
    Attn aa{a->pos, a->m, a->reach, a->gap, a->cap, a->heads, a->key_heads, a->dh, a->scale};
    Buf yy, qq = wrap(q, a->m * a->heads * a->dh), kk = wrap(k, kv_len), vv = wrap(v, kv_len);
    op_attend(yy, at(qq, 0), kk, vv, aa);
    std::memcpy(y, yy.data(), a->m * a->heads * a->dh * 4);
}
void oracle_attn_range(const oracle_attn* a, size_t i, size_t* lo, size_t* hi) {
    Attn aa{a->pos, a->m, a->reach, a->gap, a->cap, a->heads, a->key_heads, a->dh, a->scale};
    aa.range(i, lo, hi);
}
size_t oracle_attn_span(const oracle_attn* a) {
    Attn aa{a->pos, a->m, a->reach, a->gap, a->cap, a->heads, a->key_heads, a->dh, a->scale};
    size_t base = aa.base(), end = aa.pos + aa.m, sub = aa.gap + base;
    size_t span = end > sub ? end - sub : 0;
    return span < 1 ? 1 : span;
}

// ---- the model ----
void* oracle_model_new(const oracle_config* c) {
    Model* m = new Model();
    m->cfg = Config{c->vocab_size, c->d_model, c->n_heads, c->global_kv_heads, c->global_logn,
                    c->global_kshift, c->global_emb, c->global_far, c->prelude, c->core, c->coda,
                    c->window, c->max_loops, c->default_loops, c->damp, c->rope_base,
                    c->norm_eps};
    return m;
}
void oracle_model_add(void* h, const char* name, const size_t* shape, size_t ndim,
                      const float* data) {
    Model* m = (Model*)h;
    std::vector<size_t> sh(shape, shape + ndim);
    size_t n = 1;
    for (size_t s : sh) n *= s;
    m->tensors[name] = {sh, wrap(data, n)};
}
void oracle_model_set_global_cap(void* h, size_t cap) { ((Model*)h)->global_cap0 = cap; }
int oracle_model_finish(void* h) { return ((Model*)h)->finish() ? 0 : -1; }
const char* oracle_model_error(void* h) { return ((Model*)h)->error.c_str(); }
size_t oracle_model_params(void* h) { return ((Model*)h)->params(); }
void oracle_model_free(void* h) { delete (Model*)h; }

void* oracle_session_new(void* h, size_t loops) { return ((Model*)h)->session(loops); }
void oracle_session_free(void* s) { delete (Session*)s; }
size_t oracle_session_pos(void* s) { return ((Session*)s)->pos; }
void oracle_feed(void* s, const uint32_t* tokens, size_t n, size_t limit) {
    Session* se = (Session*)s;
    se->model->feed(*se, tokens, n, limit);
}
void oracle_advance(void* s, const uint32_t* tokens, size_t n, int want_logits) {
    Session* se = (Session*)s;
    se->model->advance(*se, tokens, n, want_logits != 0);
}
void oracle_step(void* s, uint32_t token) {
    Session* se = (Session*)s;
    se->model->advance(*se, &token, 1, true);
}
void oracle_logits(void* s, float* out) {
    Session* se = (Session*)s;
    std::memcpy(out, se->logits.data(), se->model->cfg.vocab_size * 4);
}
size_t oracle_state_bytes(void* s) {
    Session* se = (Session*)s;
    return se->model->state_bytes(*se);
}
// The kept buffers of model.rs:626-638: count, then each one's length and contents.
size_t oracle_kept_count(void* s) { return kept(*(Session*)s).size(); }
size_t oracle_kept_len(void* s, size_t i) { return kept(*(Session*)s)[i]->size(); }
void oracle_kept_read(void* s, size_t i, float* out, size_t n) {
    const Buf* b = kept(*(Session*)s)[i];
    std::memcpy(out, b->data(), (n < b->size() ? n : b->size()) * 4);
}

// ---- src/sample.rs ----
void* oracle_rng_new(uint64_t seed) { return new Rng(seed); }
void oracle_rng_free(void* r) { delete (Rng*)r; }
float oracle_rng_next(void* r) { return ((Rng*)r)->next_f32(); }

// sample.rs:33-93. Sorting ties: select_nth_unstable_by / sort_unstable_by leave equal
// logits in an unspecified order; a stable sort is used here.
uint32_t oracle_pick(const float* in, size_t n, const uint32_t* recent, size_t nrecent,
                     float temperature, size_t top_k, float top_p, float repeat_penalty,
                     size_t repeat_window, void* rng) {
    std::vector<float> logits(in, in + n);
    if (repeat_penalty != 1.0f) {
        size_t start = nrecent > repeat_window ? nrecent - repeat_window : 0;
        std::vector<uint32_t> seen(recent + start, recent + nrecent);
        std::sort(seen.begin(), seen.end());
        seen.erase(std::unique(seen.begin(), seen.end()), seen.end());
        for (uint32_t t : seen) {
            float& l = logits[t];
            l = l > 0.0f ? l / repeat_penalty : l * repeat_penalty;
        }
    }
    if (temperature <= 0.0f) {
        size_t b = 0;
        for (size_t i = 0; i < n; i++)
            if (logits[i] > logits[b]) b = i;
        return (uint32_t)b;
    }
    std::vector<uint32_t> ids(n);
    for (size_t i = 0; i < n; i++) ids[i] = (uint32_t)i;
    auto desc = [&](uint32_t a, uint32_t b) { return logits[a] > logits[b]; };
    if (top_k > 0 && top_k < ids.size()) {
        std::stable_sort(ids.begin(), ids.end(), desc);
        ids.resize(top_k);
    }
    if (top_p < 1.0f) std::stable_sort(ids.begin(), ids.end(), desc);
    float top = -std::numeric_limits<float>::infinity();
    for (uint32_t i : ids) top = std::fmax(top, logits[i]);
    std::vector<float> w(ids.size());
    for (size_t i = 0; i < ids.size(); i++) w[i] = std::exp((logits[ids[i]] - top) / temperature);
    if (top_p < 1.0f) {
        float total = -0.0f;
        for (float x : w) total += x;
        float enough = top_p * total, held = 0.0f;
        size_t keep = w.size();
        for (size_t i = 0; i < w.size(); i++) {
            held += w[i];
            if (held >= enough) {
                keep = i + 1;
                break;
            }
        }
        ids.resize(keep);
        w.resize(keep);
    }
    float total = -0.0f;
    for (float x : w) total += x;
    float r = ((Rng*)rng)->next_f32() * total;
    for (size_t i = 0; i < ids.size(); i++) {
        r -= w[i];
        if (r <= 0.0f) return ids[i];
    }
    return ids.back();
}

}  // extern "C"
