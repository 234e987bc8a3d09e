"""Pins the oracle (the C++ restatement of src/cpu.rs + src/model.rs) before anything is
compared against it:

* the reference's own golden data: tests/fixtures/tiny/expected.safetensors (PyTorch
  logits) under the split matrix of tests/parity.rs:15-46;
* an independent float64 statement of the model (tests/npmodel.py) past the ring's
  capacity and past a global-cache grow, which the fixture never reaches;
* chunked == token-by-token, bit for bit (true of the CPU backend by construction);
* every op against float64 brute force, with planted mistakes that must fail the same
  checks;
* src/sample.rs:95-152 and src/config.rs:125-130 known answers.
"""

import numpy as np
import pytest

import oracle as O
from npmodel import NpModel
from verify import SPLITS, check_parity

RNG = np.random.default_rng(1234)


@pytest.fixture(scope="module")
def tiny(tiny_dir):
    return O.Model(tiny_dir)


def test_fixture_parity(tiny, tiny_dir):
    reports = check_parity(tiny, tiny_dir)
    # The restatement is much tighter than the reference's 1e-4 bound.
    assert max(r.max_diff for r in reports) < 1e-6, reports


def _run(model, tokens, chunk, loops, steps=()):
    se = model.session(loops)
    se.feed(tokens, chunk)
    out = [se.logits()]
    for t in steps:
        se.step(t)
        out.append(se.logits())
    return se, out


@pytest.mark.parametrize("chunk", [3, 16, 256])
def test_chunked_equals_step_bitwise(tiny, chunk):
    toks = RNG.integers(0, 97, size=90).tolist()
    a, la = _run(tiny, toks, 1, 3, steps=[5, 6])
    b, lb = _run(tiny, toks, chunk, 3, steps=[5, 6])
    for x, y in zip(la, lb):
        assert np.array_equal(x, y)
    for x, y in zip(a.kept(), b.kept()):
        assert x.shape == y.shape and np.array_equal(x, y)


def _np_logits(npm, tokens, chunk, loops, steps):
    se = npm.session(loops)
    for i in range(0, len(tokens), chunk):
        npm.advance(se, tokens[i:i + chunk])
    out = [se["logits"]]
    for t in steps:
        npm.advance(se, [t])
        out.append(se["logits"])
    return out


def _weights(tiny_dir):
    return O.load_weights(tiny_dir)


def test_ring_wrap_against_float64(tiny, tiny_dir):
    """600 positions through rings of cap = 8 + 256 = 264 slots: every slot is rewritten."""
    cfg = tiny.cfg
    assert cfg.window + 256 < 600
    toks = RNG.integers(0, 97, size=600).tolist()
    steps = RNG.integers(0, 97, size=4).tolist()
    _, got = _run(tiny, toks, 256, 2, steps)
    want = _np_logits(NpModel(cfg, _weights(tiny_dir)), toks, 256, 2, steps)
    for g, w in zip(got, want):
        assert np.abs(g - w).max() < 1e-4
        assert int(np.argmax(g)) == int(np.argmax(w))


def test_grow_is_a_relayout(tiny_dir):
    """The global cache starts at 16 slots and doubles (model.rs:383-398, 511-513); the
    results must be those of a cache that never grows, bit for bit, and match float64."""
    small = O.Model(tiny_dir, global_cap=16)
    big = O.Model(tiny_dir)
    toks = RNG.integers(0, 97, size=70).tolist()
    a, la = _run(small, toks, 7, 3, steps=[1, 2, 3])
    b, lb = _run(big, toks, 7, 3, steps=[1, 2, 3])
    for x, y in zip(la, lb):
        assert np.array_equal(x, y)
    want = _np_logits(NpModel(big.cfg, _weights(tiny_dir)), toks, 7, 3, [1, 2, 3])
    for g, w in zip(la, want):
        assert np.abs(g - w).max() < 1e-4


def test_planted_mistake_is_caught(tiny_dir):
    """The float64 model must see a wrong loop count and a wrong window as failures."""
    m = O.Model(tiny_dir)
    toks = RNG.integers(0, 97, size=40).tolist()
    _, got = _run(m, toks, 256, 3, [])
    npm = NpModel(m.cfg, _weights(tiny_dir))
    assert np.abs(got[0] - _np_logits(npm, toks, 256, 2, [])[0]).max() > 1e-3
    cfg2 = O.Config(dict(m.cfg.raw, window=m.cfg.window + 1))
    npm2 = NpModel(cfg2, _weights(tiny_dir))
    assert np.abs(got[0] - _np_logits(npm2, toks, 256, 3, [])[0]).max() > 1e-4


# ---------------------------------------------------------------------------------------
# single ops against float64
# ---------------------------------------------------------------------------------------

def _rel(a, b):
    return float(np.abs(np.asarray(a, np.float64) - b).max() / max(np.abs(b).max(), 1e-30))


def test_dot_order():
    """cpu.rs:10-21: sixteen lane sums, then a left-to-right tail."""
    a = RNG.standard_normal(37).astype(np.float32)
    b = RNG.standard_normal(37).astype(np.float32)
    out = np.zeros(1, np.float32)
    import ctypes
    r = ctypes.c_float()
    O.lib().oracle_dot(a, b, 37, ctypes.byref(r))
    acc = np.zeros(16, np.float32)
    for c in range(2):
        acc = (acc + a[c * 16:(c + 1) * 16] * b[c * 16:(c + 1) * 16]).astype(np.float32)
    s = np.float32(-0.0)
    for v in acc:
        s = np.float32(s + v)
    t = np.float32(-0.0)
    for j in range(32, 37):
        t = np.float32(t + np.float32(a[j] * b[j]))
    assert r.value == np.float32(s + t)


@pytest.mark.parametrize("m", [1, 5])
def test_linear(m):
    rows, cols = 33, 48
    w = RNG.standard_normal((rows, cols)).astype(np.float32)
    x = RNG.standard_normal((m, cols)).astype(np.float32)
    y = O.linear(w, x, rows, cols, m).reshape(m, rows)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    assert _rel(y, ref) < 1e-5
    # a transposed weight must fail the same check
    sq = RNG.standard_normal((cols, cols)).astype(np.float32)
    ref = x.astype(np.float64) @ sq.astype(np.float64).T
    assert _rel(O.linear(sq, x, cols, cols, m).reshape(m, cols), ref) < 1e-5
    assert _rel(O.linear(sq.T.copy(), x, cols, cols, m).reshape(m, cols), ref) > 1e-2


def test_rms_l2norm_silu():
    x = RNG.standard_normal((6, 64)).astype(np.float32)
    w = RNG.standard_normal(64).astype(np.float32)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(-1, keepdims=True) + 1e-6) * w
    assert _rel(O.rms(x, w, 6, 64, 1e-6).reshape(6, 64), ref) < 1e-5
    ref = x64 / np.linalg.norm(x64, axis=-1, keepdims=True)
    assert _rel(O.l2norm(x, 6, 64).reshape(6, 64), ref) < 1e-5
    z = np.zeros((2, 64), np.float32)
    assert np.array_equal(O.l2norm(z, 2, 64), z.reshape(-1))  # max(norm, 1e-12)
    u = RNG.standard_normal(100).astype(np.float32)
    g = RNG.standard_normal(100).astype(np.float32) * 4
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert _rel(O.silu_mul(g, u), ref) < 1e-5


def test_rope():
    dh, heads, m, pos = 16, 3, 4, 1000
    inv = (1.0 / 10000.0 ** (np.arange(dh // 2) * 2 / dh)).astype(np.float32)
    c, s = O.rope_table(inv, pos, m, dh // 2)
    ang = (np.arange(pos, pos + m)[:, None] * inv[None].astype(np.float64))
    assert np.abs(c - np.cos(ang).reshape(-1)).max() < 1e-3  # f32 angle rounding
    x = RNG.standard_normal((m, heads, dh)).astype(np.float32)
    y = O.rope(x, c, s, m, heads, dh).reshape(m, heads, dh)
    c2, s2 = c.reshape(m, 1, -1).astype(np.float64), s.reshape(m, 1, -1).astype(np.float64)
    lo, hi = x[..., :dh // 2], x[..., dh // 2:]
    ref = np.concatenate([lo * c2 - hi * s2, lo * s2 + hi * c2], -1)
    assert _rel(y, ref) < 1e-6
    # a rotation keeps each pair's length
    assert np.allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1), rtol=1e-5)


def test_gla():
    m, heads, dh = 5, 2, 8
    q, k, v = (RNG.standard_normal((m, heads, dh)).astype(np.float32) for _ in range(3))
    dec = RNG.standard_normal((m, heads)).astype(np.float32)
    bias = RNG.standard_normal(heads).astype(np.float32)
    s0 = RNG.standard_normal((heads, dh, dh)).astype(np.float32)
    y, s = O.gla(s0, q, k, v, dec, bias, m, heads, dh)
    S = s0.astype(np.float64)
    ys = []
    for i in range(m):
        g = 1 / (1 + np.exp(dec[i].astype(np.float64) + bias))
        S = g[:, None, None] * S + k[i][:, :, None] * v[i][:, None, :]
        ys.append(np.einsum("ha,hab->hb", q[i], S))
    assert _rel(y.reshape(m, heads, dh), np.stack(ys)) < 1e-5
    assert _rel(s.reshape(heads, dh, dh), S) < 1e-5


def _attend64(q, k, v, pos, m, reach, gap, cap, heads, key_heads, dh, scale):
    out = np.zeros((m, heads, dh))
    group = heads // key_heads
    kk = k.reshape(key_heads, cap, dh).astype(np.float64)
    vv = v.reshape(key_heads, cap, dh).astype(np.float64)
    for i in range(m):
        p = pos + i
        lo, hi = max(0, p - reach + 1), max(0, p + 1 - gap)
        if hi <= lo:
            continue
        slots = np.arange(lo, hi) % cap
        for h in range(heads):
            s = kk[h // group, slots] @ q[i, h].astype(np.float64) * scale
            p_ = np.exp(s - s.max())
            out[i, h] = (p_ / p_.sum()) @ vv[h // group, slots]
    return out


@pytest.mark.parametrize("case", [
    dict(pos=0, m=1, reach=8, gap=0, cap=24, heads=4, key_heads=4),
    dict(pos=30, m=7, reach=8, gap=0, cap=24, heads=4, key_heads=4),    # wraps the ring
    dict(pos=50, m=9, reach=O.USIZE_MAX, gap=8, cap=64, heads=4, key_heads=2),  # global, GQA
    dict(pos=2, m=3, reach=O.USIZE_MAX, gap=8, cap=64, heads=4, key_heads=1),   # sees nothing
])
def test_attend(case):
    dh = 8
    a = dict(case, dh=dh, scale=1 / np.sqrt(dh))
    q = RNG.standard_normal((a["m"], a["heads"], dh)).astype(np.float32)
    k = RNG.standard_normal((a["key_heads"], a["cap"], dh)).astype(np.float32)
    v = RNG.standard_normal((a["key_heads"], a["cap"], dh)).astype(np.float32)
    y = O.attend(q, k, v, **a).reshape(a["m"], a["heads"], dh)
    ref = _attend64(q, k, v, **a)
    assert np.abs(y - ref).max() < 1e-5
    if a["reach"] < 100 and a["pos"] > 10:
        bad = _attend64(q, k, v, **dict(a, reach=a["reach"] + 1))
        assert np.abs(y - bad).max() > 1e-3


def test_attn_ranges():
    """ops.rs:48-66."""
    a = dict(pos=10, m=4, reach=8, gap=0, cap=24, heads=1, key_heads=1, dh=8, scale=1.0)
    assert O.attn_range(0, **a) == (3, 11)
    assert O.attn_span(**a) == 11
    g = dict(a, reach=O.USIZE_MAX, gap=12)
    assert O.attn_range(0, **g) == (0, 0)
    assert O.attn_range(3, **g) == (0, 2)


def test_store_slots():
    heads, dh, cap, pos, m = 2, 4, 5, 3, 4
    src = RNG.standard_normal((m, heads, dh)).astype(np.float32)
    c = O.store(np.zeros(heads * cap * dh, np.float32), src, pos, m, cap, heads, dh)
    c = c.reshape(heads, cap, dh)
    for i in range(m):
        assert np.array_equal(c[:, (pos + i) % cap], src[i])


# ---------------------------------------------------------------------------------------
# src/sample.rs:95-152 and src/config.rs:108-131
# ---------------------------------------------------------------------------------------

def test_pick_known_answers():
    assert O.pick([0.0, 3.0, 1.0]) == 1
    assert O.pick([0.0, 3.0, 2.0], recent=[1], repeat_penalty=2.0, repeat_window=8) == 2
    rng = O.Rng(3)
    for _ in range(200):
        assert O.pick([-9.0, 5.0, -9.0, 1.0], temperature=1.0, top_p=0.5, rng=rng) == 1
    rng = O.Rng(7)
    for _ in range(200):
        assert O.pick([5.0, 4.0, -9.0, -9.0], temperature=1.0, top_k=2, rng=rng) < 2
    assert O.pick([1.0, 1.0, 0.5]) == 0  # the first maximum wins


def test_rng_is_xorshift64star():
    r = O.Rng(5)
    s = (5 * 0x9E3779B97F4A7C15 | 1) & (2 ** 64 - 1)
    for _ in range(5):
        s ^= s >> 12
        s ^= (s << 25) & (2 ** 64 - 1)
        s ^= s >> 27
        want = np.float32(((s * 0x2545F4914F6CDD1D) & (2 ** 64 - 1)) >> 40) / np.float32(1 << 24)
        assert r.next_f32() == want


def test_think_levels(tiny):
    def cfg(dflt, mx):
        return O.Config(dict(tiny.cfg.raw, default_loops=dflt, max_loops=mx))

    levels = lambda c: [c.think_loops(t) for t in ("low", "medium", "high", "max")]
    assert levels(cfg(4, 16)) == [2, 4, 8, 16]
    assert levels(cfg(3, 6)) == [1, 3, 6, 6]
    assert levels(cfg(1, 2)) == [1, 1, 2, 2]
    with pytest.raises(ValueError):
        tiny.cfg.loops(7)
    for bad in ("loop_lora", "state_loops", "global_rope_base"):
        with pytest.raises(ValueError):
            O.Config(dict(tiny.cfg.raw, **{bad: 1}))


def test_state_bytes(tiny):
    se = tiny.session(3)
    se.feed([1, 2, 3], 256)
    c = tiny.cfg
    dh, cap = c.head_dim(), c.window + 256
    win = 2 * c.n_heads * cap * dh
    n = win * (1 + 3 + 1) + 3 * c.n_heads * dh * dh + (2 * c.global_kv_heads * 3 * dh + c.d_model)
    assert se.state_bytes() == n * 4
