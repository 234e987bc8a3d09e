"""The token loop on the GPU: the model twin (src/model.rs restated over the C ABI) against
the reference's PyTorch fixture and against the oracle (src/cpu.rs + src/model.rs
restated), on the reference's own fixture and on seeded synthetic models.

Bars: per-position logits within 1e-4 relative (‖g − c‖∞ / ‖c‖∞) of the
CPU path, identical greedy token ids, and identical ring state (every buffer the model
keeps across steps, model.rs:626-638) after a chunked prompt and after the same prompt
token by token.
"""

import numpy as np
import pytest

import oracle as O
from helpers import greedy, model_dir, rel, synth
from verify import check_parity

pytestmark = pytest.mark.gpu

TOL = 1e-4


@pytest.fixture(scope="module")
def hip(pkg):
    h = pkg.Hip(0)
    print("device:", h.name(), flush=True)
    yield h
    h.close()


@pytest.fixture(scope="module")
def tiny_hip(pkg, hip, tiny_dir):
    return pkg.Model(hip, tiny_dir)


def test_reference_fixture_split_matrix(tiny_hip, tiny_dir):
    """tests/parity.rs:15-46 on the GPU, at the reference's own tolerance (1e-4 abs)."""
    reports = check_parity(tiny_hip, tiny_dir)
    worst = max(r.max_diff for r in reports)
    print(f"max |diff| vs PyTorch fixture: {worst:.3g}; max rel {max(r.max_rel for r in reports):.3g}")
    assert max(r.max_rel for r in reports) < TOL


def _both(pkg, hip, folder, loops, global_cap=None, device_grow=False):
    g = pkg.Model(hip, folder, global_cap=global_cap, device_grow=device_grow)
    c = O.Model(folder, global_cap=global_cap)
    return g, c


def test_c1_tiny_random_greedy(pkg, hip):
    """Tiny shape, seeded N(0, 0.02) weights, a 32-token prompt, R = 2, 16 greedy tokens:
    logits at all 48 positions and the greedy ids against the oracle."""
    folder = model_dir("tiny", 1)
    g, c = _both(pkg, hip, folder, 2)
    prompt = synth.tokens(32, 97, seed=11)
    gs, cs = g.session(2), c.session(2)
    worst = 0.0
    for t in prompt:  # every prompt position, token by token
        gs.step(int(t))
        cs.step(int(t))
        worst = max(worst, rel(gs.logits(), cs.logits()))
    ids_g, ids_c = [], []
    for _ in range(16):
        lg, lc = gs.logits(), cs.logits()
        worst = max(worst, rel(lg, lc))
        ids_g.append(greedy(lg))
        ids_c.append(greedy(lc))
        gs.step(ids_g[-1])
        cs.step(ids_c[-1])
    print(f"C1: max rel {worst:.3g}; ids {ids_g}")
    assert worst < TOL
    assert ids_g == ids_c
    # the C++ decode loop (main.rs:207-223) picks the same ids
    gs2 = g.session(2)
    gs2.feed(prompt, 256)
    assert gs2.decode_greedy(16).tolist() == ids_c


@pytest.mark.parametrize("shape,loops,n", [("tiny", 2, 24), ("a86", 4, 12)])
def test_decode_greedy_device_equals_host_pick(pkg, hip, shape, loops, n):
    """Greedy decode with the pick on the device (the next step's gather reads it there)
    gives the ids of the host loop, and leaves the same session: logits, position and every
    kept buffer bit for bit."""
    folder = model_dir(shape, 1)
    m = pkg.Model(hip, folder)
    prompt = synth.tokens(40, m.cfg.raw["vocab_size"], seed=5)
    a, b = m.session(loops), m.session(loops)
    a.feed(prompt, 256)
    b.feed(prompt, 256)
    ids_host = a.decode_greedy(n).tolist()
    ids_dev = b.decode_greedy_device(n).tolist()
    print(shape, ids_host)
    assert ids_dev == ids_host
    assert a.pos == b.pos
    assert np.array_equal(a.logits(), b.logits())
    _kept_equal(a, b)
    # a second run continues from there (the device slot and ids buffer are reused)
    assert b.decode_greedy_device(3).tolist() == a.decode_greedy(3).tolist()


def _kept_equal(a, b):
    ka, kb = a.kept(), b.kept()
    assert len(ka) == len(kb)
    for i, (x, y) in enumerate(zip(ka, kb)):
        assert x.shape == y.shape, i
        assert np.array_equal(x, y), (i, float(np.abs(x - y).max()))


@pytest.mark.parametrize("chunk", [7, 256])
def test_chunked_equals_step_bitwise(tiny_hip, chunk):
    toks = synth.tokens(300, 97, seed=5)  # past cap = 264: the rings wrap
    a, b = tiny_hip.session(3), tiny_hip.session(3)
    a.feed(toks, 1)
    b.feed(toks, chunk)
    assert np.array_equal(a.logits(), b.logits())
    _kept_equal(a, b)


def test_ring_overwrite_against_oracle(pkg, hip):
    folder = model_dir("tiny", 2)
    g, c = _both(pkg, hip, folder, 3)
    toks = synth.tokens(700, 97, seed=6)
    gs, cs = g.session(3), c.session(3)
    gs.feed(toks, 256)
    cs.feed(toks, 256)
    assert rel(gs.logits(), cs.logits()) < TOL
    for t in synth.tokens(20, 97, seed=7):
        gs.step(int(t))
        cs.step(int(t))
        assert rel(gs.logits(), cs.logits()) < TOL
        assert greedy(gs.logits()) == greedy(cs.logits())


GROW = pytest.mark.parametrize("device_grow", [False, True], ids=["read_upload", "device_copy"])


@GROW
def test_global_grow(pkg, hip, device_grow):
    """Caches that start at 16 slots and double (model.rs:383-398) give the same bits as
    caches that never grow, and match the oracle: through model.rs's own sequence (a read of
    each cache inside the advance, host relayout, upload) and through the device copy."""
    folder = model_dir("tiny", 3)
    small = pkg.Model(hip, folder, global_cap=16, device_grow=device_grow)
    big = pkg.Model(hip, folder)
    c = O.Model(folder)
    toks = synth.tokens(90, 97, seed=8)
    a, b, o = small.session(2), big.session(2), c.session(2)
    for s in (a, b, o):
        s.feed(toks, 13)
    assert np.array_equal(a.logits(), b.logits())
    assert rel(a.logits(), o.logits()) < TOL
    for t in (1, 2, 3):
        a.step(t)
        b.step(t)
        o.step(t)
        assert np.array_equal(a.logits(), b.logits())
        assert rel(a.logits(), o.logits()) < TOL


def test_graphs_match_eager(pkg, hip, tiny_dir):
    """Step graphs replay the same kernels: results are bit-identical to eager launches."""
    m = pkg.Model(hip, tiny_dir)
    toks = synth.tokens(40, 97, seed=9)
    hip.set_graphs(False)
    e = m.session(3)
    e.feed(toks[:20], 8)
    le = []
    for t in toks[20:]:
        e.step(int(t))
        le.append(e.logits())
    hip.set_graphs(True)
    before = hip.graph_stats()
    g = m.session(3)
    g.feed(toks[:20], 8)
    lg = []
    for t in toks[20:]:
        g.step(int(t))
        lg.append(g.logits())
    after = hip.graph_stats()
    for x, y in zip(le, lg):
        assert np.array_equal(x, y)
    _kept_equal(e, g)
    assert after["launched"] - before["launched"] >= 10
    print("graph stats:", after)


def test_a86_short_prompt_against_oracle(pkg, hip):
    """The 86M shape (d 768, 12 x 64, FFN 4x, vocab 32000, window 4096) at R = 4: a 300-token
    prompt in chunks of 256 + 44, then 6 greedy steps."""
    folder = model_dir("a86", 2)
    g, c = _both(pkg, hip, folder, 4)
    toks = synth.tokens(300, 32000, seed=3)
    gs, cs = g.session(4), c.session(4)
    gs.feed(toks, 256)
    cs.feed(toks, 256)
    worst = rel(gs.logits(), cs.logits())
    ids = []
    for _ in range(6):
        lg, lc = gs.logits(), cs.logits()
        worst = max(worst, rel(lg, lc))
        assert greedy(lg) == greedy(lc)
        ids.append(greedy(lg))
        gs.step(ids[-1])
        cs.step(ids[-1])
    print(f"a86: max rel {worst:.3g}; ids {ids}")
    assert worst < TOL


@pytest.mark.parametrize("loops", [4, 8, 16])
def test_a86_chunked_ring_state_equals_step(pkg, hip, loops):
    """Config 3's check at full size: a 4096-token prompt in 256-token chunks leaves the
    same ring state, bit for bit, as the same prompt token by token (R = 4, 8 and 16)."""
    folder = model_dir("a86", 2)
    g = pkg.Model(hip, folder)
    toks = synth.tokens(4096, 32000, seed=4)
    a, b = g.session(loops), g.session(loops)
    a.feed(toks, 256)
    b.feed(toks, 1)
    assert np.array_equal(a.logits(), b.logits())
    _kept_equal(a, b)


def test_a86_prompt_past_the_ring_chunked_equals_step(pkg, hip):
    """Config 3's overwrite run: an 8192-token prompt at R = 4 in 256-token chunks (chunks 17
    and on overwrite ring slots the window has left, 4352 slots) leaves the same state, bit for
    bit, as the same prompt token by token; then 8 greedy steps agree."""
    folder = model_dir("a86", 2)
    g = pkg.Model(hip, folder)
    toks = synth.tokens(8192, 32000, seed=41)
    a, b = g.session(4), g.session(4)
    a.feed(toks, 256)
    b.feed(toks, 1)
    assert np.array_equal(a.logits(), b.logits())
    _kept_equal(a, b)
    assert a.decode_greedy(8).tolist() == b.decode_greedy(8).tolist()
    assert np.array_equal(a.logits(), b.logits())


@pytest.mark.parametrize("name", ["tiny", "a86"])
def test_fused_steps_match_per_op_kernels(pkg, hip, tiny_dir, name):
    """The planner's fused one-token kernels give the same bits as one launch per op."""
    folder = tiny_dir if name == "tiny" else model_dir("a86", 2)
    m = pkg.Model(hip, folder)
    vocab = m.cfg.vocab_size
    toks = synth.tokens(300, vocab, seed=12)
    runs = []
    for fuse in (False, True):
        hip.set_fusion(fuse)
        s = m.session(3 if name == "tiny" else 4)
        s.feed(toks[:260], 256)
        logits = []
        for t in toks[260:]:
            s.step(int(t))
            logits.append(s.logits())
        runs.append((s, logits, hip.last_plan()))
    hip.set_fusion(True)
    (a, la, pa), (b, lb, pb) = runs
    print(f"{name}: one-token step = {pb['ops']} ops -> {pa['kernels']} kernels unfused, "
          f"{pb['kernels']} fused")
    assert pb["kernels"] < pa["kernels"]
    if name == "a86":
        # one kernel per linear group and per attention / GLA: 5 per layer x 12 layers, the
        # inject and the head; every element-wise op rides in a prologue or epilogue
        assert pb["kernels"] <= 62, pb
    for x, y in zip(la, lb):
        assert np.array_equal(x, y)
    _kept_equal(a, b)


@GROW
def test_g86_prompt_against_oracle(pkg, hip, device_grow):
    """Config 4's model (g86: global G layers with 4 key heads, logn / kshift / emb / far on)
    at R = 4: a 700-token prompt in 256-token chunks with global caches that start at 256
    slots and double twice, then 4 greedy steps, against the oracle (both ways of growing)."""
    folder = model_dir("g86", 5)
    g, c = _both(pkg, hip, folder, 4, global_cap=256, device_grow=device_grow)
    toks = synth.tokens(700, 32000, seed=21)
    gs, cs = g.session(4), c.session(4)
    gs.feed(toks, 256)
    cs.feed(toks, 256)
    worst = rel(gs.logits(), cs.logits())
    ids = []
    for _ in range(4):
        lg, lc = gs.logits(), cs.logits()
        worst = max(worst, rel(lg, lc))
        assert greedy(lg) == greedy(lc)
        ids.append(greedy(lg))
        gs.step(ids[-1])
        cs.step(ids[-1])
    print(f"g86: max rel {worst:.3g}; ids {ids}")
    assert worst < TOL


def test_g86_long_prompt_chunked_equals_step(pkg, hip):
    """Config 4's prefill at full size: a 16384-token prompt in 256-token chunks (global caches
    grow to 32768 slots; global attention spans up to 65 superblocks) leaves the same state, bit
    for bit, as the same prompt token by token; then 16 greedy steps agree."""
    folder = model_dir("g86", 5)
    g = pkg.Model(hip, folder)
    toks = synth.tokens(16384, 32000, seed=22)
    a, b = g.session(4), g.session(4)
    a.feed(toks, 256)
    b.feed(toks, 1)
    assert np.array_equal(a.logits(), b.logits())
    _kept_equal(a, b)
    for _ in range(16):
        t = greedy(a.logits())
        assert t == greedy(b.logits())
        a.step(t)
        b.step(t)
    assert np.array_equal(a.logits(), b.logits())


def _arith_prompt(n, seed):
    """Config 5's prompt: seeded random nested arithmetic over 0-9 + - ( ) of depth at most
    10, cut to n characters and mapped through the character vocabulary (digits 17-26,
    ( 9, ) 10, + 12, - 14)."""
    rng = np.random.default_rng(seed)

    def expr(depth):
        if depth >= 10 or rng.random() < 0.3:
            return str(int(rng.integers(0, 100)))
        a, b = expr(depth + 1), expr(depth + 1)
        return "(" + a + "+-"[int(rng.integers(0, 2))] + b + ")"

    text = ""
    while len(text) < n:
        text += expr(0) + "+"
    ids = {str(d): 17 + d for d in range(10)}
    ids.update({"(": 9, ")": 10, "+": 12, "-": 14})
    return [ids[ch] for ch in text[:n]]


def test_c5_fp16_against_fp32_oracle(pkg, hip):
    """Config 5: the 86M model at R = 16 in fp16 mode, a 512-character arithmetic prompt, one
    greedy token: logits within 2e-2 relative of the fp32 oracle. fp16 mode keeps the
    chunked-equals-step invariant (bitwise)."""
    folder = model_dir("a86", 2)
    toks = _arith_prompt(512, 5)
    c = O.Model(folder)
    cs = c.session(16)
    cs.feed(toks, 256)
    want = cs.logits()
    hip.set_fp16(True)
    try:
        g = pkg.Model(hip, folder)
        a, b = g.session(16), g.session(16)
        a.feed(toks, 256)
        b.feed(toks, 1)
        got = a.logits()
        assert np.array_equal(got, b.logits())
        _kept_equal(a, b)
        err = rel(got, want)
        top = np.sort(want)[-2:]
        print(f"C5 fp16: rel {err:.3g}; greedy {greedy(got)} vs {greedy(want)} (oracle top-2 margin {top[1] - top[0]:.3g})")
        assert err < 2e-2
        if top[1] - top[0] > 4 * err * np.abs(want).max():
            assert greedy(got) == greedy(want)
    finally:
        hip.set_fp16(False)


def test_a86_fp16_mode_keeps_fp16_values(pkg, hip):
    """fp16 mode as mlx.rs keeps its Float16 arrays (mlx.rs:19-23, 53-67): with the model loaded
    in the mode, after a 300-token prompt (chunks of 256 + 44) and 4 steps at R = 4 every
    buffer the session keeps (rings, GLA states, the residual and loop states) and the logits
    hold fp16 values; chunked == token by token bitwise; within 2e-2 of the fp32 oracle."""
    folder = model_dir("a86", 2)
    toks = synth.tokens(304, 32000, seed=41)
    c = O.Model(folder)
    cs = c.session(4)
    cs.feed(toks[:300], 256)
    hip.set_fp16(True)
    try:
        g = pkg.Model(hip, folder)
        a, b = g.session(4), g.session(4)
        a.feed(toks[:300], 256)
        b.feed(toks[:300], 1)
        assert np.array_equal(a.logits(), b.logits())
        _kept_equal(a, b)
        worst = rel(a.logits(), cs.logits())
        for t in toks[300:]:
            a.step(int(t))
            cs.step(int(t))
            worst = max(worst, rel(a.logits(), cs.logits()))
        kept = a.kept()
        for i, x in enumerate(kept):
            assert np.array_equal(x, x.astype(np.float16).astype(np.float32)), i
        lg = a.logits()
        assert np.array_equal(lg, lg.astype(np.float16).astype(np.float32))
        print(f"fp16 values: {len(kept)} kept buffers; rel vs fp32 oracle {worst:.3g}")
        assert worst < 2e-2
    finally:
        hip.set_fp16(False)


def test_a86_fp16_mode_reads_half_weights(pkg, hip):
    """fp16 mode through the unchanged trait: the model uploads fp32 weights (ops.rs:77, as
    model.rs does), and the backend's linears read fp16 copies of them (half the bytes) with
    the bits of fp16 mode over the fp32 weights: a 300-token prompt (chunks of 256 + 44: the
    prompt GEMMs and their epilogues) and 8 greedy steps (the fused GEMV) at R = 4, with the
    fp16-weight kernels the ones that ran; then with step graphs and the device pick."""
    folder = model_dir("a86", 2)
    hip.set_fp16(True)
    try:
        g = pkg.Model(hip, folder)
        toks = synth.tokens(300, 32000, seed=3)
        a, b = g.session(4), g.session(4)
        hip.set_half_shadows(False)  # a: fp32 weights, rounded by each linear
        a.feed(toks, 256)
        want0 = a.logits()
        toks8, want = [], []
        for t in range(8):
            toks8.append(greedy(a.logits()))
            a.step(toks8[-1])
            want.append(a.logits())
        hip.set_half_shadows(True)  # b: the fp16 copies
        hip.set_graphs(False)
        hip.set_timing(True)
        b.feed(toks, 256)
        assert np.array_equal(b.logits(), want0)
        assert hip.kernel_stat("slm_gemm2hrw_64")["launches"] > 0
        assert hip.kernel_stat("slm_gemm2hr_64")["launches"] == 0
        hip.set_timing(False)
        hip.set_timing(True)
        for t in range(8):
            b.step(toks8[t])
            assert np.array_equal(b.logits(), want[t]), t
        assert hip.kernel_stat("slm_fghw")["launches"] > 0
        assert hip.kernel_stat("slm_fgh")["launches"] == 0
        hip.set_timing(False)
        hip.set_graphs(True)
        ids_b = b.decode_greedy_device(6).tolist()
        hip.set_half_shadows(False)
        ids_a = a.decode_greedy(6).tolist()
        assert ids_a == ids_b
        assert np.array_equal(a.logits(), b.logits())
    finally:
        hip.set_half_shadows(True)
        hip.set_timing(False)
        hip.set_graphs(True)
        hip.set_fp16(False)


def test_dropped_sessions_give_their_memory_back(pkg, hip):
    """A server makes a session per request and drops it (serve.rs:369, main.rs:308), and a Rust
    `HipBuf` frees its buffer on drop as cuda.rs's `CudaSlice` does: 40 a86 sessions at R = 16
    (about 538 MB of rings and state each), each fed a 600-token prompt (three chunks: the
    prompt lanes' copies of the scratch buffers too) and stepped, then freed, leave the
    device's free memory and the context's holdings where the first such session left them."""
    g = pkg.Model(hip, model_dir("a86", 2))
    toks = synth.tokens(600, 32000, seed=4)
    s = g.session(16)
    s.feed(toks, 256)
    s.step(1)
    del s
    free0, total, held0 = hip.mem_info()
    for i in range(40):
        s = g.session(16)
        assert s.state_bytes() > 500e6
        s.feed(toks, 256)
        s.step(int(toks[i]))
        del s
    free1, _, held1 = hip.mem_info()
    print(f"after 40 sessions: device free {free0 / 2**30:.2f} -> {free1 / 2**30:.2f} GiB of "
          f"{total / 2**30:.0f}; held {held0 / 2**20:.0f} -> {held1 / 2**20:.0f} MiB")
    assert held1 <= held0
    assert free0 - free1 < 64 << 20


# ---------------------------------------------------------------------------------------
# prompt lanes: consecutive prompt steps on several streams at once
# ---------------------------------------------------------------------------------------

class _Lanes:
    """Sets the context's prompt lanes for a block and restores them after."""

    def __init__(self, hip, n):
        self.hip, self.n = hip, n

    def __enter__(self):
        self.old = self.hip.prompt_lanes()
        self.hip.set_prompt_lanes(self.n)
        return self

    def __exit__(self, *exc):
        self.hip.set_prompt_lanes(self.old)


def test_prompt_lane_counts(pkg, hip):
    """1 to 4 lanes; anything else is refused and leaves the setting as it was."""
    n0 = hip.prompt_lanes()
    for bad in (0, 5, -1):
        with pytest.raises(pkg.SlmError):
            hip.set_prompt_lanes(bad)
        assert hip.prompt_lanes() == n0
    for n in (1, 2, 3, 4):
        hip.set_prompt_lanes(n)
        assert hip.prompt_lanes() == n
    hip.set_prompt_lanes(n0)


def _prompt(g, loops, toks):
    """main.rs:309's warm-up then the prompt, as the bench runs it."""
    s = g.session(loops)
    s.feed(toks[:16], 256)
    s.logits()
    s.feed(toks[16:], 256)
    return s


@pytest.mark.parametrize("lanes", [2, 3, 4])
def test_prompt_lanes_same_bits(pkg, hip, lanes):
    """a86 at R = 4, 16 + 2048 prompt tokens: with chunks on 2, 3 and 4 streams at once, the
    logits and every kept buffer equal one stream's bit for bit, and so do 8 greedy steps
    after (each joining the lanes first)."""
    g = pkg.Model(hip, model_dir("a86", 2))
    toks = synth.tokens(2064, 32000, seed=31)
    with _Lanes(hip, 1):
        a = _prompt(g, 4, toks)
        la = a.logits()
    with _Lanes(hip, lanes):
        st0 = hip.lane_stats()
        b = _prompt(g, 4, toks)
        lb = b.logits()
        st1 = hip.lane_stats()
    print(f"lanes {lanes}: {st1['steps'] - st0['steps']} steps on lanes, "
          f"{st1['fallbacks'] - st0['fallbacks']} on the context's stream")
    assert st1["steps"] - st0["steps"] >= 7  # 8 chunks after the warm-up; the first may grow outputs
    assert np.array_equal(la, lb)
    _kept_equal(a, b)
    assert a.decode_greedy(8).tolist() == b.decode_greedy(8).tolist()
    assert np.array_equal(a.logits(), b.logits())


def test_prompt_lanes_interleaved_sessions(pkg, hip):
    """Two sessions fed chunk by chunk in turn (consecutive steps of different sessions: no
    kept buffer in common) on 3 lanes leave the states one stream leaves feeding each alone."""
    g = pkg.Model(hip, model_dir("a86", 2))
    ta = synth.tokens(1280, 32000, seed=32)
    tb = synth.tokens(1100, 32000, seed=33)
    with _Lanes(hip, 1):
        a1 = g.session(4)
        a1.feed(ta, 256)
        b1 = g.session(8)
        b1.feed(tb, 256)
        la1, lb1 = a1.logits(), b1.logits()
    with _Lanes(hip, 3):
        a3, b3 = g.session(4), g.session(8)
        ia = ib = 0
        while ia < len(ta) or ib < len(tb):
            if ia < len(ta):
                n = min(256, len(ta) - ia)
                a3.advance(ta[ia:ia + n], ia + n == len(ta))
                ia += n
            if ib < len(tb):
                n = min(256, len(tb) - ib)
                b3.advance(tb[ib:ib + n], ib + n == len(tb))
                ib += n
        la3, lb3 = a3.logits(), b3.logits()
    assert np.array_equal(la1, la3)
    assert np.array_equal(lb1, lb3)
    _kept_equal(a1, a3)
    _kept_equal(b1, b3)


@GROW
def test_prompt_lanes_g86_growing_caches(pkg, hip, device_grow):
    """g86 (global caches doubling 256 -> 1024 inside the prompt, kshift state, 4 key heads):
    a 700-token prompt in 256- and 64-token chunks on 3 lanes equals one stream's state."""
    g = pkg.Model(hip, model_dir("g86", 5), global_cap=256, device_grow=device_grow)
    toks = synth.tokens(700, 32000, seed=34)
    for chunk in (256, 64):
        with _Lanes(hip, 1):
            a = g.session(4)
            a.feed(toks, chunk)
            la = a.logits()
        with _Lanes(hip, 3):
            b = g.session(4)
            b.feed(toks, chunk)
            lb = b.logits()
        assert np.array_equal(la, lb), chunk
        _kept_equal(a, b)


def test_prompt_lanes_tiny_every_layer_kind(tiny_hip, hip):
    """The reference fixture's shape (window, linear and global layers, R = 3): 300 tokens in
    7-token chunks (the rings wrap) on 4 lanes equal one stream's state."""
    toks = synth.tokens(300, 97, seed=5)
    with _Lanes(hip, 1):
        a = tiny_hip.session(3)
        a.feed(toks, 7)
        la = a.logits()
    with _Lanes(hip, 4):
        b = tiny_hip.session(3)
        b.feed(toks, 7)
        lb = b.logits()
    assert np.array_equal(la, lb)
    _kept_equal(a, b)


def test_prompt_lanes_fp16_rings(pkg, hip):
    """fp16 mode (fp16 weight copies and rings), a86 at R = 16, 1040 prompt tokens on 3 lanes:
    the same bits as one stream."""
    g = pkg.Model(hip, model_dir("a86", 2))
    toks = synth.tokens(1040, 32000, seed=35)
    hip.set_fp16(True)
    try:
        with _Lanes(hip, 1):
            a = _prompt(g, 16, toks)
            la = a.logits()
        with _Lanes(hip, 3):
            b = _prompt(g, 16, toks)
            lb = b.logits()
    finally:
        hip.set_fp16(False)
    assert np.array_equal(la, lb)
    _kept_equal(a, b)


def test_prompt_lanes_with_decode_steps_between(pkg, hip):
    """One session decodes (one-token steps through the step graph, on the context's stream)
    after every two prompt chunks of another (lanes 0 and 1): the lanes are joined and entered
    again around every step, and both sessions end as they do on one stream."""
    g = pkg.Model(hip, model_dir("a86", 2))
    ta = synth.tokens(300, 32000, seed=36)
    tb = synth.tokens(1300, 32000, seed=37)

    steps = synth.tokens(8, 32000, seed=38)

    def run(lanes):
        with _Lanes(hip, lanes):
            a, b = g.session(4), g.session(4)
            a.feed(ta, 256)
            st0 = hip.lane_stats()
            i = k = 0
            while i < len(tb):  # two chunks of b (lanes 0 and 1), then a step of a (a join)
                for _ in range(2):
                    n = min(256, len(tb) - i)
                    if n > 0:
                        b.advance(tb[i:i + n], i + n == len(tb))
                        i += n
                a.step(int(steps[k]))
                k += 1
            st1 = hip.lane_stats()
            return a, b, st1["steps"] - st0["steps"], a.logits(), b.logits()

    a1, b1, n1, la1, lb1 = run(1)
    a3, b3, n3, la3, lb3 = run(3)
    assert n1 == 0 and n3 >= 3
    assert np.array_equal(la1, la3)
    assert np.array_equal(lb1, lb3)
    _kept_equal(a1, a3)
    _kept_equal(b1, b3)
