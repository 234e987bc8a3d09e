"""One-launch steps (slm_step_*, opt-in): a one-token step whose planned kernels are fused
GEMVs, one-token attentions and one-token GLAs runs as one launch of 256 workgroups that runs
those kernels' work as phases. The same arithmetic runs, so every value is bit-identical to
the step replayed as a graph of separate kernels (model.rs:563-640 through the same trait
calls).
"""

import numpy as np
import pytest

import oracle as O
from helpers import model_dir, rel, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip(pkg):
    h = pkg.Hip(0)
    print("device:", h.name(), flush=True)
    yield h
    h.set_step_kernel(False)
    h.close()


def _kept_equal(a, b):
    ka, kb = a.kept(), b.kept()
    assert len(ka) == len(kb)
    for i, (x, y) in enumerate(zip(ka, kb)):
        assert x.shape == y.shape, i
        assert np.array_equal(x, y), (i, float(np.abs(x - y).max()))


def _run(hip, m, loops, toks, prompt, chunk, step_on):
    hip.set_step_kernel(step_on)
    s = m.session(loops)
    s.feed(toks[:prompt], chunk)
    out = [s.logits()]
    for t in toks[prompt:]:
        s.step(int(t))
        out.append(s.logits())
    return s, out


def test_step_kernel_available(hip):
    st = hip.step_stats()
    print("step stats:", st, flush=True)
    assert st["available"]


def test_step_launch_equals_graph_tiny(pkg, hip, tiny_dir):
    """The reference fixture (every layer kind): steps that can be one launch run as one,
    the rest replay graphs; logits and every kept buffer equal the graph path bit for bit."""
    print("tiny fixture, step on vs off", flush=True)
    m = pkg.Model(hip, tiny_dir)
    toks = synth.tokens(60, 97, seed=21)
    a, la = _run(hip, m, 3, toks, 20, 8, False)
    b, lb = _run(hip, m, 3, toks, 20, 8, True)
    for i, (x, y) in enumerate(zip(la, lb)):
        assert np.array_equal(x, y), i
    _kept_equal(a, b)
    print("step stats:", hip.step_stats(), flush=True)


def test_step_launch_equals_graph_a86(pkg, hip):
    """a86 (S and L blocks) at R = 4: a 300-token prompt, then 12 greedy-fed steps, each one
    launch; logits and kept buffers equal the graph path bit for bit, and the oracle within
    1e-4."""
    print("a86 R=4, step on vs off", flush=True)
    folder = model_dir("a86", 2)
    m = pkg.Model(hip, folder)
    toks = synth.tokens(312, 32000, seed=22)
    a, la = _run(hip, m, 4, toks, 300, 256, False)
    s0 = hip.step_stats()["launches"]
    b, lb = _run(hip, m, 4, toks, 300, 256, True)
    s1 = hip.step_stats()["launches"]
    assert s1 - s0 == 12
    for i, (x, y) in enumerate(zip(la, lb)):
        assert np.array_equal(x, y), i
    _kept_equal(a, b)
    c = O.Model(folder)
    cs = c.session(4)
    cs.feed(toks[:300], 256)
    for t in toks[300:304]:
        cs.step(int(t))
    assert rel(lb[4], cs.logits()) < 1e-4


def test_step_launch_device_pick(pkg, hip):
    """The logits GEMV's fused greedy pick as the last phase: the same ids as the host pick
    over the graph path, twice in a row."""
    print("a86 R=4, device pick in one launch", flush=True)
    folder = model_dir("a86", 2)
    m = pkg.Model(hip, folder)
    toks = synth.tokens(64, 32000, seed=23)
    hip.set_step_kernel(False)
    a = m.session(4)
    a.feed(toks, 64)
    want = a.decode_greedy(6).tolist()
    hip.set_step_kernel(True)
    b = m.session(4)
    b.feed(toks, 64)
    s0 = hip.step_stats()["launches"]
    got = b.decode_greedy_device(3).tolist() + b.decode_greedy_device(3).tolist()
    assert hip.step_stats()["launches"] - s0 >= 6
    assert got == want
    _kept_equal(a, b)


def test_step_launch_gives_up_and_recovers(pkg, hip):
    """A spin limit of 0 makes every wait give up at once: the launch ends early, the next
    read reports SLM_E_HIP once, and with the limit back the next steps are right again."""
    print("a86 R=4, forced give-up", flush=True)
    folder = model_dir("a86", 2)
    m = pkg.Model(hip, folder)
    toks = synth.tokens(40, 32000, seed=24)
    hip.set_step_kernel(True)
    a = m.session(4)
    a.feed(toks[:32], 32)
    hip.set_spin_limit(0)
    try:
        a.step(int(toks[32]))
        with pytest.raises(pkg.SlmError) as e:
            a.logits()
        assert "gave up" in str(e.value)
    finally:
        hip.set_spin_limit(1 << 24)
    b = m.session(4)
    c = m.session(4)
    hip.set_step_kernel(False)
    b.feed(toks[:32], 32)
    for t in toks[32:]:
        b.step(int(t))
    hip.set_step_kernel(True)
    c.feed(toks[:32], 32)
    for t in toks[32:]:
        c.step(int(t))
    assert np.array_equal(b.logits(), c.logits())
    _kept_equal(b, c)
