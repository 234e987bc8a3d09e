"""The token loop at its full sizes against the oracle: the benchmark sequences themselves,
not scaled-down stand-ins.

  - a86 at R = 4 (the headline configuration): 16 warm-up tokens, a 4096-token prompt in
    256-token chunks (the window fills), then 256 greedy steps, positions 4112..4367, past the
    4352-slot ring (window + 256), so that the rings overwrite (src/main.rs:285-315);
  - a86 at R = 16 (the deepest loop count the bench runs): the 4096-token prompt, 128 steps;
  - g86 at R = 4 (global layers with logn, kshift, emb and far, 4 key heads): a 16384-token
    prompt in 256-token chunks (the global caches grow to 32768 slots), 128 steps.

Bars: the logits after the prompt and at every decode step within 1e-4 relative
(‖g − c‖∞ / ‖c‖∞) of the oracle, and the greedy ids (sample.rs:48-53, the first maximum)
identical at every step. Each side picks from its own logits; the next token fed to both is
the oracle's pick.
"""

import time

import numpy as np
import pytest

import oracle as O
from helpers import greedy, model_dir, rel, synth

pytestmark = pytest.mark.gpu

TOL = 1e-4


@pytest.fixture(scope="module")
def hip(pkg):
    h = pkg.Hip(0)
    print("device:", h.name(), flush=True)
    yield h
    h.close()


def run(pkg, hip, name, seed, loops, prompt, steps, warm=0, device_grow=False):
    folder = model_dir(name, seed)
    g, c = pkg.Model(hip, folder, device_grow=device_grow), O.Model(folder)
    gs, cs = g.session(loops), c.session(loops)
    t0 = time.perf_counter()
    if warm:
        gs.feed(prompt[:warm], 256)
        cs.feed(prompt[:warm], 256)
    gs.feed(prompt, 256)
    cs.feed(prompt, 256)
    worst = rel(gs.logits(), cs.logits())
    print(f"{name} R={loops}: prompt {len(prompt)} at pos {cs.pos}, rel {worst:.3g} "
          f"({time.perf_counter() - t0:.0f} s)", flush=True)
    assert worst < TOL
    ids = []
    for t in range(steps):
        lg, lc = gs.logits(), cs.logits()
        e = rel(lg, lc)
        worst = max(worst, e)
        assert e < TOL, (t, cs.pos, e)
        assert greedy(lg) == greedy(lc), (t, cs.pos)
        ids.append(greedy(lc))
        gs.step(ids[-1])
        cs.step(ids[-1])
    e = rel(gs.logits(), cs.logits())
    worst = max(worst, e)
    assert e < TOL
    assert gs.pos == cs.pos
    print(f"{name} R={loops}: {steps} steps to pos {cs.pos}, max rel {worst:.3g}, "
          f"{len(set(ids))} distinct ids ({time.perf_counter() - t0:.0f} s)", flush=True)
    return worst, ids


def test_a86_bench_sequence_r4_past_the_ring(pkg, hip):
    prompt = synth.tokens(4096, 32000, seed=3)
    worst, ids = run(pkg, hip, "a86", 2, 4, prompt, 256, warm=16)
    assert 16 + 4096 + 256 > 4352


def test_a86_r16_prompt_4096(pkg, hip):
    prompt = synth.tokens(4096, 32000, seed=3)
    run(pkg, hip, "a86", 2, 16, prompt, 128)


@pytest.mark.parametrize("device_grow", [False, True], ids=["read_upload", "device_copy"])
def test_g86_prompt_16384(pkg, hip, device_grow):
    """The global caches grow 8192 -> 16384 -> 32768 inside the prompt: through model.rs's own
    sequence (read, host relayout, upload inside the advance) and through device copies."""
    prompt = synth.tokens(16384, 32000, seed=6)
    run(pkg, hip, "g86", 4, 4, prompt, 128, device_grow=device_grow)
