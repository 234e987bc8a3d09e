"""slm_hip_attend_noalloc (the allocation-free attention entry point) against slm_hip_attend:
the same bits, on two calls in a row (the second smaller, so the fixed scratch still holds the
first call's larger contents), through the C ABI; and its two refusals, each of which leaves
the output untouched: partials beyond the 16 MiB scratch, and a call inside a recorded step.
"""
import numpy as np
import pytest

import oracle as O
from helpers import rel

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(11)
SCRATCH_BYTES = 16 << 20


def rnd(*shape):
    return RNG.standard_normal(shape).astype(np.float32)


@pytest.fixture(scope="module")
def hip(pkg):
    h = pkg.Hip(0)
    print("device:", h.name(), flush=True)
    yield h
    h.close()


def part_bytes(a):
    """nsb · m · heads · (dp + 2) · 4: the superblock partials of one call (a window: a fixed
    count of 256-key superblocks; unbounded reach: the superblocks the keys span)."""
    m, dh = a["m"], a["dh"]
    if a["reach"] < (1 << 49):
        nsb = (a["reach"] + m - 2) // 256 + 2
    else:
        first = 0 if a["reach"] - 1 > a["pos"] else a["pos"] - (a["reach"] - 1)
        last = a["pos"] + m - 1 - a["gap"]
        nsb = last // 256 - first // 256 + 1 if last >= first else 1
    dp = 16
    while dp < dh:
        dp *= 2
    return nsb * m * a["heads"] * (dp + 2) * 4


def both(hip, a, q, k, v):
    """(slm_hip_attend's output, slm_hip_attend_noalloc's output) on the same device inputs."""
    m, heads, dh = a["m"], a["heads"], a["dh"]
    dq, dk, dv = hip.upload(q), hip.upload(k), hip.upload(v)
    y0, y1 = hip.alloc(m * heads * dh), hip.alloc(m * heads * dh)
    hip.attend(y0.ptr, dq.ptr, dk.ptr, dv.ptr, **a)
    want = y0.read()
    print("case:", {x: a[x] for x in ("pos", "m", "reach", "heads", "key_heads", "dh")}, flush=True)
    hip.attend_noalloc(y1.ptr, dq.ptr, dk.ptr, dv.ptr, **a)
    return want, y1.read()


# a prompt chunk of 256 queries against a full 4096-key window (14.6 MB of partials), then one
# query over the same ring (57 KB), a global-attention call with 4 key heads, and head size
# 128 (the general kernel) with 20 queries and then one
CALLS = [
    dict(pos=5000, m=256, reach=4096, gap=0, cap=4352, heads=12, key_heads=12, dh=64),
    dict(pos=4100, m=1, reach=4096, gap=0, cap=4352, heads=12, key_heads=12, dh=64),
    dict(pos=9000, m=40, reach=O.USIZE_MAX, gap=4096, cap=16384, heads=12, key_heads=4, dh=64),
    dict(pos=700, m=20, reach=512, gap=0, cap=600, heads=4, key_heads=2, dh=128),
    dict(pos=700, m=1, reach=512, gap=0, cap=600, heads=4, key_heads=2, dh=128),
]


def test_noalloc_equals_attend_on_calls_in_a_row(hip):
    for a in CALLS:
        a = dict(a, scale=0.125)
        assert part_bytes(a) <= SCRATCH_BYTES
        q = rnd(a["m"], a["heads"], a["dh"])
        k = rnd(a["key_heads"], a["cap"], a["dh"])
        v = rnd(a["key_heads"], a["cap"], a["dh"])
        want, got = both(hip, a, q, k, v)
        assert np.array_equal(got, want), a
        if a["m"] <= 40:  # and the oracle (a small case: the restatement runs in seconds)
            assert rel(got, O.attend(q, k, v, **a)) < 1e-5


def test_noalloc_refuses_partials_beyond_the_scratch(hip, pkg):
    a = dict(pos=5000, m=300, reach=4096, gap=0, cap=4352, heads=12, key_heads=12, dh=64, scale=0.125)
    assert part_bytes(a) > SCRATCH_BYTES
    dq = hip.upload(rnd(a["m"], a["heads"], a["dh"]))
    dk = hip.upload(rnd(a["key_heads"], a["cap"], a["dh"]))
    dv = hip.upload(rnd(a["key_heads"], a["cap"], a["dh"]))
    y = hip.upload(np.full(a["m"] * a["heads"] * a["dh"], 7.0, np.float32))
    with pytest.raises(pkg.SlmError) as e:
        hip.attend_noalloc(y.ptr, dq.ptr, dk.ptr, dv.ptr, **a)
    assert e.value.code == -3 and "fixed scratch" in str(e.value)
    assert np.all(y.read() == 7.0)
    # the same call through slm_hip_attend (its workspace grows) still runs
    hip.attend(y.ptr, dq.ptr, dk.ptr, dv.ptr, **a)
    assert np.all(np.isfinite(y.read()))


def test_noalloc_refuses_inside_a_recorded_step(hip, pkg):
    a = dict(CALLS[1], scale=0.125)
    inv = hip.upload(np.ones(32, np.float32))
    cs, sn = hip.alloc(32), hip.alloc(32)
    dq = hip.upload(rnd(a["m"], a["heads"], a["dh"]))
    dk = hip.upload(rnd(a["key_heads"], a["cap"], a["dh"]))
    dv = hip.upload(rnd(a["key_heads"], a["cap"], a["dh"]))
    y = hip.upload(np.full(a["heads"] * a["dh"], 7.0, np.float32))
    hip.rope_table(cs.ptr, sn.ptr, inv.ptr, 7, 1, 32)  # a step begins
    with pytest.raises(pkg.SlmError) as e:
        hip.attend_noalloc(y.ptr, dq.ptr, dk.ptr, dv.ptr, **a)
    assert e.value.code == -3 and "recorded step" in str(e.value)
    hip.flush()
    assert np.all(y.read() == 7.0)
    # outside the step it runs, and gives slm_hip_attend's bits
    hip.attend_noalloc(y.ptr, dq.ptr, dk.ptr, dv.ptr, **a)
    got = y.read()
    hip.attend(y.ptr, dq.ptr, dk.ptr, dv.ptr, **a)
    assert np.array_equal(got, y.read())
