"""Every operation of the C ABI on the GPU against the oracle (the restatement of
src/cpu.rs), on seeded inputs, plus the property the token loop depends on: each output is
computed the same way whatever the number of tokens in the call, so m = 1 and m = 256
give the same bits.

Tolerances: bit-exact where the kernel follows the reference's order exactly (data
movement, rms, l2norm, rope, rope_table); otherwise 2e-6 relative to the largest output
(linear, gla: MFMA / tree reassociation; silu: device expf), and for attention 1e-5
relative plus an error against float64 no larger than twice the oracle's own.
"""

import numpy as np
import pytest

import oracle as O
from helpers import attend64, rel

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(7)


@pytest.fixture(scope="module")
def hip(pkg):
    h = pkg.Hip(0)
    print("device:", h.name(), flush=True)
    yield h
    h.close()


def rnd(*shape, scale=1.0):
    return (RNG.standard_normal(shape) * scale).astype(np.float32)


def test_mfma_lane_layout(hip):
    """v_mfma_f32_16x16x4f32: lane l holds A[l%16][l/16], B[l/16][l%16] and
    D[4(l/16)+r][l%16] — the layout every linear and attention kernel assumes."""
    a = np.arange(64, dtype=np.float32)
    b = (np.arange(64, dtype=np.float32) % 7) - 3
    A = np.zeros((16, 4))
    B = np.zeros((4, 16))
    for l in range(64):
        A[l % 16, l // 16] = a[l]
        B[l // 16, l % 16] = b[l]
    D = A @ B
    out = hip.alloc(256)
    da, db = hip.upload(a), hip.upload(b)
    hip.probe_mfma(out.ptr, da.ptr, db.ptr)
    got = out.read().reshape(64, 4)
    for l in range(64):
        for r in range(4):
            assert got[l, r] == D[4 * (l // 16) + r, l % 16]


LINEAR_SHAPES = [(96, 32, 1), (2304, 768, 1), (768, 3072, 1), (32000, 768, 1), (768, 768, 5),
                 (13, 37, 3), (768, 768, 16), (768, 768, 17), (2304, 768, 256),
                 (6144, 768, 256), (768, 3072, 256), (12, 768, 256), (50, 21, 70),
                 (2300, 768, 200), (100, 1536, 100)]


@pytest.mark.parametrize("rows,cols,m", LINEAR_SHAPES)
def test_linear(hip, rows, cols, m):
    w = rnd(rows, cols, scale=0.02)
    x = rnd(m, cols)
    dw, dx, dy = hip.upload(w), hip.upload(x), hip.alloc(m * rows)
    hip.linear(dy.ptr, dw.ptr, rows, cols, dx.ptr, m)
    got = dy.read(m * rows)
    want = O.linear(w, x, rows, cols, m)
    assert rel(got, want) < 2e-6, (rows, cols, m)


@pytest.mark.parametrize("rows,cols", [(768, 768), (6144, 768), (768, 3072), (97, 32), (40, 52),
                                       (64, 1600), (8192, 768), (2300, 768), (6150, 768)])
def test_linear_same_bits_for_any_m(hip, rows, cols):
    """The decode kernel (m <= 16) and the prompt kernels (m > 16, every row tile: 32, 64,
    96 and 128 rows, ragged last tiles) run one MFMA chain."""
    m = 256
    w = rnd(rows, cols, scale=0.02)
    x = rnd(m, cols)
    dw, dx = hip.upload(w), hip.upload(x)
    full = hip.alloc(m * rows)
    hip.linear(full.ptr, dw.ptr, rows, cols, dx.ptr, m)
    ref = full.read(m * rows).reshape(m, rows)
    one = hip.alloc(rows)
    for i in [0, 1, 17, 100, 255]:
        hip.linear(one.ptr, dw.ptr, rows, cols, dx.at(i * cols), 1)
        assert np.array_equal(one.read(rows), ref[i]), i
    some = hip.alloc(16 * rows)
    hip.linear(some.ptr, dw.ptr, rows, cols, dx.at(32 * cols), 16)
    assert np.array_equal(some.read(16 * rows).reshape(16, rows), ref[32:48])
    odd = hip.alloc(33 * rows)
    hip.linear(odd.ptr, dw.ptr, rows, cols, dx.at(7 * cols), 33)
    assert np.array_equal(odd.read(33 * rows).reshape(33, rows), ref[7:40])


@pytest.mark.parametrize("groups,size", [(1, 768), (256, 768), (3072, 64), (4, 8), (5, 37)])
def test_rms_bit_exact(hip, groups, size):
    x = rnd(groups, size)
    w = rnd(size)
    dx, dw, dy = hip.upload(x), hip.upload(w), hip.alloc(groups * size)
    hip.rms(dy.ptr, dx.ptr, dw.ptr, groups, size, 1e-6)
    assert np.array_equal(dy.read(), O.rms(x, w, groups, size, 1e-6))


@pytest.mark.parametrize("heads,dh", [(12, 64), (3072, 64), (4, 8), (3, 20)])
def test_l2norm_bit_exact(hip, heads, dh):
    x = rnd(heads, dh)
    x[0] = 0.0  # max(norm, 1e-12)
    dx, dy = hip.upload(x), hip.alloc(heads * dh)
    hip.l2norm(dy.ptr, dx.ptr, heads, dh)
    assert np.array_equal(dy.read(), O.l2norm(x, heads, dh))


def test_silu_mul(hip):
    n = 256 * 3072
    g, u = rnd(n, scale=3.0), rnd(n)
    dg, du, dy = hip.upload(g), hip.upload(u), hip.alloc(n)
    hip.silu_mul(dy.ptr, dg.ptr, du.ptr, n)
    got, want = dy.read(), O.silu_mul(g, u)
    assert np.abs(got - want).max() <= 2e-6 * np.abs(want).max()


@pytest.mark.parametrize("pos,m", [(0, 1), (4095, 1), (100, 256), (20000, 3)])
def test_rope_table_and_rope_bit_exact(hip, pos, m):
    dh, heads = 64, 12
    half = dh // 2
    inv = (1.0 / np.power(np.float32(10000.0),
                          (2 * np.arange(half)).astype(np.float32) / np.float32(dh))).astype(np.float32)
    dinv = hip.upload(inv)
    dc, ds = hip.alloc(m * half), hip.alloc(m * half)
    hip.set_graphs(False)
    hip.rope_table(dc.ptr, ds.ptr, dinv.ptr, pos, m, half)
    wc, ws = O.rope_table(inv, pos, m, half)
    assert np.array_equal(dc.read(), wc) and np.array_equal(ds.read(), ws)
    x = rnd(m, heads, dh)
    dx, dy = hip.upload(x), hip.alloc(m * heads * dh)
    hip.rope(dy.ptr, dx.ptr, dc.ptr, ds.ptr, m, heads, dh)
    assert np.array_equal(dy.read(), O.rope(x, wc, ws, m, heads, dh))
    hip.set_graphs(True)


def test_data_movement_bit_exact(hip):
    m, d = 7, 40
    x, a, b = rnd(m, d), rnd(m, d), rnd(m, d)
    row, first = rnd(d), rnd(d)
    dx, da, db, drow, dfirst = (hip.upload(t) for t in (x, a, b, row, first))
    dy = hip.alloc(m * d)
    hip.copy(dy.ptr, dx.ptr, m * d)
    assert np.array_equal(dy.read(), x.reshape(-1))
    hip.add(dy.ptr, da.ptr, db.ptr, m * d)
    assert np.array_equal(dy.read(), (a + b).reshape(-1))
    hip.add_row(dy.ptr, dx.ptr, drow.ptr, m, d)
    assert np.array_equal(dy.read(), (x + row).reshape(-1))
    hip.mix(dy.ptr, da.ptr, db.ptr, m * d, np.float32(0.3))
    assert np.array_equal(dy.read(), (a + np.float32(0.3) * (b - a)).reshape(-1))
    hip.shift(dy.ptr, dfirst.ptr, dx.ptr, m, d)
    assert np.array_equal(dy.read(), np.concatenate([first[None], x[:-1]]).reshape(-1))
    f = rnd(m)
    hip.scale_rows(dy.ptr, dx.ptr, f, d)
    assert np.array_equal(dy.read(), (x * f[:, None]).reshape(-1))
    hip.scale_rows(dy.ptr, dx.ptr, f[:1], d)
    assert np.array_equal(dy.read(d), x[0] * f[0])
    dc = hip.alloc(m * 10)
    hip.columns(dc.ptr, dx.ptr, m, d, 13, 10)
    assert np.array_equal(dc.read(), x[:, 13:23].reshape(-1))
    w = rnd(50, d)
    dw = hip.upload(w)
    ids = np.array([3, 49, 0, 3, 7, 7, 1], dtype=np.uint32)
    hip.gather(dy.ptr, dw.ptr, ids, d)
    assert np.array_equal(dy.read(), w[ids].reshape(-1))


def test_store_wraps_the_ring(hip):
    heads, dh, cap = 3, 8, 20
    cache = np.zeros((heads, cap, dh), np.float32)
    dcache = hip.upload(cache)
    for pos, m in [(0, 5), (5, 20), (25, 1), (37, 9)]:
        src = rnd(m, heads, dh)
        dsrc = hip.upload(src)
        hip.store(dcache.ptr, dsrc.ptr, pos, m, cap, heads, dh)
        cache = O.store(cache, src, pos, m, cap, heads, dh).reshape(heads, cap, dh)
        assert np.array_equal(dcache.read(), cache.reshape(-1))


def test_bounds_are_checked_before_launch(hip, pkg):
    dy, dx = hip.alloc(10), hip.alloc(10)
    with pytest.raises(pkg.SlmError) as e:
        hip.copy(dy.ptr, dx.ptr, 11)
    assert e.value.code == -5
    dw = hip.alloc(4 * 8)  # 16 rows of 2
    hip.gather(dy.ptr, dw.ptr, np.array([15], np.uint32), 2)
    with pytest.raises(pkg.SlmError):
        hip.gather(dy.ptr, dw.ptr, np.array([16], np.uint32), 2)  # id past the rows
    with pytest.raises(pkg.SlmError):
        hip.linear(dy.ptr, dw.ptr, 10, 4, dx.ptr, 3)  # x too short


@pytest.mark.parametrize("m,heads,dh", [(1, 12, 64), (256, 12, 64), (37, 4, 8), (5, 2, 16),
                                        (300, 3, 16), (96, 2, 32), (70, 2, 128)])
def test_gla(hip, m, heads, dh):
    q, k, v = rnd(m, heads, dh), rnd(m, heads, dh), rnd(m, heads, dh)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    dec = rnd(m, heads)
    bias = rnd(heads) - 3
    s0 = rnd(heads, dh, dh, scale=0.1)
    bufs = [hip.upload(t) for t in (q, k, v, dec, bias, s0)]
    dq, dk, dv, dd, db, ds = bufs
    dy = hip.alloc(m * heads * dh)
    hip.gla(dy.ptr, ds.ptr, dq.ptr, dk.ptr, dv.ptr, dd.ptr, db.ptr, m, heads, dh)
    wy, wst = O.gla(s0, q, k, v, dec, bias, m, heads, dh)
    assert rel(dy.read(), wy) < 2e-6
    assert rel(ds.read(), wst) < 2e-6
    # token by token leaves the same bits
    ds2 = hip.upload(s0)
    dy1 = hip.alloc(heads * dh)
    ys = []
    for i in range(m):
        hip.gla(dy1.ptr, ds2.ptr, dq.at(i * heads * dh), dk.at(i * heads * dh),
                dv.at(i * heads * dh), dd.at(i * heads), db.ptr, 1, heads, dh)
        ys.append(dy1.read())
    assert np.array_equal(np.concatenate(ys), dy.read())
    assert np.array_equal(ds2.read(), ds.read())


def test_gla_unaligned_inputs(hip):
    """q, k and v one float past 16-byte alignment: the prompt kernel copies single floats,
    more pieces per token row than the workgroup has threads."""
    m, heads, dh = 45, 2, 64
    q, k, v = rnd(m, heads, dh), rnd(m, heads, dh), rnd(m, heads, dh)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    dec, bias, s0 = rnd(m, heads), rnd(heads) - 3, rnd(heads, dh, dh, scale=0.1)
    pads = [hip.upload(np.concatenate([np.zeros(1, np.float32), t.ravel()])) for t in (q, k, v)]
    dd, db, ds = hip.upload(dec), hip.upload(bias), hip.upload(s0)
    dy = hip.alloc(m * heads * dh)
    hip.gla(dy.ptr, ds.ptr, pads[0].at(1), pads[1].at(1), pads[2].at(1), dd.ptr, db.ptr, m, heads, dh)
    wy, wst = O.gla(s0, q, k, v, dec, bias, m, heads, dh)
    assert rel(dy.read(), wy) < 2e-6
    assert rel(ds.read(), wst) < 2e-6
    # the same bits as from aligned inputs
    al = [hip.upload(t) for t in (q, k, v)]
    ds2, dy2 = hip.upload(s0), hip.alloc(m * heads * dh)
    hip.gla(dy2.ptr, ds2.ptr, al[0].ptr, al[1].ptr, al[2].ptr, dd.ptr, db.ptr, m, heads, dh)
    assert np.array_equal(dy.read(), dy2.read())
    assert np.array_equal(ds.read(), ds2.read())


ATTN_CASES = [
    dict(pos=0, m=1, reach=8, gap=0, cap=24, heads=4, key_heads=4, dh=8),
    dict(pos=30, m=7, reach=8, gap=0, cap=24, heads=4, key_heads=4, dh=8),
    dict(pos=50, m=9, reach=O.USIZE_MAX, gap=8, cap=64, heads=4, key_heads=2, dh=8),
    dict(pos=2, m=3, reach=O.USIZE_MAX, gap=8, cap=64, heads=4, key_heads=1, dh=8),
    dict(pos=4100, m=1, reach=4096, gap=0, cap=4352, heads=12, key_heads=12, dh=64),
    dict(pos=5000, m=256, reach=4096, gap=0, cap=4352, heads=12, key_heads=12, dh=64),
    # a filling window: superblock slots no query sees yet, a diagonal cut inside a segment
    dict(pos=272, m=256, reach=4096, gap=0, cap=4352, heads=12, key_heads=12, dh=64),
    dict(pos=100, m=50, reach=64, gap=0, cap=200, heads=4, key_heads=2, dh=16),
    dict(pos=9000, m=40, reach=O.USIZE_MAX, gap=4096, cap=16384, heads=12, key_heads=4, dh=64),
    dict(pos=600, m=33, reach=200, gap=0, cap=456, heads=6, key_heads=3, dh=32),
    dict(pos=700, m=20, reach=512, gap=0, cap=600, heads=4, key_heads=2, dh=128),
    dict(pos=300, m=5, reach=O.USIZE_MAX, gap=0, cap=320, heads=2, key_heads=2, dh=256),
    # one-token kernel edges: sixteen query heads per key head, head sizes 48 and 4, and a
    # span whose superblock partials do not fit its LDS (combined by a second kernel)
    dict(pos=1000, m=3, reach=O.USIZE_MAX, gap=0, cap=1100, heads=16, key_heads=1, dh=64),
    dict(pos=400, m=4, reach=300, gap=0, cap=512, heads=4, key_heads=2, dh=48),
    dict(pos=90, m=2, reach=64, gap=0, cap=100, heads=2, key_heads=1, dh=4),
    dict(pos=9000, m=2, reach=O.USIZE_MAX, gap=0, cap=9100, heads=16, key_heads=1, dh=64),
    # rings of exactly the one-token kernel's superblock count (cap = 256 x slots): its
    # workgroups copy ring slots before they read the position. Wrapped; the oldest key on a
    # superblock boundary at 4607 (one slot holds no key); grouped heads; a global span
    dict(pos=5000, m=3, reach=4096, gap=0, cap=4352, heads=12, key_heads=12, dh=64),
    dict(pos=4605, m=3, reach=4096, gap=0, cap=4352, heads=12, key_heads=12, dh=64),
    dict(pos=2000, m=2, reach=512, gap=0, cap=768, heads=4, key_heads=2, dh=32),
    dict(pos=700, m=2, reach=O.USIZE_MAX, gap=0, cap=768, heads=4, key_heads=1, dh=64),
]


@pytest.mark.parametrize("case", ATTN_CASES, ids=lambda c: f"p{c['pos']}m{c['m']}kh{c['key_heads']}")
def test_attend(hip, case):
    a = dict(case, scale=float(1 / np.sqrt(case["dh"])))
    m, heads, kh, dh, cap = a["m"], a["heads"], a["key_heads"], a["dh"], a["cap"]
    q = rnd(m, heads, dh)
    k = rnd(kh, cap, dh)
    v = rnd(kh, cap, dh)
    dq, dk, dv, dy = hip.upload(q), hip.upload(k), hip.upload(v), hip.alloc(m * heads * dh)
    hip.attend(dy.ptr, dq.ptr, dk.ptr, dv.ptr, **a)
    got = dy.read()
    want = O.attend(q, k, v, **a)
    exact = attend64(q, k, v, **a)
    # both are fp32 sums over up to thousands of keys in different orders: the GPU is
    # judged against float64 no worse than the reference's own order is
    assert rel(got, want) < 1e-5
    assert rel(got, exact) <= 2 * rel(want, exact) + 1e-7
    # each query alone (m = 1 at its own position) gives the same bits
    d1 = hip.alloc(heads * dh)
    for i in sorted({0, m // 2, m - 1}):
        hip.attend(d1.ptr, dq.at(i * heads * dh), dk.ptr, dv.ptr, **dict(a, pos=a["pos"] + i, m=1))
        assert np.array_equal(d1.read(), got[i * heads * dh:(i + 1) * heads * dh]), i


# ---------------------------------------------------------------------------------------
# fused one-token kernels: each pattern the planner fuses, against one launch per op
# ---------------------------------------------------------------------------------------

def _step(hip, body, inv, cs, sn, fuse):
    """Records one step (rope_table .. flush) and runs it fused or unfused."""
    hip.set_fusion(fuse)
    hip.rope_table(cs.ptr, sn.ptr, inv.ptr, 7, 1, 32)
    body()
    hip.flush()
    plan = hip.last_plan()
    hip.set_fusion(True)
    return plan


def test_read_ahead_of_a_step_output(hip):
    """A replayed one-token step graph whose output the host read right after its last replay
    copies that range into mapped host memory behind the step, and the next read of it waits
    for the copy; a read of another range, or one after other work, takes the usual copy.
    Every read returns what the device holds."""
    d = 768
    inv = hip.upload((1.0 / 10000.0 ** (np.arange(32) * 2 / 64)).astype(np.float32))
    cs, sn = hip.alloc(32), hip.alloc(32)
    w = hip.upload(rnd(d, d, scale=0.02))
    x = hip.upload(rnd(d))
    y = hip.alloc(d)

    def step():
        hip.rope_table(cs.ptr, sn.ptr, inv.ptr, 7, 1, 32)
        hip.linear(y.ptr, w.ptr, d, d, x.ptr, 1)
        hip.flush([y.ptr])

    def eager():
        hip.set_graphs(False)
        try:
            step()
            return y.read()
        finally:
            hip.set_graphs(True)

    want = eager()
    r0 = hip.read_ahead_stats()
    for _ in range(5):  # capture, a read that teaches the graph, replays copied ahead
        step()
        assert np.array_equal(y.read(), want)
    r1 = hip.read_ahead_stats()
    assert r1 - r0 >= 3, (r0, r1)
    step()  # another range: the usual copy (and the graph learns that one)
    assert np.array_equal(y.read(100), want[:100])
    step()
    assert np.array_equal(y.read(), want)
    step()
    assert np.array_equal(y.read(), want)
    z = rnd(d)
    dz = hip.upload(z)
    step()  # other work on the output after the replay: the read sees it
    hip.copy(y.ptr, dz.ptr, d)
    assert np.array_equal(y.read(), z)
    x2 = rnd(d)
    hip.upload_into(x, x2)  # new input: each replay's copy follows the device
    want2 = eager()
    assert not np.array_equal(want2, want)
    for _ in range(3):
        step()
        assert np.array_equal(y.read(), want2)
    assert hip.read_ahead_stats() > r1


FUSION_CASES = ["plain", "rms", "resid", "silu", "rope_store", "l2_decay", "combine", "side_copy",
                "split_fold", "split_flush", "gla_l2", "rounds", "row_offset"]


@pytest.mark.parametrize("tile", [0, 16, 12, 8, 4], ids=["tile_auto", "tile16", "tile12", "tile8", "tile4"])
@pytest.mark.parametrize("fp16", [False, True], ids=["fp32", "fp16"])
@pytest.mark.parametrize("case", FUSION_CASES)
def test_fusion_pattern(hip, case, fp16, tile):
    """Every fused one-token pattern gives the bits of one launch per op, with the fused
    GEMV's rows per tile chosen by the planner or forced to 16, 12, 8 or 4 (each row's chain is
    the same whatever the tile: the rope and SiLU row pairs, the residual, the split
    partials and the pick follow their rows)."""
    d, heads, dh, hid, cap = 768, 12, 64, 3072, 4352
    inv = hip.upload((1.0 / 10000.0 ** (np.arange(32) * 2 / 64)).astype(np.float32))
    cs, sn = hip.alloc(32), hip.alloc(32)
    wsq = hip.upload(rnd(d, d, scale=0.02))
    wqkv = hip.upload(rnd(3 * d, d, scale=0.02))
    wqkvg = hip.upload(rnd(4 * d, d, scale=0.02))
    wdec = hip.upload(rnd(heads, d, scale=0.02))
    wup = hip.upload(rnd(2 * hid, d, scale=0.02))
    wdown = hip.upload(rnd(d, hid, scale=0.02))
    whead = hip.upload(rnd(32000, d, scale=0.02))
    xh = hip.upload(rnd(hid))
    bias = hip.upload(rnd(heads))
    hn = hip.upload(rnd(dh))
    s0 = rnd(heads, dh, dh, scale=0.1)
    x = hip.upload(rnd(d))
    res = hip.upload(rnd(d))
    nw = hip.upload(rnd(d))
    kring = hip.upload(rnd(heads, cap, dh))
    vring = hip.upload(rnd(heads, cap, dh))
    q = hip.upload(rnd(heads, dh))

    def outs():
        return {k: hip.alloc(n) for k, n in
                dict(n=d, y=4 * d, q=d, k=d, t=d, up=2 * hid, g=hid, dd=heads, s=d,
                     kr=heads * cap * dh, vr=heads * cap * dh, att=d, h=d, z=d, y2=d,
                     S=heads * dh * dh, lg=32000).items()}

    def body(o):
        if case == "plain":
            hip.linear(o["y"].ptr, wsq.ptr, d, d, x.ptr, 1)
        elif case == "rms":
            hip.rms(o["n"].ptr, x.ptr, nw.ptr, 1, d, 1e-6)
            hip.linear(o["y"].ptr, wsq.ptr, d, d, o["n"].ptr, 1)
        elif case == "resid":
            hip.linear(o["y"].ptr, wsq.ptr, d, d, x.ptr, 1)
            hip.add(o["t"].ptr, res.ptr, o["y"].ptr, d)
        elif case == "silu":
            hip.linear(o["up"].ptr, wup.ptr, 2 * hid, d, x.ptr, 1)
            hip.silu_mul(o["g"].ptr, o["up"].ptr, o["up"].at(hid), hid)
        elif case == "rope_store":
            hip.rms(o["n"].ptr, x.ptr, nw.ptr, 1, d, 1e-6)
            hip.linear(o["y"].ptr, wqkv.ptr, 3 * d, d, o["n"].ptr, 1)
            hip.rope(o["q"].ptr, o["y"].ptr, cs.ptr, sn.ptr, 1, heads, dh)
            hip.rope(o["k"].ptr, o["y"].at(d), cs.ptr, sn.ptr, 1, heads, dh)
            hip.store(o["kr"].ptr, o["k"].ptr, 4100, 1, cap, heads, dh)
            hip.store(o["vr"].ptr, o["y"].at(2 * d), 4100, 1, cap, heads, dh)
        elif case == "l2_decay":
            hip.linear(o["y"].ptr, wqkvg.ptr, 4 * d, d, x.ptr, 1)
            hip.l2norm(o["q"].ptr, o["y"].ptr, heads, dh)
            hip.l2norm(o["k"].ptr, o["y"].at(d), heads, dh)
            hip.linear(o["dd"].ptr, wdec.ptr, heads, d, x.ptr, 1)
        elif case == "combine":
            hip.attend(o["att"].ptr, q.ptr, kring.ptr, vring.ptr, pos=5000, m=1, reach=4096,
                       gap=0, cap=cap, heads=heads, key_heads=heads, dh=dh, scale=0.125)
            hip.linear(o["y"].ptr, wsq.ptr, d, d, o["att"].ptr, 1)
            hip.add(o["t"].ptr, res.ptr, o["y"].ptr, d)
        elif case == "side_copy":
            hip.linear(o["y"].ptr, wsq.ptr, d, d, x.ptr, 1)
            hip.copy(o["s"].ptr, x.ptr, d)
            hip.add(o["t"].ptr, o["s"].ptr, o["y"].ptr, d)
        elif case == "split_fold":  # a 3072-column linear's splits fold in the next prologue
            hip.linear(o["h"].ptr, wdown.ptr, d, hid, xh.ptr, 1)
            hip.add(o["t"].ptr, res.ptr, o["h"].ptr, d)
            hip.rms(o["n"].ptr, o["t"].ptr, nw.ptr, 1, d, 1e-6)
            hip.linear(o["y"].ptr, wsq.ptr, d, d, o["n"].ptr, 1)
        elif case == "split_flush":  # ... or in a kernel of their own
            hip.linear(o["h"].ptr, wdown.ptr, d, hid, xh.ptr, 1)
            hip.add(o["t"].ptr, res.ptr, o["h"].ptr, d)
        elif case == "row_offset":  # a prologue op reading another's output at an offset
            hip.add(o["up"].ptr, xh.ptr, xh.ptr, 2 * d)
            hip.copy(o["s"].ptr, o["up"].at(d), d)
            hip.rms(o["n"].ptr, o["s"].ptr, nw.ptr, 1, d, 1e-6)
            hip.linear(o["y"].ptr, wsq.ptr, d, d, o["n"].ptr, 1)
        elif case == "rounds":  # 2000 tiles: each workgroup takes several rounds of two
            hip.rms(o["n"].ptr, x.ptr, nw.ptr, 1, d, 1e-6)
            hip.linear(o["lg"].ptr, whead.ptr, 32000, d, o["n"].ptr, 1)
        elif case == "gla_l2":  # the L mixer: the l2norms move into the GLA kernel
            hip.linear(o["y"].ptr, wqkvg.ptr, 4 * d, d, x.ptr, 1)
            hip.l2norm(o["q"].ptr, o["y"].ptr, heads, dh)
            hip.l2norm(o["k"].ptr, o["y"].at(d), heads, dh)
            hip.linear(o["dd"].ptr, wdec.ptr, heads, d, x.ptr, 1)
            hip.gla(o["z"].ptr, o["S"].ptr, o["q"].ptr, o["k"].ptr, o["y"].at(2 * d), o["dd"].ptr,
                    bias.ptr, 1, heads, dh)
            hip.rms(o["y2"].ptr, o["z"].ptr, hn.ptr, heads, dh, 1e-6)
            hip.silu_mul(o["z"].ptr, o["y"].at(3 * d), o["y2"].ptr, d)

    got = []
    hip.set_fp16(fp16)
    hip.set_tile_rows(tile)
    try:
        for fuse in (False, True):
            o = outs()
            hip.write(o["S"], s0)
            plan = _step(hip, lambda: body(o), inv, cs, sn, fuse)
            got.append(({k: b.read() for k, b in o.items()}, plan))
    finally:
        hip.set_tile_rows(0)
        hip.set_fp16(False)
    (a, pa), (b, pb) = got
    print(case, "unfused", pa, "fused", pb)
    assert pb["kernels"] <= pa["kernels"]
    if case not in ("plain", "split_flush"):  # a fold with no kernel to join runs alone
        assert pb["kernels"] < pa["kernels"]
    for k in a:
        assert np.array_equal(a[k], b[k]), (case, k, float(np.abs(a[k] - b[k]).max()))


def test_bounded_wait_that_gives_up_is_reported(hip, pkg):
    """A fused kernel's bounded LDS wait that gives up sets the fault word; the next read
    returns SLM_E_HIP once. Forced from the host with a spin limit of 0 (every such wait
    gives up at once, and every kernel still runs to its end); with the default limit the
    same step runs clean and gives the per-op kernels' bits."""
    d = 768
    inv = hip.upload((1.0 / 10000.0 ** (np.arange(32) * 2 / 64)).astype(np.float32))
    cs, sn = hip.alloc(32), hip.alloc(32)
    w = hip.upload(rnd(d, d, scale=0.02))
    x, nw, res = hip.upload(rnd(d)), hip.upload(rnd(d)), hip.upload(rnd(d))
    n, y, t = hip.alloc(d), hip.alloc(d), hip.alloc(d)

    def body():  # the block input chain: residual add, rms, GEMV (rms syncs the prologue)
        hip.add(t.ptr, res.ptr, x.ptr, d)
        hip.rms(n.ptr, t.ptr, nw.ptr, 1, d, 1e-6)
        hip.linear(y.ptr, w.ptr, d, d, n.ptr, 1)

    _step(hip, body, inv, cs, sn, False)
    want = y.read()
    hip.set_spin_limit(0)
    try:
        _step(hip, body, inv, cs, sn, True)
        with pytest.raises(pkg.SlmError) as e:
            y.read()
        assert e.value.code == -2 and "gave up" in str(e.value)
        y.read()  # reported once
    finally:
        hip.set_spin_limit(1 << 24)
    _step(hip, body, inv, cs, sn, True)
    assert np.array_equal(y.read(), want)


# ---------------------------------------------------------------------------------------
# prompt row chains: the element-wise ops between two GEMMs as one launch per chain
# ---------------------------------------------------------------------------------------

def _pick(x):
    """sample.rs:48-53: b = 0, then b = i whenever x[i] > x[b]."""
    b = 0
    for i in range(1, len(x)):
        if x[i] > x[b]:
            b = i
    return b


@pytest.mark.parametrize("case", ["random", "ties", "nan_first", "nan_inside", "all_neg_inf",
                                  "signed_zero", "short", "odd"])
def test_argmax_picks_like_the_reference(hip, case):
    """The device pick gives the reference's greedy index: the first maximum, NaNs never
    chosen, a NaN at 0 keeping 0; written to the token slot and the ids slot."""
    n = {"short": 1, "odd": 1025}.get(case, 32000)
    x = rnd(n)
    if case == "ties":
        x[[7, 900, 31000]] = 9.0
    if case == "nan_first":
        x[0] = np.nan
        x[5] = 50.0
    if case == "nan_inside":
        x[[3, 100, 20000]] = np.nan
        x[4000] = 7.0
    if case == "all_neg_inf":
        x[:] = -np.inf
    if case == "signed_zero":
        x[:] = -1.0
        x[10] = -0.0
        x[20] = 0.0
    want = _pick(x)
    dx = hip.upload(x)
    tok = hip.alloc(2)
    ids = hip.alloc(4)
    hip.argmax(tok.ptr, ids.ptr, 4, 2, dx.ptr, n)
    hip.flush()
    got_tok = int(tok.read(2).view(np.int64)[0])
    got_id = int(ids.read(4).view(np.uint32)[2])
    assert got_tok == want and got_id == want, (case, got_tok, got_id, want)


def _pick_rows(case, rows, cols=64):
    """Weights whose GEMV with x = e0 gives y = w[:, 0] exactly (the other columns meet zeros):
    the pick cases of test_argmax_picks_like_the_reference, as logits of a linear."""
    w = rnd(rows, cols)
    c = w[:, 0]
    if case == "ties":
        c[[7, rows // 2, rows - 3]] = 9.0
    if case == "nan_first":
        c[0] = np.nan
        c[5] = 50.0
    if case == "nan_inside":
        c[[3, rows // 3, rows - 1]] = np.nan
        c[rows // 2] = 7.0
    if case == "all_neg_inf":
        c[:] = -np.inf
    if case == "signed_zero":
        c[:] = -1.0
        c[10] = -0.0
        c[20] = 0.0
    return w


@pytest.mark.parametrize("tile", [0, 12, 4], ids=["tile_auto", "tile12", "tile4"])
@pytest.mark.parametrize("rows", [32000, 40])
@pytest.mark.parametrize("case", ["random", "ties", "nan_first", "nan_inside", "all_neg_inf",
                                  "signed_zero"])
def test_pick_fused_into_the_logits_gemv(hip, case, rows, tile):
    """The greedy pick after a one-token linear, inside a step: fused into the GEMV's epilogue
    (each workgroup's first maximum into a 64-bit atomic maximum, the last workgroup writes the
    pick) it gives the standalone kernel's index, the reference's first maximum, with no
    slm_argmax launch; and every replay of the step's graph picks afresh (the key and the
    counter are cleared by the launch that used them). With the planner's tiles and 4-row
    tiles."""
    cols = 64
    inv = hip.upload((1.0 / 10000.0 ** (np.arange(32) * 2 / 64)).astype(np.float32))
    cs, sn = hip.alloc(32), hip.alloc(32)
    x = np.zeros(cols, np.float32)
    x[0] = 1.0
    dx, dw = hip.upload(x), hip.upload(_pick_rows(case, rows))
    y, tok, ids = hip.alloc(rows), hip.alloc(2), hip.alloc(4)

    def body():
        hip.linear(y.ptr, dw.ptr, rows, cols, dx.ptr, 1)
        hip.argmax(tok.ptr, ids.ptr, 4, 2, y.ptr, rows)

    def picked():
        return int(tok.read(2).view(np.int64)[0]), int(ids.read(4).view(np.uint32)[2])

    hip.set_tile_rows(tile)
    try:
        plans = {}
        got = {}
        for fuse in (False, True):
            hip.write(tok, np.zeros(2, np.float32))
            hip.write(ids, np.zeros(4, np.float32))
            plans[fuse] = _step(hip, body, inv, cs, sn, fuse)
            got[fuse] = picked()
        yv = y.read()
        want = _pick(yv)
        assert got[True] == (want, want) and got[False] == (want, want), (case, got, want)
        assert plans[True]["kernels"] < plans[False]["kernels"]
        # eagerly, with the launches counted: no slm_argmax
        hip.set_graphs(False)
        hip.set_timing(True)
        try:
            _step(hip, body, inv, cs, sn, True)
            assert hip.kernel_stat("slm_argmax")["launches"] == 0
            assert hip.kernel_stat("slm_fg")["launches"] == 1
        finally:
            hip.set_timing(False)
            hip.set_graphs(True)
        assert picked() == (want, want)
        # graph replays with new weights each time: each pick is fresh
        for seed in range(4):
            w = _pick_rows("random", rows)
            w[(seed * 997) % rows, 0] = 20.0 + seed
            hip.write(dw, w)
            _step(hip, body, inv, cs, sn, True)
            assert picked() == ((seed * 997) % rows,) * 2, seed
    finally:
        hip.set_tile_rows(0)


ROW_CASES = ["attn_in", "attn_in_dead", "gla_in_dead", "mlp", "mlp_dead", "inplace", "overlap"]
# the GEMM whose epilogue takes the dead ops over (fp16 mode: the same names with "2h")
ROW_EPI_GEMM = {"attn_in_dead": ["slm_gemm2r_64"], "gla_in_dead": ["slm_gemm2n_64"],
                "mlp_dead": [f"slm_gemm2s_{b}" for b in (32, 64, 96, 128)]}


def _fp16_weight_kernel(name):
    """slm_gemm2r_64 -> slm_gemm2hrw_64: the fp16-mode GEMM over fp16 weights."""
    head, tile = name.rsplit("_", 1)
    return head.replace("gemm2", "gemm2h") + "w_" + tile


@pytest.mark.parametrize("fp16", [False, True], ids=["fp32", "fp16"])
@pytest.mark.parametrize("m", [37, 256])
@pytest.mark.parametrize("case", ROW_CASES)
def test_row_chain(hip, case, m, fp16):
    """A prompt chunk's element-wise ops fused into row chains give the bits of one launch
    per op, for in-place updates, operands read from an earlier op's output at an offset,
    a shared vector read by every row and outputs overwritten later in the chain; where the
    ops after a GEMM are dead, that GEMM's epilogue kernel is the one that ran. In fp32 and
    in fp16 mode."""
    hip.set_fp16(fp16)
    try:
        _row_chain(hip, case, m, fp16)
    finally:
        hip.set_fp16(False)


def _row_chain(hip, case, m, fp16):
    d, heads, dh, hid, cap, pos = 768, 12, 64, 3072, 4352, 100
    if case == "attn_in_dead":
        pos = cap - 20  # the ring slots wrap inside the chunk
    inv = hip.upload((1.0 / 10000.0 ** (np.arange(32) * 2 / 64)).astype(np.float32))
    cs, sn = hip.alloc(m * 32), hip.alloc(m * 32)
    wsq = hip.upload(rnd(d, d, scale=0.02))
    wqkv = hip.upload(rnd(3 * d, d, scale=0.02))
    wqkvg = hip.upload(rnd(4 * d, d, scale=0.02))
    wup = hip.upload(rnd(2 * hid, d, scale=0.02))
    wdown = hip.upload(rnd(d, hid, scale=0.02))
    x = hip.upload(rnd(m, d))
    res = hip.upload(rnd(m, d))
    row = hip.upload(rnd(d))
    nw = hip.upload(rnd(d))
    kr0, vr0 = rnd(heads, cap, dh), rnd(heads, cap, dh)

    def outs():
        o = {k: hip.alloc(n) for k, n in
             dict(y=m * 3 * d, y4=m * 4 * d, gt=m * d, q=m * d, k=m * d, k2=m * d, v=m * d, up=m * 2 * hid, g=m * hid,
                  u=m * hid, h=m * hid, dn=m * d, t=m * d, n=m * d, z=m * d, s=m * d,
                  y2=m * d, a=m * d // 2, b=m * d, c2=m * d // 2).items()}
        # the rings: Ops::zeros_cache, fp16 values in fp16 mode (the QKV GEMM's epilogue and
        # the row chain's stores then round what they write)
        o["kr"], o["vr"] = hip.alloc_cache(heads, cap, dh), hip.alloc_cache(heads, cap, dh)
        hip.write(o["kr"], kr0)
        hip.write(o["vr"], vr0)
        return o

    def body(o):
        if case == "attn_in":
            hip.linear(o["y"].ptr, wqkv.ptr, 3 * d, d, x.ptr, m)
            hip.columns(o["q"].ptr, o["y"].ptr, m, 3 * d, 0, d)
            hip.rope(o["q"].ptr, o["q"].ptr, cs.ptr, sn.ptr, m, heads, dh)
            hip.columns(o["k"].ptr, o["y"].ptr, m, 3 * d, d, d)
            hip.rope(o["k2"].ptr, o["k"].ptr, cs.ptr, sn.ptr, m, heads, dh)
            hip.columns(o["v"].ptr, o["y"].ptr, m, 3 * d, 2 * d, d)
            hip.store(o["kr"].ptr, o["k2"].ptr, pos, m, cap, heads, dh)
            hip.store(o["vr"].ptr, o["v"].ptr, pos, m, cap, heads, dh)
            hip.linear(o["t"].ptr, wsq.ptr, d, d, o["q"].ptr, m)
        elif case == "attn_in_dead":  # model.rs:417-432 as the model issues it: the column
            # scratch k is overwritten before anything reads it, so the QKV GEMM rotates q and k
            # and writes the rings itself
            hip.linear(o["y"].ptr, wqkv.ptr, 3 * d, d, x.ptr, m)
            hip.columns(o["k"].ptr, o["y"].ptr, m, 3 * d, 0, d)
            hip.rope(o["q"].ptr, o["k"].ptr, cs.ptr, sn.ptr, m, heads, dh)
            hip.columns(o["k"].ptr, o["y"].ptr, m, 3 * d, d, d)
            hip.rope(o["k2"].ptr, o["k"].ptr, cs.ptr, sn.ptr, m, heads, dh)
            hip.columns(o["v"].ptr, o["y"].ptr, m, 3 * d, 2 * d, d)
            hip.store(o["kr"].ptr, o["k2"].ptr, pos, m, cap, heads, dh)
            hip.store(o["vr"].ptr, o["v"].ptr, pos - 7, m, cap, heads, dh)  # its own slots
            hip.linear(o["k"].ptr, wsq.ptr, d, d, o["q"].ptr, m)
        elif case == "gla_in_dead":  # model.rs:434-440: the QKVG GEMM normalises q and k per
            # head and writes v and the gate itself (the column scratch k is dead)
            hip.linear(o["y4"].ptr, wqkvg.ptr, 4 * d, d, x.ptr, m)
            hip.columns(o["k"].ptr, o["y4"].ptr, m, 4 * d, 0, d)
            hip.l2norm(o["q"].ptr, o["k"].ptr, m * heads, dh)
            hip.columns(o["k"].ptr, o["y4"].ptr, m, 4 * d, d, d)
            hip.l2norm(o["k2"].ptr, o["k"].ptr, m * heads, dh)
            hip.columns(o["v"].ptr, o["y4"].ptr, m, 4 * d, 2 * d, d)
            hip.columns(o["gt"].ptr, o["y4"].ptr, m, 4 * d, 3 * d, d)
            hip.linear(o["k"].ptr, wsq.ptr, d, d, o["q"].ptr, m)
        elif case == "mlp":  # a split GEMM's fold opens the second chain
            hip.linear(o["up"].ptr, wup.ptr, 2 * hid, d, x.ptr, m)
            hip.columns(o["g"].ptr, o["up"].ptr, m, 2 * hid, 0, hid)
            hip.columns(o["u"].ptr, o["up"].ptr, m, 2 * hid, hid, hid)
            hip.silu_mul(o["h"].ptr, o["g"].ptr, o["u"].ptr, m * hid)
            hip.linear(o["dn"].ptr, wdown.ptr, d, hid, o["h"].ptr, m)
            hip.add(o["t"].ptr, res.ptr, o["dn"].ptr, m * d)
            hip.rms(o["n"].ptr, o["t"].ptr, nw.ptr, m, d, 1e-6)
            hip.linear(o["z"].ptr, wsq.ptr, d, d, o["n"].ptr, m)
        elif case == "mlp_dead":  # up, gate and amp are overwritten before anything reads
            # them: the up GEMM writes the SiLU pair's product itself
            hip.linear(o["up"].ptr, wup.ptr, 2 * hid, d, x.ptr, m)
            hip.columns(o["g"].ptr, o["up"].ptr, m, 2 * hid, 0, hid)
            hip.columns(o["u"].ptr, o["up"].ptr, m, 2 * hid, hid, hid)
            hip.silu_mul(o["h"].ptr, o["g"].ptr, o["u"].ptr, m * hid)
            hip.linear(o["dn"].ptr, wdown.ptr, d, hid, o["h"].ptr, m)
            hip.copy(o["g"].ptr, o["h"].ptr, m * hid)
            hip.add(o["u"].ptr, o["h"].ptr, o["g"].ptr, m * hid)
            hip.linear(o["up"].ptr, wup.ptr, 2 * hid, d, o["dn"].ptr, m)
        elif case == "inplace":
            hip.linear(o["t"].ptr, wsq.ptr, d, d, x.ptr, m)
            hip.add(o["t"].ptr, o["t"].ptr, res.ptr, m * d)
            hip.rms(o["t"].ptr, o["t"].ptr, nw.ptr, m, d, 1e-6)
            hip.add_row(o["t"].ptr, o["t"].ptr, row.ptr, m, d)
            hip.mix(o["z"].ptr, o["t"].ptr, res.ptr, m * d, 0.3)
            hip.copy(o["s"].ptr, o["z"].ptr, m * d)
            hip.l2norm(o["n"].ptr, o["s"].ptr, m * heads, dh)
        elif case == "overlap":
            hip.linear(o["t"].ptr, wsq.ptr, d, d, x.ptr, m)
            hip.add(o["y2"].ptr, o["t"].ptr, res.ptr, m * d)
            hip.columns(o["a"].ptr, o["y2"].ptr, m, d, d // 4, d // 2)
            hip.rope(o["b"].ptr, o["y2"].ptr, cs.ptr, sn.ptr, m, heads, dh)
            hip.add_row(o["z"].ptr, o["b"].ptr, row.ptr, m, d)
            hip.add(o["y2"].ptr, o["z"].ptr, o["y2"].ptr, m * d)
            hip.rms(o["n"].ptr, o["y2"].ptr, nw.ptr, m, d, 1e-6)
            hip.columns(o["c2"].ptr, o["n"].ptr, m, d, 0, d // 2)
            hip.copy(o["s"].ptr, o["y2"].ptr, m * d)

    got = []
    for fuse in (True, False, True):  # (the first pass grows the backend's buffers)
        o = outs()
        hip.set_fusion(fuse)
        last = len(got) == 2
        if last:  # eager launches, counted by kernel
            hip.set_graphs(False)
            hip.set_timing(True)
        try:
            hip.rope_table(cs.ptr, sn.ptr, inv.ptr, pos, m, 32)
            body(o)
            hip.flush()
            plan = hip.last_plan()
            # (fp16 mode: the fp16-weight kernel, "...w_", reading the context's fp16 copy of
            # the weights)
            epi = sum(hip.kernel_stat(_fp16_weight_kernel(n) if fp16 else n)["launches"]
                      for n in ROW_EPI_GEMM.get(case, [])) if last else 0
        finally:
            hip.set_fusion(True)
            if last:
                hip.set_timing(False)
                hip.set_graphs(True)
        got.append(({k: b.read() for k, b in o.items()}, plan))
    _, (a, pa), (b, pb) = got
    print(case, m, "unfused", pa, "fused", pb)
    assert pb["kernels"] < pa["kernels"]
    if case in ROW_EPI_GEMM:
        assert epi == 1, (case, m, fp16, epi)
    for k in a:
        assert np.array_equal(a[k], b[k]), (case, m, k, float(np.abs(a[k] - b[k]).max()))


# ---------------------------------------------------------------------------------------
# fp16 mode: linears round their operands to fp16 at fp16 MFMAs, sum in fp32 and round the
# result to fp16; every operation's result is rounded to fp16 (mlx.rs's Float16 arrays)
# ---------------------------------------------------------------------------------------

def _is_f16(a):
    a = np.asarray(a, np.float32)
    return np.array_equal(a, a.astype(np.float16).astype(np.float32))


@pytest.mark.parametrize("rows,cols", [(768, 768), (2304, 768), (768, 3072), (40, 128)])
def test_linear_fp16(hip, rows, cols):
    """Every m (the small-m GEMV and the GEMM) against float64 sums of the fp16-rounded
    operands (their products are exact in fp32, so only the fp32 sums differ) rounded to fp16:
    the result holds fp16 values, each the fp16 rounding of the float64 sum except where the
    fp32 sum falls on the other side of a rounding boundary (then one fp16 step, or for sums
    near zero the fp32 sum's own error, away); and the same bits for a row whatever m is."""
    w = rnd(rows, cols, scale=0.05)
    x = rnd(256, cols)
    dw, dx = hip.upload(w), hip.upload(x)
    w16 = w.astype(np.float16).astype(np.float64)
    x16 = x.astype(np.float16).astype(np.float64)
    want = x16 @ w16.T
    want16 = want.astype(np.float16).astype(np.float32)
    hip.set_fp16(True)
    try:
        got = {}
        for m in (1, 5, 37, 256):
            dy = hip.alloc(m * rows)
            hip.linear(dy.ptr, dw.ptr, rows, cols, dx.ptr, m)
            got[m] = dy.read().reshape(m, rows)
            assert _is_f16(got[m]), m
            step = np.spacing(np.abs(want16[:m]).astype(np.float16)).astype(np.float32)
            tol = step + 1e-6 * np.abs(want).max()  # (fp32 summation error, absolute)
            assert np.all(np.abs(got[m] - want16[:m]) <= tol), m
            assert np.mean(got[m] == want16[:m]) > 0.99, m
        for m in (1, 5, 37):
            assert np.array_equal(got[m], got[256][:m]), m
        # fp16 rounding is visible: the fp32 path gives other values
        dy = hip.alloc(rows)
        hip.set_fp16(False)
        hip.linear(dy.ptr, dw.ptr, rows, cols, dx.ptr, 1)
        assert not np.array_equal(dy.read(), got[1][0])
    finally:
        hip.set_fp16(False)


def test_linear_fp16_rejects_ragged_columns(hip):
    dw, dx, dy = hip.alloc(16 * 40), hip.alloc(40), hip.alloc(16)
    hip.set_fp16(True)
    try:
        with pytest.raises(Exception):
            hip.linear(dy.ptr, dw.ptr, 16, 40, dx.ptr, 1)
    finally:
        hip.set_fp16(False)


def test_fp16_mode_values(hip):
    """fp16 mode keeps every buffer's values in fp16, as mlx.rs's Float16 arrays (mlx.rs:19-23,
    53-67): an upload rounds (mlx.rs:61-63); add, add_row, mix, scale_rows and rope give
    mlx.rs's rounding points over fp32 arithmetic bit for bit (each fp16 array operation is the
    fp32 one rounded to nearest even: numpy below); rms rounds its fp32 quotient before the
    weight (mlx.rs:178-185); rms, l2norm, silu_mul and the GLA give fp16 values within fp16
    roundings of float64, the GLA's state too."""
    f16 = lambda a: np.asarray(a, np.float32).astype(np.float16).astype(np.float32)  # noqa: E731
    n, heads, dh, m = 1536, 12, 64, 3
    a, b = rnd(n), rnd(n)
    hip.set_fp16(True)
    try:
        da, db = hip.upload(a), hip.upload(b)
        a16, b16 = da.read(), db.read()
        assert np.array_equal(a16, f16(a)) and np.array_equal(b16, f16(b))
        y = hip.alloc(n)
        hip.add(y.ptr, da.ptr, db.ptr, n)
        assert np.array_equal(y.read(), f16(a16 + b16))
        hip.add_row(y.ptr, da.ptr, db.ptr, 2, n // 2)
        assert np.array_equal(y.read(), f16(a16 + np.tile(b16[:n // 2], 2)))
        t = np.float32(0.3)
        hip.mix(y.ptr, da.ptr, db.ptr, n, float(t))
        assert np.array_equal(y.read(), f16(a16 + f16(f16(b16 - a16) * f16(t))))
        f = np.array([1.7, -0.25], np.float32)
        hip.scale_rows(y.ptr, da.ptr, f, n // 2)
        assert np.array_equal(y.read(), f16(a16 * np.repeat(f16(f), n // 2)))
        # rope over one token of 12 heads, cos / sin rows as fp16 values
        half = dh // 2
        c16, s16 = f16(rnd(half)), f16(rnd(half))
        dc, ds = hip.upload(c16), hip.upload(s16)
        x = f16(rnd(heads, dh))
        dx, yr = hip.upload(x), hip.alloc(heads * dh)
        hip.rope(yr.ptr, dx.ptr, dc.ptr, ds.ptr, 1, heads, dh)
        lo, hi = x[:, :half], x[:, half:]
        want = np.concatenate([f16(f16(lo * c16) - f16(hi * s16)), f16(f16(lo * s16) + f16(hi * c16))], 1)
        assert np.array_equal(yr.read().reshape(heads, dh), want)
        # rms, l2norm, silu_mul: fp16 values, within fp16 roundings of float64
        w = f16(rnd(dh))
        dw, yn = hip.upload(w), hip.alloc(heads * dh)
        hip.rms(yn.ptr, dx.ptr, dw.ptr, heads, dh, 1e-6)
        x64 = x.astype(np.float64)
        r = 1.0 / np.sqrt((x64 * x64).mean(1, keepdims=True) + 1e-6)
        got = yn.read().reshape(heads, dh)
        assert _is_f16(got)
        assert np.allclose(got, x64 * r * w, rtol=2e-3, atol=1e-6)
        hip.l2norm(yn.ptr, dx.ptr, heads, dh)
        got = yn.read().reshape(heads, dh)
        assert _is_f16(got)
        assert np.allclose(got, x64 / np.sqrt((x64 * x64).sum(1, keepdims=True)), rtol=1e-3, atol=1e-6)
        hip.silu_mul(y.ptr, da.ptr, db.ptr, n)
        g64, u64 = a16.astype(np.float64), b16.astype(np.float64)
        assert _is_f16(y.read())
        assert np.allclose(y.read(), g64 / (1 + np.exp(-g64)) * u64, rtol=3e-3, atol=1e-6)
        # the GLA over m tokens: output and state in fp16
        q, k, v = f16(rnd(m, heads, dh, scale=0.2)), f16(rnd(m, heads, dh, scale=0.2)), f16(rnd(m, heads, dh))
        dec, bias = f16(rnd(m, heads)), f16(rnd(heads))
        s0 = f16(rnd(heads, dh, dh, scale=0.1))
        S = hip.upload(s0)
        yg = hip.alloc(m * heads * dh)
        hip.gla(yg.ptr, S.ptr, hip.upload(q).ptr, hip.upload(k).ptr, hip.upload(v).ptr,
                hip.upload(dec).ptr, hip.upload(bias).ptr, m, heads, dh)
        st = s0.astype(np.float64)
        want = np.zeros((m, heads, dh))
        for i in range(m):
            dd = 1.0 / (1.0 + np.exp(dec[i] + bias))
            st = st * dd[:, None, None] + k[i][:, :, None] * v[i][:, None, :]
            want[i] = np.einsum("hd,hde->he", q[i], st)
        gy, gs = yg.read().reshape(m, heads, dh), S.read().reshape(heads, dh, dh)
        assert _is_f16(gy) and _is_f16(gs)
        assert np.abs(gs - st).max() <= 4e-3 * np.abs(st).max()
        assert np.abs(gy - want).max() <= 8e-3 * np.abs(want).max()
    finally:
        hip.set_fp16(False)


# ---------------------------------------------------------------------------------------
# fp16 weights (slm_hip_alloc_half): fp16 mode with half the weight bytes, the same bits
# ---------------------------------------------------------------------------------------

def test_half_upload_rounds_to_nearest_even(hip):
    """Upload into an fp16 allocation rounds like numpy's float16 (IEEE binary16, ties to even:
    subnormals, the overflow threshold, signed zeros, infinities, NaN); read widens back."""
    tiny = np.float32(2.0 ** -24)
    x = np.array([1 + 2 ** -11, 1 + 3 * 2 ** -11, 1 - 2 ** -12, 65504, 65519.99, 65520, -65520,
                  tiny, tiny / 2, tiny * 1.5, tiny * 2.5, 2 ** -14 - tiny / 2, -0.0, 0.0, np.inf,
                  -np.inf, np.nan, 3.14159, -2.71828e-3, 1e-8, 6e4, 2 ** -15 * 1.25],
                 dtype=np.float32)
    x = np.concatenate([x, rnd(4099, scale=10.0), rnd(1000, scale=1e-5)])
    b = hip.upload_half(x)
    got = b.read(x.size)
    with np.errstate(over="ignore"):  # (the values past 65504 round to infinity)
        want = x.astype(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


@pytest.mark.parametrize("rows,cols", [(768, 768), (2304, 768), (6144, 768), (768, 3072),
                                       (12, 768), (2300, 768), (100, 1536), (8192, 768)])
def test_linear_half_weights_equal_fp16_mode(hip, rows, cols):
    """fp16 weights give fp16 mode's bits on the same weights in fp32, for every m (the
    small-m GEMV and each GEMM row tile), eagerly; and refuse to run outside fp16 mode."""
    w = rnd(rows, cols, scale=0.05)
    x = rnd(256, cols)
    dw, dh, dx = hip.upload(w), hip.upload_half(w), hip.upload(x)
    hip.set_fp16(True)
    try:
        for m in (1, 5, 16, 17, 37, 256):
            a, b, c = hip.alloc(m * rows), hip.alloc(m * rows), hip.alloc(m * rows)
            hip.set_half_shadows(False)  # fp32 weights rounded by the linear itself
            hip.linear(a.ptr, dw.ptr, rows, cols, dx.ptr, m)
            hip.set_half_shadows(True)  # fp32 weights through the context's fp16 copy
            hip.linear(c.ptr, dw.ptr, rows, cols, dx.ptr, m)
            hip.linear(b.ptr, dh.ptr, rows, cols, dx.ptr, m)
            assert np.array_equal(a.read(), b.read()), m
            assert np.array_equal(a.read(), c.read()), m
    finally:
        hip.set_half_shadows(True)
        hip.set_fp16(False)
    with pytest.raises(Exception):
        hip.linear(hip.alloc(rows).ptr, dh.ptr, rows, cols, dx.ptr, 1)


@pytest.mark.parametrize("case", ["plain", "rms", "resid", "silu", "rope_store", "split_fold", "rounds"])
def test_fused_step_half_weights(hip, case):
    """Inside a step (the fused GEMV slm_fghw): fp16 weights give the fused fp16-mode bits of the
    same weights in fp32, and the unfused ones."""
    d, hid, heads, dh, cap = 768, 3072, 12, 64, 4352
    inv = hip.upload((1.0 / 10000.0 ** (np.arange(32) * 2 / 64)).astype(np.float32))
    cs, sn = hip.alloc(32), hip.alloc(32)
    shapes = {"plain": (d, d), "rms": (3 * d, d), "resid": (d, d), "silu": (2 * hid, d),
              "rope_store": (3 * d, d), "split_fold": (d, hid), "rounds": (32000, d)}
    rows, cols = shapes[case]
    w = rnd(rows, cols, scale=0.02)
    dw, dh16 = hip.upload(w), hip.upload_half(w)
    x, res, nw = hip.upload(rnd(cols)), hip.upload(rnd(rows)), hip.upload(rnd(cols))
    xn, y, o1 = hip.alloc(cols), hip.alloc(rows), hip.alloc(rows)
    kc, vc = hip.alloc(heads * cap * dh), hip.alloc(heads * cap * dh)
    q, k, h = hip.alloc(d), hip.alloc(d), hip.alloc(hid)

    def body(wp):
        def run():
            src = x.ptr
            if case == "rms":
                hip.rms(xn.ptr, x.ptr, nw.ptr, 1, cols, 1e-5)
                src = xn.ptr
            hip.linear(y.ptr, wp, rows, cols, src, 1)
            if case == "resid":
                hip.add(o1.ptr, res.ptr, y.ptr, rows)
            if case == "silu":
                hip.silu_mul(h.ptr, y.ptr, y.at(hid), hid)
            if case == "rope_store":
                hip.rope(q.ptr, y.ptr, cs.ptr, sn.ptr, 1, heads, dh)
                hip.rope(k.ptr, y.at(d), cs.ptr, sn.ptr, 1, heads, dh)
                hip.store(kc.ptr, k.ptr, 4300, 1, cap, heads, dh)
                hip.store(vc.ptr, y.at(2 * d), 4300, 1, cap, heads, dh)
        return run

    def outs():
        r = [y.read()]
        if case == "resid":
            r.append(o1.read())
        if case == "silu":
            r.append(h.read())
        if case == "rope_store":
            r += [q.read(), k.read(), kc.read()[:heads * dh], vc.read()[:heads * dh]]
        return r

    hip.set_fp16(True)
    try:
        got = {}
        for name, wp, fuse in (("f32w", dw.ptr, True), ("half", dh16.ptr, True),
                               ("half_unfused", dh16.ptr, False), ("shadow", dw.ptr, True)):
            hip.set_half_shadows(name == "shadow")
            _step(hip, body(wp), inv, cs, sn, fuse)
            got[name] = outs()
    finally:
        hip.set_half_shadows(True)
        hip.set_fp16(False)
    for name in ("half", "half_unfused", "shadow"):
        for a, b in zip(got["f32w"], got[name]):
            assert np.array_equal(a, b), (case, name)


def test_half_shadow_follows_the_weights(hip):
    """fp16 mode's fp16 copy of a weight buffer is dropped whenever the fp32 buffer changes: an
    upload into it, an operation writing it (outside a step and inside one, before the linear
    in the same step), and a free and a new buffer at the same address. Each result equals
    fp16 mode over the fp32 weights with no copies."""
    inv = hip.upload((1.0 / 10000.0 ** (np.arange(32) * 2 / 64)).astype(np.float32))
    cs, sn = hip.alloc(32), hip.alloc(32)
    rows, cols = 768, 768
    w1, w2 = rnd(rows, cols, scale=0.02), rnd(rows, cols, scale=0.02)
    dw, src, dx = hip.upload(w1), hip.upload(w2), hip.upload(rnd(cols))
    y = hip.alloc(rows)

    def want(w):
        hip.set_half_shadows(False)
        t = hip.upload(w)
        o = hip.alloc(rows)
        hip.linear(o.ptr, t.ptr, rows, cols, dx.ptr, 1)
        hip.set_half_shadows(True)
        return o.read()

    hip.set_fp16(True)
    try:
        r1, r2 = want(w1), want(w2)
        hip.linear(y.ptr, dw.ptr, rows, cols, dx.ptr, 1)
        assert np.array_equal(y.read(), r1)
        hip.upload_into(dw, w2)  # an upload into the weights
        hip.linear(y.ptr, dw.ptr, rows, cols, dx.ptr, 1)
        assert np.array_equal(y.read(), r2)
        hip.copy(dw.ptr, hip.upload(w1.ravel()).ptr, rows * cols)  # an operation writing them
        hip.linear(y.ptr, dw.ptr, rows, cols, dx.ptr, 1)
        assert np.array_equal(y.read(), r1)

        def body():  # inside a step: the write comes before the linear that reads the weights
            hip.copy(dw.ptr, src.ptr, rows * cols)
            hip.linear(y.ptr, dw.ptr, rows, cols, dx.ptr, 1)
        _step(hip, body, inv, cs, sn, True)
        assert np.array_equal(y.read(), r2)
        hip.upload_into(dw, w1)
        hip.linear(y.ptr, dw.ptr, rows, cols, dx.ptr, 1)
        assert np.array_equal(y.read(), r1)
        addr = dw.ptr
        dw.free()
        dw2 = hip.upload(w2)  # (the pool may give the same address back)
        print("same address again:", dw2.ptr == addr)
        hip.linear(y.ptr, dw2.ptr, rows, cols, dx.ptr, 1)
        assert np.array_equal(y.read(), r2)
    finally:
        hip.set_fp16(False)


# ---------------------------------------------------------------------------------------
# fp16 rings (slm_hip_alloc_cache in fp16 mode): stores round to fp16, attention widens the
# halves exactly, so everything equals fp32 rings holding the same values
# ---------------------------------------------------------------------------------------

def _f16(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


# the ATTN_CASES the fp16 kernels take (head size at most 64, a multiple of 8, 64+ slots)
HALF_ATTN_CASES = [c for c in ATTN_CASES if c["dh"] <= 64 and c["dh"] % 8 == 0 and c["cap"] >= 64]


@pytest.mark.parametrize("case", HALF_ATTN_CASES, ids=lambda c: f"p{c['pos']}m{c['m']}kh{c['key_heads']}d{c['dh']}")
def test_half_rings_store_and_attend(hip, case):
    """A ring from slm_hip_alloc_cache in fp16 mode holds halves: a store rounds to nearest
    even, and attention over it (the one-token kernel at m = 1, the prompt kernel at m > 1,
    and the allocation-free entry point) gives, bit for bit, attention over fp32 rings that
    hold the same values."""
    a = dict(case, scale=float(1 / np.sqrt(case["dh"])))
    m, heads, kh, dh, cap = a["m"], a["heads"], a["key_heads"], a["dh"], a["cap"]
    k, v = _f16(rnd(kh, cap, dh)), _f16(rnd(kh, cap, dh))
    q = rnd(m, heads, dh)
    new_k, new_v = rnd(m, kh, dh), rnd(m, kh, dh)
    hip.set_fp16(True)
    try:
        hk, hv = hip.alloc_cache(kh, cap, dh), hip.alloc_cache(kh, cap, dh)
    finally:
        hip.set_fp16(False)
    fk, fv = hip.alloc_cache(kh, cap, dh), hip.alloc_cache(kh, cap, dh)  # fp32 outside fp16 mode
    hip.write(hk, k)
    hip.write(hv, v)
    hip.write(fk, k)
    hip.write(fv, v)
    assert np.array_equal(hk.read(), k.ravel())
    # the new rows: rounded by the store into the fp16 ring, stored pre-rounded into the fp32 one
    spos = a["pos"]
    sk, sv = hip.upload(new_k), hip.upload(new_v)
    sk16, sv16 = hip.upload(_f16(new_k)), hip.upload(_f16(new_v))
    hip.store(hk.ptr, sk.ptr, spos, m, cap, kh, dh)
    hip.store(hv.ptr, sv.ptr, spos, m, cap, kh, dh)
    hip.store(fk.ptr, sk16.ptr, spos, m, cap, kh, dh)
    hip.store(fv.ptr, sv16.ptr, spos, m, cap, kh, dh)
    assert np.array_equal(hk.read(), fk.read())
    assert np.array_equal(hv.read(), fv.read())
    dq = hip.upload(q)
    y16, y32, yna = (hip.alloc(m * heads * dh) for _ in range(3))
    hip.attend(y16.ptr, dq.ptr, hk.ptr, hv.ptr, **a)
    hip.attend(y32.ptr, dq.ptr, fk.ptr, fv.ptr, **a)
    assert np.array_equal(y16.read(), y32.read())
    hip.attend_noalloc(yna.ptr, dq.ptr, hk.ptr, hv.ptr, **a)
    assert np.array_equal(yna.read(), y32.read())
    # against the oracle on the rounded values
    want = O.attend(q, fk.read().reshape(kh, cap, dh), fv.read().reshape(kh, cap, dh), **a)
    assert rel(y16.read(), want) < 1e-5


def test_half_ring_refusals(hip):
    """fp16 rings only where the fp16 kernels run: other shapes get fp32 caches; a ring pair
    of mixed kinds is refused."""
    hip.set_fp16(True)
    try:
        small = hip.alloc_cache(2, 32, 8)     # fewer than 64 slots: fp32
        wide = hip.alloc_cache(2, 128, 128)   # head size above 64: fp32
        half = hip.alloc_cache(2, 128, 64)
    finally:
        hip.set_fp16(False)
    hip.write(small, np.arange(2 * 32 * 8, dtype=np.float32) + 0.1)
    assert np.array_equal(small.read(), np.arange(2 * 32 * 8, dtype=np.float32) + 0.1)  # fp32 kept
    hip.write(wide, np.full(2 * 128 * 128, 0.1, np.float32))
    assert np.array_equal(wide.read(), np.full(2 * 128 * 128, 0.1, np.float32))
    hip.write(half, np.full(2 * 128 * 64, 0.1, np.float32))
    assert np.array_equal(half.read(), _f16(np.full(2 * 128 * 64, 0.1, np.float32)))  # rounded
    f32 = hip.alloc(2 * 128 * 64)
    q, y = hip.upload(rnd(1, 4, 64)), hip.alloc(4 * 64)
    with pytest.raises(pkg_error()):
        hip.attend(y.ptr, q.ptr, half.ptr, f32.ptr, pos=10, m=1, reach=64, gap=0, cap=128, heads=4,
                   key_heads=2, dh=64, scale=0.125)
    with pytest.raises(pkg_error()):  # an fp16 ring is not an fp32 buffer
        hip.copy(y.ptr, half.ptr, 4 * 64)


def pkg_error():
    import slm_use_amd
    return slm_use_amd.SlmError


@pytest.mark.parametrize("fp16", [False, True], ids=["fp32", "fp16"])
def test_grow_cache(hip, fp16):
    """slm_hip_grow_cache: every head's rows at the start of its doubled rows, zeros after, for
    fp32 and fp16 caches (model.rs:383-398's relayout)."""
    kh, cap, dh = 3, 96, 64
    x = _f16(rnd(kh, cap, dh))
    hip.set_fp16(fp16)
    try:
        old, new = hip.alloc_cache(kh, cap, dh), hip.alloc_cache(kh, 2 * cap, dh)
    finally:
        hip.set_fp16(False)
    hip.write(old, x)
    hip.grow_cache(new, old, kh, cap, dh)
    want = np.zeros((kh, 2 * cap, dh), np.float32)
    want[:, :cap] = x
    assert np.array_equal(new.read(), want.ravel())


@pytest.mark.parametrize("fuse", [True, False], ids=["fused", "per_op"])
def test_half_rings_in_a_decode_step(hip, fuse):
    """The one-token attention block with fp16 rings inside a step: the QKV linear's rope and
    ring-store epilogue (fused) or the per-op store kernel writes rounded values, and the
    attention after it reads them; the same bits as the same step over fp32 rings whose
    contents are those halves."""
    d, heads, dh, cap, pos = 768, 12, 64, 4352, 4400
    inv = hip.upload((1.0 / 10000.0 ** (np.arange(32) * 2 / 64)).astype(np.float32))
    cs, sn = hip.alloc(32), hip.alloc(32)
    wqkv = hip.upload(rnd(3 * d, d, scale=0.02))
    x = hip.upload(rnd(d))
    k0, v0 = _f16(rnd(heads, cap, dh)), _f16(rnd(heads, cap, dh))
    hip.set_fp16(True)
    try:
        rings = {"h": (hip.alloc_cache(heads, cap, dh), hip.alloc_cache(heads, cap, dh))}
        rings["f"] = (hip.alloc(heads * cap * dh), hip.alloc(heads * cap * dh))
        got = {}
        for name, (kr, vr) in rings.items():
            hip.write(kr, k0)
            hip.write(vr, v0)
            y, q, k, att = hip.alloc(3 * d), hip.alloc(d), hip.alloc(d), hip.alloc(d)

            def body():
                hip.linear(y.ptr, wqkv.ptr, 3 * d, d, x.ptr, 1)
                hip.rope(q.ptr, y.ptr, cs.ptr, sn.ptr, 1, heads, dh)
                hip.rope(k.ptr, y.at(d), cs.ptr, sn.ptr, 1, heads, dh)
                hip.store(kr.ptr, k.ptr, pos, 1, cap, heads, dh)
                hip.store(vr.ptr, y.at(2 * d), pos, 1, cap, heads, dh)
                hip.attend(att.ptr, q.ptr, kr.ptr, vr.ptr, pos=pos, m=1, reach=4096, gap=0,
                           cap=cap, heads=heads, key_heads=heads, dh=dh, scale=0.125)
            if name == "f":  # the fp32 rings get the rounded new rows: store them rounded
                def body():  # noqa: F811
                    hip.linear(y.ptr, wqkv.ptr, 3 * d, d, x.ptr, 1)
                    hip.rope(q.ptr, y.ptr, cs.ptr, sn.ptr, 1, heads, dh)
                    hip.rope(k.ptr, y.at(d), cs.ptr, sn.ptr, 1, heads, dh)
            _step(hip, body, inv, cs, sn, fuse)
            if name == "f":
                kk, vv = _f16(k.read()), _f16(y.read()[2 * d:])
                hip.store(kr.ptr, hip.upload(kk).ptr, pos, 1, cap, heads, dh)
                hip.store(vr.ptr, hip.upload(vv).ptr, pos, 1, cap, heads, dh)
                hip.attend(att.ptr, q.ptr, kr.ptr, vr.ptr, pos=pos, m=1, reach=4096, gap=0,
                           cap=cap, heads=heads, key_heads=heads, dh=dh, scale=0.125)
            got[name] = (kr.read(), vr.read(), att.read(), q.read())
    finally:
        hip.set_fp16(False)
    for a, b in zip(got["h"], got["f"]):
        assert np.array_equal(a, b)
