"""The C-ABI library without a GPU: it loads, exports every function include/*.h declares,
and reports a missing device as SLM_NO_DEVICE rather than failing (src/cuda.rs:72-83)."""

import ctypes
import subprocess

import pytest


def test_library_exports_every_declared_symbol(pkg):
    names = pkg.header_symbols()
    assert len(names) > 30
    missing = [n for n in names if not hasattr(pkg.lib, n)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", str(pkg.LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert set(names) <= exported


def test_every_trait_method_has_an_entry_point(pkg):
    """src/ops.rs:68-228: each Ops method maps to one slm_hip_* function."""
    methods = ["name", "zeros", "upload", "read", "flush", "gather", "copy", "shift", "columns",
               "linear", "add", "add_row", "scale_rows", "mix", "rms", "silu_mul", "rope_table",
               "rope", "l2norm", "gla", "store", "attend"]
    alias = {"zeros": "alloc"}
    names = set(pkg.header_symbols())
    for m in methods:
        assert f"slm_hip_{alias.get(m, m)}" in names, m


def test_code_object_is_gfx950(pkg):
    lib = pkg.lib
    size = ctypes.c_size_t.in_dll(lib, "slm_code_object_size").value
    blob = (ctypes.c_ubyte * size).in_dll(lib, "slm_code_object")
    data = bytes(blob)
    assert b"gfx950" in data
    assert b"slm_linear_small_v" in data and b"slm_attn_part_4" in data


def test_no_device_is_not_an_error(pkg):
    try:
        import torch

        if torch.cuda.device_count() > 0:
            pytest.skip("a GPU is present")
    except ImportError:
        pass
    with pytest.raises(pkg.NoDevice):
        pkg.Hip(0)
    assert pkg.lib.slm_hip_last_error(None) == b"no usable AMD GPU"


def _ref_pick(l):
    """sample.rs:48-53 as written: b = 0, b = i whenever l[i] > l[b]."""
    b = 0
    for i in range(len(l)):
        if l[i] > l[b]:
            b = i
    return b


def test_host_greedy_pick(pkg):
    """The twin's host pick (slm_pick_greedy, two passes) against sample.rs's loop as written and
    against the oracle's pick: ties (the first wins), NaN at 0 and inside, all -inf, +-0,
    infinities, one and 1025 elements, and random logits of the vocabulary's size."""
    import numpy as np
    import oracle as O

    nan, inf = float("nan"), float("inf")
    cases = [[0.0], [1.0, 1.0, 0.5], [0.0, 3.0, 1.0], [nan, 5.0, 9.0], [1.0, nan, 2.0, nan],
             [-inf, -inf, -inf], [-0.0, 0.0, -0.0], [0.0, -0.0], [-1.0, inf, inf], [-inf, nan, -inf],
             [nan, nan], [3.0, 2.0, 3.0, 3.0], list(np.arange(1025, dtype=np.float32) % 7)]
    rng = np.random.default_rng(5)
    for _ in range(40):
        x = rng.standard_normal(32000).astype(np.float32)
        if rng.random() < 0.5:
            x[rng.integers(0, 32000, 3)] = x.max()  # ties at the maximum
        if rng.random() < 0.3:
            x[rng.integers(0, 32000, 5)] = nan
        cases.append(list(x))
    for c in cases:
        a = np.asarray(c, dtype=np.float32)
        want = _ref_pick(a.tolist())
        assert pkg.pick_greedy(a) == want == O.pick(a), c[:8]
