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
