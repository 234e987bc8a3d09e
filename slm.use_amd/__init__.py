"""slm.use_amd — the MI355X (gfx950) backend for SLM.use's token loop.

The product is `libslm_hip.so` (built by `build.py`): the C ABI of include/slm_hip.h, one
entry point per method of the reference's `Ops` trait (src/ops.rs:68-228), over
hand-written gfx950 kernels loaded with hipModuleLoadData; plus the model twin of
include/slm_model.h, which drives that ABI exactly as src/model.rs drives the trait.

This module is a thin ctypes binding of both, for tests and benchmarks. Importing it
fails loudly when the library is not built; opening a context fails loudly without a GPU.
There is no fallback path: every operation runs the HIP kernels.
"""

from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
LIB_PATH = PKG / "libslm_hip.so"
HEADERS = [ROOT / "include" / "slm_hip.h", ROOT / "include" / "slm_model.h"]

SLM_OK, SLM_NO_DEVICE = 0, 1
CODES = {-1: "SLM_E_INVALID", -2: "SLM_E_HIP", -3: "SLM_E_UNSUPPORTED", -4: "SLM_E_MEMORY",
         -5: "SLM_E_BOUNDS"}
USIZE_MAX = 2 ** 64 - 1


class SlmError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{CODES.get(code, code)}: {msg}")
        self.code = code


class NoDevice(RuntimeError):
    pass


class Attn(C.Structure):
    """slm_attn, src/ops.rs:34-46."""

    _fields_ = [(n, C.c_size_t) for n in
                ("pos", "m", "reach", "gap", "cap", "heads", "key_heads", "dh")] + [
        ("scale", C.c_float)]


if not LIB_PATH.exists():
    raise ImportError(f"{LIB_PATH} is not built: run `python slm.use_amd/build.py` "
                      "(or __graft_entry__.build())")

lib = C.CDLL(str(LIB_PATH))

_p = C.c_void_p
_sz = C.c_size_t
_f = C.c_float
_i = C.c_int
_u32p = C.POINTER(C.c_uint32)
_f32p = C.POINTER(C.c_float)

_SIGS = {
    "slm_hip_open": (_i, [_i, C.POINTER(_p)]),
    "slm_hip_close": (None, [_p]),
    "slm_hip_last_error": (C.c_char_p, [_p]),
    "slm_hip_name": (_i, [_p, C.c_char_p, _sz]),
    "slm_hip_alloc": (_i, [_p, _sz, C.POINTER(_p)]),
    "slm_hip_alloc_half": (_i, [_p, _sz, C.POINTER(_p)]),
    "slm_hip_get_fp16": (_i, [_p, C.POINTER(_i)]),
    "slm_hip_free": (_i, [_p, _p]),
    "slm_hip_upload": (_i, [_p, _p, _f32p, _sz]),
    "slm_hip_read": (_i, [_p, _f32p, _p, _sz]),
    "slm_hip_flush": (_i, [_p, C.POINTER(_p), _sz]),
    "slm_hip_gather": (_i, [_p, _p, _p, _u32p, _sz, _sz]),
    "slm_hip_gather_dev": (_i, [_p, _p, _p, _p, _sz, _sz]),
    "slm_hip_argmax": (_i, [_p, _p, _p, _sz, _sz, _p, _sz]),
    "slm_hip_copy": (_i, [_p, _p, _p, _sz]),
    "slm_hip_shift": (_i, [_p, _p, _p, _p, _sz, _sz]),
    "slm_hip_columns": (_i, [_p, _p, _p, _sz, _sz, _sz, _sz]),
    "slm_hip_linear": (_i, [_p, _p, _p, _sz, _sz, _p, _sz]),
    "slm_hip_add": (_i, [_p, _p, _p, _p, _sz]),
    "slm_hip_add_row": (_i, [_p, _p, _p, _p, _sz, _sz]),
    "slm_hip_scale_rows": (_i, [_p, _p, _p, _f32p, _sz, _sz]),
    "slm_hip_mix": (_i, [_p, _p, _p, _p, _sz, _f]),
    "slm_hip_rms": (_i, [_p, _p, _p, _p, _sz, _sz, _f]),
    "slm_hip_silu_mul": (_i, [_p, _p, _p, _p, _sz]),
    "slm_hip_rope_table": (_i, [_p, _p, _p, _p, _sz, _sz, _sz]),
    "slm_hip_rope": (_i, [_p, _p, _p, _p, _p, _sz, _sz, _sz]),
    "slm_hip_l2norm": (_i, [_p, _p, _p, _sz, _sz]),
    "slm_hip_gla": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _sz, _sz, _sz]),
    "slm_hip_store": (_i, [_p, _p, _p, _sz, _sz, _sz, _sz, _sz]),
    "slm_hip_attend": (_i, [_p, _p, _p, _p, _p, _p, C.POINTER(Attn)]),
    "slm_hip_attend_noalloc": (_i, [_p, _p, _p, _p, _p, _p, C.POINTER(Attn)]),
    "slm_hip_set_graphs": (_i, [_p, _i]),
    "slm_hip_set_step_kernel": (_i, [_p, _i]),
    "slm_hip_step_stats": (_i, [_p, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64), C.POINTER(C.c_int)]),
    "slm_hip_set_prompt_lanes": (_i, [_p, _i]),
    "slm_hip_read_ahead_stats": (_i, [_p, C.POINTER(C.c_uint64)]),
    "slm_hip_get_prompt_lanes": (_i, [_p, C.POINTER(C.c_int)]),
    "slm_hip_prompt_lane_stats": (_i, [_p, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
    "slm_hip_set_fusion": (_i, [_p, _i]),
    "slm_hip_set_fp16": (_i, [_p, _i]),
    "slm_hip_graph_stats": (_i, [_p, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64),
                                 C.POINTER(C.c_uint64)]),
    "slm_hip_last_plan": (_i, [_p, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
    "slm_hip_set_timing": (_i, [_p, C.c_int]),
    "slm_hip_kernel_stat": (_i, [_p, C.c_char_p, C.POINTER(C.c_longlong), C.POINTER(C.c_double),
                                 C.POINTER(C.c_double)]),
    "slm_hip_probe_mfma": (_i, [_p, _p, _p, _p]),
    "slm_hip_set_spin_limit": (_i, [_p, C.c_longlong]),
    "slm_hip_stream": (_i, [_p, C.POINTER(_p)]),
    "slm_hip_set_half_shadows": (_i, [_p, _i]),
    "slm_hip_set_tile_rows": (_i, [_p, _i]),
    "slm_hip_alloc_cache": (_i, [_p, _sz, _sz, _sz, C.POINTER(_p)]),
    "slm_hip_grow_cache": (_i, [_p, _p, _p, _sz, _sz, _sz]),
    "slm_hip_mem_info": (_i, [_p, C.POINTER(_sz), C.POINTER(_sz), C.POINTER(_sz)]),
    "slm_model_load": (_i, [_p, C.c_char_p, C.POINTER(_p)]),
    "slm_model_free": (None, [_p]),
    "slm_model_error": (C.c_char_p, [_p]),
    "slm_model_params": (_sz, [_p]),
    "slm_model_set_global_cap": (_i, [_p, _sz]),
    "slm_model_set_device_grow": (_i, [_p, _i]),
    "slm_session_new": (_i, [_p, _sz, C.POINTER(_p)]),
    "slm_session_free": (None, [_p]),
    "slm_session_pos": (_sz, [_p]),
    "slm_session_loops": (_sz, [_p]),
    "slm_session_feed": (_i, [_p, _u32p, _sz, _sz]),
    "slm_session_advance": (_i, [_p, _u32p, _sz, _i]),
    "slm_session_step": (_i, [_p, C.c_uint32]),
    "slm_session_logits": (_i, [_p, _f32p]),
    "slm_session_state_bytes": (_sz, [_p]),
    "slm_session_kept_count": (_sz, [_p]),
    "slm_session_kept_len": (_sz, [_p, _sz]),
    "slm_session_kept_read": (_i, [_p, _sz, _f32p, _sz]),
    "slm_session_decode_greedy": (_i, [_p, _sz, _u32p]),
    "slm_pick_greedy": (_sz, [_f32p, _sz]),
    "slm_session_decode_greedy_device": (_i, [_p, _sz, _u32p]),
}
for _name, (_res, _args) in _SIGS.items():
    _fn = getattr(lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _fp(a: np.ndarray):
    return a.ctypes.data_as(_f32p)


def _up(a: np.ndarray):
    return a.ctypes.data_as(_u32p)


class Buffer:
    """A device buffer of n floats owned by a Hip context."""

    def __init__(self, hip: "Hip", ptr: int, n: int):
        self.hip, self.ptr, self.n = hip, ptr, n

    def at(self, offset: int) -> int:
        """The pointer of the `At { buf, offset }` view (ops.rs:13-17)."""
        return self.ptr + 4 * offset

    def read(self, n: int | None = None) -> np.ndarray:
        return self.hip.read(self, self.n if n is None else n)

    def free(self):
        if self.ptr:
            self.hip.check(lib.slm_hip_free(self.hip.ctx, self.ptr))
            self.ptr = 0


class Hip:
    """A backend context: one device, one stream (slm_hip_open)."""

    def __init__(self, device: int = 0):
        ctx = _p()
        rc = lib.slm_hip_open(device, C.byref(ctx))
        if rc == SLM_NO_DEVICE:
            raise NoDevice(lib.slm_hip_last_error(None).decode())
        if rc != SLM_OK:
            raise SlmError(rc, lib.slm_hip_last_error(None).decode())
        self.ctx = ctx.value

    def close(self):
        if getattr(self, "ctx", None):
            lib.slm_hip_close(self.ctx)
            self.ctx = None

    def __del__(self):
        self.close()

    def check(self, rc: int):
        if rc != SLM_OK:
            raise SlmError(rc, lib.slm_hip_last_error(self.ctx).decode())

    def name(self) -> str:
        buf = C.create_string_buffer(256)
        self.check(lib.slm_hip_name(self.ctx, buf, 256))
        return buf.value.decode()

    def alloc(self, n: int) -> Buffer:
        p = _p()
        self.check(lib.slm_hip_alloc(self.ctx, n, C.byref(p)))
        return Buffer(self, p.value, max(n, 1))

    def upload(self, data) -> Buffer:
        a = _f32(data).reshape(-1)
        b = self.alloc(a.size)
        self.check(lib.slm_hip_upload(self.ctx, b.ptr, _fp(a), a.size))
        return b

    def upload_into(self, buf: Buffer, data, offset: int = 0):
        """slm_hip_upload into an existing buffer, at `offset` floats."""
        a = _f32(data).reshape(-1)
        self.check(lib.slm_hip_upload(self.ctx, buf.at(offset), _fp(a), a.size))

    def upload_half(self, data) -> Buffer:
        """fp16 weights (slm_hip_alloc_half): `data` rounded to fp16; read() widens them back."""
        a = _f32(data).reshape(-1)
        p = _p()
        self.check(lib.slm_hip_alloc_half(self.ctx, a.size, C.byref(p)))
        b = Buffer(self, p.value, max(a.size, 1))
        self.check(lib.slm_hip_upload(self.ctx, b.ptr, _fp(a), a.size))
        return b

    def alloc_cache(self, heads: int, cap: int, dh: int) -> Buffer:
        """Ops::zeros_cache (slm_hip_alloc_cache): fp16 values in fp16 mode where the fp16
        attention kernels take the shape, else fp32. Its pointer is the cache's start only."""
        p = _p()
        self.check(lib.slm_hip_alloc_cache(self.ctx, heads, cap, dh, C.byref(p)))
        return Buffer(self, p.value, max(heads * cap * dh, 1))

    def grow_cache(self, dst: Buffer, src: Buffer, heads: int, cap: int, dh: int):
        self.check(lib.slm_hip_grow_cache(self.ctx, dst.ptr, src.ptr, heads, cap, dh))

    def get_fp16(self) -> bool:
        on = C.c_int()
        self.check(lib.slm_hip_get_fp16(self.ctx, C.byref(on)))
        return bool(on.value)

    def write(self, buf: Buffer, data, offset: int = 0):
        a = _f32(data).reshape(-1)
        self.check(lib.slm_hip_upload(self.ctx, buf.at(offset), _fp(a), a.size))

    def read(self, buf: Buffer | int, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.float32)
        ptr = buf.ptr if isinstance(buf, Buffer) else buf
        self.check(lib.slm_hip_read(self.ctx, _fp(out), ptr, n))
        return out

    def set_graphs(self, on: bool):
        self.check(lib.slm_hip_set_graphs(self.ctx, int(on)))

    def set_step_kernel(self, on: bool):
        self.check(lib.slm_hip_set_step_kernel(self.ctx, int(on)))

    def step_stats(self):
        a, b, c = C.c_uint64(), C.c_uint64(), C.c_int()
        self.check(lib.slm_hip_step_stats(self.ctx, C.byref(a), C.byref(b), C.byref(c)))
        return dict(launches=a.value, programs=b.value, available=bool(c.value))

    def read_ahead_stats(self) -> int:
        n = C.c_uint64()
        self.check(lib.slm_hip_read_ahead_stats(self.ctx, C.byref(n)))
        return n.value

    def set_prompt_lanes(self, n: int):
        self.check(lib.slm_hip_set_prompt_lanes(self.ctx, int(n)))

    def prompt_lanes(self) -> int:
        n = C.c_int()
        self.check(lib.slm_hip_get_prompt_lanes(self.ctx, C.byref(n)))
        return n.value

    def lane_stats(self):
        a, b = C.c_uint64(), C.c_uint64()
        self.check(lib.slm_hip_prompt_lane_stats(self.ctx, C.byref(a), C.byref(b)))
        return dict(steps=a.value, fallbacks=b.value)

    def last_plan(self):
        a, b = C.c_uint64(), C.c_uint64()
        self.check(lib.slm_hip_last_plan(self.ctx, C.byref(a), C.byref(b)))
        return dict(ops=a.value, kernels=b.value)

    def set_timing(self, on: bool):
        """Per-kernel HIP-event timing of launches made outside graphs (resets the stats)."""
        self.check(lib.slm_hip_set_timing(self.ctx, int(on)))

    def kernel_stat(self, name: str):
        n, us, b = C.c_longlong(), C.c_double(), C.c_double()
        self.check(lib.slm_hip_kernel_stat(self.ctx, name.encode(), C.byref(n), C.byref(us),
                                           C.byref(b)))
        return dict(launches=n.value, us=us.value, bytes=b.value)

    def set_fusion(self, on: bool):
        self.check(lib.slm_hip_set_fusion(self.ctx, int(on)))

    def set_fp16(self, on: bool):
        """fp16 mode: every linear rounds its operands to fp16 at fp16 MFMAs (sums in fp32)."""
        self.check(lib.slm_hip_set_fp16(self.ctx, int(on)))

    def graph_stats(self):
        a, b, c = C.c_uint64(), C.c_uint64(), C.c_uint64()
        self.check(lib.slm_hip_graph_stats(self.ctx, C.byref(a), C.byref(b), C.byref(c)))
        return dict(launched=a.value, captured=b.value, eager=c.value)

    # -- operations: pointers are ints (Buffer.ptr or Buffer.at(offset)) --
    def flush(self, keep=()):
        arr = (_p * max(len(keep), 1))(*keep)
        self.check(lib.slm_hip_flush(self.ctx, arr, len(keep)))

    def gather(self, y, w, ids, d):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        self.check(lib.slm_hip_gather(self.ctx, y, w, _up(ids), ids.size, d))

    def gather_dev(self, y, w, tok, rows, d):
        self.check(lib.slm_hip_gather_dev(self.ctx, y, w, tok, rows, d))

    def argmax(self, tok, ids, ids_cap, slot, x, n):
        self.check(lib.slm_hip_argmax(self.ctx, tok, ids, ids_cap, slot, x, n))

    def copy(self, y, x, n):
        self.check(lib.slm_hip_copy(self.ctx, y, x, n))

    def shift(self, y, first, x, m, d):
        self.check(lib.slm_hip_shift(self.ctx, y, first, x, m, d))

    def columns(self, y, x, m, stride, off, length):
        self.check(lib.slm_hip_columns(self.ctx, y, x, m, stride, off, length))

    def linear(self, y, w, rows, cols, x, m):
        self.check(lib.slm_hip_linear(self.ctx, y, w, rows, cols, x, m))

    def add(self, y, a, b, n):
        self.check(lib.slm_hip_add(self.ctx, y, a, b, n))

    def add_row(self, y, x, row, m, d):
        self.check(lib.slm_hip_add_row(self.ctx, y, x, row, m, d))

    def scale_rows(self, y, x, f, d):
        f = _f32(f).reshape(-1)
        self.check(lib.slm_hip_scale_rows(self.ctx, y, x, _fp(f), f.size, d))

    def mix(self, y, a, b, n, t):
        self.check(lib.slm_hip_mix(self.ctx, y, a, b, n, t))

    def rms(self, y, x, w, groups, size, eps):
        self.check(lib.slm_hip_rms(self.ctx, y, x, w, groups, size, eps))

    def silu_mul(self, y, g, u, n):
        self.check(lib.slm_hip_silu_mul(self.ctx, y, g, u, n))

    def rope_table(self, cs, sn, inv, pos, m, half):
        self.check(lib.slm_hip_rope_table(self.ctx, cs, sn, inv, pos, m, half))

    def rope(self, y, x, cs, sn, m, heads, dh):
        self.check(lib.slm_hip_rope(self.ctx, y, x, cs, sn, m, heads, dh))

    def l2norm(self, y, x, heads, dh):
        self.check(lib.slm_hip_l2norm(self.ctx, y, x, heads, dh))

    def gla(self, y, s, q, k, v, decay, bias, m, heads, dh):
        self.check(lib.slm_hip_gla(self.ctx, y, s, q, k, v, decay, bias, m, heads, dh))

    def store(self, cache, src, pos, m, cap, heads, dh):
        self.check(lib.slm_hip_store(self.ctx, cache, src, pos, m, cap, heads, dh))

    def attend(self, y, q, k, v, **a):
        args = Attn(**a)
        self.check(lib.slm_hip_attend(self.ctx, y, None, q, k, v, C.byref(args)))

    def attend_noalloc(self, y, q, k, v, **a):
        """attend with its partials in the device's fixed scratch (no allocation)."""
        args = Attn(**a)
        self.check(lib.slm_hip_attend_noalloc(self.ctx, y, None, q, k, v, C.byref(args)))

    def stream(self) -> int:
        s = _p()
        self.check(lib.slm_hip_stream(self.ctx, C.byref(s)))
        return s.value or 0

    def set_tile_rows(self, rows: int):
        """Fused GEMV rows per tile: 0 = the planner's choice, or 16, 12, 8, 4."""
        self.check(lib.slm_hip_set_tile_rows(self.ctx, int(rows)))

    def set_half_shadows(self, on: bool):
        """fp16 mode's fp16 copies of the weights its linears read (on by default)."""
        self.check(lib.slm_hip_set_half_shadows(self.ctx, int(on)))

    def mem_info(self):
        """(free, total) bytes of the device and the bytes this context holds."""
        f, t, h = _sz(), _sz(), _sz()
        self.check(lib.slm_hip_mem_info(self.ctx, C.byref(f), C.byref(t), C.byref(h)))
        return f.value, t.value, h.value

    def set_spin_limit(self, polls: int):
        """Polls a fused kernel's bounded wait makes before it gives up (0: at once)."""
        self.check(lib.slm_hip_set_spin_limit(self.ctx, polls))

    def probe_mfma(self, out, a, b):
        self.check(lib.slm_hip_probe_mfma(self.ctx, out, a, b))


class Model:
    """The model twin (include/slm_model.h) on a Hip context."""

    def __init__(self, hip: Hip, folder, global_cap: int | None = None,
                 device_grow: bool = False):
        import json

        self.hip = hip
        self.cfg = _Cfg(json.loads((Path(folder) / "config.json").read_text()))
        h = _p()
        rc = lib.slm_model_load(hip.ctx, str(folder).encode(), C.byref(h))
        if rc != SLM_OK:
            raise SlmError(rc, lib.slm_model_error(None).decode())
        self.h = h.value
        if global_cap is not None:
            self.check(lib.slm_model_set_global_cap(self.h, global_cap))
        # grow global caches as model.rs:383-398 does (read, host relayout, upload) unless
        # device_grow asks for the device-copy relayout
        self.check(lib.slm_model_set_device_grow(self.h, int(device_grow)))

    def check(self, rc: int):
        if rc != SLM_OK:
            raise SlmError(rc, lib.slm_model_error(self.h).decode())

    def params(self) -> int:
        return lib.slm_model_params(self.h)

    def session(self, loops: int | None = None) -> "Session":
        s = _p()
        self.check(lib.slm_session_new(self.h, loops or 0, C.byref(s)))
        return Session(self, s.value)

    def free(self):
        if getattr(self, "h", None):
            lib.slm_model_free(self.h)
            self.h = None

    def __del__(self):
        # sessions hold a reference to the model, so they are gone first
        if getattr(self, "hip", None) is not None and self.hip.ctx:
            self.free()


class Session:
    def __init__(self, model: Model, h: int):
        self.model, self.h = model, h

    def __del__(self):
        if getattr(self, "h", None) and self.model.hip.ctx and self.model.h:
            lib.slm_session_free(self.h)
            self.h = None

    @property
    def pos(self) -> int:
        return lib.slm_session_pos(self.h)

    @property
    def loops(self) -> int:
        return lib.slm_session_loops(self.h)

    def feed(self, tokens, limit: int = 256):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        self.model.check(lib.slm_session_feed(self.h, _up(t), t.size, limit))

    def advance(self, tokens, want_logits: bool):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        self.model.check(lib.slm_session_advance(self.h, _up(t), t.size, int(want_logits)))

    def step(self, token: int):
        self.model.check(lib.slm_session_step(self.h, int(token)))

    def logits(self) -> np.ndarray:
        out = np.empty(self.model.cfg.vocab_size, dtype=np.float32)
        self.model.check(lib.slm_session_logits(self.h, _fp(out)))
        return out

    def state_bytes(self) -> int:
        return lib.slm_session_state_bytes(self.h)

    def kept(self) -> list:
        out = []
        for i in range(lib.slm_session_kept_count(self.h)):
            n = lib.slm_session_kept_len(self.h, i)
            a = np.empty(n, dtype=np.float32)
            self.model.check(lib.slm_session_kept_read(self.h, i, _fp(a), n))
            out.append(a)
        return out

    def decode_greedy(self, n: int) -> np.ndarray:
        ids = np.empty(n, dtype=np.uint32)
        self.model.check(lib.slm_session_decode_greedy(self.h, n, _up(ids)))
        return ids

    def decode_greedy_device(self, n: int) -> np.ndarray:
        """decode_greedy with the pick on the device: no logits read-back between steps."""
        ids = np.empty(n, dtype=np.uint32)
        self.model.check(lib.slm_session_decode_greedy_device(self.h, n, _up(ids)))
        return ids


class _Cfg:
    def __init__(self, d):
        self.raw = d
        self.vocab_size = int(d["vocab_size"])
        self.d_model = int(d["d_model"])
        self.n_heads = int(d["n_heads"])
        self.default_loops = int(d["default_loops"])

    def head_dim(self):
        return self.d_model // self.n_heads


def header_symbols() -> list:
    """Every function declared in include/*.h."""
    import re

    names = []
    for h in HEADERS:
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"^\s*[\w\s\*]+?\b(slm_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def pick_greedy(logits) -> int:
    """sample.rs:48-53's greedy pick, as the model twin's host decode loop runs it."""
    a = np.ascontiguousarray(logits, dtype=np.float32)
    return int(lib.slm_pick_greedy(_fp(a), a.size))
