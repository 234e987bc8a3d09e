"""ORACLE — test infrastructure only (tests/, the smoke check and bench.py's CPU-baseline
leg). ctypes binding of liboracle.so, the C++ restatement of the reference's CPU backend
and model (src/cpu.rs, src/model.rs, src/sample.rs), plus the config loader of
src/config.rs:20-105.

Nothing in the product imports this module.
"""

from __future__ import annotations

import ctypes as C
import json
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
_szp = C.POINTER(C.c_size_t)


class AttnArgs(C.Structure):
    """src/ops.rs:34-46."""

    _fields_ = [(n, C.c_size_t) for n in
                ("pos", "m", "reach", "gap", "cap", "heads", "key_heads", "dh")] + [
        ("scale", C.c_float)]


class _Cfg(C.Structure):
    _fields_ = [
        ("vocab_size", C.c_size_t), ("d_model", C.c_size_t), ("n_heads", C.c_size_t),
        ("global_kv_heads", C.c_size_t), ("global_logn", C.c_uint32),
        ("global_kshift", C.c_uint32), ("global_emb", C.c_uint32), ("global_far", C.c_uint32),
        ("prelude", C.c_char_p), ("core", C.c_char_p), ("coda", C.c_char_p),
        ("window", C.c_size_t), ("max_loops", C.c_size_t), ("default_loops", C.c_size_t),
        ("damp", C.c_float), ("rope_base", C.c_float), ("norm_eps", C.c_float)]


def build(quiet: bool = True, force: bool = False) -> Path:
    """Compiles liboracle.so with oracle/Makefile (`force`: even when it is up to date)."""
    out = subprocess.run(["make", "-C", str(HERE)] + (["-B"] if force else []), capture_output=True,
                         text=True)
    if out.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + out.stdout + out.stderr)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        build()
    L = C.CDLL(str(LIB_PATH))
    sz, f = C.c_size_t, C.c_float
    sig = {
        "oracle_dot": (None, [_f32p, _f32p, sz, C.POINTER(C.c_float)]),
        "oracle_linear": (None, [_f32p, _f32p, sz, sz, _f32p, sz]),
        "oracle_rms": (None, [_f32p, _f32p, _f32p, sz, sz, f]),
        "oracle_l2norm": (None, [_f32p, _f32p, sz, sz]),
        "oracle_silu_mul": (None, [_f32p, _f32p, _f32p, sz]),
        "oracle_rope_table": (None, [_f32p, _f32p, _f32p, sz, sz, sz]),
        "oracle_rope": (None, [_f32p, _f32p, _f32p, _f32p, sz, sz, sz]),
        "oracle_gla": (None, [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, sz, sz, sz]),
        "oracle_store": (None, [_f32p, _f32p, sz, sz, sz, sz, sz]),
        "oracle_attend": (None, [_f32p, _f32p, _f32p, _f32p, C.POINTER(AttnArgs), sz]),
        "oracle_attn_range": (None, [C.POINTER(AttnArgs), sz, _szp, _szp]),
        "oracle_attn_span": (sz, [C.POINTER(AttnArgs)]),
        "oracle_model_new": (C.c_void_p, [C.POINTER(_Cfg)]),
        "oracle_model_add": (None, [C.c_void_p, C.c_char_p, _szp, sz, _f32p]),
        "oracle_model_set_global_cap": (None, [C.c_void_p, sz]),
        "oracle_model_finish": (C.c_int, [C.c_void_p]),
        "oracle_model_error": (C.c_char_p, [C.c_void_p]),
        "oracle_model_params": (sz, [C.c_void_p]),
        "oracle_model_free": (None, [C.c_void_p]),
        "oracle_session_new": (C.c_void_p, [C.c_void_p, sz]),
        "oracle_session_free": (None, [C.c_void_p]),
        "oracle_session_pos": (sz, [C.c_void_p]),
        "oracle_feed": (None, [C.c_void_p, _u32p, sz, sz]),
        "oracle_advance": (None, [C.c_void_p, _u32p, sz, C.c_int]),
        "oracle_step": (None, [C.c_void_p, C.c_uint32]),
        "oracle_logits": (None, [C.c_void_p, _f32p]),
        "oracle_state_bytes": (sz, [C.c_void_p]),
        "oracle_kept_count": (sz, [C.c_void_p]),
        "oracle_kept_len": (sz, [C.c_void_p, sz]),
        "oracle_kept_read": (None, [C.c_void_p, sz, _f32p, sz]),
        "oracle_rng_new": (C.c_void_p, [C.c_uint64]),
        "oracle_rng_free": (None, [C.c_void_p]),
        "oracle_rng_next": (C.c_float, [C.c_void_p]),
        "oracle_pick": (C.c_uint32, [_f32p, sz, _u32p, sz, f, sz, f, f, sz, C.c_void_p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------------------------------
# src/config.rs
# ---------------------------------------------------------------------------------------

class Config:
    """`config.json` as src/config.rs:20-79 reads it (unknown keys are ignored)."""

    def __init__(self, d: dict):
        self.raw = dict(d)
        self.vocab_size = int(d["vocab_size"])
        self.d_model = int(d["d_model"])
        self.n_heads = int(d["n_heads"])
        self.global_kv_heads = int(d.get("global_kv_heads", 4))
        self.global_rope_base = float(d.get("global_rope_base", 0.0))
        self.global_logn = int(d.get("global_logn", 0))
        self.global_kshift = int(d.get("global_kshift", 0))
        self.global_emb = int(d.get("global_emb", 0))
        self.global_far = int(d.get("global_far", 0))
        self.prelude = str(d["prelude"])
        self.core = str(d["core"])
        self.coda = str(d["coda"])
        self.window = int(d["window"])
        self.max_loops = int(d["max_loops"])
        self.default_loops = int(d["default_loops"])
        self.loop_lora = int(d.get("loop_lora", 0))
        self.state_loops = int(d.get("state_loops", 0))
        self.damp = float(d.get("damp", 1.0))
        self.rope_base = float(d["rope_base"])
        self.norm_eps = float(d["norm_eps"])
        if self.loop_lora != 0:
            raise ValueError("loop_lora models are not supported")
        if self.state_loops != 0:
            raise ValueError("state_loops models are not supported")
        if self.global_rope_base != 0.0:
            raise ValueError("global_rope_base is not supported")

    @classmethod
    def load(cls, folder) -> "Config":
        return cls(json.loads((Path(folder) / "config.json").read_text(encoding="utf-8")))

    def head_dim(self) -> int:
        return self.d_model // self.n_heads

    def think_loops(self, level: str) -> int:
        """config.rs:85-94, with the aliases of config.rs:10-18."""
        level = {"none": "low", "minimal": "low", "xhigh": "max"}.get(level, level)
        d = self.default_loops
        return {"low": max(d // 2, 1), "medium": d, "high": min(d * 2, self.max_loops),
                "max": self.max_loops}[level]

    def loops(self, n=None) -> int:
        """config.rs:96-105."""
        if not self.core:
            return 0
        n = self.default_loops if n is None else n
        if not (1 <= n <= self.max_loops):
            raise ValueError(f"loops must be between 1 and {self.max_loops}")
        return n

    def _c(self) -> _Cfg:
        c = _Cfg()
        for k in ("vocab_size", "d_model", "n_heads", "global_kv_heads", "global_logn",
                  "global_kshift", "global_emb", "global_far", "window", "max_loops",
                  "default_loops", "damp", "rope_base", "norm_eps"):
            setattr(c, k, getattr(self, k))
        c.prelude, c.core, c.coda = (s.encode() for s in (self.prelude, self.core, self.coda))
        return c


def load_weights(folder) -> dict:
    """model.safetensors, f32 only (src/model.rs:36-54)."""
    from safetensors.numpy import load_file

    w = load_file(str(Path(folder) / "model.safetensors"))
    for name, t in w.items():
        if t.dtype != np.float32:
            raise ValueError(f"{name}: expected f32 weights")
    return w


# ---------------------------------------------------------------------------------------
# src/model.rs
# ---------------------------------------------------------------------------------------

CHUNK = 256  # model.rs:27


class Model:
    def __init__(self, folder=None, *, cfg: Config | None = None, weights: dict | None = None,
                 global_cap: int | None = None):
        L = lib()
        self.cfg = cfg if cfg is not None else Config.load(folder)
        weights = weights if weights is not None else load_weights(folder)
        self._c = self.cfg._c()
        self.h = L.oracle_model_new(C.byref(self._c))
        if global_cap is not None:
            L.oracle_model_set_global_cap(self.h, global_cap)
        for name, t in weights.items():
            t = _f32(t)
            shape = (C.c_size_t * t.ndim)(*t.shape)
            L.oracle_model_add(self.h, name.encode(), shape, t.ndim, t.reshape(-1))
        if L.oracle_model_finish(self.h) != 0:
            raise ValueError(L.oracle_model_error(self.h).decode())

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.oracle_model_free(self.h)
            self.h = None

    def params(self) -> int:
        return lib().oracle_model_params(self.h)

    def session(self, loops=None) -> "Session":
        return Session(self, self.cfg.loops(loops))


class Session:
    def __init__(self, model: Model, loops: int):
        self.model = model
        self.loops = loops
        self.h = lib().oracle_session_new(model.h, loops)

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.oracle_session_free(self.h)
            self.h = None

    @property
    def pos(self) -> int:
        return lib().oracle_session_pos(self.h)

    def feed(self, tokens, limit: int = CHUNK):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        lib().oracle_feed(self.h, t, t.size, limit)

    def advance(self, tokens, want_logits: bool):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        lib().oracle_advance(self.h, t, t.size, int(want_logits))

    def step(self, token: int):
        lib().oracle_step(self.h, int(token))

    def logits(self) -> np.ndarray:
        out = np.empty(self.model.cfg.vocab_size, dtype=np.float32)
        lib().oracle_logits(self.h, out)
        return out

    def state_bytes(self) -> int:
        return lib().oracle_state_bytes(self.h)

    def kept(self) -> list:
        """Every buffer that outlives a step, in model.rs:626-638 order (logits first)."""
        L = lib()
        out = []
        for i in range(L.oracle_kept_count(self.h)):
            n = L.oracle_kept_len(self.h, i)
            a = np.empty(n, dtype=np.float32)
            L.oracle_kept_read(self.h, i, a, n)
            out.append(a)
        return out


# ---------------------------------------------------------------------------------------
# src/sample.rs
# ---------------------------------------------------------------------------------------

class Rng:
    def __init__(self, seed: int):
        self.h = lib().oracle_rng_new(seed)

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.oracle_rng_free(self.h)
            self.h = None

    def next_f32(self) -> float:
        return lib().oracle_rng_next(self.h)


def pick(logits, recent=(), temperature=0.0, top_k=0, top_p=1.0, repeat_penalty=1.0,
         repeat_window=0, rng: Rng | None = None) -> int:
    rng = rng or Rng(0)
    lg = _f32(logits)
    rc = np.ascontiguousarray(recent, dtype=np.uint32)
    return int(lib().oracle_pick(lg, lg.size, rc, rc.size, temperature, top_k, top_p,
                                 repeat_penalty, repeat_window, rng.h))


# ---------------------------------------------------------------------------------------
# single ops (host arrays in, host arrays out)
# ---------------------------------------------------------------------------------------

def linear(w, x, rows, cols, m):
    y = np.empty(m * rows, dtype=np.float32)
    lib().oracle_linear(y, _f32(w).reshape(-1), rows, cols, _f32(x).reshape(-1), m)
    return y


def rms(x, w, groups, size, eps):
    y = np.empty(groups * size, dtype=np.float32)
    lib().oracle_rms(y, _f32(x).reshape(-1), _f32(w), groups, size, eps)
    return y


def l2norm(x, heads, dh):
    y = np.empty(heads * dh, dtype=np.float32)
    lib().oracle_l2norm(y, _f32(x).reshape(-1), heads, dh)
    return y


def silu_mul(g, u):
    g, u = _f32(g).reshape(-1), _f32(u).reshape(-1)
    y = np.empty(g.size, dtype=np.float32)
    lib().oracle_silu_mul(y, g, u, g.size)
    return y


def rope_table(inv, pos, m, half):
    c = np.empty(m * half, dtype=np.float32)
    s = np.empty(m * half, dtype=np.float32)
    lib().oracle_rope_table(c, s, _f32(inv), pos, m, half)
    return c, s


def rope(x, cos, sin, m, heads, dh):
    y = np.empty(m * heads * dh, dtype=np.float32)
    lib().oracle_rope(y, _f32(x).reshape(-1), _f32(cos), _f32(sin), m, heads, dh)
    return y


def gla(s, q, k, v, decay, bias, m, heads, dh):
    """Returns (y, new state)."""
    st = _f32(s).reshape(-1).copy()
    y = np.empty(m * heads * dh, dtype=np.float32)
    lib().oracle_gla(y, st, _f32(q).reshape(-1), _f32(k).reshape(-1), _f32(v).reshape(-1),
                     _f32(decay).reshape(-1), _f32(bias), m, heads, dh)
    return y, st


def store(cache, src, pos, m, cap, heads, dh):
    c = _f32(cache).reshape(-1).copy()
    lib().oracle_store(c, _f32(src).reshape(-1), pos, m, cap, heads, dh)
    return c


def attend(q, k, v, **a):
    args = AttnArgs(**a)
    y = np.empty(args.m * args.heads * args.dh, dtype=np.float32)
    k, v = _f32(k).reshape(-1), _f32(v).reshape(-1)
    lib().oracle_attend(y, _f32(q).reshape(-1), k, v, C.byref(args), k.size)
    return y


def attn_range(i, **a):
    lo, hi = C.c_size_t(), C.c_size_t()
    lib().oracle_attn_range(C.byref(AttnArgs(**a)), i, C.byref(lo), C.byref(hi))
    return lo.value, hi.value


def attn_span(**a):
    return lib().oracle_attn_span(C.byref(AttnArgs(**a)))


USIZE_MAX = 2 ** 64 - 1
