"""Shared helpers for the GPU tests."""

import os
import sys
import tempfile
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT / "slm.use_amd"))

import synth  # noqa: E402


def model_dir(name: str, seed: int) -> Path:
    """A synthetic model folder (cached under the temp dir for the process's lifetime)."""
    base = Path(os.environ.get("SLM_MODEL_CACHE", tempfile.gettempdir())) / "slm_models"
    return synth.write_model(base / f"{name}-{seed}", name, seed)


def rel(a, b) -> float:
    """||a - b||_inf / ||b||_inf."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def greedy(logits) -> int:
    """src/sample.rs:48-53: fold(0, |b, (i, v)| if v > logits[b] { i } else { b }) — the
    first maximum wins, a NaN never wins, and a NaN at index 0 keeps index 0."""
    x = np.asarray(logits, np.float32)
    b = 0
    for i in np.flatnonzero(x > x[0]) if not np.isnan(x[0]) else ():
        if x[i] > x[b]:
            b = int(i)
    return b


def attend64(q, k, v, pos, m, reach, gap, cap, heads, key_heads, dh, scale):
    """Softmax attention in float64 over positions picked by number (ops.rs:48-66)."""
    out = np.zeros((m, heads, dh))
    group = heads // key_heads
    kk = np.asarray(k, np.float64).reshape(key_heads, cap, dh)
    vv = np.asarray(v, np.float64).reshape(key_heads, cap, dh)
    q = np.asarray(q, np.float64).reshape(m, heads, dh)
    for i in range(m):
        p = pos + i
        lo, hi = max(0, p - reach + 1), max(0, p + 1 - gap)
        if hi <= lo:
            continue
        slots = np.arange(lo, hi) % cap
        for h in range(heads):
            s = kk[h // group, slots] @ q[i, h] * scale
            e = np.exp(s - s.max())
            out[i, h] = (e / e.sum()) @ vv[h // group, slots]
    return out.reshape(-1)
