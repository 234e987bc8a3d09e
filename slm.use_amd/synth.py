"""Seeded random-weight models in the reference's layout (model.safetensors + config.json),
for parity tests and benchmarks. There is no network for checkpoints, so every model here
is synthetic.

Initialisation (the reference fixture's scheme, tools/make_fixture.py:55-60 via PyTorch
defaults, restated): every matrix N(0, 0.02), every norm weight 1, GLA decay bias
ln(u / (1 - u)) with u = 0.1 · 0.01^(h / (H - 1)). Unlike the fixture, `loop_embed` and
`decay.weight` are N(0, 0.02) too, so that add_row and the decay linear carry signal.
Numbers come from numpy's PCG64 generator (`numpy.random.default_rng(seed)`), drawn in
the order the tensors are listed by `tensor_specs`.

Weight names and shapes follow src/model.rs:114-153 and 226-251.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np

TINY = dict(vocab_size=97, d_model=32, n_heads=4, global_kv_heads=2, global_rope_base=0.0,
            global_logn=16, global_kshift=1, global_emb=1, global_far=1,
            mlp_mult=4.0, prelude="S", core="LS", coda="SG", window=8, max_loops=6,
            loop_lora=0, default_loops=3, state_loops=0, damp=1.0, rope_base=10000.0,
            norm_eps=1e-6)

# 86M-class: d 768, 12 x 64 heads, FFN 4x, vocab 32000, window 4096, no G layers.
A86 = dict(vocab_size=32000, d_model=768, n_heads=12, global_kv_heads=4, global_rope_base=0.0,
           global_logn=0, global_kshift=0, global_emb=0, global_far=0, mlp_mult=4.0,
           prelude="SS", core="LS", coda="SS", window=4096, max_loops=16, loop_lora=0,
           default_loops=4, state_loops=0, damp=1.0, rope_base=10000.0, norm_eps=1e-6)

# The same dims with global layers: prelude SG, coda SG, 4 key heads, logn/kshift/emb/far on.
G86 = dict(A86, prelude="SG", coda="SG", global_logn=4096, global_kshift=1, global_emb=1,
           global_far=1)

CONFIGS = {"tiny": TINY, "a86": A86, "g86": G86}


def tensor_specs(cfg: dict):
    """(name, shape, kind) in generation order; kind is 'mat', 'ones' or 'decay_bias'."""
    d, H = cfg["d_model"], cfg["n_heads"]
    dh = d // H
    hidden = int(round(cfg.get("mlp_mult", 4.0) * d))
    kd = cfg["global_kv_heads"] * dh
    out = []
    for part in ("prelude", "core", "coda"):
        for i, kind in enumerate(cfg[part]):
            p = f"{part}.{i}"
            if kind == "S":
                out += [(f"{p}.mixer.qkv.weight", (3 * d, d), "mat"),
                        (f"{p}.mixer.o.weight", (d, d), "mat")]
            elif kind == "L":
                out += [(f"{p}.mixer.qkvg.weight", (4 * d, d), "mat"),
                        (f"{p}.mixer.decay.weight", (H, d), "mat"),
                        (f"{p}.mixer.decay.bias", (H,), "decay_bias"),
                        (f"{p}.mixer.head_norm.weight", (dh,), "ones"),
                        (f"{p}.mixer.o.weight", (d, d), "mat")]
            elif kind == "G":
                out += [(f"{p}.mixer.q.weight", (d, d), "mat"),
                        (f"{p}.mixer.kv.weight", (2 * kd, d), "mat"),
                        (f"{p}.mixer.o.weight", (d, d), "mat")]
                if cfg.get("global_emb", 0):
                    out.append((f"{p}.mixer.norm_e.weight", (d,), "ones"))
            else:
                raise ValueError(f"unknown layer type {kind}")
            out += [(f"{p}.norm1.weight", (d,), "ones"), (f"{p}.norm2.weight", (d,), "ones"),
                    (f"{p}.mlp.up.weight", (2 * hidden, d), "mat"),
                    (f"{p}.mlp.down.weight", (d, hidden), "mat")]
    if cfg["core"]:
        out += [("inject_e.weight", (d, d), "mat"),
                ("loop_embed.weight", (cfg["max_loops"], d), "mat")]
    out += [("embed.weight", (cfg["vocab_size"], d), "mat"), ("norm_f.weight", (d,), "ones")]
    return out


def make_weights(cfg: dict, seed: int) -> dict:
    rng = np.random.default_rng(seed)
    w = {}
    for name, shape, kind in tensor_specs(cfg):
        if kind == "mat":
            w[name] = (rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02))
        elif kind == "ones":
            w[name] = np.ones(shape, dtype=np.float32)
        else:
            H = shape[0]
            h = np.arange(H, dtype=np.float64)
            u = 0.1 * 0.01 ** (h / max(H - 1, 1))
            w[name] = np.log(u / (1 - u)).astype(np.float32)
    return w


def write_model(folder, cfg: dict | str, seed: int) -> Path:
    """Writes config.json and model.safetensors into `folder` (created if needed)."""
    from safetensors.numpy import save_file

    if isinstance(cfg, str):
        cfg = CONFIGS[cfg]
    folder = Path(folder)
    folder.mkdir(parents=True, exist_ok=True)
    stamp = folder / ".synth"
    key = json.dumps([cfg, seed], sort_keys=True)
    if stamp.exists() and stamp.read_text() == key and (folder / "model.safetensors").exists():
        return folder
    (folder / "config.json").write_text(json.dumps(cfg, indent=1))
    save_file(make_weights(cfg, seed), str(folder / "model.safetensors"))
    stamp.write_text(key)
    return folder


def tokens(n: int, vocab: int, seed: int) -> np.ndarray:
    """n uniform token ids in [0, vocab)."""
    return np.random.default_rng(seed).integers(0, vocab, size=n, dtype=np.int64).astype(np.uint32)
