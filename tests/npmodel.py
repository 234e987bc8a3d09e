"""An independent float64 statement of the Looped Hybrid Reasoner, written from the
mathematics (src/model.rs:1-15 and the op definitions of src/ops.rs) rather than from the
oracle's code: no rings, no caches, no chunking — every layer keeps the full history of
keys and values as plain lists and attention picks positions by number. It pins what the
reference's fixture cannot reach: ring wrap past `cap = window + 256`, and global caches
that have grown.
"""

import numpy as np


def rms(x, w, eps):
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * w


def silu(g):
    return g / (1.0 + np.exp(-g))


class NpModel:
    def __init__(self, cfg, weights):
        self.cfg = cfg
        self.w = {k: v.astype(np.float64) for k, v in weights.items()}
        dh = cfg.head_dim()
        j = np.arange(dh // 2, dtype=np.float64)
        self.inv = 1.0 / cfg.rope_base ** (2 * j / dh)

    def session(self, loops):
        c = self.cfg
        hist = lambda kinds: [dict(k=[], v=[], s=np.zeros((c.n_heads, c.head_dim(), c.head_dim())),
                                   prev=np.zeros(c.d_model)) for _ in kinds]
        return dict(pos=0, loops=loops, prelude=hist(c.prelude),
                    core=[hist(c.core) for _ in range(loops)], coda=hist(c.coda), logits=None)

    def _rope(self, x, p):
        """x: [heads, dh] at position p; half-split rotation."""
        a = p * self.inv
        c, s = np.cos(a), np.sin(a)
        h = x.shape[-1] // 2
        lo, hi = x[..., :h], x[..., h:]
        return np.concatenate([lo * c - hi * s, lo * s + hi * c], axis=-1)

    def _attend(self, q, keys, vals, lo, hi, group):
        """q: [heads, dh]; keys/vals: lists indexed by position of [key_heads, dh]."""
        heads, dh = q.shape
        out = np.zeros((heads, dh))
        if hi <= lo:
            return out
        K = np.stack(keys[lo:hi])  # [n, kh, dh]
        V = np.stack(vals[lo:hi])
        for h in range(heads):
            s = K[:, h // group] @ q[h] / np.sqrt(dh)
            p = np.exp(s - s.max())
            out[h] = (p / p.sum()) @ V[:, h // group]
        return out

    def _block(self, prefix, kind, st, x, e0, pos):
        c, W = self.cfg, self.w
        d, H, dh = c.d_model, c.n_heads, c.head_dim()
        n = rms(x, W[prefix + ".norm1.weight"], c.norm_eps)
        m = x.shape[0]
        h = None
        if kind == "S":
            qkv = n @ W[prefix + ".mixer.qkv.weight"].T
            for i in range(m):
                p = pos + i
                st["k"].append(self._rope(qkv[i, d:2 * d].reshape(H, dh), p))
                st["v"].append(qkv[i, 2 * d:].reshape(H, dh))
            y = np.zeros((m, d))
            for i in range(m):
                p = pos + i
                q = self._rope(qkv[i, :d].reshape(H, dh), p)
                y[i] = self._attend(q, st["k"], st["v"], max(0, p - c.window + 1), p + 1, 1).reshape(-1)
            h = y @ W[prefix + ".mixer.o.weight"].T
        elif kind == "L":
            mix = n @ W[prefix + ".mixer.qkvg.weight"].T
            dec = n @ W[prefix + ".mixer.decay.weight"].T + W[prefix + ".mixer.decay.bias"]
            y = np.zeros((m, H, dh))
            for i in range(m):
                q = mix[i, :d].reshape(H, dh)
                k = mix[i, d:2 * d].reshape(H, dh)
                v = mix[i, 2 * d:3 * d].reshape(H, dh)
                q = q / np.maximum(np.linalg.norm(q, axis=-1, keepdims=True), 1e-12)
                k = k / np.maximum(np.linalg.norm(k, axis=-1, keepdims=True), 1e-12)
                g = 1.0 / (1.0 + np.exp(dec[i]))  # sigmoid(-(decay + bias)) per head
                st["s"] = g[:, None, None] * st["s"] + k[:, :, None] * v[:, None, :]
                y[i] = np.einsum("ha,hab->hb", q, st["s"])
            y = rms(y, W[prefix + ".mixer.head_norm.weight"], c.norm_eps).reshape(m, d)
            y = silu(mix[:, 3 * d:]) * y
            h = y @ W[prefix + ".mixer.o.weight"].T
        else:
            kh, kd = c.global_kv_heads, c.global_kv_heads * dh
            if c.global_emb:
                n = n + rms(e0, W[prefix + ".mixer.norm_e.weight"], c.norm_eps)
            q = n @ W[prefix + ".mixer.q.weight"].T
            kv = n @ W[prefix + ".mixer.kv.weight"].T
            if c.global_logn:
                f = np.log1p(np.arange(pos, pos + m, dtype=np.float64)) / np.log(c.global_logn)
                q = q * f[:, None]
            if c.global_kshift:
                shifted = np.concatenate([st["prev"][None], n[:-1]], axis=0)
                keys = (shifted @ W[prefix + ".mixer.kv.weight"].T)[:, :kd]
                st["prev"] = n[-1].copy()
            else:
                keys = kv[:, :kd]
            for i in range(m):
                st["k"].append(keys[i].reshape(kh, dh))
                st["v"].append(kv[i, kd:].reshape(kh, dh))
            far = c.window if c.global_far else 0
            if pos + m > far:
                y = np.zeros((m, d))
                for i in range(m):
                    p = pos + i
                    y[i] = self._attend(q[i].reshape(H, dh), st["k"], st["v"], 0, p + 1 - far,
                                        H // kh).reshape(-1) if p + 1 > far else 0.0
                h = y @ W[prefix + ".mixer.o.weight"].T
        if h is not None:
            x = x + h
        n = rms(x, W[prefix + ".norm2.weight"], c.norm_eps)
        up = n @ W[prefix + ".mlp.up.weight"].T
        hidden = up.shape[1] // 2
        y = silu(up[:, :hidden]) * up[:, hidden:]
        return x + y @ W[prefix + ".mlp.down.weight"].T

    def advance(self, se, tokens):
        c, W = self.cfg, self.w
        pos = se["pos"]
        e0 = W["embed.weight"][np.asarray(tokens)]
        x = e0.copy()
        for i, k in enumerate(c.prelude):
            x = self._block(f"prelude.{i}", k, se["prelude"][i], x, e0, pos)
        if c.core:
            e_proj = x @ W["inject_e.weight"].T
            s = x
            for r in range(se["loops"]):
                x = s + e_proj + W["loop_embed.weight"][r]
                for i, k in enumerate(c.core):
                    x = self._block(f"core.{i}", k, se["core"][r][i], x, e0, pos)
                s = x if c.damp == 1.0 else s + c.damp * (x - s)
            x = s
        for i, k in enumerate(c.coda):
            x = self._block(f"coda.{i}", k, se["coda"][i], x, e0, pos)
        last = rms(x[-1], W["norm_f.weight"], c.norm_eps)
        se["logits"] = last @ W["embed.weight"].T
        se["pos"] += len(tokens)
