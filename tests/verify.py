"""The reference's verify harness, src/verify.rs:40-119, for any model with the
session/feed/step/logits API (the oracle and the HIP model twin both have it)."""

from dataclasses import dataclass

import numpy as np
from safetensors.numpy import load_file


@dataclass
class Report:
    steps: int
    checked: int
    max_diff: float
    max_rel: float
    same_argmax: bool


@dataclass
class Expected:
    tokens: list
    loops: int
    positions: list
    logits: np.ndarray


def expected(folder, vocab) -> Expected:
    """verify.rs:46-63: `tokens`, `loops`, `positions` and `logits` (positions x vocab)."""
    st = load_file(str(folder / "expected.safetensors"))
    e = Expected(tokens=[int(t) for t in st["tokens"]], loops=int(st["loops"][0]),
                 positions=[int(p) for p in st["positions"]],
                 logits=st["logits"].reshape(-1).astype(np.float32))
    if e.logits.size != len(e.positions) * vocab:
        raise ValueError("expected logits do not match positions x vocab")
    e.logits = e.logits.reshape(len(e.positions), vocab)
    return e


def argmax(l) -> int:
    """verify.rs:40-44: the first maximum wins."""
    b = 0
    for i in range(len(l)):
        if l[i] > l[b]:
            b = i
    return b


def run_split(model, folder, split: int, chunk: int) -> Report:
    """verify.rs:79-119: read the prompt in chunks up to `split`, then step the rest."""
    v = model.cfg.vocab_size
    e = expected(folder, v)
    se = model.session(e.loops)
    r = Report(len(e.tokens), 0, 0.0, 0.0, True)

    def check(want):
        got = se.logits()
        r.max_diff = max(r.max_diff, float(np.abs(got - want).max()))
        r.max_rel = max(r.max_rel, float(np.abs(got - want).max() / np.abs(want).max()))
        r.same_argmax &= argmax(got) == argmax(want)
        r.checked += 1

    def want(p):
        return e.logits[e.positions.index(p)] if p in e.positions else None

    if split > 0:
        se.feed(e.tokens[:split], chunk)
        w = want(split - 1)
        if w is None:
            raise ValueError(f"no reference at position {split - 1}")
        check(w)
    for t in range(split, len(e.tokens)):
        se.step(e.tokens[t])
        w = want(t)
        if w is not None:
            check(w)
    return r


# tests/parity.rs:13 and :22-45
TOLERANCE = 1e-4
SPLITS = [(1, 1), (5, 2), (8, 8), (9, 3), (20, 7), (30, 16), (39, 256), (40, 5), (40, 40)]


def check_parity(model, folder):
    """tests/parity.rs:15-46 for any backend."""
    plain = run_split(model, folder, 0, 1)
    assert plain.checked == 40
    assert plain.max_diff < TOLERANCE, plain
    assert plain.same_argmax, plain
    reports = [plain]
    for split, chunk in SPLITS:
        r = run_split(model, folder, split, chunk)
        assert r.checked == 41 - split, (split, r)
        assert r.max_diff < TOLERANCE, (split, chunk, r)
        assert r.same_argmax, (split, chunk, r)
        reports.append(r)
    return reports
