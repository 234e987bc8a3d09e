"""Token-loop benchmark on one MI355X: the reference's `slm bench` sequence
(src/main.rs:285-315) on the 86M-class synthetic model, at R = 4, 8 and 16.

    python bench.py [--gpus 1] [--steps 256] [--warmup 16] [--no-cpu] [--no-g86] [--no-fp16]

Workload (one GPU): model "a86" (d 768, 12 x 64 heads, FFN 4x, vocab 32000, window 4096,
prelude SS / core LS / coda SS, seeded N(0, 0.02) fp32 weights). For each R in 4, 8, 16 (the
loop counts main.rs:134-135 bench over) a new session reads 16 warm-up tokens, then a
4096-token uniform-random prompt in 256-token chunks (timed: prefill tok/s, including the
final logits read, main.rs:200-205) — which fills the sliding window — then decodes greedily,
reading the logits back every token (main.rs:207-223): `--warmup` untimed tokens, then
`--steps` timed ones. With the defaults the positions run to 4384, past the 4352-slot ring
(window + 256), so the rings overwrite as in the reference bench. A "step" is one decoded
token; `value` is decode tok/s at R = 4, the headline configuration.

Also printed, in the same JSON line: `r4`, `r8`, `r16` (decode and prefill tok/s with their
HBM and MFMA roofline fractions), `g86` (the 16384-token prompt of the global-attention
model, config C4, then 128 decode steps), `roofline` (the dominant decode kernel, the fused
one-token GEMV slm_fg, against HBM: its launches over `--timed-steps` more decode steps, each
timed by the start and stop events of hipExtModuleLaunchKernel on the backend's stream, which
carry the dispatch's own begin and end timestamps), and `cpu_baseline` (the oracle, a C++
restatement of src/cpu.rs + src/model.rs, OpenMP over the host's cores, on a bounded sample
of the same workload).
"""

from __future__ import annotations

import argparse
import ctypes as C
import importlib.util
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
HBM_PEAK = 8.0e12            # bytes/s, MI355X
FP32_MFMA_PEAK = 157.3e12    # flop/s, MI355X dense fp32 matrix


def package():
    spec = importlib.util.spec_from_file_location(
        "slm_use_amd", ROOT / "slm.use_amd" / "__init__.py",
        submodule_search_locations=[str(ROOT / "slm.use_amd")])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["slm_use_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------------------
# algorithmic work of the token loop
# ---------------------------------------------------------------------------------------

def block_linears(cfg, kind, pos_plus_m_over_far=True):
    d, H = cfg["d_model"], cfg["n_heads"]
    dh = d // H
    hid = int(round(cfg.get("mlp_mult", 4.0) * d))
    kd = cfg["global_kv_heads"] * dh
    if kind == "S":
        mix = [(3 * d, d), (d, d)]
    elif kind == "L":
        mix = [(4 * d, d), (H, d), (d, d)]
    else:
        mix = [(d, d), (2 * kd, d)] + ([(2 * kd, d)] if cfg["global_kshift"] else [])
        mix += [(d, d)] if pos_plus_m_over_far else []
    return mix + [(2 * hid, d), (d, hid)]


def step_linears(cfg, loops):
    """(rows, cols) of every linear of one m = 1 advance, in call order (model.rs:563-624)."""
    out = []
    for k in cfg["prelude"]:
        out += block_linears(cfg, k)
    if cfg["core"]:
        out.append((cfg["d_model"], cfg["d_model"]))
        for _ in range(loops):
            for k in cfg["core"]:
                out += block_linears(cfg, k)
    for k in cfg["coda"]:
        out += block_linears(cfg, k)
    out.append((cfg["vocab_size"], cfg["d_model"]))
    return out


def instances(cfg, loops):
    kinds = cfg["prelude"] + cfg["core"] * loops + cfg["coda"]
    return {k: kinds.count(k) for k in "SLG"}


def decode_bytes(cfg, loops, pos):
    """Algorithmic HBM bytes of one decoded token at position `pos`: every weight read as
    executed, the K/V window read and the new K/V written, GLA state read + written."""
    d, H, W = cfg["d_model"], cfg["n_heads"], cfg["window"]
    dh = d // H
    n = instances(cfg, loops)
    w = sum(r * c for r, c in step_linears(cfg, loops))
    keys = min(pos + 1, W)
    far = W if cfg.get("global_far") else 0
    gkeys = max(pos + 1 - far, 0)
    kd = cfg["global_kv_heads"] * dh
    return 4 * (w + n["S"] * (2 * keys * d + 2 * d) + n["L"] * 2 * H * dh * dh
                + n["G"] * (2 * gkeys * kd + 2 * kd))


def prefill_flops(cfg, loops, start, count):
    """Algorithmic flops of reading `count` prompt tokens from position `start`."""
    d, H, W = cfg["d_model"], cfg["n_heads"], cfg["window"]
    dh = d // H
    n = instances(cfg, loops)
    lin = 2 * sum(r * c for r, c in step_linears(cfg, loops)[:-1])  # no logits per token
    p = np.arange(start, start + count)
    keys = np.minimum(p + 1, W).sum()
    far = W if cfg.get("global_far") else 0
    gkeys = np.maximum(p + 1 - far, 0).sum()
    return (lin * count + n["S"] * 4 * d * keys + n["G"] * 4 * d * gkeys
            + n["L"] * 4 * H * dh * dh * count)


# ---------------------------------------------------------------------------------------
# the CPU baseline: the oracle on the host cores
# ---------------------------------------------------------------------------------------

def cpu_baseline(folder, cfg, loops, prompt, decode_tokens):
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as O

    cores = os.cpu_count() or 1
    omp = int(os.environ.get("OMP_NUM_THREADS", cores))
    m = O.Model(folder)
    se = m.session(loops)
    se.feed(prompt[:16], 256)
    t = time.perf_counter()
    se.feed(prompt, 256)
    se.logits()
    fill_s = time.perf_counter() - t
    ids = []
    t = time.perf_counter()
    for _ in range(decode_tokens):
        ids.append(O.pick(se.logits()))
        se.step(ids[-1])
    dec_s = time.perf_counter() - t
    return dict(value=round(decode_tokens / dec_s, 2), unit="tok/s", cores=omp, kind="port",
                sample=(f"oracle (C++ restatement of src/cpu.rs + src/model.rs, OpenMP) on the "
                        f"same model and prompt: 16 + {len(prompt)} prompt tokens in 256-chunks, "
                        f"then {decode_tokens} greedy decode steps timed (of the GPU run's "
                        f"steps); {omp} threads of {cores} visible cores"),
                prefill_tok_s=round(len(prompt) / fill_s, 1), ids=ids)


# ---------------------------------------------------------------------------------------

def traffic():
    """HBM bytes per slm_fg launch in the a86 decode step, as the committed counter profile
    measured them (FETCH_SIZE and WRITE_SIZE passes, each scaled by what the same counter reads
    for a copy of known size); None when the profile is absent."""
    f = ROOT / "profiles" / "slm_fg_a86_decode_traffic.md"
    if not f.exists():
        return None
    for ln in f.read_text().splitlines():
        if ln.startswith("traffic_bytes_per_launch:"):
            return int(ln.split(":")[1])
    return None


def cpu_model() -> str:
    try:
        for ln in Path("/proc/cpuinfo").read_text().splitlines():
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def window_note(cfg, h):
    """What the timed positions do to the sliding-window rings (cap = window + 256 slots)."""
    cap = cfg["window"] + 256
    first, last = h["decode_from_pos"], h["decode_to_pos"]
    full = "window full" if first >= cfg["window"] else f"window filling ({first} of {cfg['window']})"
    if last < cap:
        return f"{full}; positions {first}..{last}, below the {cap}-slot ring's wrap"
    if first >= cap:
        return f"{full}; positions {first}..{last}, the rings overwriting"
    return f"{full}; positions {first}..{last}, the rings wrapping at {cap}"


def under_profiler() -> bool:
    """Is this process running under rocprofv3 (its tool library preloaded)?"""
    return ("rocprofiler" in os.environ.get("LD_PRELOAD", "")
            or any(k.startswith("ROCPROF") for k in os.environ))


def run_loops(model, cfg, prompt, loops, warmup, steps):
    """The reference bench sequence at one loop count: 16 warm-up tokens, the timed prompt,
    untimed then timed greedy decode. Returns (prefill tok/s, decode tok/s, first timed
    position, ids of the warm-up and timed steps, the session)."""
    se = model.session(loops)
    se.feed(prompt[:16], 256)  # main.rs:309
    se.logits()
    t = time.perf_counter()
    se.feed(prompt, 256)
    se.logits()
    fill_s = time.perf_counter() - t
    ids = se.decode_greedy(warmup).tolist() if warmup else []
    se.logits()
    pos0 = se.pos
    t = time.perf_counter()
    ids += se.decode_greedy(steps).tolist()
    se.logits()  # waits for the last step
    dec_s = time.perf_counter() - t
    return len(prompt) / fill_s, steps / dec_s, pos0, ids, se


def g86_leg(pkg, hip, synth, device_grow=False):
    """Config C4: the g86 model (global layers with logn, kshift, emb, far, 4 key heads), a
    16384-token prompt at R = 4 in 256-token chunks (the global caches grow 8192 -> 16384 ->
    32768), then 128 greedy decode steps. The caches grow by model.rs:383-398's own sequence
    (read, host relayout, upload inside the advance) or, with `device_grow`, by device
    copies (the optional grow_cache trait method)."""
    cache = Path(os.environ.get("SLM_MODEL_CACHE", "/tmp")) / "slm_models"
    folder = synth.write_model(cache / "g86-4", "g86", 4)
    cfg = synth.G86
    prompt = synth.tokens(16384, cfg["vocab_size"], seed=6)
    model = pkg.Model(hip, folder, device_grow=device_grow)
    se = model.session(4)
    t = time.perf_counter()
    se.feed(prompt, 256)
    se.logits()
    fill_s = time.perf_counter() - t
    pos0 = se.pos
    g0 = hip.graph_stats()
    # the first step (position 16384) doubles the global caches to 32768 slots: model.rs's
    # grow moves them through the host there; it is timed on its own as well
    t = time.perf_counter()
    se.decode_greedy(1)
    se.logits()
    first_s = time.perf_counter() - t
    t1 = time.perf_counter()
    se.decode_greedy(127)
    se.logits()
    rest_s = time.perf_counter() - t1
    dec_s = time.perf_counter() - t
    g1 = hip.graph_stats()
    fl = prefill_flops(cfg, 4, 0, len(prompt))
    bpt = np.mean([decode_bytes(cfg, 4, p) for p in range(pos0, pos0 + 128)])
    out = {"prompt_tokens": len(prompt), "prefill_tok_s": round(len(prompt) / fill_s, 1),
           "prefill_tflops": round(fl / fill_s / 1e12, 2),
           "prefill_frac": round(fl / fill_s / FP32_MFMA_PEAK, 4),
           "decode_tok_s": round(128 / dec_s, 1), "decode_from_pos": pos0,
           "first_step_ms": round(first_s * 1e3, 2),
           "decode_tok_s_after_first": round(127 / rest_s, 1),
           "first_step": "grows the global caches 16384 -> 32768 slots",
           "decode_bytes_per_token": round(bpt),
           "decode_frac": round(bpt * 128 / dec_s / HBM_PEAK, 4),
           "layers": "SG|LS|SG", "loops": 4,
           "decode_graphs": {k: g1[k] - g0[k] for k in g1},
           "grow": ("device copies (grow_cache, an optional trait method)" if device_grow else
                    "model.rs:383-398 as written: read + host relayout + upload inside the advance")}
    del se, model
    return out


def fp16_leg(pkg, hip, folder, a, prompt, fl):
    """The same workload in fp16 mode (the --fp16 analogue, slm_hip_set_fp16, set before the
    model loads as mlx.rs fixes its dtype): every buffer holds fp16 values — uploads round,
    every operation rounds what it writes at mlx.rs's rounding points; the linears read fp16
    copies of the weights (half the bytes) at fp16 MFMAs with fp32 sums; the rings hold halves."""
    hip.set_fp16(True)
    model = pkg.Model(hip, folder)
    s16 = model.session(a.loops)
    s16.feed(prompt[:16], 256)
    s16.logits()
    t = time.perf_counter()
    s16.feed(prompt, 256)
    s16.logits()
    fill16_s = time.perf_counter() - t
    if a.warmup:
        s16.decode_greedy(a.warmup)
    s16.logits()
    t = time.perf_counter()
    s16.decode_greedy(a.steps)
    s16.logits()
    dec16_s = time.perf_counter() - t
    # per-kernel time of a few more steps, launched eagerly with every launch timed
    hip.set_graphs(False)
    hip.set_timing(True)
    s16.decode_greedy(a.timed_steps)
    s16.logits()
    names = ("slm_fghw", "slm_attn_dec16_4", "slm_gla1_4")
    kern = {n: hip.kernel_stat(n) for n in names}
    hip.set_timing(False)
    hip.set_graphs(not a.no_graphs)
    del s16, model
    hip.set_fp16(False)
    fp16 = {"decode_tok_s": round(a.steps / dec16_s, 2), "prefill_tok_s": round(len(prompt) / fill16_s, 1),
            "us_per_step_by_kernel": {n: round(v["us"] / max(a.timed_steps, 1), 1) for n, v in kern.items()},
            "us_per_launch_by_kernel": {n: round(v["us"] / max(v["launches"], 1), 2) for n, v in kern.items()},
            "rings": "fp16 (slm_hip_alloc_cache in fp16 mode): K/V bytes halved",
            "prefill_tflops": round(fl / fill16_s / 1e12, 2),
            "path": "the trait's calls unchanged: slm_hip_set_fp16(1), then the model's fp32 uploads",
            "note": "every buffer holds fp16 values (uploads and every op's output rounded, "
                    "mlx.rs:19-23, 53-67); linears read fp16 copies of the weights the backend "
                    "makes on first use, operands at v_mfma_f32_16x16x16f16 (fp32 sums); "
                    "checked at 2e-2 vs the fp32 oracle (config C5), chunked == token by token "
                    "bitwise"}
    log(f"fp16 mode: prefill {fp16['prefill_tok_s']} tok/s, decode {fp16['decode_tok_s']} tok/s")
    return fp16


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--loops", type=int, nargs="+", default=[4, 8, 16],
                    help="loop counts to bench (the first is the headline)")
    ap.add_argument("--prompt", type=int, default=4096)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-steps", type=int, default=32)
    ap.add_argument("--no-graphs", action="store_true")
    ap.add_argument("--tile-rows", type=int, default=0,
                    help="fused GEMV rows per tile (0: the planner's choice; 16, 8 or 4)")
    ap.add_argument("--prompt-lanes", type=int, default=0,
                    help="streams consecutive prompt chunks run on (0: the backend's default)")
    ap.add_argument("--no-fp16", action="store_true", help="skip the fp16-mode leg")
    ap.add_argument("--no-g86", action="store_true", help="skip the g86 16K-prompt leg (config C4)")
    ap.add_argument("--timed-steps", type=int, default=16,
                    help="decode steps whose kernels are timed one by one for the roofline")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="only copy this many MiB four times through slm_hip_copy and exit (a "
                         "known-size workload that calibrates the FETCH_SIZE/WRITE_SIZE counters)")
    a = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print(f"bench.py runs on one GPU: --gpus {a.gpus} (WORLD_SIZE {world}) is not "
              "supported; the token loop has no multi-GPU path here", file=sys.stderr)
        sys.exit(2)

    pkg = package()
    sys.path.insert(0, str(ROOT / "slm.use_amd"))
    import synth

    if a.copy_mib:
        hip = pkg.Hip(0)
        n = a.copy_mib << 18  # floats
        src, dst = hip.alloc(n), hip.alloc(n)
        for _ in range(4):
            hip.copy(dst.ptr, src.ptr, n)
        dst.read(4)
        log(f"copied {a.copy_mib} MiB four times")
        hip.close()
        return

    cache = Path(os.environ.get("SLM_MODEL_CACHE", "/tmp")) / "slm_models"
    folder = synth.write_model(cache / "a86-2", "a86", 2)
    cfg = synth.A86
    prompt = synth.tokens(a.prompt, cfg["vocab_size"], seed=3)

    if under_profiler() and not a.no_graphs:
        # rocprofv3's kernel tracing of step-graph launches has crashed inside the profiler's
        # own library here (twice); profiled runs launch the same kernels eagerly
        log("under rocprofv3: step graphs off (--no-graphs)")
        a.no_graphs = True
    hip = pkg.Hip(0)
    if a.no_graphs:
        hip.set_graphs(False)
    if a.tile_rows:
        hip.set_tile_rows(a.tile_rows)
    if a.prompt_lanes:
        hip.set_prompt_lanes(a.prompt_lanes)
    log("device:", hip.name(), "prompt lanes:", hip.prompt_lanes())
    model = pkg.Model(hip, folder)
    per_r = {}
    head = a.loops[0]
    for r in a.loops:
        prefill, tok_s, pos0, ids, se = run_loops(model, cfg, prompt, r, a.warmup, a.steps)
        bpt = np.mean([decode_bytes(cfg, r, p) for p in range(pos0, pos0 + a.steps)])
        fl = prefill_flops(cfg, r, 16, len(prompt))
        per_r[r] = {"decode_tok_s": round(tok_s, 2), "ms_per_token": round(1e3 / tok_s, 4),
                    "decode_from_pos": pos0, "decode_to_pos": pos0 + a.steps - 1,
                    "decode_bytes_per_token": round(bpt),
                    "decode_hbm_frac": round(bpt * tok_s / HBM_PEAK, 4),
                    "prefill_tok_s": round(prefill, 1), "prefill_flops_per_token": round(fl / len(prompt)),
                    "prefill_tflops": round(fl * prefill / len(prompt) / 1e12, 2),
                    "prefill_mfma_frac": round(fl * prefill / len(prompt) / FP32_MFMA_PEAK, 4),
                    "state_bytes": se.state_bytes()}
        log(f"R={r}: prefill {prefill:.1f} tok/s, decode {tok_s:.1f} tok/s "
            f"(pos {pos0}..{pos0 + a.steps - 1})")
        if r == head:
            head_ids, head_se = ids, se
        else:
            del se
    se = head_se
    tok_s = per_r[head]["decode_tok_s"]
    # the same greedy loop with the pick on the device (the logits stay on the GPU; each step's
    # embedding gather reads the previous step's pick there): the opt-in fast path, after
    # untimed steps of its own (its step graph's capture and first-call set-up)
    if a.warmup:
        se.decode_greedy_device(a.warmup)
    se.logits()
    t = time.perf_counter()
    se.decode_greedy_device(a.steps)
    se.logits()
    dev_s = time.perf_counter() - t
    dev_pick = {"value": round(a.steps / dev_s, 1), "unit": "tok/s", "steps": a.steps,
                "from_pos": se.pos - a.steps,
                "note": "greedy decode with slm_hip_argmax on the device instead of the per-token "
                        "logits read-back and host pick; the same ids (tests/test_gpu_model.py)"}
    log(f"decode, device pick: {dev_pick['value']} tok/s")
    stats = hip.graph_stats()
    # dominant kernel: the fused decode GEMV (slm_fg), every launch of `--timed-steps` more
    # decode steps timed by the dispatch's own timestamps (eager launches: the same kernels
    # the step graph holds)
    hip.set_graphs(False)
    hip.set_timing(True)
    se.decode_greedy(a.timed_steps)
    se.logits()
    kern = {n: hip.kernel_stat(n) for n in ("slm_fg", "slm_attn_dec_4", "slm_gla1_4")}
    attn_launch_us = kern["slm_attn_dec_4"]["us"] / max(kern["slm_attn_dec_4"]["launches"], 1)
    hip.set_timing(False)
    hip.set_graphs(not a.no_graphs)
    fg = kern["slm_fg"]
    per_launch = fg["us"] / 1e6 / max(fg["launches"], 1)
    bpl = fg["bytes"] / max(fg["launches"], 1)
    gemv_bw = bpl / per_launch if per_launch else 0.0
    log(f"slm_fg: {fg['launches']} launches, {per_launch * 1e6:.2f} us/launch, "
        f"{bpl / 1e6:.2f} MB/launch, {gemv_bw / 1e9:.0f} GB/s")
    share = {n: round(v["us"] / max(a.timed_steps, 1), 1) for n, v in kern.items()}

    # the same workload in fp16 mode (the --fp16 analogue: every buffer's values in fp16)
    fp16 = None
    if not a.no_fp16:
        fp16 = fp16_leg(pkg, hip, folder, argparse.Namespace(loops=head, warmup=a.warmup, steps=a.steps,
                                                            timed_steps=a.timed_steps, no_graphs=a.no_graphs),
                        prompt, prefill_flops(cfg, head, 16, len(prompt)))
    del se, head_se
    g86 = None
    if not a.no_g86:
        log("g86: 16384-token prompt at R=4, then 128 decode steps ...")
        g86 = g86_leg(pkg, hip, synth)
        log(f"g86: prefill {g86['prefill_tok_s']} tok/s, decode {g86['decode_tok_s']} tok/s")
        dg = g86_leg(pkg, hip, synth, device_grow=True)
        g86["with_device_grow"] = {k: dg[k] for k in ("prefill_tok_s", "prefill_frac", "decode_tok_s",
                                                      "decode_frac", "first_step_ms",
                                                      "decode_tok_s_after_first", "grow")}
        log(f"g86 (device grow): prefill {dg['prefill_tok_s']} tok/s, decode {dg['decode_tok_s']} tok/s")

    cpu = None
    if not a.no_cpu:
        n = min(a.cpu_steps, a.steps)
        log(f"CPU baseline: oracle prefill {len(prompt)} + decode {n} at R={head} ...")
        cpu = cpu_baseline(folder, cfg, head, prompt, n)
        same = cpu.pop("ids") == head_ids[:n]
        cpu["same_greedy_ids_as_gpu"] = bool(same)
        cpu["cpu_model"] = cpu_model()
        log(f"CPU: prefill {cpu['prefill_tok_s']} tok/s, decode {cpu['value']} tok/s, "
            f"same ids: {same}")

    h = per_r[head]
    line = {
        "metric": "decode tok/s @R=4/8/16 full 4096 window; prefill tok/s; % HBM/MFMA peak",
        "value": h["decode_tok_s"],
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": h["ms_per_token"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded N(0,0.02) fp32 weights, uniform random token ids",
        "config": {"workload": f"a86 decode at R={head} after 16 + {len(prompt)} prompt tokens "
                               f"({window_note(cfg, h)}), greedy, logits read back every token",
                   "loops": head, "d_model": 768, "heads": 12, "head_dim": 64,
                   "ffn": 3072, "vocab": 32000, "window": 4096, "layers": "SS|LS|SS",
                   "prompt_tokens": len(prompt), "decode_from_pos": h["decode_from_pos"]},
        "roofline": {"bound": "hbm", "achieved": round(gemv_bw / 1e9, 1), "peak": 8000.0,
                     "unit": "GB/s", "frac": round(gemv_bw / HBM_PEAK, 4), "traffic": traffic(),
                     "kernel": "slm_fg", "launches": fg["launches"],
                     "bytes_per_launch": round(bpl), "us_per_launch": round(per_launch * 1e6, 3),
                     "timing": "kernel begin/end timestamps (hipExtModuleLaunchKernel events), eager launches",
                     "us_per_step_by_kernel": share,
                     "attn_dec_us_per_launch": round(attn_launch_us, 2)},
        "decode_roofline": {"bound": "hbm", "bytes_per_token": h["decode_bytes_per_token"],
                            "achieved": round(h["decode_bytes_per_token"] * h["decode_tok_s"] / 1e9, 1),
                            "peak": 8000.0, "unit": "GB/s", "frac": h["decode_hbm_frac"]},
        "prefill": {"value": h["prefill_tok_s"], "unit": "tok/s", "prompt_tokens": len(prompt),
                    "flops_per_token": h["prefill_flops_per_token"],
                    "achieved_tflops": h["prefill_tflops"], "peak_tflops": FP32_MFMA_PEAK / 1e12,
                    "frac": h["prefill_mfma_frac"], "prompt_lanes": hip.prompt_lanes(),
                    "lanes_note": "consecutive 256-token chunks on that many streams at once, "
                                  "each lane writing its own copies of the step's scratch; "
                                  "model.rs's calls unchanged (the flush keep lists)"},
    }
    for r in a.loops:
        line[f"r{r}"] = per_r[r]
    line.update({
        "g86": g86,
        "decode_device_pick": dev_pick,
        "graphs": stats,
        "fp16_mode": fp16,
        "cpu_baseline": cpu,
        "reference_published": {"decode_tok_s_rtx5080": {"r4": 209, "r8": 123, "r16": 67},
                                "prefill_tok_s_rtx5080": {"r4": 2819, "r8": 1630, "r16": 884},
                                "note": "README.md:143-149; different GPU and model dims"},
    })
    print(json.dumps(line), flush=True)
    del model
    hip.close()


if __name__ == "__main__":
    main()
