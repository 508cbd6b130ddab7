"""Decode benchmark of the HIP token loop (BASELINE.json metric, config 2).

One "step" = one Sampler.Generate pass over one batch: Forge-98M shape
(12 layers, d 768, 12 heads, ctx 1024, V 16384), fp32, batch 1, a 64-token
PCG32(42) prompt, 256 greedy tokens with the KV cache, random-init weights
(new Random(1234), GptModel init).  Inputs are resident on the device before
the timed region; only the 256 ids come back per step.

value = generated tokens / wall time of the K timed steps (prefill included).
roofline: the decode kernel's algorithmic HBM bytes per launch (per token:
every weight once + the KV rows read and written + two embedding rows; one
fused launch runs all 255 cached greedy steps) over its duration, timed with
HIP events on the session stream inside the library.
cpu_baseline: the oracle's restatement of the reference CPU algorithm
(full-window recompute per token, Sampler.Generate semantics) on this host,
on the first tokens of the same workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "forge-lm_amd"))

HBM_PEAK_GBS = 8000.0

C2 = dict(vocab_size=16384, context_length=1024, d_model=768, n_layers=12, n_heads=12)
PROMPT_LEN, NEW_TOKENS = 64, 256


def decode_bytes_per_step(c, attended: float, batch: int = 1, esize: int = 4) -> float:
    """Algorithmic bytes of one decode step (every weight once, tied head, KV read+write, embeddings)."""
    d, L, V = c["d_model"], c["n_layers"], c["vocab_size"]
    weights = esize * (L * (12 * d * d + 13 * d) + V * d + 2 * d)
    per_seq = esize * (L * 2 * d * attended + L * 2 * d + 2 * d)
    return weights + batch * per_seq


def cpu_baseline(weights_seed: int, prompt, gpu_ids, budget_tokens: int = 96):
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    threads = min(16, os.cpu_count() or 1)
    O.set_threads(threads)
    oc = O.Config(*[C2[k] for k in ("vocab_size", "context_length", "d_model", "n_layers", "n_heads")])
    w = O.init_weights(oc, weights_seed)
    t0 = time.perf_counter()
    ids = O.generate(oc, w, prompt, budget_tokens, kv_cached=False)
    dt = time.perf_counter() - t0
    return {
        "value": budget_tokens / dt, "unit": "tok/s", "cores": threads, "kind": "port",
        "sample": (f"reference CPU algorithm (C++ restatement, full-window recompute per token as "
                   f"Sampler.Generate does) on the C2 weights and prompt: first {budget_tokens} of "
                   f"{NEW_TOKENS} tokens, {dt:.1f} s, {threads} threads"),
        "ids_match_gpu": bool((ids == gpu_ids[:budget_tokens]).all()),
    }


def copy_calibration(mib: int, reps: int) -> dict:
    """Times the library's plain copy kernel (fh_buffer_copy) on `mib` MiB: the
    known-size kernel whose FETCH_SIZE / WRITE_SIZE counters scale the decode
    kernel's counters to bytes."""
    import forge_hip as fhp
    nbytes = mib << 20
    be = fhp.HipBackend(0)
    src, dst = fhp.DeviceBuffer(be, nbytes), fhp.DeviceBuffer(be, nbytes)
    dst.copy_from(src)  # warm-up
    ms = [dst.copy_from(src) for _ in range(reps)]
    src.free()
    dst.free()
    be.dispose()
    best = min(ms)
    return {"copy_bytes": nbytes, "reps": reps, "ms_min": round(best, 4), "ms_mean": round(sum(ms) / len(ms), 4),
            "read_plus_write_GBs": round(2 * nbytes / best / 1e6, 1)}


def profiled_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed counter summary, or None."""
    path = os.path.join(ROOT, "profiles", "decode_step_c2_traffic.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:") and kernel in line:
                    return int(line.split(":", 1)[1].split()[0])
    except OSError:
        pass
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-tokens", type=int, default=96,
                    help="tokens of the workload the CPU baseline runs (about 15-25 s on 16 cores)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only time the plain copy kernel on MIB MiB and print its line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs one GPU only: the token loop of one batch-1 sequence is a single-GPU "
              f"workload and this build has no multi-GPU path (asked for --gpus {args.gpus}).", file=sys.stderr)
        sys.exit(2)

    if args.copy_calibration:
        print(json.dumps(copy_calibration(args.copy_calibration, max(1, args.steps))), flush=True)
        return

    import numpy as np
    import forge_hip as fhp

    cfg = fhp.ModelConfig(**C2)
    be = fhp.HipBackend(0)
    model = fhp.GptModel(cfg, be, seed=1234)
    prompt = fhp.TrainingRandom(42).ids(cfg.vocab_size, PROMPT_LEN)

    for _ in range(args.warmup):
        ids = fhp.Sampler.generate(model, prompt, NEW_TOKENS, 0.0, 0, None)
    decode_ms, prefill_ms = [], []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        ids = fhp.Sampler.generate(model, prompt, NEW_TOKENS, 0.0, 0, None)
        t = fhp.Sampler.last_timing
        decode_ms.append(t["decode_ms"])
        prefill_ms.append(t["prefill_ms"])
    wall = time.perf_counter() - t0
    assert len(ids) == NEW_TOKENS

    n_dec = NEW_TOKENS - 1  # step 0 comes from the prefill forward
    avg_step_s = float(np.mean(decode_ms)) / 1e3 / n_dec
    # decode step n attends positions 0..P+n-1 (P+n keys)
    attended = np.mean([PROMPT_LEN + n for n in range(1, NEW_TOKENS)])
    step_bytes = decode_bytes_per_step(C2, attended)
    achieved = step_bytes / avg_step_s / 1e9
    value = args.steps * NEW_TOKENS / wall
    fused = os.environ.get("FORGE_HIP_FUSED_DECODE", "1") != "0"
    kernel = "k_decode_step<768>" if fused else "decode step graph (generic kernels)"
    # the fused greedy path runs every cached step in one launch; the generic
    # path launches one graph per step
    tokens_per_launch = n_dec if fused else 1
    out = {
        "metric": "decode tok/s, Forge-98M shape fp32 bs1 (prompt 64 + 256 greedy)",
        "value": round(value, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (random-init weights from new Random(1234); PCG32(42) prompt ids)",
        "config": {"workload": "C2: Forge-98M shape (L12 d768 H12 ctx1024 V16384) fp32, batch 1, "
                               "prompt 64 + 256 greedy, KV cache", "batch": 1, "prompt_len": PROMPT_LEN,
                   "new_tokens": NEW_TOKENS},
        "decode_tok_s": round(n_dec / (float(np.mean(decode_ms)) / 1e3), 2),
        "decode_us_per_token": round(avg_step_s * 1e6, 2),
        "prefill_tok_s": round(PROMPT_LEN / (float(np.mean(prefill_ms)) / 1e3), 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic(kernel) if fused else None,
                     "kernel": kernel, "tokens_per_launch": tokens_per_launch,
                     "bytes_per_launch": int(step_bytes * tokens_per_launch),
                     "launch_us": round(avg_step_s * tokens_per_launch * 1e6, 2)},
        "device": be.device_name,
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(1234, prompt, ids, args.cpu_tokens)
    model.dispose()
    be.dispose()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
