"""Decode benchmark of the HIP token loop (BASELINE.json metric).

Default workload (config 2, the headline): one "step" = one Sampler.Generate
pass over one batch: Forge-98M shape (12 layers, d 768, 12 heads, ctx 1024,
V 16384), fp32, batch 1, a 64-token PCG32(42) prompt, 256 greedy tokens with
the KV cache, random-init weights (new Random(1234), GptModel init).  Inputs
are resident on the device before the timed region; only the ids come back
per step.

value = generated tokens / wall time of the K timed steps (prefill included).
roofline: the decode kernel's algorithmic HBM bytes per launch (per token:
every weight once + the KV rows read and written + two embedding rows; one
fused launch runs all 255 cached greedy steps) over its duration, timed with
HIP events on the session stream inside the library.
cpu_baseline: the oracle's restatement of the reference CPU algorithm
(full-window recompute per token, Sampler.Generate semantics) on this host's
cores (up to the 16 CPUs a GPU job is given on this pool): the whole C2
workload; for the other configurations the first tokens of the same workload,
extrapolated to the whole run by the FLOPs of each step's window.

The default line also carries the rest of BASELINE's metric, measured in the
same run: "sampled_decode" (config 3), "bs32_decode" (config 4, batch 32) and
"prefill" (config 5, bf16 prefill), each with its own roofline and CPU baseline
(a capped sample, extrapolated), and "stream": the drop-in seam as the CLI drives
it (Sampler.generate_stream at the generate command's sampling defaults) against
one fh_generate call (--no-extra leaves these out).  roofline.achievable is this
box's copy and read bandwidth measured in the same run.  Each configuration also
runs alone:
  --workload c3  sampling path (T 0.7, top-k 30, penalty 1.1, no-repeat 4-gram),
                 prompt 32 + 512 tokens; roofline over one decode step
  --workload c4  batch 32, prompts 512 (PCG32 seeds 42 + b) + 512 greedy;
                 roofline over one batched decode step (weights + 32 KV windows)
  --workload c5  Forge-220M shape, bf16 weights/activations, fp32 accumulation,
                 batch 8 x 1024-token prompts + 128 greedy (every step
                 re-prefills the full window); value = prefill tok/s, roofline
                 = prefill FLOPs / prefill time against the bf16 MFMA peak

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extra] [--workload c2|c3|c4|c5]
                       [--new N] [--prompt P] [--copy-calibration MIB]
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "forge-lm_amd"))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0

C2 = dict(vocab_size=16384, context_length=1024, d_model=768, n_layers=12, n_heads=12)
C5 = dict(vocab_size=16384, context_length=1024, d_model=1024, n_layers=16, n_heads=16)
DIMS = ("vocab_size", "context_length", "d_model", "n_layers", "n_heads")
PROMPT_LEN, NEW_TOKENS = 64, 256

# name -> shape, dtype, batch, prompt length, new tokens, sampling (T, k, penalty, ngram, rng seed)
WORKLOADS = {
    "c2": dict(shape=C2, dtype="f32", batch=1, prompt=PROMPT_LEN, new=NEW_TOKENS, sampling=None,
               desc="C2: Forge-98M shape (L12 d768 H12 ctx1024 V16384) fp32, batch 1, prompt 64 + 256 greedy, "
                    "KV cache"),
    "c3": dict(shape=C2, dtype="f32", batch=1, prompt=32, new=512, sampling=(0.7, 30, 1.1, 4, 1),
               desc="C3: Forge-98M shape fp32, batch 1, prompt 32 + 512 sampled (T 0.7, top-k 30, repetition "
                    "penalty 1.1, no-repeat-ngram 4, Random(1) uniforms), KV cache"),
    "c4": dict(shape=C2, dtype="f32", batch=32, prompt=512, new=512, sampling=None,
               desc="C4: Forge-98M shape fp32, batch 32, prompts 512 + 512 greedy, KV cache (windows 513..1023)"),
    "c5": dict(shape=C5, dtype="bf16", batch=8, prompt=1024, new=128, sampling=None,
               desc="C5: Forge-220M shape (L16 d1024 H16 ctx1024 V16384) bf16 weights and activations, fp32 "
                    "accumulation, batch 8, prompts 1024 + 128 greedy (every step re-prefills the window)"),
}


def decode_bytes_per_step(c, attended: float, batch: int = 1, esize: int = 4) -> float:
    """Algorithmic bytes of one decode step (every weight once, tied head, KV read+write, embeddings)."""
    d, L, V = c["d_model"], c["n_layers"], c["vocab_size"]
    weights = esize * (L * (12 * d * d + 13 * d) + V * d + 2 * d)
    per_seq = esize * (L * 2 * d * attended + L * 2 * d + 2 * d)
    return weights + batch * per_seq


def prefill_flops(c, T: int, batch: int) -> float:
    """FLOPs of one bf16 prefill forward as the library runs it: layers 0..L-2 in
    full (the linear layers, causal QK^T and PV over every row), the last layer's
    qkv on every row (it fills the K/V caches) and the rest of it (attention of
    the last query over T keys, attn.proj, mlp.fc, mlp.proj) on the last row of
    each sequence, which is all that the head reads; then the last-row head.
    The full last layer would add 2 (T - 1) (9 d^2 + d T) per sequence."""
    d, L, V = c["d_model"], c["n_layers"], c["vocab_size"]
    full = 2.0 * T * (L - 1) * 12 * d * d + 2.0 * (L - 1) * d * T * (T + 1)
    last = 2.0 * T * 3 * d * d + 2.0 * 9 * d * d + 4.0 * d * T
    return batch * (full + last + 2.0 * V * d)


def prompts_for(name: str, w: dict, vocab: int):
    import numpy as np
    import forge_hip as fhp
    if w["batch"] == 1:
        return fhp.TrainingRandom(42).ids(vocab, w["prompt"])
    return np.stack([fhp.TrainingRandom(42 + b).ids(vocab, w["prompt"]) for b in range(w["batch"])])


def bf16_round(x):
    """fp32 -> nearest-even bf16 -> fp32 (what a bf16 session stores)."""
    import numpy as np
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def window_flops(c, T: int) -> float:
    """FLOPs of one reference decode step (Sampler.Generate recomputes the whole
    window of T rows, GptModel.cs:202-222): every linear layer and the tied head
    over T rows, plus QK^T and PV over the full T x T score matrix of every head."""
    d, L, V = c["d_model"], c["n_layers"], c["vocab_size"]
    return 2.0 * T * (L * 12 * d * d + V * d) + 4.0 * L * d * T * T


def host_cpu():
    """(logical CPUs, CPU model name) of this host."""
    model = platform.processor() or "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return os.cpu_count() or 1, model


def cpu_baseline(name: str, w: dict, prompts, gpu_ids, budget_tokens: int):
    """The oracle (reference CPU algorithm, full-window recompute) on a bounded sample
    of the workload, extrapolated to the whole workload by window FLOPs."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    nproc, model_name = host_cpu()
    # a GPU job on this pool is given 16 CPUs whatever the host shows (more threads
    # would only contend with other jobs' threads)
    threads = min(16, nproc)
    O.set_threads(threads)
    oc = O.Config(*[w["shape"][k] for k in DIMS])
    wt = O.init_weights(oc, 1234)
    if w["dtype"] == "bf16":
        wt = bf16_round(wt)
    prompt = prompts if prompts.ndim == 1 else prompts[0]
    gpu0 = gpu_ids if w["batch"] == 1 else gpu_ids[0]
    n = min(budget_tokens, w["new"])
    kw = {}
    if w["sampling"]:
        T, k, pen, ng, seed = w["sampling"]
        kw = dict(temperature=T, top_k=k, uniforms=O.net_random_doubles(seed, n), penalty=pen, ngram=ng)
    t0 = time.perf_counter()
    ids = O.generate(oc, wt, prompt, n, kv_cached=False, **kw)
    dt = time.perf_counter() - t0
    # step j of the workload recomputes a window of min(P + j, ctx) rows; the sample
    # ran steps 0..n-1, the workload runs w["new"] steps per sequence, batch of them
    ctx = w["shape"]["context_length"]
    cost = [window_flops(w["shape"], min(w["prompt"] + j, ctx)) for j in range(w["new"])]
    full_s = dt * sum(cost) / sum(cost[:n]) * w["batch"]
    whole = n == w["new"] and w["batch"] == 1
    what = "sequence 0 of %d, " % w["batch"] if w["batch"] > 1 else ""
    out = {
        "value": w["batch"] * w["new"] / full_s, "unit": "tok/s", "cores": threads, "kind": "port",
        "host_cpus": nproc, "cpu_model": model_name,
        "sample": (f"reference CPU algorithm (C++ restatement, full-window recompute per token as "
                   f"Sampler.Generate does) on the {name.upper()} weights and prompt: the whole workload "
                   f"({w['new']} tokens) ran in {dt:.1f} s on {threads} threads" if whole else
                   f"reference CPU algorithm (C++ restatement, full-window recompute per token as "
                   f"Sampler.Generate does) on the {name.upper()} weights and prompt: {what}steps 0..{n - 1} "
                   f"of {w['new']} ran in {dt:.1f} s on {threads} threads ({n / dt:.3g} tok/s); value = the "
                   f"whole workload ({w['batch']} x {w['new']} tokens) extrapolated by the FLOPs of each "
                   f"step's window: {full_s:.0f} s (cap: {n} steps of sequence 0)"),
        "sample_tok_s": n / dt,
        "ids_match_gpu": bool((np.asarray(ids) == np.asarray(gpu0)[:n]).all()),
    }
    if name == "c5":
        # every C5 token is a full 1024-token window forward: also quote it as window tokens/s
        out["window_tok_s"] = n * w["prompt"] / dt
    return out


def copy_calibration(mib: int, reps: int) -> dict:
    """Times the library's plain copy kernel (fh_buffer_copy) on `mib` MiB -- the
    known-size kernel whose FETCH_SIZE / WRITE_SIZE counters scale the decode
    kernel's counters to bytes -- and its read-only pass (fh_buffer_checksum, one
    read of every byte): what this box's HBM sustains for a plain copy and a plain
    read, next to the vendor peak."""
    import forge_hip as fhp
    nbytes = mib << 20
    be = fhp.HipBackend(0)
    src, dst = fhp.DeviceBuffer(be, nbytes), fhp.DeviceBuffer(be, nbytes)
    dst.copy_from(src)  # warm-up
    ms = [dst.copy_from(src) for _ in range(reps)]
    src.checksum()
    rms = [src.checksum()[1] for _ in range(reps)]
    src.free()
    dst.free()
    be.dispose()
    best, rbest = min(ms), min(rms)
    return {"copy_bytes": nbytes, "reps": reps, "ms_min": round(best, 4), "ms_mean": round(sum(ms) / len(ms), 4),
            "read_plus_write_GBs": round(2 * nbytes / best / 1e6, 1),
            "read_ms_min": round(rbest, 4), "read_GBs": round(nbytes / rbest / 1e6, 1)}


def achievable(reps: int = 5) -> dict:
    """The box's sustained HBM rates measured in this run (1 GiB, best of `reps`)."""
    c = copy_calibration(1024, reps)
    return {"copy_read_plus_write_GBs": c["read_plus_write_GBs"], "read_GBs": c["read_GBs"],
            "how": "fh_buffer_copy (grid-stride 16-byte copy) and fh_buffer_checksum (4 loads in flight per "
                   "thread) on 1 GiB, best of %d; frac_of_achievable = achieved / read_GBs" % reps}


TRAFFIC_PROFILE = os.path.join("profiles", "decode_step_c2_traffic.md")
TRAFFIC_PROFILE_2 = os.path.join("profiles", "decode_sampled_c3_traffic.md")
TRAFFIC_PROFILE_C4 = os.path.join("profiles", "decode_batched_c4_traffic.md")
TRAFFIC_PROFILE_C5 = os.path.join("profiles", "prefill_c5_traffic.md")


def profiled_traffic(kernel: str, path: str = TRAFFIC_PROFILE):
    """(HBM bytes per launch of `kernel`, HBM / algorithmic bytes of `kernel`, what
    build they were counted on) from a committed counter summary (rocprofv3 --pmc
    runs; the counters cannot be read inside this run); None where it has none."""
    value, ratio, build, where = None, None, None, None
    try:
        with open(os.path.join(ROOT, path)) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:") and kernel in line:
                    value = int(line.split(":", 1)[1].split()[0])
                elif line.startswith("traffic_ratio:") and kernel in line:
                    ratio = float(line.split(":", 1)[1].split()[0])
                elif line.startswith("measured_on:"):
                    build = line.split(":", 1)[1].strip()
                elif line.startswith("counted_at:"):
                    where = line.split(":", 1)[1].strip()
                elif line.startswith("extra_bytes_per_step:") and kernel in line:
                    value = int(line.split(":", 1)[1].split()[0])
    except OSError:
        pass
    return value, ratio, (f"{build}, {where}" if where else build)


def run_workload(name: str, args, steps: int, warmup: int, with_cpu: bool, new: int = 0, prompt: int = 0,
                 cpu_budget: int = 0) -> dict:
    import numpy as np
    import forge_hip as fhp

    w = dict(WORKLOADS[name])
    if new:
        w["new"] = new
        w["desc"] += f" (shortened to {new} new tokens)"
    if prompt:
        w["prompt"] = prompt
        w["desc"] += f" (prompt length {prompt}, a profiling run)"
    c = w["shape"]
    cfg = fhp.ModelConfig(**c)
    be = fhp.HipBackend(0)
    model = fhp.GptModel(cfg, be, seed=1234, batch=w["batch"], dtype=w["dtype"])
    prompts = prompts_for(name, w, cfg.vocab_size)
    B, P, NEW = w["batch"], w["prompt"], w["new"]

    def one():
        if w["sampling"]:
            T, k, pen, ng, seed = w["sampling"]
            return fhp.Sampler.generate(model, prompts, NEW, T, k, fhp.Random(seed), None, pen, ng)
        return fhp.Sampler.generate(model, prompts, NEW, 0.0, 0, None)

    for _ in range(warmup):
        ids = one()
    decode_ms, prefill_ms, timings = [], [], []
    t0 = time.perf_counter()
    for _ in range(steps):
        ids = one()
        t = fhp.Sampler.last_timing
        timings.append(t)
        decode_ms.append(t["decode_ms"])
        prefill_ms.append(t["prefill_ms"])
    wall = time.perf_counter() - t0
    n_out = len(ids) if B == 1 else sum(len(r) for r in ids)
    assert n_out == B * NEW, (n_out, B * NEW)

    n_dec = NEW - 1  # step 0 comes from the prefill forward
    dec_s = float(np.mean(decode_ms)) / 1e3
    pre_s = float(np.mean(prefill_ms)) / 1e3
    if n_dec == 0 and name != "c5":
        raise SystemExit("--new must be at least 2 for a decode workload (token 0 comes from the prefill)")
    avg_step_s = dec_s / n_dec if n_dec else 0.0
    ctx = c["context_length"]
    value = steps * B * NEW / wall
    out = {
        "metric": None, "value": round(value, 2), "unit": "tok/s", "n_gpus": 1, "steps": steps,
        "warmup": warmup, "ms_per_step": round(wall / steps * 1e3, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": w["dtype"],
        "data": "synthetic (random-init weights from new Random(1234); PCG32 prompt ids, seed 42 + sequence)",
        "config": {"workload": w["desc"], "batch": B, "prompt_len": P, "new_tokens": NEW},
    }
    if name == "c5":
        c5_traffic, _, c5_build = profiled_traffic("prefill forward", TRAFFIC_PROFILE_C5)
        flops = prefill_flops(c, min(P, ctx), B)
        tflops = flops / pre_s / 1e12
        pre_tok = B * min(P, ctx) / pre_s
        out.update({
            "metric": "prefill tok/s, Forge-220M shape bf16 bs8 x 1024-token prompts",
            "value": round(pre_tok, 1),
            "ms_per_step": round(pre_s * 1e3, 3),
            "decode_tok_s_reprefill": round(B * n_dec / dec_s, 1) if n_dec else None,
            "reprefill_ms_per_step": round(avg_step_s * 1e3, 3),
            "whole_job_tok_s": round(value, 2),
            "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(tflops / BF16_PEAK_TFLOPS, 4), "traffic": c5_traffic,
                         "kernel": "prefill forward (GEMM, attention, LayerNorm, head kernels)",
                         "flops_per_launch": flops, "launch_us": round(pre_s * 1e6, 1)},
        })
        if c5_traffic is not None:
            out["roofline"]["traffic_source"] = f"{TRAFFIC_PROFILE_C5} (counted on {c5_build})"
        # the timed unit is one prefill forward; value is its token rate
        out["steps"] = steps
    else:
        # decode step n attends P+n keys (positions 0..P+n-1 plus itself), n = 1..NEW-1
        attended = float(np.mean([min(P + n, ctx) for n in range(1, NEW)]))
        step_bytes = decode_bytes_per_step(c, attended, batch=B)
        achieved = step_bytes / avg_step_s / 1e9
        rt = timings[-1]["route"]
        N = fhp._native
        # one launch runs every cached step: greedy (in-kernel argmax) or top-k sampled (in-kernel draw)
        persistent = bool(rt & N.FH_ROUTE_FUSED_STEP) and (not w["sampling"] or bool(rt & N.FH_ROUTE_FUSED_SAMPLER))
        if persistent:
            kernel = "k_decode_step<768, 12, sampled>" if w["sampling"] else "k_decode_step<768>"
        elif rt & N.FH_ROUTE_FUSED_STEP:
            kernel = "k_decode_step<768> + k_sample_row (one launch of each per sampled token)"
        else:
            kernel = "decode step graph (generic kernels)"
        tokens_per_launch = n_dec if persistent else 1
        traffic, traffic_src = None, None
        if persistent and name == "c2":
            traffic, _, build = profiled_traffic(kernel)
            traffic_src = f"{TRAFFIC_PROFILE} (counted on {build})" if traffic is not None else None
        elif persistent and name == "c3":
            traffic, _, build = profiled_traffic(kernel, TRAFFIC_PROFILE_2)
            traffic_src = f"{TRAFFIC_PROFILE_2} (counted on {build})" if traffic is not None else None
        elif not persistent and name == "c4":
            extra, ratio, build = profiled_traffic(kernel, TRAFFIC_PROFILE_C4)
            if extra is not None:
                # the counted bytes above the algorithmic ones (split-K partial sums, which
                # do not grow with the window) added to this run's algorithmic bytes
                traffic = int((step_bytes + extra) * tokens_per_launch)
                traffic_src = (f"{TRAFFIC_PROFILE_C4}: {extra / 1e9:.3f} GB per step above the algorithmic "
                               f"bytes ({build}; ratio {ratio:.4f} there), added to this run's algorithmic bytes")
        out.update({
            "decode_tok_s": round(B * n_dec / dec_s, 2),
            "decode_us_per_step": round(avg_step_s * 1e6, 2),
            "prefill_tok_s": round(B * P / pre_s, 2),
            "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(achieved / HBM_PEAK_GBS, 4),
                         "traffic": traffic,
                         "kernel": kernel, "tokens_per_launch": tokens_per_launch,
                         "bytes_per_launch": int(step_bytes * tokens_per_launch),
                         "launch_us": round(avg_step_s * tokens_per_launch * 1e6, 2)},
        })
        if traffic is not None:
            out["roofline"]["traffic_source"] = traffic_src
        if name == "c2":
            out["metric"] = "decode tok/s, Forge-98M shape fp32 bs1 (prompt 64 + 256 greedy)"
            out["decode_us_per_token"] = out.pop("decode_us_per_step")
        elif name == "c3":
            out["metric"] = "decode tok/s, Forge-98M shape fp32 bs1 sampled (prompt 32 + 512)"
        else:
            out["metric"] = "decode tok/s, Forge-98M shape fp32 bs32 (prompt 512 + 512 greedy)"
    out["device"] = be.device_name
    if with_cpu:
        # C2 runs the whole workload (BASELINE's CPU plan); the others a capped sample
        budget = cpu_budget or args.cpu_tokens or {"c2": 256, "c3": 96, "c4": 12, "c5": 2}[name]
        out["cpu_baseline"] = cpu_baseline(name, w, prompts, ids, budget)
    model.dispose()
    be.dispose()
    return out


def run_stream(steps: int, warmup: int) -> dict:
    """The drop-in seam as the CLI drives it: Sampler.generate_stream (fh_generate_begin /
    fh_generate_next, 16 steps per call) at the `generate` command's defaults -- temperature
    0.8, top-k 40, no repetition controls, the tokenizer's EOS id set (Program.cs:642-644,
    671-673) -- on the C2 shape and prompt, against one fh_generate call with the same
    options.  The EOS id is one the run never draws, so every one of the 256 steps runs
    (a model that emits no EOS within --tokens)."""
    import ctypes
    import numpy as np
    import forge_hip as fhp
    N = fhp._native
    w = WORKLOADS["c2"]
    cfg = fhp.ModelConfig(**w["shape"])
    be = fhp.HipBackend(0)
    model = fhp.GptModel(cfg, be, seed=1234)
    prompt = prompts_for("c2", w, cfg.vocab_size)
    NEW, T, K, CHUNK = w["new"], 0.8, 40, 16
    drawn = set(int(i) for i in fhp.Sampler.generate(model, prompt, NEW, T, K, fhp.Random(1)))
    eos = min(set(range(cfg.vocab_size)) - drawn)

    def one():
        return list(fhp.Sampler.generate(model, prompt, NEW, T, K, fhp.Random(1), eos))

    def stream():
        return list(fhp.Sampler.generate_stream(model, prompt, NEW, T, K, fhp.Random(1), eos, chunk=CHUNK))

    def timed(fn):
        for _ in range(warmup):
            fn()
        t0 = time.perf_counter()
        for _ in range(steps):
            ids = fn()
        return ids, (time.perf_counter() - t0) / steps

    ids_one, s_one = timed(one)
    ids_stream, s_stream = timed(stream)
    route = ctypes.c_int32()
    N.check(N.lib().fh_last_route(model.handle, ctypes.byref(route)))
    model.dispose()
    be.dispose()
    return {
        "metric": "decode tok/s through Sampler.generate_stream, Forge-98M shape fp32 bs1, CLI sampling defaults",
        "value": round(NEW / s_stream, 2), "unit": "tok/s", "steps": steps, "warmup": warmup,
        "config": {"workload": f"C2 shape and prompt (64 ids), 256 tokens, temperature {T}, top-k {K}, penalty 1, "
                               f"no n-gram ban, EOS id {eos} (never drawn), {CHUNK} steps per fh_generate_next, "
                               f"Random(1) uniforms"},
        "stream_us_per_token": round(s_stream / NEW * 1e6, 2),
        "one_shot_us_per_token": round(s_one / NEW * 1e6, 2),
        "stream_over_one_shot": round(s_stream / s_one, 4),
        "ids_equal_one_shot": ids_stream == ids_one and len(ids_one) == NEW,
        "in_kernel_sampler": bool(route.value & N.FH_ROUTE_FUSED_SAMPLER),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="c2")
    ap.add_argument("--new", type=int, default=0,
                    help="generate this many tokens instead of the workload's count (short profiling runs)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="C2 only: leave out the bs32 decode (C4) and prefill (C5) sub-objects")
    ap.add_argument("--cpu-tokens", type=int, default=0,
                    help="tokens of the workload the CPU baseline runs (default: about 10-25 s on 16 cores)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only time the plain copy kernel (and the read-only pass) on MIB MiB and print its line")
    ap.add_argument("--prompt", type=int, default=0,
                    help="prompt length instead of the workload's (profiling runs, e.g. C4 near window 1023)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs one GPU only: the token loop of one batch-1 sequence is a single-GPU "
              f"workload and this build has no multi-GPU path (asked for --gpus {args.gpus}).", file=sys.stderr)
        sys.exit(2)

    if args.copy_calibration:
        print(json.dumps(copy_calibration(args.copy_calibration, max(1, args.steps))), flush=True)
        return
    line = run_workload(args.workload, args, args.steps, args.warmup, not args.no_cpu, args.new, args.prompt)
    ach = achievable()
    if "roofline" in line and line["roofline"]["unit"] == "GB/s":
        line["roofline"]["achievable"] = ach
        line["roofline"]["frac_of_achievable_read"] = round(line["roofline"]["achieved"] / ach["read_GBs"], 4)
    if args.workload == "c2" and not args.no_extra and not args.new and not args.prompt:
        # the rest of the metric ("bs1/bs32 ... prefill tok/s"), two timed passes each, each
        # with its CPU baseline (a capped sample, extrapolated; the cap is in its text)
        keep = ("value", "unit", "ms_per_step", "steps", "warmup", "dtype", "config", "roofline",
                "decode_tok_s", "decode_us_per_step", "prefill_tok_s", "decode_tok_s_reprefill",
                "reprefill_ms_per_step", "whole_job_tok_s", "metric", "cpu_baseline")
        for key, wl in (("sampled_decode", "c3"), ("bs32_decode", "c4"), ("prefill", "c5")):
            sub = run_workload(wl, args, 2, 1, not args.no_cpu)
            if "roofline" in sub and sub["roofline"]["unit"] == "GB/s":
                sub["roofline"]["frac_of_achievable_read"] = round(sub["roofline"]["achieved"] / ach["read_GBs"], 4)
            line[key] = {k: sub[k] for k in keep if k in sub}
        line["stream"] = run_stream(2, 1)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
