"""Per-hand-off timeline of the persistent batch-1 decode kernel.

    python -m forge_hip.trace [--steps N] [--repeat R]

Creates a C2-shape session (Forge-98M shape fp32, new Random(1234) weights) with
FORGE_HIP_TRACE=1, generates N greedy tokens from the 64-id PCG32(42) prompt R
times, and prints, for layer 1 of the launch's sixth token, when each phase of
each block happened (min / median / max over the 256 blocks, microseconds from the
first block's "x ready"), then the head of that token.  The marks come from
fh_debug_fused_trace; the phases are those of k_decode_step (decode_fast.hip):

  c A x ready         control wave: the layer's input x gathered
  d A put             data waves: q/k/v columns computed and published
  c B qkv ready       attention blocks: q, k, v of their head gathered
  d B kv in / scores  attention waves: cached K/V rows landed / scores done
  c B part written    attention blocks: the block's partial (o, max, sum) published
  c C parts gathered  every block: its XCD's attention partials gathered
  c C combined        ... and combined into o of the XCD's heads
  d C put             attn.proj partial sums over the XCD's heads published
  c C px2 slices      the block's columns of the 8 XCD partials gathered (cross-XCD)
  c C x2 ready        x2 all-gathered within the XCD
  d D put / c D h     mlp.fc + GELU published / the XCD's h slice gathered
  d E put             mlp.proj partial sums published
  c E px slices       the block's columns of the 8 XCD partials gathered (cross-XCD)
  c E x written       x of the block's columns published
  c A x ready L2      the next layer's x all-gathered
"""
from __future__ import annotations

import argparse
import ctypes
import os

import numpy as np

NAMES = {0: "c A x ready", 1: "c B qkv ready", 2: "c B part written", 3: "c C o ready", 7: "c C px2 slices",
         4: "c C x2 ready", 5: "c D h ready", 8: "c E px slices", 6: "c E x written", 9: "c A x ready L2",
         13: "c C parts gathered", 15: "c C combined", 16: "c H x final", 17: "c H records out",
         18: "c H argmax", 19: "c H next x",
         32: "d A sync", 33: "d A put", 34: "d B sync", 35: "d B attn", 36: "d C sync", 37: "d C put",
         38: "d D sync", 39: "d D put", 40: "d E sync", 41: "d E put", 42: "d A loads landed", 43: "d B kv in",
         44: "d B scores", 45: "d C arrive", 46: "d H logits"}
ORDER = [0, 32, 33, 42, 1, 34, 43, 44, 35, 2, 13, 15, 3, 36, 37, 7, 4, 38, 39, 5, 40, 41, 8, 6, 9]
HEAD = [16, 46, 17, 18, 19]
PER = 64


def collect(steps: int = 256, repeat: int = 3):
    """(timestamps [256, 64] in us from the first x ready, us per token of the last launch)."""
    os.environ["FORGE_HIP_TRACE"] = "1"
    from . import _native as N
    from .model import GptModel, HipBackend, ModelConfig, TrainingRandom
    from .sampler import Sampler
    be = HipBackend(0)
    m = GptModel(ModelConfig(16384, 1024, 768, 12, 12), be, seed=1234)
    prompt = TrainingRandom(42).ids(16384, 64)
    for _ in range(repeat):
        Sampler.generate(m, prompt, steps, 0.0, 0, None)
    us_tok = Sampler.last_timing["decode_ms"] * 1000 / (steps - 1)
    raw = np.zeros(256 * PER, np.uint64)
    N.check(N.lib().fh_debug_fused_trace(m.handle, raw.ctypes.data, raw.size))
    m.dispose()
    be.dispose()
    tr = raw.reshape(256, PER).astype(np.int64)
    xcd = tr[:, 12].copy()
    valid = tr > 1000
    t0 = tr[:, 0][tr[:, 0] > 0].min()
    return (tr - t0) * 0.01, valid, xcd, us_tok


def report(T, valid, xcd, us_tok) -> str:
    out = [f"decode: {us_tok:.2f} us per token",
           "%-20s %8s %8s %8s   (layer 1 of token 5; us from the first x ready)" % ("event", "min", "median", "max")]

    def row(i):
        v = T[valid[:, i], i]
        if len(v):
            out.append("%-20s %8.2f %8.2f %8.2f   (n=%d)" % (NAMES[i], v.min(), np.median(v), v.max(), len(v)))

    for i in ORDER:
        row(i)
    out.append("head of token 5:")
    for i in HEAD:
        row(i)
    out.append("per XCD: last partial | C o ready min/med/max | px2 max | x2 ready median")
    for x in range(8):
        sel = xcd == x
        att = sel & valid[:, 2]
        out.append("  xcd %d  %6.2f | %6.2f %6.2f %6.2f | %6.2f | %6.2f" % (
            x, T[att, 2].max() if att.any() else -1, T[sel, 3].min(), np.median(T[sel, 3]), T[sel, 3].max(),
            T[sel, 7].max(), np.median(T[sel, 4])))
    return "\n".join(out)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--repeat", type=int, default=3)
    a = ap.parse_args()
    print(report(*collect(a.steps, a.repeat)), flush=True)


if __name__ == "__main__":
    main()
