"""Writes the committed golden vectors from the CPU oracle.

Run from the repo root: ``python tests/golden/make_golden.py``.  Every vector is
produced by oracle/forge_oracle.cpp (the reference algorithm restated in C++,
full recompute per token as Sampler.Generate does); nothing here runs
reference code.  The tests check that the oracle still reproduces these files
and that the GPU path matches them.

Files:
  c1_greedy.npz      config 1 (L4 d128 H4 ctx128 V2256, weights seed 1234, prompt
                     PCG32(42) x16, 200 greedy tokens): ids, per-step top-5 ids and
                     logits, top-2 margins, full logits at steps 0, 112, 113, 199
  tiny_forward.npz   V32/ctx8/d16/L2/H2 (InferenceTests.Small), weights seed 6,
                     Forward logits [T, V] of ids {3,1,4,1,5}
  net_random.npz     first 1000 NextDouble() of seeds 0, 1, 42 from the restated
                     System.Random (parity against .NET itself is unpinned)
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle as O  # noqa: E402

C1 = O.Config(2256, 128, 128, 4, 4)
TINY = O.Config(32, 8, 16, 2, 2)


def c1_greedy():
    w = O.init_weights(C1, 1234)
    prompt = O.pcg32_ids(42, C1.vocab_size, 16)
    ids, logits = O.generate(C1, w, prompt, 200, kv_cached=False, return_logits=True)
    order = np.argsort(-logits, axis=1, kind="stable")[:, :5]
    top_logits = np.take_along_axis(logits, order, axis=1)
    margins = top_logits[:, 0] - top_logits[:, 1]
    steps = np.array([0, 112, 113, 199], np.int32)
    np.savez_compressed(os.path.join(HERE, "c1_greedy.npz"), prompt=prompt, ids=ids, top5_ids=order.astype(np.int32),
                        top5_logits=top_logits, margins=margins, full_steps=steps, full_logits=logits[steps])


def tiny_forward():
    w = O.init_weights(TINY, 6)
    ids = np.array([3, 1, 4, 1, 5], np.int32)
    np.savez_compressed(os.path.join(HERE, "tiny_forward.npz"), ids=ids, logits=O.forward(TINY, w, ids))


def net_random():
    np.savez_compressed(os.path.join(HERE, "net_random.npz"),
                        **{f"seed{s}": O.net_random_doubles(s, 1000) for s in (0, 1, 42)})


if __name__ == "__main__":
    O.build()
    c1_greedy()
    tiny_forward()
    net_random()
    print("golden vectors written to", HERE)
