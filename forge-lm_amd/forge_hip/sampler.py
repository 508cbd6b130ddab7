"""Sampler mirror (src/LLM.Core/Inference/Sampler.cs) running on the device.

``Sampler.generate`` keeps Sampler.Generate's observable contract
(Sampler.cs:78-109): the same validation errors, exactly ``max_new_tokens``
ids unless ``eos_id`` is yielded (the eos id itself is yielded), the window
left-truncated to ContextLength with positions restarting at 0, and one
``NextDouble`` drawn per sampled step (temperature > 0) from the caller's
Random.  The whole loop, including ApplyRepetitionControls and Sample, runs
on the GPU; only the ids come back.
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional, Sequence

import numpy as np

from . import _native as N
from .model import GptModel, HipBackend, Random


def _validate_repetition(repetition_penalty: float, no_repeat_ngram_size: int):
    if not math.isfinite(repetition_penalty) or repetition_penalty < 1.0:
        raise ValueError("Repetition penalty must be finite and >= 1.")
    if no_repeat_ngram_size < 0:
        raise ValueError("No-repeat n-gram size must be >= 0.")


class Sampler:
    last_timing = None

    @staticmethod
    def generate(model: GptModel, prompt_tokens, max_new_tokens: int, temperature: float, top_k: int,
                 rng: Optional[Random], eos_id: Optional[int] = None, repetition_penalty: float = 1.0,
                 no_repeat_ngram_size: int = 0, return_logits: bool = False):
        """Returns ids [batch, n] (or a 1-D list for batch 1), plus logits if asked.

        ``prompt_tokens`` is one prompt (1-D) or ``batch`` prompts of equal length (2-D).
        """
        if model is None or prompt_tokens is None:
            raise ValueError("model and prompt_tokens are required")
        prompts = np.ascontiguousarray(prompt_tokens, np.int32)
        single = prompts.ndim == 1
        if single:
            prompts = prompts[None, :]
        if prompts.shape[1] == 0:
            raise ValueError("Need at least one prompt token.")
        if max_new_tokens < 0:
            raise ValueError("maxNewTokens must be >= 0")
        V = model.config.vocab_size
        if eos_id is not None and not (0 <= eos_id < V):
            raise ValueError("EOS token must be inside the model vocabulary.")
        _validate_repetition(repetition_penalty, no_repeat_ngram_size)
        if not math.isfinite(temperature):
            raise ValueError("Temperature must be finite.")
        B, P = prompts.shape
        uniforms = None
        if temperature > 0:
            if rng is None:
                raise ValueError("rng is required when temperature > 0")
            # one NextDouble per sampled step, per sequence (sequence-major); a single
            # sequence consumes only the steps it ran (it stops after yielding eos)
            uniforms = np.ascontiguousarray(rng.peek_doubles(B * max_new_tokens), np.float64)
        opts = N.Sampling(float(temperature), int(top_k), float(repetition_penalty), int(no_repeat_ngram_size),
                          -1 if eos_id is None else int(eos_id), 0)
        out = np.zeros((B, max(1, max_new_tokens)), np.int32)
        counts = np.zeros(B, np.int32)
        dump = np.empty((B, max(1, max_new_tokens), V), np.float32) if return_logits else None
        N.check(N.lib().fh_generate(model.handle, prompts.ctypes.data, B, P, int(max_new_tokens), ctypes.byref(opts),
                                    None if uniforms is None else uniforms.ctypes.data, out.ctypes.data,
                                    counts.ctypes.data, None if dump is None else dump.ctypes.data))
        pre, dec = ctypes.c_double(), ctypes.c_double()
        nc, nr = ctypes.c_int32(), ctypes.c_int32()
        N.check(N.lib().fh_last_timing(model.handle, ctypes.byref(pre), ctypes.byref(dec), ctypes.byref(nc),
                                       ctypes.byref(nr)))
        route = ctypes.c_int32()
        N.check(N.lib().fh_last_route(model.handle, ctypes.byref(route)))
        Sampler.last_timing = {"prefill_ms": pre.value, "decode_ms": dec.value, "cached_steps": nc.value,
                               "reprefill_steps": nr.value, "route": route.value}
        if uniforms is not None:
            rng.skip(int(counts[0]) if B == 1 else B * max_new_tokens)
        ids = [out[b, :counts[b]].copy() for b in range(B)]
        if single:
            ids = ids[0]
        if return_logits:
            lg = [dump[b, :counts[b]].copy() for b in range(B)]
            return ids, (lg[0] if single else lg)
        return ids

    @staticmethod
    def generate_stream(model: GptModel, prompt_tokens, max_new_tokens: int, temperature: float, top_k: int,
                        rng: Optional[Random], eos_id: Optional[int] = None, repetition_penalty: float = 1.0,
                        no_repeat_ngram_size: int = 0, chunk: int = 16):
        """Sampler.Generate as the reference's iterator (Sampler.cs:78-109): yields one id
        at a time for a single prompt, running ``chunk`` device steps per round trip
        (fh_generate_begin / fh_generate_next).  Stops after yielding ``eos_id``."""
        if model is None or prompt_tokens is None:
            raise ValueError("model and prompt_tokens are required")
        prompt = np.ascontiguousarray(prompt_tokens, np.int32)
        if prompt.ndim != 1:
            raise ValueError("generate_stream takes one prompt")
        if prompt.size == 0:
            raise ValueError("Need at least one prompt token.")
        if max_new_tokens < 0:
            raise ValueError("maxNewTokens must be >= 0")
        V = model.config.vocab_size
        if eos_id is not None and not (0 <= eos_id < V):
            raise ValueError("EOS token must be inside the model vocabulary.")
        _validate_repetition(repetition_penalty, no_repeat_ngram_size)
        if not math.isfinite(temperature):
            raise ValueError("Temperature must be finite.")
        if chunk < 1:
            raise ValueError("chunk must be positive")
        if model.batch != 1:
            raise ValueError("generate_stream runs a batch-1 session")
        uniforms = None
        if temperature > 0:
            if rng is None:
                raise ValueError("rng is required when temperature > 0")
            uniforms = np.ascontiguousarray(rng.peek_doubles(max_new_tokens), np.float64)
        opts = N.Sampling(float(temperature), int(top_k), float(repetition_penalty), int(no_repeat_ngram_size),
                          -1 if eos_id is None else int(eos_id), 0)
        N.check(N.lib().fh_generate_begin(model.handle, prompt.ctypes.data, 1, prompt.size, int(max_new_tokens),
                                          ctypes.byref(opts), None if uniforms is None else uniforms.ctypes.data))
        out = np.zeros(max(1, max_new_tokens), np.int32)
        counts = np.zeros(1, np.int32)
        produced = ctypes.c_int32()
        yielded = 0
        try:
            while yielded < max_new_tokens:
                N.check(N.lib().fh_generate_next(model.handle, int(chunk), None, out.ctypes.data,
                                                 counts.ctypes.data, ctypes.byref(produced)))
                n = int(counts[0])
                for i in range(yielded, n):
                    yielded = i + 1  # one NextDouble per yielded (sampled) step
                    yield int(out[i])
                if n < produced.value or produced.value >= max_new_tokens:  # eos yielded, or done
                    break
        finally:
            if uniforms is not None:
                rng.skip(yielded)

    @staticmethod
    def sample_device_logits(backend: HipBackend, logits_dev_ptr, vocab: int, history: Sequence[int],
                             temperature: float, top_k: int, u01: float, repetition_penalty: float = 1.0,
                             no_repeat_ngram_size: int = 0) -> int:
        """ApplyRepetitionControls + Sample on a device logit row (fh_sample_logits)."""
        h = np.ascontiguousarray(history, np.int32)
        opts = N.Sampling(float(temperature), int(top_k), float(repetition_penalty), int(no_repeat_ngram_size), -1, 0)
        out = ctypes.c_int32()
        N.check(N.lib().fh_sample_logits(backend.handle, logits_dev_ptr if isinstance(logits_dev_ptr, ctypes.c_void_p) else ctypes.c_void_p(logits_dev_ptr), vocab,
                                         h.ctypes.data if h.size else None, h.size, ctypes.byref(opts), float(u01),
                                         ctypes.byref(out)))
        return out.value
