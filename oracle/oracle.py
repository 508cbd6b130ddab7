"""ctypes front end of the CPU oracle -- TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg may
import this module.  It loads ``oracle/build/libforge_oracle.so`` (built from
``oracle/forge_oracle.cpp`` by ``oracle/Makefile``), a C++ restatement of the
reference CPU backend, GptModel forward and Sampler; see the header of
forge_oracle.cpp for which reference lines each function follows and which
check pins it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "build", "libforge_oracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_c_int, _c_float, _c_double = ctypes.c_int, ctypes.c_float, ctypes.c_double


def build() -> str:
    """Compiles the oracle with its Makefile (always; make skips up-to-date work)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.or_set_threads.argtypes = [_c_int]
        L.or_net_random_doubles.argtypes = [_c_int, _c_int, _f64p]
        L.or_pcg32_ids.argtypes = [_c_int, _c_int, _c_int, _i32p]
        L.or_param_count.argtypes = [_c_int] * 5
        L.or_param_count.restype = ctypes.c_int64
        L.or_init_weights.argtypes = [_c_int] * 6 + [_f32p]
        L.or_matmul_nn.argtypes = [_f32p, _f32p, _f32p, _c_int, _c_int, _c_int]
        L.or_matmul_nt.argtypes = [_f32p, _f32p, _f32p, _c_int, _c_int, _c_int]
        L.or_dot.argtypes = [_f32p, _f32p, _c_int]
        L.or_dot.restype = _c_float
        L.or_layernorm.argtypes = [_f32p, _f32p, _f32p, _f32p, _c_int, _c_int, _c_float]
        L.or_softmax.argtypes = [_f32p, _c_int, _c_int]
        L.or_gelu.argtypes = [_f32p, _f32p, _c_int]
        L.or_greedy.argtypes = [_f32p, _c_int]
        L.or_greedy.restype = _c_int
        L.or_sample.argtypes = [_f32p, _c_int, _c_float, _c_int, _c_double]
        L.or_sample.restype = _c_int
        L.or_apply_repetition_controls.argtypes = [_f32p, _c_int, _i32p, _c_int, _c_float, _c_int]
        L.or_forward.argtypes = [_c_int] * 5 + [_f32p, _i32p, _c_int, _f32p]
        L.or_generate.argtypes = ([_c_int] * 5 + [_f32p, _i32p, _c_int, _c_int, _c_float, _c_int,
                                                  ctypes.c_void_p, _c_int, _c_float, _c_int, _c_int,
                                                  _i32p, ctypes.c_void_p])
        L.or_generate.restype = _c_int
        _lib = L
    return _lib


@dataclass(frozen=True)
class Config:
    """ModelConfig (src/LLM.Core/Model/ModelConfig.cs:8-25)."""
    vocab_size: int
    context_length: int
    d_model: int
    n_layers: int
    n_heads: int

    @property
    def dims(self):
        return (self.vocab_size, self.context_length, self.d_model, self.n_layers, self.n_heads)


def set_threads(n: int) -> None:
    lib().or_set_threads(int(n))


def net_random_doubles(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float64)
    lib().or_net_random_doubles(seed, n, out)
    return out


def pcg32_ids(seed: int, max_excl: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    lib().or_pcg32_ids(seed, max_excl, n, out)
    return out


def param_count(cfg: Config) -> int:
    return int(lib().or_param_count(*cfg.dims))


def init_weights(cfg: Config, seed: int) -> np.ndarray:
    w = np.empty(param_count(cfg), dtype=np.float32)
    lib().or_init_weights(*cfg.dims, seed, w)
    return w


def matmul_nn(a, b):
    a = np.ascontiguousarray(a, np.float32); b = np.ascontiguousarray(b, np.float32)
    y = np.empty((a.shape[0], b.shape[1]), np.float32)
    lib().or_matmul_nn(a, b, y, a.shape[0], a.shape[1], b.shape[1])
    return y


def matmul_nt(a, b):
    a = np.ascontiguousarray(a, np.float32); b = np.ascontiguousarray(b, np.float32)
    y = np.empty((a.shape[0], b.shape[0]), np.float32)
    lib().or_matmul_nt(a, b, y, a.shape[0], a.shape[1], b.shape[0])
    return y


def dot(x, y) -> float:
    x = np.ascontiguousarray(x, np.float32); y = np.ascontiguousarray(y, np.float32)
    return float(lib().or_dot(x, y, x.size))


def layernorm(x, w, b, eps=1e-5):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().or_layernorm(x, np.ascontiguousarray(w, np.float32), np.ascontiguousarray(b, np.float32),
                       out, x.shape[0], x.shape[1], eps)
    return out


def softmax(x):
    x = np.array(x, np.float32, copy=True, order="C")
    lib().or_softmax(x, x.shape[0], x.shape[1])
    return x


def gelu(x):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().or_gelu(x, y, x.size)
    return y


def greedy(logits) -> int:
    return int(lib().or_greedy(np.ascontiguousarray(logits, np.float32), len(logits)))


def sample(logits, temperature: float, top_k: int, u01: float) -> int:
    return int(lib().or_sample(np.ascontiguousarray(logits, np.float32), len(logits),
                               temperature, top_k, u01))


def apply_repetition_controls(logits, history, penalty: float, ngram: int) -> np.ndarray:
    out = np.array(logits, np.float32, copy=True)
    h = np.ascontiguousarray(history, np.int32)
    lib().or_apply_repetition_controls(out, out.size, h, h.size, penalty, ngram)
    return out


def forward(cfg: Config, weights: np.ndarray, ids) -> np.ndarray:
    ids = np.ascontiguousarray(ids, np.int32)
    out = np.empty((ids.size, cfg.vocab_size), np.float32)
    lib().or_forward(*cfg.dims, weights, ids, ids.size, out)
    return out


def generate(cfg: Config, weights: np.ndarray, prompt, max_new: int, temperature: float = 0.0,
             top_k: int = 0, uniforms=None, eos: int = -1, penalty: float = 1.0, ngram: int = 0,
             kv_cached: bool = True, return_logits: bool = False):
    """Sampler.Generate (Sampler.cs:78-109) for one sequence.

    Returns ``ids`` or ``(ids, logits[n, V])``; logits are the raw ForwardLast rows.
    """
    prompt = np.ascontiguousarray(prompt, np.int32)
    out = np.empty(max(max_new, 1), np.int32)
    u = None
    if temperature > 0:
        u = np.ascontiguousarray(uniforms, np.float64)
        assert u.size >= max_new
    lg = np.empty((max(max_new, 1), cfg.vocab_size), np.float32) if return_logits else None
    n = lib().or_generate(*cfg.dims, weights, prompt, prompt.size, max_new, temperature, top_k,
                          None if u is None else u.ctypes.data, eos, penalty, ngram, int(kv_cached),
                          out, None if lg is None else lg.ctypes.data)
    ids = out[:n].copy()
    if return_logits:
        return ids, lg[:n].copy()
    return ids
