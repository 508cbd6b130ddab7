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
        L.or_pcg32_stream.argtypes = [_c_int, ctypes.c_uint64, _c_int, _i32p,
                                      np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")]
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
        i64, vp = ctypes.c_int64, ctypes.c_void_p
        L.or_op_matmul.argtypes = [_c_int, _f32p, _f32p, _f32p] + [_c_int] * 5
        L.or_op_pack_heads.argtypes = [_f32p, _c_int, _f32p] + [_c_int] * 5
        L.or_op_unpack_heads.argtypes = [_f32p, _f32p] + [_c_int] * 6
        L.or_op_add_bias.argtypes = [_f32p, _f32p, _c_int, _c_int]
        L.or_op_sum_rows.argtypes = [_f32p, _f32p, _c_int, _c_int]
        L.or_op_add_in_place.argtypes = [_f32p, _f32p, i64]
        L.or_op_copy_block.argtypes = [_f32p, _c_int, _f32p] + [_c_int] * 7
        L.or_op_scale.argtypes = [_f32p, i64, _c_float]
        L.or_op_transpose.argtypes = [_f32p, _f32p, _c_int, _c_int]
        L.or_op_layernorm_forward.argtypes = [_f32p] * 6 + [_c_int, _c_int, _c_float]
        L.or_op_layernorm_backward.argtypes = [_f32p] * 8 + [_c_int, _c_int]
        L.or_op_softmax_backward.argtypes = [_f32p, _f32p, _f32p, _c_int, _c_int]
        L.or_op_gelu_backward.argtypes = [_f32p, _f32p, _f32p, i64]
        L.or_op_embedding_forward.argtypes = [_f32p, _i32p, _c_int, _f32p, _c_int]
        L.or_op_embedding_backward.argtypes = [_f32p, _i32p, _c_int, _f32p, _c_int]
        L.or_op_causal_mask.argtypes = [_f32p, i64, _c_int]
        L.or_op_cross_entropy_forward.argtypes = [vp, _i32p, vp, _c_int, _c_int, _c_int]
        L.or_op_cross_entropy_forward.restype = _c_float
        L.or_op_cross_entropy_backward.argtypes = [vp, _i32p, vp, _c_int, _c_int, _c_int]
        L.or_op_sum_squares.argtypes = [_f32p, i64]
        L.or_op_sum_squares.restype = _c_double
        L.or_op_adamw.argtypes = [_f32p, _f32p, _f32p, _f32p, i64] + [_c_float] * 5 + [_c_int, _c_int]
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


def pcg32_stream(seed: int, increment: int, bounds) -> np.ndarray:
    """TrainingRandom's seeding (TrainingRandom.cs:13-20) with a given odd increment;
    draw i is NextUInt32 when bounds[i] == 0, else Next(bounds[i]) (:33-46)."""
    b = np.ascontiguousarray(bounds, dtype=np.int32)
    out = np.empty(b.size, dtype=np.uint32)
    lib().or_pcg32_stream(seed, increment, b.size, b, out)
    return out


def param_count(cfg: Config) -> int:
    return int(lib().or_param_count(*cfg.dims))


def init_weights(cfg: Config, seed: int) -> np.ndarray:
    w = np.empty(param_count(cfg), dtype=np.float32)
    lib().or_init_weights(*cfg.dims, seed, w)
    return w


def param_layout(cfg: Config) -> list:
    """[(name, offset, shape)] of the flat registry array, in GptModel's registration
    order (GptModel.cs:53-91): tok_emb [V,d], pos_emb [ctx,d], per block ln1.{w,b},
    attn.qkv.{w [d,3d], b}, attn.proj.{w [d,d], b}, ln2.{w,b}, mlp.fc.{w [d,4d], b},
    mlp.proj.{w [4d,d], b}, then ln_f.{w,b}."""
    V, ctx, d, L, _ = cfg.dims
    shapes = [("tok_emb", (V, d)), ("pos_emb", (ctx, d))]
    for i in range(L):
        p = f"blocks.{i}."
        shapes += [(p + "ln1.w", (d,)), (p + "ln1.b", (d,)), (p + "attn.qkv.w", (d, 3 * d)),
                   (p + "attn.qkv.b", (3 * d,)), (p + "attn.proj.w", (d, d)), (p + "attn.proj.b", (d,)),
                   (p + "ln2.w", (d,)), (p + "ln2.b", (d,)), (p + "mlp.fc.w", (d, 4 * d)),
                   (p + "mlp.fc.b", (4 * d,)), (p + "mlp.proj.w", (4 * d, d)), (p + "mlp.proj.b", (d,))]
    shapes += [("ln_f.w", (d,)), ("ln_f.b", (d,))]
    out, off = [], 0
    for name, shp in shapes:
        out.append((name, off, shp))
        off += int(np.prod(shp))
    assert off == param_count(cfg)
    return out


def params(cfg: Config, weights: np.ndarray) -> dict:
    """name -> view of `weights` with the tensor's shape."""
    return {n: weights[o:o + int(np.prod(s))].reshape(s) for n, o, s in param_layout(cfg)}


def trained_like(cfg: Config, weights: np.ndarray, seed: int, ln_w_std: float = 0.1, ln_b_std: float = 0.05,
                 bias_std: float = 0.05) -> np.ndarray:
    """A copy of `weights` whose LayerNorm and Linear vectors are no longer the
    initial (1, 0) and 0 (GptModel.cs:65-66, 90-91): every LayerNorm weight becomes
    1 + N(0, ln_w_std), every LayerNorm bias N(0, ln_b_std) and every Linear bias
    N(0, bias_std), drawn from numpy's seeded generator.  Matrices are kept.  With
    these values the LayerNorm affine (CpuBackend.cs:396) and AddBias
    (Layers.cs:35) change every output, as they do in a trained checkpoint."""
    out = np.array(weights, np.float32, copy=True)
    rng = np.random.default_rng(seed)
    for name, off, shp in param_layout(cfg):
        n = int(np.prod(shp))
        if name.endswith(("ln1.w", "ln2.w", "ln_f.w")):
            out[off:off + n] = (1.0 + ln_w_std * rng.standard_normal(n)).astype(np.float32)
        elif name.endswith(("ln1.b", "ln2.b", "ln_f.b")):
            out[off:off + n] = (ln_b_std * rng.standard_normal(n)).astype(np.float32)
        elif name.endswith(".b"):
            out[off:off + n] = (bias_std * rng.standard_normal(n)).astype(np.float32)
    return out


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


# ---- the rest of CpuBackend (training ops), in place on float32 arrays ------------------
# Each wraps the or_op_* restatement in forge_oracle.cpp; arrays are modified in place
# where the reference method writes, as the C# methods do on Tensor.Data.

def _f(x):
    assert isinstance(x, np.ndarray) and x.dtype == np.float32 and x.flags.c_contiguous
    return x


def op_matmul(mode: str, a, b, y, M, K, N, accumulate=False, slots=1):
    """MatMulNN/NT/TN and the Batched variants (CpuBackend.cs:37-221), into y."""
    lib().or_op_matmul({"nn": 0, "nt": 1, "tn": 2}[mode], _f(a), _f(b), _f(y), slots, M, K, N, int(accumulate))


def op_pack_heads(src, src_cols, dst, batch, T, H, hd, col_base):
    lib().or_op_pack_heads(_f(src), src_cols, _f(dst), batch, T, H, hd, col_base)


def op_unpack_heads(src, dst, dst_cols, batch, T, H, hd, col_base):
    lib().or_op_unpack_heads(_f(src), _f(dst), dst_cols, batch, T, H, hd, col_base)


def op_add_bias(y, bias, rows, cols):
    lib().or_op_add_bias(_f(y), _f(bias), rows, cols)


def op_sum_rows(dy, dbias, rows, cols):
    lib().or_op_sum_rows(_f(dy), _f(dbias), rows, cols)


def op_add_in_place(dst, src):
    lib().or_op_add_in_place(_f(dst), _f(src), dst.size)


def op_copy_block(src, src_cols, dst, dst_cols, src_row, src_col, dst_row, dst_col, rows, cols):
    lib().or_op_copy_block(_f(src), src_cols, _f(dst), dst_cols, src_row, src_col, dst_row, dst_col, rows, cols)


def op_scale(x, factor):
    lib().or_op_scale(_f(x), x.size, factor)


def op_transpose(x, out, rows, cols):
    lib().or_op_transpose(_f(x), _f(out), rows, cols)


def op_layernorm_forward(x, w, b, out, mean, rstd, rows, cols, eps):
    lib().or_op_layernorm_forward(_f(x), _f(w), _f(b), _f(out), _f(mean), _f(rstd), rows, cols, eps)


def op_layernorm_backward(dout, x, w, mean, rstd, dx, dw, db, rows, cols):
    lib().or_op_layernorm_backward(_f(dout), _f(x), _f(w), _f(mean), _f(rstd), _f(dx), _f(dw), _f(db), rows, cols)


def op_softmax_forward(x, rows, cols):
    lib().or_softmax(_f(x), rows, cols)


def op_softmax_backward(dout, s, dx, rows, cols):
    lib().or_op_softmax_backward(_f(dout), _f(s), _f(dx), rows, cols)


def op_scaled_causal_softmax_forward(scores, rows, T, scale):
    """ITensorBackend.cs:117-122: Scale, CausalMask, SoftmaxForward."""
    op_scale(scores, scale)
    op_causal_mask(scores, T)
    op_softmax_forward(scores, rows, T)


def op_scaled_softmax_backward(dout, s, dx, rows, cols, scale):
    """ITensorBackend.cs:125-130: SoftmaxBackward, then Scale."""
    op_softmax_backward(dout, s, dx, rows, cols)
    op_scale(dx, scale)


def op_gelu_forward(x, out):
    lib().or_gelu(_f(x), _f(out), x.size)


def op_gelu_backward(dout, x, dx):
    lib().or_op_gelu_backward(_f(dout), _f(x), _f(dx), x.size)


def op_embedding_forward(table, indices, out, D):
    idx = np.ascontiguousarray(indices, np.int32)
    lib().or_op_embedding_forward(_f(table), idx, idx.size, _f(out), D)


def op_embedding_backward(dout, indices, dtable, D):
    idx = np.ascontiguousarray(indices, np.int32)
    lib().or_op_embedding_backward(_f(dout), idx, idx.size, _f(dtable), D)


def op_causal_mask(scores, T):
    lib().or_op_causal_mask(_f(scores), scores.size, T)


def op_cross_entropy_forward(logits, targets, probs, T, V, ignore) -> float:
    """probs may be logits itself (the in-place form)."""
    tg = np.ascontiguousarray(targets, np.int32)
    return float(lib().or_op_cross_entropy_forward(_f(logits).ctypes.data, tg, _f(probs).ctypes.data, T, V, ignore))


def op_cross_entropy_backward(probs, targets, dlogits, T, V, ignore):
    tg = np.ascontiguousarray(targets, np.int32)
    lib().or_op_cross_entropy_backward(_f(probs).ctypes.data, tg, _f(dlogits).ctypes.data, T, V, ignore)


def op_sum_squares(x) -> float:
    return float(lib().or_op_sum_squares(_f(x), x.size))


def op_adamw(w, g, m, v, lr, beta1, beta2, eps, weight_decay, step, is_matrix):
    lib().or_op_adamw(_f(w), _f(g), _f(m), _f(v), w.size, lr, beta1, beta2, eps, weight_decay, step, int(is_matrix))
