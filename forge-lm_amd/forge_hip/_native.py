"""ctypes binding of libforge_hip.so (include/forge_hip.h).

The library is built in-tree by ``forge-lm_amd/csrc/Makefile`` into
``forge-lm_amd/build/libforge_hip.so``.  There is no fallback: if the library
is missing or a GPU call fails, the error is raised.
"""
from __future__ import annotations

import ctypes
import os

_PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG_ROOT, "build", "libforge_hip.so")

FH_OK = 0
FH_ERR_INVALID = -1
FH_ERR_RANGE = -2
FH_ERR_HIP = -3
FH_ERR_OOM = -4
FH_ERR_STATE = -5
FH_ERR_UNSUPPORTED = -6
FH_ERR_DATA = -7

FH_DTYPE_F32 = 0
FH_DTYPE_BF16 = 1
# fh_last_route bits
FH_ROUTE_FUSED_STEP, FH_ROUTE_FUSED_EPILOGUES, FH_ROUTE_ATTN_IN_PROJ, FH_ROUTE_UNFUSED = 1, 2, 4, 8
FH_ROUTE_FUSED_SAMPLER, FH_ROUTE_RETRIED, FH_ROUTE_FALLBACK = 16, 32, 64

# Every symbol include/forge_hip.h declares (checked by the CPU tests).
EXPORTS = (
    "fh_last_error", "fh_version", "fh_random_doubles", "fh_context_create", "fh_context_destroy",
    "fh_context_info", "fh_context_memory", "fh_buffer_alloc", "fh_buffer_free", "fh_buffer_write", "fh_buffer_read",
    "fh_buffer_copy", "fh_buffer_checksum", "fh_matmul_nn",
    "fh_session_create", "fh_session_destroy", "fh_param_count", "fh_param_info",
    "fh_session_init_random", "fh_init_weights", "fh_session_load_weights", "fh_session_read_param", "fh_forward_last",
    "fh_generate", "fh_last_timing", "fh_last_route", "fh_debug_fused_trace", "fh_sample_logits", "fh_sample_logits_noalloc",
    "fh_checkpoint_info", "fh_session_load_checkpoint", "fh_sha256", "fh_generate_begin", "fh_generate_next",
    # op-level ITensorBackend
    "fh_op_matmul_nn", "fh_op_matmul_nt", "fh_op_matmul_tn", "fh_op_pack_heads", "fh_op_unpack_heads",
    "fh_op_add_bias", "fh_op_sum_rows", "fh_op_add_in_place", "fh_op_copy", "fh_op_scale", "fh_op_zero",
    "fh_op_copy_block", "fh_op_transpose", "fh_op_layernorm_forward", "fh_op_layernorm_backward",
    "fh_op_softmax_forward", "fh_op_scaled_causal_softmax_forward", "fh_op_softmax_backward",
    "fh_op_gelu_forward", "fh_op_gelu_backward", "fh_op_embedding_forward", "fh_op_embedding_backward",
    "fh_op_causal_mask", "fh_op_cross_entropy_forward", "fh_op_begin_loss_accumulation",
    "fh_op_end_loss_accumulation", "fh_op_cross_entropy_backward", "fh_op_sum_squares",
    "fh_op_global_sum_squares", "fh_op_adamw_step",
)


class ModelDesc(ctypes.Structure):
    _fields_ = [("vocab_size", ctypes.c_int32), ("context_length", ctypes.c_int32),
                ("d_model", ctypes.c_int32), ("n_layers", ctypes.c_int32), ("n_heads", ctypes.c_int32),
                ("max_batch", ctypes.c_int32), ("dtype", ctypes.c_int32), ("reserved", ctypes.c_int32)]


class Sampling(ctypes.Structure):
    _fields_ = [("temperature", ctypes.c_float), ("top_k", ctypes.c_int32),
                ("repetition_penalty", ctypes.c_float), ("no_repeat_ngram", ctypes.c_int32),
                ("eos_id", ctypes.c_int32), ("reserved", ctypes.c_int32)]


class HipError(RuntimeError):
    """A libforge_hip call returned a negative status."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"{msg} (status {code})")
        self.code = code


class ArgumentError(HipError, ValueError):
    """FH_ERR_INVALID / FH_ERR_RANGE: the reference's ArgumentException family."""


class InvalidDataError(HipError, ValueError):
    """FH_ERR_DATA: the reference's InvalidDataException (malformed or corrupted checkpoint)."""


class InvalidOperationError(HipError):
    """FH_ERR_STATE: the reference's InvalidOperationException (a call out of order)."""


_lib = None


def lib():
    """Loads the library once; raises FileNotFoundError if it was never built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise FileNotFoundError(
            f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`")
    L = ctypes.CDLL(LIB_PATH)
    vp, i32, i64, f32, f64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_double
    P = ctypes.POINTER
    L.fh_last_error.argtypes = [ctypes.c_char_p, ctypes.c_size_t]
    L.fh_version.restype = ctypes.c_char_p
    L.fh_random_doubles.argtypes = [i32, ctypes.c_int, vp]
    L.fh_context_create.argtypes = [ctypes.c_int, P(vp)]
    L.fh_context_destroy.argtypes = [vp]
    L.fh_context_info.argtypes = [vp, ctypes.c_char_p, ctypes.c_size_t, P(ctypes.c_uint64), P(i32)]
    L.fh_context_memory.argtypes = [vp, P(ctypes.c_uint64), P(ctypes.c_uint64)]
    L.fh_buffer_alloc.argtypes = [vp, ctypes.c_size_t, P(vp)]
    L.fh_buffer_free.argtypes = [vp, vp]
    L.fh_buffer_checksum.argtypes = [vp, vp, ctypes.c_size_t, P(ctypes.c_uint64), P(f32)]
    L.fh_buffer_write.argtypes = [vp, vp, vp, ctypes.c_size_t]
    L.fh_buffer_read.argtypes = [vp, vp, vp, ctypes.c_size_t]
    L.fh_buffer_copy.argtypes = [vp, vp, vp, ctypes.c_size_t, P(ctypes.c_float)]
    L.fh_matmul_nn.argtypes = [vp, vp, vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    L.fh_session_create.argtypes = [vp, P(ModelDesc), P(vp)]
    L.fh_session_destroy.argtypes = [vp]
    L.fh_param_count.argtypes = [P(ModelDesc)]
    L.fh_param_count.restype = i64
    L.fh_param_info.argtypes = [P(ModelDesc), ctypes.c_int, ctypes.c_char_p, ctypes.c_size_t, P(i64)]
    L.fh_session_init_random.argtypes = [vp, i32]
    L.fh_init_weights.argtypes = [P(ModelDesc), i32, vp, i64]
    L.fh_session_load_weights.argtypes = [vp, P(vp), ctypes.c_int]
    L.fh_session_read_param.argtypes = [vp, ctypes.c_int, vp, i64]
    L.fh_forward_last.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, vp]
    L.fh_generate.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, P(Sampling), vp, vp, vp, vp]
    L.fh_last_timing.argtypes = [vp, P(f64), P(f64), P(i32), P(i32)]
    L.fh_last_route.argtypes = [vp, P(i32)]
    L.fh_debug_fused_trace.argtypes = [vp, vp, ctypes.c_int]
    L.fh_sample_logits.argtypes = [vp, vp, ctypes.c_int, vp, ctypes.c_int, P(Sampling), f64, P(i32)]
    L.fh_sample_logits_noalloc.argtypes = L.fh_sample_logits.argtypes
    L.fh_checkpoint_info.argtypes = [ctypes.c_char_p, P(ModelDesc), ctypes.c_char_p, ctypes.c_size_t, ctypes.c_int]
    L.fh_session_load_checkpoint.argtypes = [vp, ctypes.c_char_p]
    L.fh_sha256.argtypes = [vp, ctypes.c_size_t, vp]
    L.fh_generate_begin.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, P(Sampling), vp]
    L.fh_generate_next.argtypes = [vp, ctypes.c_int, vp, vp, vp, P(i32)]
    ci, cf = ctypes.c_int, ctypes.c_float
    for mm in ("nn", "nt", "tn"):
        getattr(L, f"fh_op_matmul_{mm}").argtypes = [vp, vp, vp, vp, ci, ci, ci, ci, ci]
    L.fh_op_pack_heads.argtypes = [vp, vp, ci, vp, ci, ci, ci, ci, ci]
    L.fh_op_unpack_heads.argtypes = [vp, vp, vp, ci, ci, ci, ci, ci, ci]
    L.fh_op_add_bias.argtypes = [vp, vp, vp, ci, ci]
    L.fh_op_sum_rows.argtypes = [vp, vp, vp, ci, ci]
    L.fh_op_add_in_place.argtypes = [vp, vp, vp, i64]
    L.fh_op_copy.argtypes = [vp, vp, vp, i64]
    L.fh_op_scale.argtypes = [vp, vp, i64, cf]
    L.fh_op_zero.argtypes = [vp, vp, i64]
    L.fh_op_copy_block.argtypes = [vp, vp, ci, vp, ci, ci, ci, ci, ci, ci, ci]
    L.fh_op_transpose.argtypes = [vp, vp, vp, ci, ci]
    L.fh_op_layernorm_forward.argtypes = [vp, vp, vp, vp, vp, vp, vp, ci, ci, cf]
    L.fh_op_layernorm_backward.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, vp, ci, ci]
    L.fh_op_softmax_forward.argtypes = [vp, vp, ci, ci]
    L.fh_op_scaled_causal_softmax_forward.argtypes = [vp, vp, ci, ci, cf]
    L.fh_op_softmax_backward.argtypes = [vp, vp, vp, vp, ci, ci, cf]
    L.fh_op_gelu_forward.argtypes = [vp, vp, vp, i64]
    L.fh_op_gelu_backward.argtypes = [vp, vp, vp, vp, i64]
    L.fh_op_embedding_forward.argtypes = [vp, vp, ci, vp, ci, vp, ci]
    L.fh_op_embedding_backward.argtypes = [vp, vp, vp, ci, vp, ci, ci]
    L.fh_op_causal_mask.argtypes = [vp, vp, i64, ci]
    L.fh_op_cross_entropy_forward.argtypes = [vp, vp, vp, vp, ci, ci, ci, P(f32)]
    L.fh_op_begin_loss_accumulation.argtypes = [vp]
    L.fh_op_end_loss_accumulation.argtypes = [vp, P(f32)]
    L.fh_op_cross_entropy_backward.argtypes = [vp, vp, vp, vp, ci, ci, ci]
    L.fh_op_sum_squares.argtypes = [vp, vp, i64, P(f64)]
    L.fh_op_global_sum_squares.argtypes = [vp, P(vp), P(i64), ci, P(f64)]
    L.fh_op_adamw_step.argtypes = [vp, vp, vp, vp, vp, i64, cf, cf, cf, cf, cf, ci, ci]
    _lib = L
    return L


def last_error() -> str:
    buf = ctypes.create_string_buffer(1024)
    lib().fh_last_error(buf, len(buf))
    return buf.value.decode(errors="replace")


def check(code: int) -> int:
    """Raises on a negative status; returns non-negative values unchanged."""
    if code >= 0:
        return code
    msg = last_error()
    if code in (FH_ERR_INVALID, FH_ERR_RANGE):
        raise ArgumentError(code, msg)
    if code == FH_ERR_DATA:
        raise InvalidDataError(code, msg)
    if code == FH_ERR_STATE:
        raise InvalidOperationError(code, msg)
    raise HipError(code, msg)
