"""forge_hip: MI355X (gfx950) backend for ForgeLM's autoregressive token loop.

The compute lives in ``libforge_hip.so`` (HIP kernels + C ABI, ``csrc/``); this
package is the host-side mirror of the reference's model/sampler interface
over that ABI, plus the op-level ITensorBackend (``tensor_backend``) on the
library's ``fh_op_*`` entry points.
"""
from ._native import ArgumentError, HipError, InvalidDataError, InvalidOperationError, LIB_PATH, lib  # noqa: F401
from .model import (BackendSelection, DeviceBuffer, GptModel, HipBackend, ModelConfig, ModelPreset, PRESETS,  # noqa: F401
                    Random, TrainingRandom, get_preset, registry)
from .sampler import Sampler  # noqa: F401
from .checkpoint import Checkpoint  # noqa: F401
from .chat import Chat  # noqa: F401
from .tensor_backend import HipTensorBackend, Tensor  # noqa: F401
