"""Checkpoint: FORGEMODEL1 files into a HIP session.

Mirrors ``Checkpoint.Load`` / ``LoadWithMetadata`` of the reference
(src/LLM.Core/Checkpoint/Checkpoint.cs:116-126, 174-250): the file is parsed,
validated and SHA-256-checked by the library (``fh_checkpoint_info``,
``fh_session_load_checkpoint``); a malformed or corrupted file raises
``InvalidDataError`` (the reference's InvalidDataException) with LoadCore's
message.  The optimizer moments of a training checkpoint are checksummed and
dropped, as ``Load`` (restoreTrainingState: false) drops them.
"""
from __future__ import annotations

import ctypes
import os

from . import _native as N
from .model import GptModel, HipBackend, ModelConfig


class Checkpoint:
    @staticmethod
    def read_config(path: str, verify: bool = True):
        """(ModelConfig, model name) of a checkpoint; verify=True also checks the SHA-256 trailer."""
        desc = N.ModelDesc()
        name = ctypes.create_string_buffer(256)
        N.check(N.lib().fh_checkpoint_info(os.fsencode(path), ctypes.byref(desc), name, len(name), int(verify)))
        cfg = ModelConfig(desc.vocab_size, desc.context_length, desc.d_model, desc.n_layers, desc.n_heads)
        return cfg, name.value.decode("utf-8", errors="replace")

    @staticmethod
    def load(path: str, backend: HipBackend, batch: int = 1, dtype: str = "f32") -> GptModel:
        """Checkpoint.Load(path, backend): a session of the checkpoint's configuration with its weights."""
        cfg, name = Checkpoint.read_config(path, verify=False)
        model = GptModel(cfg, backend, batch=batch, dtype=dtype, name=name)
        try:
            N.check(N.lib().fh_session_load_checkpoint(model.handle, os.fsencode(path)))
        except Exception:
            model.dispose()
            raise
        return model
