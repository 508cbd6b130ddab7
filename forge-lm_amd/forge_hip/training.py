"""The reference's training model over an ``ITensorBackend``.

A mirror of the layer classes (src/LLM.Core/Model/Layers.cs), the training half of
``GptModel`` (GptModel.cs:38-99, 124-290), ``Parameters`` (Parameters.cs) and the
``AdamW`` optimizer (src/LLM.Core/Training/AdamW.cs), written against the
``ITensorBackend`` method names so that ``HipTensorBackend`` runs them on the
device: every forward and backward op is an ``fh_op_*`` launch, gradients and Adam
moments stay device-resident, and the host sees them only through
``EnsureHostCurrent``.  Layer caching follows the reference's low-memory mode
(attention rebuilds packed Q/K/V and probabilities in backward; the MLP recomputes
its GELU output).
"""
from __future__ import annotations

import ctypes
import math
from typing import Dict, List, Sequence

import numpy as np

from . import _native as N
from .model import ModelConfig, _desc, registry
from .tensor_backend import Tensor

IGNORE_INDEX = -1


class Parameters:
    """Named weights and same-shaped gradients in registration order (Parameters.cs)."""

    def __init__(self, backend=None):
        self._backend = backend
        self._map: Dict[str, tuple] = {}
        self._names: List[str] = []

    def Add(self, name: str, *shape: int) -> Tensor:
        if name in self._map:
            raise ValueError(f"Duplicate parameter name '{name}'.")
        w, g = Tensor(*shape), Tensor(*shape)
        self._map[name] = (w, g)
        self._names.append(name)
        return w

    def Weight(self, name: str) -> Tensor:
        return self._map[name][0]

    def Grad(self, name: str) -> Tensor:
        return self._map[name][1]

    @property
    def Names(self) -> List[str]:
        return list(self._names)

    @property
    def Gradients(self) -> List[Tensor]:
        return [self._map[n][1] for n in self._names]

    @property
    def Count(self) -> int:
        return sum(self._map[n][0].Length for n in self._names)

    def ZeroGrads(self) -> None:
        for n in self._names:
            g = self._map[n][1]
            if self._backend is not None:
                self._backend.Zero(g)
            else:
                g.Zero()


class Linear:
    """y = x @ W + b (Layers.cs:10-55); backward accumulates dW, dB and returns dX."""

    def __init__(self, b, w, dw, bias, dbias):
        self._b, self._w, self._dw, self._bias, self._dbias = b, w, dw, bias, dbias
        self._x = None

    @property
    def In(self):
        return self._w.Shape[0]

    @property
    def Out(self):
        return self._w.Shape[1]

    def Forward(self, x: Tensor, cacheX: bool = True) -> Tensor:
        self._x = x if cacheX else None
        t = x.Shape[0]
        y = Tensor(t, self.Out)
        self._b.MatMulNN(x, self._w, y, t, self.In, self.Out)
        self._b.AddBias(y, self._bias, t, self.Out)
        return y

    def Backward(self, dY: Tensor, x: Tensor = None) -> Tensor:
        if x is None:
            if self._x is None:
                raise RuntimeError("Forward must run before Backward.")
            x = self._x
        self._x = None
        t = x.Shape[0]
        self._b.MatMulTN(x, dY, self._dw, self.In, t, self.Out, True)
        self._b.SumRows(dY, self._dbias, t, self.Out)
        dX = Tensor(t, self.In)
        self._b.MatMulNT(dY, self._w, dX, t, self.Out, self.In)
        return dX


class TiedOutputProjection:
    """logits = x @ table^T, gradient into the shared table (Layers.cs:62-96)."""

    def __init__(self, b, table, dtable):
        self._b, self._table, self._dtable = b, table, dtable
        self._x = None

    def Forward(self, x: Tensor) -> Tensor:
        self._x = x
        V, D = self._table.Shape
        logits = Tensor(x.Shape[0], V)
        self._b.MatMulNT(x, self._table, logits, x.Shape[0], D, V)
        return logits

    def Backward(self, dLogits: Tensor) -> Tensor:
        x, self._x = self._x, None
        V, D = self._table.Shape
        rows = x.Shape[0]
        self._b.MatMulTN(dLogits, x, self._dtable, V, rows, D, True)
        dX = Tensor(rows, D)
        self._b.MatMulNN(dLogits, self._table, dX, rows, V, D)
        return dX


class LayerNorm:
    """Row LayerNorm with cached statistics (Layers.cs:102-141), eps 1e-5."""

    EPS = 1e-5

    def __init__(self, b, w, dw, bias, dbias):
        self._b, self._w, self._dw, self._bias, self._dbias = b, w, dw, bias, dbias
        self._x = self._mean = self._rstd = None

    def Forward(self, x: Tensor) -> Tensor:
        self._x = x
        t, C = x.Shape[0], self._w.Shape[0]
        y = Tensor(t, C)
        self._mean, self._rstd = Tensor(t), Tensor(t)
        self._b.LayerNormForward(x, self._w, self._bias, y, self._mean, self._rstd, t, C, self.EPS)
        return y

    def Backward(self, dY: Tensor) -> Tensor:
        if self._x is None:
            raise RuntimeError("Forward must run before Backward.")
        t, C = self._x.Shape[0], self._w.Shape[0]
        dX = Tensor(t, C)
        self._b.LayerNormBackward(dY, self._x, self._w, self._mean, self._rstd, dX, self._dw, self._dbias, t, C)
        self._x = self._mean = self._rstd = None
        return dX


class MultiHeadAttention:
    """Causal multi-head attention over slot-packed heads (Layers.cs:143-291)."""

    def __init__(self, b, n_heads: int, d_model: int, qkv: Linear, proj: Linear):
        self._b, self._H, self._D = b, n_heads, d_model
        self._hd = d_model // n_heads
        self._inv_scale = np.float32(1.0) / np.float32(math.sqrt(np.float32(self._hd)))
        self.Qkv, self.Proj = qkv, proj
        self._qkv = None
        self._t = 0
        self._batch = 1

    def _packed(self, qkv: Tensor, batch: int, t: int):
        slots, hd = batch * self._H, self._hd
        q, k, v = Tensor(slots * t, hd), Tensor(slots * t, hd), Tensor(slots * t, hd)
        self._b.PackQkvHeads(qkv, q, k, v, batch, t, self._H, hd)
        probs = Tensor(slots * t, t)
        self._b.BatchedMatMulNT(q, k, probs, slots, t, hd, t)
        self._b.ScaledCausalSoftmaxForward(probs, slots * t, t, float(self._inv_scale))
        return q, k, v, probs

    def Forward(self, x: Tensor, batch: int = 1) -> Tensor:
        rows = x.Shape[0]
        if batch < 1 or rows % batch:
            raise ValueError(f"Row count {rows} must be a multiple of batch size {batch}.")
        t = rows // batch
        self._t, self._batch = t, batch
        qkv = self.Qkv.Forward(x)
        q, k, v, probs = self._packed(qkv, batch, t)
        slots, hd = batch * self._H, self._hd
        ctx = Tensor(slots * t, hd)
        self._b.BatchedMatMulNN(probs, v, ctx, slots, t, t, hd)
        concat = Tensor(rows, self._D)
        self._b.UnpackHeads(ctx, concat, batch, t, self._H, hd, 0)
        self._qkv = qkv
        return self.Proj.Forward(concat)

    def Backward(self, dY: Tensor) -> Tensor:
        t, batch = self._t, self._batch
        slots, hd = batch * self._H, self._hd
        dConcat = self.Proj.Backward(dY)
        if self._qkv is None:
            raise RuntimeError("Forward must run before Backward.")
        q, k, v, probs = self._packed(self._qkv, batch, t)
        self._qkv = None
        dCtx = Tensor(slots * t, hd)
        self._b.PackHeads(dConcat, dCtx, batch, t, self._H, hd, 0)
        dProbs = Tensor(slots * t, t)
        self._b.BatchedMatMulNT(dCtx, v, dProbs, slots, t, hd, t)
        dV = Tensor(slots * t, hd)
        self._b.BatchedMatMulTN(probs, dCtx, dV, slots, t, t, hd)
        dScores = Tensor(slots * t, t)
        self._b.ScaledSoftmaxBackward(dProbs, probs, dScores, slots * t, t, float(self._inv_scale))
        dQ = Tensor(slots * t, hd)
        self._b.BatchedMatMulNN(dScores, k, dQ, slots, t, t, hd)
        dK = Tensor(slots * t, hd)
        self._b.BatchedMatMulTN(dScores, q, dK, slots, t, t, hd)
        dQkv = Tensor(dY.Shape[0], 3 * self._D)
        self._b.UnpackQkvHeads(dQ, dK, dV, dQkv, batch, t, self._H, hd)
        return self.Qkv.Backward(dQkv)


class Mlp:
    """fc -> GELU -> proj, GELU output recomputed in backward (Layers.cs:293-333)."""

    def __init__(self, b, fc: Linear, proj: Linear):
        self._b, self.Fc, self.Proj = b, fc, proj
        self._fc_out = None

    def Forward(self, x: Tensor) -> Tensor:
        self._fc_out = self.Fc.Forward(x)
        h = Tensor(x.Shape[0], self.Fc.Out)
        self._b.GeluForward(self._fc_out, h)
        return self.Proj.Forward(h, cacheX=False)

    def Backward(self, dY: Tensor) -> Tensor:
        if self._fc_out is None:
            raise RuntimeError("Forward must run before Backward.")
        h = Tensor(*self._fc_out.Shape)
        self._b.GeluForward(self._fc_out, h)
        dH = self.Proj.Backward(dY, h)
        dA = Tensor(*dH.Shape)
        self._b.GeluBackward(dH, self._fc_out, dA)
        self._fc_out = None
        return self.Fc.Backward(dA)


class Embedding:
    """Row gather with scatter-add backward (Layers.cs:335-362)."""

    def __init__(self, b, table, dtable):
        self._b, self._table, self._dtable = b, table, dtable
        self._idx = None

    def Forward(self, indices: Sequence[int]) -> Tensor:
        self._idx = np.ascontiguousarray(np.asarray(indices, np.int32))
        D = self._table.Shape[1]
        out = Tensor(self._idx.size, D)
        self._b.EmbeddingForward(self._table, self._idx, out, D)
        return out

    def Backward(self, dOut: Tensor) -> None:
        if self._idx is None:
            raise RuntimeError("Forward must run before Backward.")
        self._b.EmbeddingBackward(dOut, self._idx, self._dtable, self._table.Shape[1])


class TransformerBlock:
    """Pre-LN block: x += Attn(LN1(x)); x += Mlp(LN2(x)) (Layers.cs:364-405)."""

    def __init__(self, b, ln1, attn, ln2, mlp):
        self._b, self.Ln1, self.Attn, self.Ln2, self.Mlp = b, ln1, attn, ln2, mlp

    def Forward(self, x: Tensor, batch: int = 1) -> Tensor:
        a = self.Attn.Forward(self.Ln1.Forward(x), batch)
        self._b.AddInPlace(a, x)
        m = self.Mlp.Forward(self.Ln2.Forward(a))
        self._b.AddInPlace(m, a)
        return m

    def Backward(self, dY: Tensor) -> Tensor:
        dX2 = Tensor(*dY.Shape)
        self._b.Copy(dY, dX2)
        self._b.AddInPlace(dX2, self.Ln2.Backward(self.Mlp.Backward(dY)))
        dX = Tensor(*dY.Shape)
        self._b.Copy(dX2, dX)
        self._b.AddInPlace(dX, self.Ln1.Backward(self.Attn.Backward(dX2)))
        return dX


class TrainableGptModel:
    """GptModel's forward / ForwardBackward over an ITensorBackend (GptModel.cs:38-290).

    Weights come from ``new Random(seed)`` as the reference constructor draws them
    (``fh_init_weights``), or from a registry-order array via ``load_weights``."""

    def __init__(self, config: ModelConfig, backend, seed: int = 1234, name: str = "Forge"):
        if not name.strip() or len(name) > 64:
            raise ValueError("Model name must contain 1-64 non-whitespace characters.")
        self.Config, self.Name, self._b = config, name, backend
        p = Parameters(backend)
        d, L = config.d_model, config.n_layers
        for pname, numel in registry(config):
            p.Add(pname, *self._shape(pname, numel))
        self.Params = p
        W = lambda n: (p.Weight(n), p.Grad(n))  # noqa: E731
        self._tok = Embedding(backend, *W("tok_emb"))
        self._pos = Embedding(backend, *W("pos_emb"))
        self._blocks = []
        for i in range(L):
            pre = f"blocks.{i}."

            def lin(nm):
                return Linear(backend, *W(pre + nm + ".w"), *W(pre + nm + ".b"))

            def ln(nm):
                return LayerNorm(backend, *W(pre + nm + ".w"), *W(pre + nm + ".b"))

            attn = MultiHeadAttention(backend, config.n_heads, d, lin("attn.qkv"), lin("attn.proj"))
            self._blocks.append(TransformerBlock(backend, ln("ln1"), attn, ln("ln2"),
                                                 Mlp(backend, lin("mlp.fc"), lin("mlp.proj"))))
        self._lnf = LayerNorm(backend, *W("ln_f.w"), *W("ln_f.b"))
        self._head = TiedOutputProjection(backend, *W("tok_emb"))
        w = np.empty(p.Count, np.float32)
        desc = _desc(config, 1, "f32")
        N.check(N.lib().fh_init_weights(ctypes.byref(desc), int(seed), w.ctypes.data, w.size))
        self.load_weights(w)

    def _shape(self, name: str, numel: int):
        c = self.Config
        if name == "tok_emb":
            return (c.vocab_size, c.d_model)
        if name == "pos_emb":
            return (c.context_length, c.d_model)
        if name.endswith(".w") and numel > c.d_model:  # a matrix [in, out]
            rows = c.d_model if not name.endswith("mlp.proj.w") else 4 * c.d_model
            return (rows, numel // rows)
        return (numel,)

    def load_weights(self, flat: np.ndarray) -> None:
        """Registry-order fp32 weights into the parameters (host write + invalidate)."""
        flat = np.ascontiguousarray(flat, np.float32).reshape(-1)
        if flat.size != self.Params.Count:
            raise ValueError(f"expected {self.Params.Count} floats, got {flat.size}")
        o = 0
        for n in self.Params.Names:
            t = self.Params.Weight(n)
            t.Data[:] = flat[o:o + t.Length]
            o += t.Length
            self._b.InvalidateDeviceCache(t)

    def _validate(self, ids, allow_ignore=False):
        out = np.ascontiguousarray(np.asarray(ids, np.int64).reshape(-1))
        V = self.Config.vocab_size
        bad = (out < 0) | (out >= V)
        if allow_ignore:
            bad &= out != IGNORE_INDEX
        if bad.any():
            i = int(np.argmax(bad))
            what = "Target id" if allow_ignore else "Token id"
            raise ValueError(f"{what} {int(out[i])} out of range [0,{V}).")
        return out.astype(np.int32)

    def _forward_core(self, tokens: np.ndarray, batch: int) -> Tensor:
        t = tokens.size // batch
        x = self._tok.Forward(tokens)
        self._b.AddInPlace(x, self._pos.Forward(np.tile(np.arange(t, dtype=np.int32), batch)))
        for blk in self._blocks:
            x = blk.Forward(x, batch)
        return self._head.Forward(self._lnf.Forward(x))

    def Forward(self, tokens: Sequence[int]) -> Tensor:
        toks = self._validate(tokens)
        if toks.size == 0:
            raise ValueError("Need at least one token.")
        if toks.size > self.Config.context_length:
            raise ValueError(f"Sequence length {toks.size} exceeds ContextLength {self.Config.context_length}.")
        logits = self._forward_core(toks, 1)
        self._b.EnsureHostCurrent(logits)
        return logits

    def ForwardBackward(self, inputs, targets, batch: int = 1, gradientScale: float = 1.0) -> float:
        """Forward, mean cross-entropy (ignore -1), backward accumulating every gradient
        (GptModel.cs:161-250).  Gradients are not zeroed here."""
        inp, tgt = self._validate(inputs), self._validate(targets, allow_ignore=True)
        if batch < 1:
            raise ValueError("batch must be >= 1.")
        if inp.size != tgt.size:
            raise ValueError(f"inputs ({inp.size}) and targets ({tgt.size}) must have equal length.")
        if inp.size % batch:
            raise ValueError(f"inputs length {inp.size} is not a multiple of batch {batch}.")
        t = inp.size // batch
        if t == 0 or t > self.Config.context_length:
            raise ValueError(f"Sequence length {t} must be in [1, {self.Config.context_length}].")
        if not math.isfinite(gradientScale) or gradientScale <= 0:
            raise ValueError("Gradient scale must be finite and > 0.")
        logits = self._forward_core(inp, batch)
        rows, V = logits.Shape[0], self.Config.vocab_size
        loss = self._b.CrossEntropyForward(logits, tgt, logits, rows, V, IGNORE_INDEX)
        self._b.CrossEntropyBackward(logits, tgt, logits, rows, V, IGNORE_INDEX)
        if gradientScale != 1.0:
            self._b.Scale(logits, gradientScale)
        dX = self._lnf.Backward(self._head.Backward(logits))
        for blk in reversed(self._blocks):
            dX = blk.Backward(dX)
        self._pos.Backward(dX)
        self._tok.Backward(dX)
        return loss


class AdamW:
    """AdamW with lazily created, device-resident moments (AdamW.cs)."""

    def __init__(self, backend=None):
        self._b = backend
        self._state: Dict[str, tuple] = {}
        self.StepCount = 0

    def Step(self, p: Parameters, lr: float, beta1: float = 0.9, beta2: float = 0.95, eps: float = 1e-8,
             weightDecay: float = 0.1) -> None:
        self.StepCount += 1
        for name in p.Names:
            w, g = p.Weight(name), p.Grad(name)
            if name not in self._state:
                st = (Tensor(*w.Shape), Tensor(*w.Shape))
                if self._b is not None:
                    self._b.Zero(st[0])
                    self._b.Zero(st[1])
                self._state[name] = st
            m, v = self._state[name]
            self._b.AdamWStep(w, g, m, v, lr, beta1, beta2, eps, weightDecay, self.StepCount)
