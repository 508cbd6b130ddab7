"""The op-level ``ITensorBackend`` of the ``hip`` backend.

Mirrors ``ITensorBackend`` (src/LLM.Core/Tensor/ITensorBackend.cs:18-266) and the
``Tensor`` it works on (src/LLM.Core/Tensor/Tensor.cs) so that model, training and
test code written against the reference's interface runs on libforge_hip's
``fh_op_*`` entry points.  Method names and argument meanings are the reference's.

Residency follows the reference's device backends (CudaBackend.cs:520-600): a
tensor's device copy is created on first use and is authoritative once a kernel
has written it.  ``EnsureHostCurrent`` downloads a device-written tensor,
``InvalidateDeviceCache`` marks the host copy authoritative after a direct write
to ``Data`` (the next kernel re-uploads); writing ``Data`` without it leaves the
kernels on the stale device copy, as the contract states.
"""
from __future__ import annotations

import ctypes
import weakref
from typing import Optional, Sequence

import numpy as np

from . import _native as N
from .model import DeviceBuffer, HipBackend


class Tensor:
    """Dense row-major float32 tensor (Tensor.cs): ``Tensor(*shape)`` is zeros,
    ``Tensor(data, *shape)`` wraps a copy-free float32 view of ``data``."""

    def __init__(self, *args):
        if args and not isinstance(args[0], (int, np.integer)):
            data = np.ascontiguousarray(np.asarray(args[0], dtype=np.float32).reshape(-1))
            shape = tuple(int(s) for s in args[1:]) or (data.size,)
            if int(np.prod(shape)) != data.size:
                raise ValueError(f"data of {data.size} floats does not fill shape {shape}")
        else:
            shape = tuple(int(s) for s in args)
            if not shape or any(s < 0 for s in shape):
                raise ValueError("a tensor needs a non-negative shape")
            data = np.zeros(int(np.prod(shape)), np.float32)
        self.Data = data
        self.Shape = shape
        self.DeviceResource = None

    @property
    def Rank(self) -> int:
        return len(self.Shape)

    @property
    def Length(self) -> int:
        return self.Data.size

    @property
    def Rows(self) -> int:
        return self.Shape[-2]

    @property
    def Cols(self) -> int:
        return self.Shape[-1]

    def Zero(self) -> None:
        self.Data[:] = 0.0

    def Clone(self) -> "Tensor":
        return Tensor(self.Data.copy(), *self.Shape)

    def __repr__(self) -> str:
        return f"Tensor([{','.join(str(s) for s in self.Shape)}])"


class _Entry:
    """A tensor's device copy: host_stale = a kernel wrote it since the last download;
    device_stale = the host copy is authoritative (never uploaded, or invalidated)."""

    __slots__ = ("buf", "host_stale", "device_stale", "backend", "__weakref__")

    def __init__(self, backend, buf):
        self.backend = backend
        self.buf = buf
        self.host_stale = False
        self.device_stale = True


def _bucket(nbytes: int) -> int:
    """Allocation size class: 256-byte granules up to 64 KiB, then steps of an
    eighth of the power of two (waste below 12.5%)."""
    n = max(256, int(nbytes))
    if n <= 65536:
        return (n + 255) // 256 * 256
    step = 1 << (n.bit_length() - 4)
    return (n + step - 1) // step * step


class HipTensorBackend:
    """``ITensorBackend`` on one device (the ``hip`` backend's op-level half)."""

    def __init__(self, device: int = 0, backend: Optional[HipBackend] = None):
        self._owns = backend is None
        self.backend = backend if backend is not None else HipBackend(device)
        self._ctx = self.backend.handle
        # device storage of collected tensors goes back to per-size free lists and
        # is reused (the reference's device backends do the same, CudaBackend.cs:496-515);
        # every use of a buffer is ordered on the context's stream, so reuse is safe
        self._free = {}
        self._all = []

    # ---- residency -----------------------------------------------------------------
    def _release(self, size: int, buf: DeviceBuffer) -> None:
        if self._free is not None:
            self._free.setdefault(size, []).append(buf)

    def _entry(self, t: Tensor) -> _Entry:
        e = t.DeviceResource
        if e is None or e.backend is not self:
            size = _bucket(t.Data.nbytes)
            pool = self._free.get(size)
            if pool:
                buf = pool.pop()
            else:
                buf = DeviceBuffer(self.backend, size)
                self._all.append(buf)
            e = _Entry(self, buf)
            t.DeviceResource = e
            weakref.finalize(e, self._release, size, buf)
        return e

    def _read(self, t: Tensor):
        e = self._entry(t)
        if e.device_stale:
            if t.Data.size:
                e.buf.write(t.Data)
            e.device_stale = False
        return e.buf.ptr

    def _write(self, t: Tensor, preserve: bool = False):
        """Device pointer of an output; with ``preserve`` the kernel keeps (or adds to)
        the current contents, so an authoritative host copy is uploaded first."""
        e = self._entry(t)
        if preserve and e.device_stale:
            if t.Data.size:
                e.buf.write(t.Data)
        e.device_stale = False
        e.host_stale = True
        return e.buf.ptr

    def InvalidateDeviceCache(self, t: Tensor) -> None:
        e = t.DeviceResource
        if e is not None and e.backend is self:
            e.device_stale = True
            e.host_stale = False

    def EnsureHostCurrent(self, t: Tensor) -> None:
        e = t.DeviceResource
        if e is not None and e.backend is self and e.host_stale:
            t.Data[:] = e.buf.read(np.float32, t.Data.size)
            e.host_stale = False

    # ---- matmuls -------------------------------------------------------------------
    def _matmul(self, fn, a, b, y, slots, M, K, N_, accumulate):
        pa, pb = self._read(a), self._read(b)
        py = self._write(y, preserve=accumulate)
        N.check(fn(self._ctx, pa, pb, py, slots, M, K, N_, int(bool(accumulate))))

    def MatMulNN(self, a, b, y, M, K, N_, accumulate=False):
        self._matmul(N.lib().fh_op_matmul_nn, a, b, y, 1, M, K, N_, accumulate)

    def MatMulNT(self, a, b, y, M, K, N_, accumulate=False):
        self._matmul(N.lib().fh_op_matmul_nt, a, b, y, 1, M, K, N_, accumulate)

    def MatMulTN(self, a, b, y, M, K, N_, accumulate=False):
        self._matmul(N.lib().fh_op_matmul_tn, a, b, y, 1, M, K, N_, accumulate)

    def BatchedMatMulNN(self, a, b, y, slots, M, K, N_, accumulate=False):
        self._matmul(N.lib().fh_op_matmul_nn, a, b, y, slots, M, K, N_, accumulate)

    def BatchedMatMulNT(self, a, b, y, slots, M, K, N_, accumulate=False):
        self._matmul(N.lib().fh_op_matmul_nt, a, b, y, slots, M, K, N_, accumulate)

    def BatchedMatMulTN(self, a, b, y, slots, M, K, N_, accumulate=False):
        self._matmul(N.lib().fh_op_matmul_tn, a, b, y, slots, M, K, N_, accumulate)

    # ---- head packing ----------------------------------------------------------------
    def PackHeads(self, src, dst, batch, T, nHeads, headDim, colBase):
        ps = self._read(src)
        N.check(N.lib().fh_op_pack_heads(self._ctx, ps, src.Cols, self._write(dst), batch, T, nHeads, headDim,
                                         colBase))

    def UnpackHeads(self, src, dst, batch, T, nHeads, headDim, colBase):
        ps = self._read(src)
        N.check(N.lib().fh_op_unpack_heads(self._ctx, ps, self._write(dst, preserve=True), dst.Cols, batch, T,
                                           nHeads, headDim, colBase))

    def PackQkvHeads(self, src, q, k, v, batch, T, nHeads, headDim):
        """ITensorBackend.cs:58-65."""
        d = nHeads * headDim
        self.PackHeads(src, q, batch, T, nHeads, headDim, 0)
        self.PackHeads(src, k, batch, T, nHeads, headDim, d)
        self.PackHeads(src, v, batch, T, nHeads, headDim, 2 * d)

    def UnpackQkvHeads(self, q, k, v, dst, batch, T, nHeads, headDim):
        """ITensorBackend.cs:68-76."""
        d = nHeads * headDim
        self.Zero(dst)
        self.UnpackHeads(q, dst, batch, T, nHeads, headDim, 0)
        self.UnpackHeads(k, dst, batch, T, nHeads, headDim, d)
        self.UnpackHeads(v, dst, batch, T, nHeads, headDim, 2 * d)

    # ---- elementwise / rows ------------------------------------------------------------
    def AddBias(self, y, bias, rows, cols):
        pb = self._read(bias)
        N.check(N.lib().fh_op_add_bias(self._ctx, self._write(y, preserve=True), pb, rows, cols))

    def SumRows(self, dY, dBias, rows, cols):
        pd = self._read(dY)
        N.check(N.lib().fh_op_sum_rows(self._ctx, pd, self._write(dBias, preserve=True), rows, cols))

    def AddInPlace(self, dst, src):
        if dst.Length != src.Length:
            raise ValueError("AddInPlace needs equal lengths")
        ps = self._read(src)
        N.check(N.lib().fh_op_add_in_place(self._ctx, self._write(dst, preserve=True), ps, dst.Length))

    def Copy(self, src, dst):
        if dst.Length != src.Length:
            raise ValueError("Copy needs equal lengths")
        ps = self._read(src)
        N.check(N.lib().fh_op_copy(self._ctx, ps, self._write(dst), src.Length))

    def CopyBlock(self, src, dst, srcRow, srcCol, dstRow, dstCol, rows, cols):
        if (srcRow + rows) * src.Cols > src.Length or (dstRow + rows) * dst.Cols > dst.Length:
            raise ValueError("block rows outside a tensor")
        ps = self._read(src)
        N.check(N.lib().fh_op_copy_block(self._ctx, ps, src.Cols, self._write(dst, preserve=True), dst.Cols, srcRow,
                                         srcCol, dstRow, dstCol, rows, cols))

    def Scale(self, x, factor):
        N.check(N.lib().fh_op_scale(self._ctx, self._write(x, preserve=True), x.Length, float(factor)))

    def Transpose(self, x, output, rows, cols):
        px = self._read(x)
        N.check(N.lib().fh_op_transpose(self._ctx, px, self._write(output), rows, cols))

    # ---- LayerNorm / softmax / GELU ---------------------------------------------------------
    def LayerNormForward(self, x, w, b, output, mean, rstd, rows, cols, eps):
        px, pw, pb = self._read(x), self._read(w), self._read(b)
        N.check(N.lib().fh_op_layernorm_forward(self._ctx, px, pw, pb, self._write(output), self._write(mean),
                                                self._write(rstd), rows, cols, float(eps)))

    def LayerNormBackward(self, dOut, x, w, mean, rstd, dX, dW, dB, rows, cols):
        pd, px, pw, pm, pr = (self._read(t) for t in (dOut, x, w, mean, rstd))
        N.check(N.lib().fh_op_layernorm_backward(self._ctx, pd, px, pw, pm, pr, self._write(dX),
                                                 self._write(dW, preserve=True), self._write(dB, preserve=True),
                                                 rows, cols))

    def SoftmaxForward(self, x, rows, cols):
        N.check(N.lib().fh_op_softmax_forward(self._ctx, self._write(x, preserve=True), rows, cols))

    def SoftmaxBackward(self, dOut, softmaxOut, dX, rows, cols):
        pd, ps = self._read(dOut), self._read(softmaxOut)
        N.check(N.lib().fh_op_softmax_backward(self._ctx, pd, ps, self._write(dX), rows, cols, 1.0))

    def ScaledCausalSoftmaxForward(self, scores, rows, T, scale):
        N.check(N.lib().fh_op_scaled_causal_softmax_forward(self._ctx, self._write(scores, preserve=True), rows, T,
                                                            float(scale)))

    def ScaledSoftmaxBackward(self, dOut, softmaxOut, dX, rows, cols, scale):
        pd, ps = self._read(dOut), self._read(softmaxOut)
        N.check(N.lib().fh_op_softmax_backward(self._ctx, pd, ps, self._write(dX), rows, cols, float(scale)))

    def GeluForward(self, x, output):
        px = self._read(x)
        N.check(N.lib().fh_op_gelu_forward(self._ctx, px, self._write(output), x.Length))

    def GeluBackward(self, dOut, x, dX):
        pd, px = self._read(dOut), self._read(x)
        N.check(N.lib().fh_op_gelu_backward(self._ctx, pd, px, self._write(dX), x.Length))

    # ---- embedding / mask -----------------------------------------------------------------
    @staticmethod
    def _ints(a: Sequence[int]) -> np.ndarray:
        return np.ascontiguousarray(np.asarray(a, dtype=np.int32).reshape(-1))

    def EmbeddingForward(self, table, indices, output, D):
        idx = self._ints(indices)
        pt = self._read(table)
        N.check(N.lib().fh_op_embedding_forward(self._ctx, pt, table.Length // D, idx.ctypes.data, idx.size,
                                                self._write(output), D))

    def EmbeddingBackward(self, dOut, indices, dTable, D):
        idx = self._ints(indices)
        pd = self._read(dOut)
        N.check(N.lib().fh_op_embedding_backward(self._ctx, pd, idx.ctypes.data, idx.size,
                                                 self._write(dTable, preserve=True), dTable.Length // D, D))

    def CausalMask(self, scores, T):
        N.check(N.lib().fh_op_causal_mask(self._ctx, self._write(scores, preserve=True), scores.Length, T))

    # ---- cross-entropy ------------------------------------------------------------------------
    def CrossEntropyForward(self, logits, targets, probs, T, V, ignoreIndex) -> float:
        tg = self._ints(targets)
        pl = self._read(logits)
        pp = self._write(probs, preserve=probs is logits)
        loss = ctypes.c_float()
        N.check(N.lib().fh_op_cross_entropy_forward(self._ctx, pl, tg.ctypes.data, pp, T, V, ignoreIndex,
                                                    ctypes.byref(loss)))
        return float(loss.value)

    def BeginLossAccumulation(self) -> None:
        N.check(N.lib().fh_op_begin_loss_accumulation(self._ctx))

    def EndLossAccumulation(self) -> float:
        out = ctypes.c_float()
        N.check(N.lib().fh_op_end_loss_accumulation(self._ctx, ctypes.byref(out)))
        return float(out.value)

    def CrossEntropyBackward(self, probs, targets, dLogits, T, V, ignoreIndex):
        tg = self._ints(targets)
        pp = self._read(probs)
        pd = self._write(dLogits, preserve=dLogits is probs)
        N.check(N.lib().fh_op_cross_entropy_backward(self._ctx, pp, tg.ctypes.data, pd, T, V, ignoreIndex))

    # ---- reductions, optimizer, housekeeping -----------------------------------------------------
    def Zero(self, t):
        """Zeroes host and device copies (CudaBackend.Zero, CudaBackend.cs:600-609)."""
        t.Zero()
        N.check(N.lib().fh_op_zero(self._ctx, self._write(t), t.Length))
        t.DeviceResource.host_stale = False

    def SumSquares(self, t) -> float:
        out = ctypes.c_double()
        N.check(N.lib().fh_op_sum_squares(self._ctx, self._read(t), t.Length, ctypes.byref(out)))
        return float(out.value)

    def GlobalSumSquares(self, tensors) -> float:
        tensors = list(tensors)
        if not tensors:
            return 0.0
        ptrs = (ctypes.c_void_p * len(tensors))(*[self._read(t).value for t in tensors])
        sizes = (ctypes.c_int64 * len(tensors))(*[t.Length for t in tensors])
        out = ctypes.c_double()
        N.check(N.lib().fh_op_global_sum_squares(self._ctx, ptrs, sizes, len(tensors), ctypes.byref(out)))
        return float(out.value)

    def AdamWStep(self, w, g, m, v, lr, beta1, beta2, eps, weightDecay, step):
        pg = self._read(g)
        N.check(N.lib().fh_op_adamw_step(self._ctx, self._write(w, preserve=True), pg, self._write(m, preserve=True),
                                         self._write(v, preserve=True), w.Length, float(lr), float(beta1),
                                         float(beta2), float(eps), float(weightDecay), int(step), int(w.Rank > 1)))

    def DumpStats(self, tag: str) -> None:
        pass

    def Dispose(self) -> None:
        self._free = None
        for buf in self._all:
            buf.free()
        self._all = []
        if self._owns and self.backend is not None:
            self.backend.dispose()
        self.backend = None
