"""Training through the hip backend: the reference's model layers (Layers.cs), the
training half of GptModel and AdamW over HipTensorBackend (forge_hip.training).

CPU: the host-side initial weights (fh_init_weights, the GptModel constructor's draw
from new Random(seed)) equal the oracle's bit for bit, and the parameter registry has
the reference's shapes and count.  GPU: the model-level tests of the reference's
device-backend contract (GpuBackendTests.cs:602-720): full-model forward against the
oracle, a batched finite-difference gradient check of every parameter, and a small
batch that overfits under SGD; plus the same batch under AdamW with device-resident
moments (BatchedModelTests.cs:243-273).
"""
import numpy as np
import pytest

TINY = (12, 6, 8, 1, 2)  # GpuBackendTests.Tiny


@pytest.mark.parametrize("shape,seed", [(TINY, 42), ((32, 8, 16, 2, 2), 7), ((2256, 128, 128, 4, 4), 1234)])
def test_init_weights_match_oracle(fhp, oracle, shape, seed):
    cfg = fhp.ModelConfig(*shape)
    n = sum(k for _, k in fhp.registry(cfg))
    w = np.empty(n, np.float32)
    desc = fhp.model._desc(cfg, 1, "f32")
    import ctypes
    fhp._native.check(fhp.lib().fh_init_weights(ctypes.byref(desc), seed, w.ctypes.data, n))
    np.testing.assert_array_equal(w.view(np.uint32), oracle.init_weights(oracle.Config(*shape), seed).view(np.uint32))


def test_parameter_shapes(fhp):
    # GptModel.cs:53-91 registration: matrices are [in, out], the tied table [V, d]
    class NoBackend:
        def InvalidateDeviceCache(self, t):
            pass
    m = fhp.TrainableGptModel(fhp.ModelConfig(*TINY), NoBackend(), seed=1)
    P = m.Params
    assert P.Weight("tok_emb").Shape == (12, 8) and P.Weight("pos_emb").Shape == (6, 8)
    assert P.Weight("blocks.0.attn.qkv.w").Shape == (8, 24)
    assert P.Weight("blocks.0.mlp.fc.w").Shape == (8, 32)
    assert P.Weight("blocks.0.mlp.proj.w").Shape == (32, 8)
    assert P.Weight("blocks.0.ln1.w").Shape == (8,) and np.all(P.Weight("blocks.0.ln1.w").Data == 1)
    assert P.Count == sum(k for _, k in fhp.registry(fhp.ModelConfig(*TINY)))
    assert P.Names[-2:] == ["ln_f.w", "ln_f.b"]


@pytest.fixture(scope="module")
def tb(fhp):
    b = fhp.HipTensorBackend(0)
    yield b
    b.Dispose()


@pytest.mark.gpu
def test_model_forward_matches_oracle(fhp, oracle, tb):
    # GpuBackendTests.Model_ForwardMatchesCpu (1e-3), and a 2-layer 128-wide model
    for shape, seed, toks in [(TINY, 42, [3, 1, 4, 1, 5, 2]), ((512, 64, 128, 2, 4), 9, list(range(0, 400, 7)))]:
        m = fhp.TrainableGptModel(fhp.ModelConfig(*shape), tb, seed=seed)
        got = m.Forward(toks)
        ref = oracle.forward(oracle.Config(*shape), oracle.init_weights(oracle.Config(*shape), seed), toks)
        err = np.abs(got.Data.reshape(ref.shape) - ref) / np.maximum(1.0, np.abs(ref))
        assert err.max() <= 1e-3, (shape, err.max())


@pytest.mark.gpu
def test_model_gradient_check_batched(fhp, tb):
    # GpuBackendTests.Model_GradientCheck_Batched: every parameter, eps 1e-3, tol 2e-2
    m = fhp.TrainableGptModel(fhp.ModelConfig(*TINY), tb, seed=123)
    inputs = [1, 2, 3, 4, 0, 5, 5, 4, 3, 2, 1, 0]
    targets = [2, 3, 4, 5, 1, 0, 4, 3, 2, 1, 0, 5]
    eps, tol = 1e-3, 2e-2
    m.Params.ZeroGrads()
    loss = m.ForwardBackward(inputs, targets, 2)
    assert loss > 0 and np.isfinite(loss)
    analytic = {}
    for n in m.Params.Names:
        g = m.Params.Grad(n)
        tb.EnsureHostCurrent(g)
        analytic[n] = g.Data.copy()
    worst, where = 0.0, ""
    for n in m.Params.Names:
        w = m.Params.Weight(n)
        for i in range(w.Length):
            orig = w.Data[i]
            w.Data[i] = orig + np.float32(eps)
            tb.InvalidateDeviceCache(w)
            hi = m.ForwardBackward(inputs, targets, 2)
            w.Data[i] = orig - np.float32(eps)
            tb.InvalidateDeviceCache(w)
            lo = m.ForwardBackward(inputs, targets, 2)
            w.Data[i] = orig
            tb.InvalidateDeviceCache(w)
            num = (hi - lo) / (2 * eps)
            err = abs(num - analytic[n][i]) / max(1.0, abs(num))
            if err > worst:
                worst, where = err, f"{n}[{i}] numeric={num:.6g} analytic={analytic[n][i]:.6g}"
    print(f"batched grad-check max rel/abs err {worst:.4g} ({where})", flush=True)
    assert worst < tol, where


@pytest.mark.gpu
def test_overfit_small_batch_sgd_and_adamw(fhp, tb):
    # GpuBackendTests.Overfit_SmallBatchLossDrops (200 host SGD steps on device
    # gradients), then the same batch under AdamW with device moments
    inputs = [0, 1, 2, 3, 4, 5, 5, 4, 3, 2, 1, 0]
    targets = [1, 2, 3, 4, 5, 0, 4, 3, 2, 1, 0, 5]
    m = fhp.TrainableGptModel(fhp.ModelConfig(*TINY), tb, seed=5)
    m.Params.ZeroGrads()
    initial = m.ForwardBackward(inputs, targets, 2)
    for _ in range(200):
        m.Params.ZeroGrads()
        m.ForwardBackward(inputs, targets, 2)
        for n in m.Params.Names:
            w, g = m.Params.Weight(n), m.Params.Grad(n)
            tb.EnsureHostCurrent(g)
            tb.EnsureHostCurrent(w)
            w.Data -= np.float32(0.05) * g.Data
            tb.InvalidateDeviceCache(w)
    m.Params.ZeroGrads()
    final = m.ForwardBackward(inputs, targets, 2)
    print(f"SGD overfit loss {initial:.4f} -> {final:.4f}", flush=True)
    assert final < 0.2 * initial
    m2 = fhp.TrainableGptModel(fhp.ModelConfig(*TINY), tb, seed=5)
    opt = fhp.AdamW(tb)
    m2.Params.ZeroGrads()
    first = m2.ForwardBackward(inputs, targets, 2)
    for _ in range(100):
        m2.Params.ZeroGrads()
        m2.ForwardBackward(inputs, targets, 2)
        opt.Step(m2.Params, lr=0.01, weightDecay=0.0)
    m2.Params.ZeroGrads()
    last = m2.ForwardBackward(inputs, targets, 2)
    print(f"AdamW overfit loss {first:.4f} -> {last:.4f}", flush=True)
    assert opt.StepCount == 100 and last < 0.2 * first
