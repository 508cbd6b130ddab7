"""Host-side initial weights and the parameter registry (CPU only).

fh_init_weights draws the GptModel constructor's initial weights from
new Random(seed) (src/LLM.Core/Model/GptModel.cs:38-99, Tensor.FillNormal
Tensor.cs:79-91) into a host array; they equal the oracle's bit for bit.  The
registry (fh_param_info) has the reference's names, order and sizes
(GptModel.cs:53-91).
"""
import ctypes

import numpy as np
import pytest

TINY = (12, 6, 8, 1, 2)  # GpuBackendTests.Tiny


@pytest.mark.parametrize("shape,seed", [(TINY, 42), ((32, 8, 16, 2, 2), 7), ((2256, 128, 128, 4, 4), 1234)])
def test_init_weights_match_oracle(fhp, oracle, shape, seed):
    cfg = fhp.ModelConfig(*shape)
    n = sum(k for _, k in fhp.registry(cfg))
    w = np.empty(n, np.float32)
    desc = fhp.model._desc(cfg, 1, "f32")
    fhp._native.check(fhp.lib().fh_init_weights(ctypes.byref(desc), seed, w.ctypes.data, n))
    np.testing.assert_array_equal(w.view(np.uint32), oracle.init_weights(oracle.Config(*shape), seed).view(np.uint32))


def test_registry_names_and_sizes(fhp):
    # GptModel.cs:53-91: tok_emb [V,d], pos_emb [ctx,d], per block ln1, attn.qkv [d,3d],
    # attn.proj [d,d], ln2, mlp.fc [d,4d], mlp.proj [4d,d] (weights then biases), ln_f
    V, ctx, d, L, H = TINY
    reg = fhp.registry(fhp.ModelConfig(*TINY))
    want = [("tok_emb", V * d), ("pos_emb", ctx * d)]
    for i in range(L):
        p = f"blocks.{i}."
        want += [(p + "ln1.w", d), (p + "ln1.b", d), (p + "attn.qkv.w", d * 3 * d), (p + "attn.qkv.b", 3 * d),
                 (p + "attn.proj.w", d * d), (p + "attn.proj.b", d), (p + "ln2.w", d), (p + "ln2.b", d),
                 (p + "mlp.fc.w", d * 4 * d), (p + "mlp.fc.b", 4 * d), (p + "mlp.proj.w", 4 * d * d),
                 (p + "mlp.proj.b", d)]
    want += [("ln_f.w", d), ("ln_f.b", d)]
    assert reg == want
