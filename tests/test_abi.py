"""C ABI surface of libforge_hip.so and the host-side mirror, without a GPU."""
import ctypes
import os
import re

import numpy as np
import pytest

from conftest import ROOT


def header_symbols():
    text = open(os.path.join(ROOT, "include", "forge_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fh_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(fhp):
    lib = fhp.lib()
    syms = header_symbols()
    assert len(syms) >= 17
    for s in syms:
        assert hasattr(lib, s), f"{s} declared in include/forge_hip.h but not exported"
    assert sorted(fhp._native.EXPORTS) == syms


def test_no_gpu_reports_error_instead_of_crashing(fhp):
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU driver is present")
    with pytest.raises(fhp.HipError):
        fhp.HipBackend(0)


def test_random_doubles_match_oracle_and_published_values(fhp, oracle):
    # library and oracle restate System.Random independently
    for seed in (0, 1, 42, -7, 2**31 - 1, -2**31):
        np.testing.assert_array_equal(fhp.Random(seed).next_doubles(500), oracle.net_random_doubles(seed, 500))
    # published outputs of the seeded .NET generator: new Random(1).Next() x3 and
    # new Random(0).NextDouble() (Next() = InternalSample, NextDouble = sample/int.MaxValue)
    r1 = fhp.Random(1).next_doubles(3)
    assert [int(round(x * 2147483647)) for x in r1] == [534011718, 237820880, 1002897798]
    assert abs(fhp.Random(0).next_double() - 0.7262432699679598) < 1e-15


def test_param_count_and_registry(fhp, oracle):
    for shape in [(32, 8, 16, 2, 2), (16384, 1024, 768, 12, 12), (16384, 1024, 1024, 16, 16)]:
        c = fhp.ModelConfig(*shape)
        reg = fhp.registry(c)
        assert sum(n for _, n in reg) == c.parameter_count() == oracle.param_count(oracle.Config(*shape))
    names = [n for n, _ in fhp.registry(fhp.ModelConfig(32, 8, 16, 2, 2))]
    assert names[:4] == ["tok_emb", "pos_emb", "blocks.0.ln1.w", "blocks.0.ln1.b"]
    assert names[-2:] == ["ln_f.w", "ln_f.b"] and len(names) == 2 + 2 * 12 + 2
    assert fhp.ModelConfig(16384, 1024, 768, 12, 12).parameter_count() == 98_425_344
    assert fhp.ModelConfig(16384, 1024, 1024, 16, 16).parameter_count() == 219_367_424


def test_param_info_rejects_bad_shapes(fhp):
    from forge_hip import _native as N
    L = fhp.lib()
    bad = N.ModelDesc(32, 8, 15, 2, 2, 1, 0, 0)  # DModel not divisible by NHeads
    assert L.fh_param_count(ctypes.byref(bad)) == -1
    assert "divisible" in N.last_error()
    big = N.ModelDesc(32, 8, 2048, 2, 16, 1, 0, 0)
    assert L.fh_param_count(ctypes.byref(big)) == -1


def test_model_config_validation(fhp):
    with pytest.raises(ValueError, match="divisible"):
        fhp.ModelConfig(32, 8, 15, 2, 2)
    with pytest.raises(ValueError, match="VocabSize"):
        fhp.ModelConfig(0, 8, 16, 2, 2)
    assert fhp.ModelConfig(32, 8, 16, 2, 2).head_dim == 8
    assert fhp.get_preset("FORGE-98M").parameter_count(16257) == 97_934_592
    with pytest.raises(ValueError, match="Unknown model preset"):
        fhp.get_preset("forge-nope")


def test_backend_selection_semantics(fhp):
    # BackendSelectionTests.cs:8-56, with `hip` first in the auto order
    BS = fhp.BackendSelection
    probes = []

    def factory_all_fail_but_cpu(name):
        probes.append(name)
        if name != "cpu":
            raise RuntimeError(f"{name} unavailable")
        return "CPU"

    skipped = []
    assert BS.create("auto", False, factory_all_fail_but_cpu, lambda c, e: skipped.append(c)) == ("cpu", "CPU")
    assert probes == ["hip", "cuda", "cpu"] and skipped == ["hip", "cuda"]
    probes.clear()
    assert BS.create("AUTO", True, factory_all_fail_but_cpu)[0] == "cpu"
    assert probes == ["hip", "cuda", "gpu", "cpu"]
    assert BS.create("auto", False, lambda n: n.upper()) == ("hip", "HIP")
    with pytest.raises(RuntimeError):  # explicit choices fail loudly
        BS.create("hip", False, factory_all_fail_but_cpu)
    with pytest.raises(ValueError, match="unknown backend"):
        BS.create("metal", False, factory_all_fail_but_cpu)


def test_generate_validation_before_device_work(fhp):
    class Stub:  # validation runs before any device call
        config = fhp.ModelConfig(32, 8, 16, 2, 2)
        handle = None
    S = fhp.Sampler
    with pytest.raises(ValueError, match="prompt"):
        S.generate(Stub(), [], 1, 1.0, 0, fhp.Random(1))
    with pytest.raises(ValueError, match="maxNewTokens"):
        S.generate(Stub(), [1], -1, 1.0, 0, fhp.Random(1))
    with pytest.raises(ValueError, match="penalty"):
        S.generate(Stub(), [1], 1, 1.0, 0, fhp.Random(1), repetition_penalty=0.9)
    with pytest.raises(ValueError, match="n-gram"):
        S.generate(Stub(), [1], 1, 1.0, 0, fhp.Random(1), no_repeat_ngram_size=-1)
    with pytest.raises(ValueError, match="EOS"):
        S.generate(Stub(), [1], 1, 1.0, 0, fhp.Random(1), eos_id=32)
    with pytest.raises(ValueError, match="Temperature"):
        S.generate(Stub(), [1], 1, float("nan"), 0, fhp.Random(1))


def test_op_entry_points_reject_a_null_context(fhp):
    # every fh_op_* validates its context before touching a device
    import ctypes as C
    L = fhp.lib()
    buf = (C.c_float * 4)()
    loss, dbl = C.c_float(), C.c_double()
    calls = [
        lambda: L.fh_op_matmul_nn(None, buf, buf, buf, 1, 1, 1, 1, 0),
        lambda: L.fh_op_scale(None, buf, 4, 2.0),
        lambda: L.fh_op_zero(None, buf, 4),
        lambda: L.fh_op_layernorm_forward(None, buf, buf, buf, buf, buf, buf, 1, 4, 1e-5),
        lambda: L.fh_op_cross_entropy_forward(None, buf, (C.c_int32 * 1)(0), buf, 1, 4, -1, C.byref(loss)),
        lambda: L.fh_op_begin_loss_accumulation(None),
        lambda: L.fh_op_sum_squares(None, buf, 4, C.byref(dbl)),
        lambda: L.fh_op_adamw_step(None, buf, buf, buf, buf, 4, 1e-3, 0.9, 0.95, 1e-8, 0.1, 1, 1),
    ]
    for call in calls:
        assert call() == fhp._native.FH_ERR_INVALID
        assert "null context" in fhp._native.last_error()


def test_init_weights_rejects_a_wrong_size(fhp):
    import ctypes as C
    cfg = fhp.ModelConfig(32, 8, 16, 2, 2)
    desc = fhp.model._desc(cfg, 1, "f32")
    w = np.empty(10, np.float32)
    assert fhp.lib().fh_init_weights(C.byref(desc), 1, w.ctypes.data, 10) == fhp._native.FH_ERR_INVALID
    assert "registry holds" in fhp._native.last_error()
