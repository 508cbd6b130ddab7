"""FORGEMODEL1 checkpoint ingest (Checkpoint.Load, src/LLM.Core/Checkpoint/Checkpoint.cs:116-250).

CPU tests: the library's SHA-256 against hashlib, and header / payload / checksum
validation through fh_checkpoint_info (no GPU needed), including the reference's
own checkpoint tests (tests/LLM.Core.Tests/CheckpointTests.cs: bad magic, truncated
payload, same-size corruption caught by the checksum).  The GPU test loads a
checkpoint into a session and compares its logits with the same weights loaded
directly and with the oracle.
"""
import ctypes
import hashlib
import json
import os
import struct

import numpy as np
import pytest

ARCH = "forge-gpt2-tied-v1"


def training_header(has_moments=False):
    # Checkpoint.TrainingHeader, property order as declared (Checkpoint.cs:35-58)
    return {"GlobalStep": 2, "AdamStep": 2 if has_moments else 0, "SamplerRandomState": 1, "SamplerRandomIncrement": 3,
            "SamplerEpoch": 0, "SamplerCursor": 0, "SamplerStart": 0, "SamplerStride": 8, "SamplerChunkCount": 4,
            "SamplerContextLength": 8, "HasOptimizerState": has_moments, "TotalSteps": 2, "MaxLr": 0.001,
            "MinLr": 0.0001, "WarmupSteps": 1, "WeightDecay": 0.1, "GradClip": 1.0, "BatchSize": 1,
            "AccumulationSteps": 1, "TrainingContextLength": 8, "DataIdentity": "data",
            "TokenizerIdentity": "tokenizer"}


def write_checkpoint(path, cfg, names, weights, name="Forge-Test", arch=ARCH, training=True, moments=None,
                     header_override=None):
    """A FORGEMODEL1 file as Checkpoint.WriteHeaderAndWeights lays it out (Checkpoint.cs:143-166):
    magic, int32 JSON length, the Header JSON (System.Text.Json defaults: declared order,
    PascalCase, compact), registry-order fp32, optional Adam M/V per tensor, SHA-256."""
    hdr = {"VocabSize": cfg[0], "ContextLength": cfg[1], "DModel": cfg[2], "NLayers": cfg[3], "NHeads": cfg[4],
           "ModelName": name, "Architecture": arch, "Names": list(names),
           "Training": training_header(moments is not None) if training else None}
    if header_override:
        hdr.update(header_override)
    js = json.dumps(hdr, separators=(",", ":")).encode()
    body = b"FORGEMODEL1" + struct.pack("<i", len(js)) + js + np.ascontiguousarray(weights, "<f4").tobytes()
    if moments is not None:
        body += np.ascontiguousarray(moments, "<f4").tobytes()
    with open(path, "wb") as f:
        f.write(body + hashlib.sha256(body).digest())


SMALL = (32, 8, 16, 2, 2)  # CheckpointTests.Small


@pytest.fixture
def small(fhp, tmp_path):
    cfg = fhp.ModelConfig(*SMALL)
    reg = fhp.registry(cfg)
    names = [n for n, _ in reg]
    total = sum(n for _, n in reg)
    w = np.random.default_rng(42).standard_normal(total).astype(np.float32) * 0.02
    return cfg, names, w, tmp_path


@pytest.mark.parametrize("n", [0, 1, 3, 55, 56, 57, 63, 64, 65, 127, 128, 1000, 1 << 16])
def test_sha256_matches_hashlib(fhp, n):
    data = np.random.default_rng(n).integers(0, 256, n, dtype=np.uint8).tobytes()
    out = (ctypes.c_uint8 * 32)()
    buf = ctypes.create_string_buffer(data, max(n, 1))
    fhp._native.check(fhp.lib().fh_sha256(buf, n, out))
    assert bytes(out) == hashlib.sha256(data).digest()


def test_header_round_trip_and_verify(fhp, small):
    cfg, names, w, tmp = small
    p = str(tmp / "m.forge")
    write_checkpoint(p, SMALL, names, w, name="Forge-Test")
    got, name = fhp.Checkpoint.read_config(p, verify=True)
    assert (got.vocab_size, got.context_length, got.d_model, got.n_layers, got.n_heads) == SMALL
    assert name == "Forge-Test"


def test_training_checkpoint_with_moments_verifies(fhp, small):
    cfg, names, w, tmp = small
    p = str(tmp / "m.forge")
    moments = np.random.default_rng(1).standard_normal(2 * w.size).astype(np.float32)
    write_checkpoint(p, SMALL, names, w, moments=moments)
    fhp.Checkpoint.read_config(p, verify=True)


def test_bad_magic_throws(fhp, tmp_path):
    # CheckpointTests.Load_BadMagicThrows
    p = str(tmp_path / "bad.forge")
    open(p, "wb").write(b"NOTACHECKPOINT!")
    with pytest.raises(fhp.InvalidDataError, match="is not a current FORGEMODEL1 checkpoint"):
        fhp.Checkpoint.read_config(p)


def test_truncated_payload_throws(fhp, small):
    # CheckpointTests.Load_TruncatedPayloadThrows: 4 bytes chopped
    cfg, names, w, tmp = small
    p = str(tmp / "m.forge")
    write_checkpoint(p, SMALL, names, w)
    data = open(p, "rb").read()
    open(p, "wb").write(data[:-4])
    with pytest.raises(fhp.InvalidDataError, match="Checkpoint payload is"):
        fhp.Checkpoint.read_config(p)


def test_same_size_corruption_fails_checksum(fhp, small):
    # CheckpointTests.TrainingCheckpoint_SameSizeCorruptionFailsChecksum: the last payload byte flipped
    cfg, names, w, tmp = small
    p = str(tmp / "m.forge")
    write_checkpoint(p, SMALL, names, w)
    data = bytearray(open(p, "rb").read())
    data[-33] ^= 1
    open(p, "wb").write(bytes(data))
    fhp.Checkpoint.read_config(p, verify=False)  # the header alone is still valid
    with pytest.raises(fhp.InvalidDataError, match="checksum"):
        fhp.Checkpoint.read_config(p, verify=True)


@pytest.mark.parametrize("kind,msg", [
    ("arch", "Unsupported checkpoint architecture 'gpt-neox'"),
    ("name", "missing its Forge model name"),
    ("training", "missing its training-state header"),
    ("names", "parameter names do not match the model registry"),
    ("short", "too short to contain its checksum"),
    ("hdrlen", "Implausible header length"),
    ("json", "header failed to parse"),
])
def test_load_core_rejections(fhp, small, kind, msg):
    cfg, names, w, tmp = small
    p = str(tmp / "m.forge")
    if kind == "arch":
        write_checkpoint(p, SMALL, names, w, arch="gpt-neox")
    elif kind == "name":
        write_checkpoint(p, SMALL, names, w, name="   ")
    elif kind == "training":
        write_checkpoint(p, SMALL, names, w, training=False)
    elif kind == "names":
        bad = list(names)
        bad[2], bad[3] = bad[3], bad[2]
        write_checkpoint(p, SMALL, bad, w)
    elif kind == "short":
        open(p, "wb").write(b"FORGEMODEL1" + b"\0" * 20)
    elif kind == "hdrlen":
        body = b"FORGEMODEL1" + struct.pack("<i", -5) + b"\0" * 64
        open(p, "wb").write(body + hashlib.sha256(body).digest())
    else:
        js = b'{"VocabSize":32,'
        body = b"FORGEMODEL1" + struct.pack("<i", len(js)) + js
        open(p, "wb").write(body + hashlib.sha256(body).digest())
    with pytest.raises(fhp.InvalidDataError, match=msg):
        fhp.Checkpoint.read_config(p)


def test_invalid_model_config_is_an_argument_error(fhp, small):
    cfg, names, w, tmp = small
    p = str(tmp / "m.forge")
    write_checkpoint(p, SMALL, names, w, header_override={"DModel": 15})
    with pytest.raises(fhp.ArgumentError, match="must be divisible by NHeads"):
        fhp.Checkpoint.read_config(p)


def test_missing_file_is_an_argument_error(fhp, tmp_path):
    with pytest.raises(fhp.ArgumentError, match="Could not find file"):
        fhp.Checkpoint.read_config(str(tmp_path / "none.forge"))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_checkpoint_loads_into_a_session(fhp, oracle, tmp_path, dtype):
    # CheckpointTests.RoundTrip_BitwiseEqualWeightsAndLogits through the HIP session:
    # the loaded weights read back bit for bit (bf16: as the direct load rounds them)
    # and ForwardLast matches the directly loaded session exactly and the oracle
    # within the fp32 / bf16 bars
    shape = (2256, 128, 128, 4, 4)
    ocfg = oracle.Config(*shape)
    # trained-like: LayerNorm and bias vectors away from their initial 1 / 0
    w = oracle.trained_like(ocfg, oracle.init_weights(ocfg, 1234), 77)
    be = fhp.HipBackend(0)
    cfg = fhp.ModelConfig(*shape)
    names = [n for n, _ in fhp.registry(cfg)]
    p = str(tmp_path / "c1.forge")
    write_checkpoint(p, shape, names, w, name="Forge-C1",
                     moments=np.zeros(2 * w.size, np.float32))
    m = fhp.Checkpoint.load(p, be, dtype=dtype)
    assert m.name == "Forge-C1"
    direct = fhp.GptModel(cfg, be, dtype=dtype)
    direct.load_weights(w)
    assert np.array_equal(m.read_weights().view(np.uint32), direct.read_weights().view(np.uint32))
    ids = fhp.TrainingRandom(42).ids(shape[0], 16)
    a = m.forward_last(ids)
    b = direct.forward_last(ids)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    if dtype == "f32":
        ref = oracle.forward(ocfg, w, ids)[-1]
        assert np.max(np.abs(a[0] - ref) / np.maximum(1.0, np.abs(ref))) <= 1e-4
    # a corrupted file leaves no session behind and raises the data error
    data = bytearray(open(p, "rb").read())
    data[len(data) // 2] ^= 0x10
    open(p, "wb").write(bytes(data))
    with pytest.raises(fhp.InvalidDataError, match="checksum"):
        fhp.Checkpoint.load(p, be, dtype=dtype)
    m.dispose()
    direct.dispose()
    be.dispose()


@pytest.mark.gpu
def test_checkpoint_of_released_shape_decodes_on_the_fused_step(fhp, oracle, tmp_path):
    # a FORGEMODEL1 file of the released Forge-98M configuration (V 16257, ctx 512,
    # MODEL_CARD.md:16-17) with trained-like parameters: loaded through
    # fh_session_load_checkpoint, which also builds the fused decode step's tiles
    # from it, then 48 greedy ids in one fused launch equal the oracle's
    shape = (16257, 512, 768, 12, 12)
    ocfg = oracle.Config(*shape)
    w = oracle.trained_like(ocfg, oracle.init_weights(ocfg, 5), 6)
    be = fhp.HipBackend(0)
    names = [n for n, _ in fhp.registry(fhp.ModelConfig(*shape))]
    p = str(tmp_path / "forge98m.forge")
    write_checkpoint(p, shape, names, w, name="Forge-98M")
    m = fhp.Checkpoint.load(p, be)
    prompt = fhp.TrainingRandom(42).ids(shape[0], 64)
    ids = fhp.Sampler.generate(m, prompt, 48, 0.0, 0, None)
    assert fhp.Sampler.last_timing["route"] == fhp._native.FH_ROUTE_FUSED_STEP
    oracle.set_threads(8)
    np.testing.assert_array_equal(ids, oracle.generate(ocfg, w, prompt, 48))
    m.dispose()
    be.dispose()
