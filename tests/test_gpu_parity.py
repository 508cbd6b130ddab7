"""Parity of the HIP token loop with the CPU oracle, through the C ABI.

Bars: greedy token ids bit-identical; per-step logits
within rel/abs 1e-4 for fp32 (|a-e| <= tol*max(1,|e|), the reference's
GpuBackendTests.NearRel metric, tests/LLM.Core.Tests/GpuBackendTests.cs:83-102).

Most token-loop tests load "trained-like" parameters (oracle.trained_like): the
initial weights with every LayerNorm weight 1 + N(0, 0.1), LayerNorm bias
N(0, 0.05) and Linear bias N(0, 0.05).  At the initial values (1, 0, 0) the
LayerNorm affine and every bias add are exact no-ops, so an indexing mistake in
them would pass unseen; a trained checkpoint has neither.
"""
import os

import numpy as np
import pytest

from conftest import GOLDEN

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-4


def rel_err(a, e):
    a = np.asarray(a, np.float64)
    e = np.asarray(e, np.float64)
    return float(np.max(np.abs(a - e) / np.maximum(1.0, np.abs(e))))


@pytest.fixture(scope="module")
def backend(fhp):
    be = fhp.HipBackend(0)
    print(f"device: {be.device_name}, {be.compute_units} CUs", flush=True)
    yield be
    be.dispose()


def make_model(fhp, oracle, backend, shape, seed, batch=1, dtype="f32", trained=True):
    """A session and the oracle's copy of its parameters: the GptModel initial weights
    from new Random(seed), made trained-like unless trained=False."""
    cfg = fhp.ModelConfig(*shape)
    ocfg = oracle.Config(*shape)
    w = oracle.init_weights(ocfg, seed)
    if trained:
        w = oracle.trained_like(ocfg, w, seed + 1000)
    m = fhp.GptModel(cfg, backend, batch=batch, dtype=dtype)
    m.load_weights(w)
    return m, ocfg, w


def route(fhp):
    return fhp.Sampler.last_timing["route"]


def assert_greedy_parity(ids, lg, rids, rlg, tol, what=""):
    """Greedy ids equal and logits within tol at every step, except that a run may
    part at a near tie: at the first differing step both ids must be within 2 tol of
    the top of the oracle's logits (any fp32 summation order may pick either), and
    the steps after it are not compared.  Returns the number of agreeing steps."""
    ids, rids = np.asarray(ids), np.asarray(rids)
    n = min(len(ids), len(rids))
    diff = np.nonzero(ids[:n] != rids[:n])[0]
    same = int(diff[0]) if diff.size else n
    upto = min(n, same + 1)
    assert rel_err(lg[:upto], rlg[:upto]) <= tol, what
    if same < n:
        row = np.asarray(rlg[same], np.float64)
        top = row.max()
        gap = top - min(row[ids[same]], row[rids[same]])
        assert gap <= 2 * tol * max(1.0, abs(top)), f"{what}: ids part at step {same} with a margin of {gap:.3g}"
    return same


@pytest.mark.parametrize("prompt,steps", [([1, 2], 12), (list(np.arange(12) % 32), 6), ([3, 1], 1)])
def test_tiny_generate_with_slides(fhp, oracle, backend, prompt, steps):
    # InferenceTests.Small; the first case slides after 6 steps, the second starts past ctx
    m, oc, w = make_model(fhp, oracle, backend, (32, 8, 16, 2, 2), 8)
    ids, lg = fhp.Sampler.generate(m, prompt, steps, 0.0, 0, None, return_logits=True)
    rids, rlg = oracle.generate(oc, w, prompt, steps, return_logits=True)
    np.testing.assert_array_equal(ids, rids)
    assert rel_err(lg, rlg) <= TOL_F32
    m.dispose()


def test_forward_last_matches_golden(fhp, oracle, backend):
    g = np.load(os.path.join(GOLDEN, "tiny_forward.npz"))
    m, oc, w = make_model(fhp, oracle, backend, (32, 8, 16, 2, 2), 6, trained=False)
    out = m.forward_last(g["ids"])
    assert out.shape == (1, 32)
    assert rel_err(out[0], g["logits"][-1]) <= TOL_F32
    m.dispose()


def test_init_random_matches_oracle_bitwise(fhp, oracle, backend):
    shape = (2256, 128, 128, 4, 4)
    m = fhp.GptModel(fhp.ModelConfig(*shape), backend, seed=1234)
    np.testing.assert_array_equal(m.read_weights(), oracle.init_weights(oracle.Config(*shape), 1234))
    m.dispose()


def test_c1_greedy_matches_golden(fhp, oracle, backend):
    g = np.load(os.path.join(GOLDEN, "c1_greedy.npz"))
    m = fhp.GptModel(fhp.ModelConfig(2256, 128, 128, 4, 4), backend, seed=1234)
    ids, lg = fhp.Sampler.generate(m, g["prompt"], 200, 0.0, 0, None, return_logits=True)
    np.testing.assert_array_equal(ids, g["ids"])
    got_top = np.take_along_axis(lg, g["top5_ids"].astype(np.int64), axis=1)
    assert rel_err(got_top, g["top5_logits"]) <= TOL_F32
    assert rel_err(lg[g["full_steps"]], g["full_logits"]) <= TOL_F32
    t = fhp.Sampler.last_timing
    assert t["cached_steps"] == 112 and t["reprefill_steps"] == 87  # slide from step 113 on
    m.dispose()


@pytest.mark.parametrize("params", ["init", "trained"])
def test_c2_greedy_matches_oracle(fhp, oracle, backend, params):
    # Forge-98M shape, fp32, prompt 64 + 256 greedy, on the fused
    # decode step: 256 ids bit-identical, logits within 1e-4 at every step, and the
    # greedy run without a logits dump (the in-kernel argmax) gives the same ids
    shape = (16384, 1024, 768, 12, 12)
    m, oc, w = make_model(fhp, oracle, backend, shape, 1234, trained=params == "trained")
    prompt = fhp.TrainingRandom(42).ids(16384, 64)
    ids, lg = fhp.Sampler.generate(m, prompt, 256, 0.0, 0, None, return_logits=True)
    assert route(fhp) & fhp._native.FH_ROUTE_FUSED_STEP
    fast = fhp.Sampler.generate(m, prompt, 256, 0.0, 0, None)
    assert route(fhp) == fhp._native.FH_ROUTE_FUSED_STEP
    oracle.set_threads(8)
    rids, rlg = oracle.generate(oc, w, prompt, 256, return_logits=True)
    top2 = np.sort(rlg, axis=1)[:, -2:]
    print(f"min top-2 margin {float(np.min(top2[:, 1] - top2[:, 0])):.4g}", flush=True)
    np.testing.assert_array_equal(ids, rids)
    np.testing.assert_array_equal(fast, rids)
    err = rel_err(lg, rlg)
    print(f"max logit rel/abs err over 256 steps: {err:.3g}", flush=True)
    assert err <= TOL_F32
    m.dispose()


@pytest.mark.parametrize("params", ["init", "trained"])
def test_c2_generic_decode_path_matches_oracle(fhp, oracle, backend, monkeypatch, params):
    """The same workload on the generic multi-kernel decode path (fused step off)."""
    monkeypatch.setenv("FORGE_HIP_FUSED_DECODE", "0")
    shape = (16384, 1024, 768, 12, 12)
    m, oc, w = make_model(fhp, oracle, backend, shape, 99, trained=params == "trained")
    prompt = fhp.TrainingRandom(7).ids(16384, 48)
    ids, lg = fhp.Sampler.generate(m, prompt, 64, 0.0, 0, None, return_logits=True)
    assert route(fhp) & fhp._native.FH_ROUTE_FUSED_EPILOGUES and not route(fhp) & fhp._native.FH_ROUTE_FUSED_STEP
    rids, rlg = oracle.generate(oc, w, prompt, 64, return_logits=True)
    np.testing.assert_array_equal(ids, rids)
    assert rel_err(lg, rlg) <= TOL_F32
    m.dispose()


def test_fused_greedy_without_dump_matches_dump_run(fhp, oracle, backend):
    """Greedy without a logits dump takes the in-kernel argmax; ids equal the dumped run's."""
    shape = (16384, 1024, 768, 12, 12)
    m, oc, w = make_model(fhp, oracle, backend, shape, 5)
    prompt = fhp.TrainingRandom(11).ids(16384, 20)
    ids_fast = fhp.Sampler.generate(m, prompt, 64, 0.0, 0, None)
    ids_dump, _ = fhp.Sampler.generate(m, prompt, 64, 0.0, 0, None, return_logits=True)
    np.testing.assert_array_equal(ids_fast, ids_dump)
    np.testing.assert_array_equal(ids_fast, oracle.generate(oc, w, prompt, 64))
    m.dispose()


@pytest.mark.parametrize("V", [200, 512, 768, 2816, 16257])
def test_d768_vocab_sizes_greedy_matches_oracle(fhp, oracle, backend, V):
    """The fused step's head gives each of its 256 blocks ceil(V / 256) vocabulary
    rows: 200 leaves 56 blocks and some data waves without rows, 512 and 768 give
    2 and 3 rows, 2816 splits 11 rows unevenly over three data waves, and 16257 (the
    released Forge-98M vocabulary, MODEL_CARD.md:16) leaves the last block one row
    and the one before it a partial set.  With and without the logits dump."""
    shape = (V, 1024, 768, 2, 12)
    m, oc, w = make_model(fhp, oracle, backend, shape, 21)
    prompt = fhp.TrainingRandom(3).ids(V, 30)
    ids, lg = fhp.Sampler.generate(m, prompt, 40, 0.0, 0, None, return_logits=True)
    assert route(fhp) & fhp._native.FH_ROUTE_FUSED_STEP
    rids, rlg = oracle.generate(oc, w, prompt, 40, return_logits=True)
    np.testing.assert_array_equal(ids, rids)
    assert rel_err(lg, rlg) <= TOL_F32
    np.testing.assert_array_equal(fhp.Sampler.generate(m, prompt, 40, 0.0, 0, None), rids)
    assert route(fhp) == fhp._native.FH_ROUTE_FUSED_STEP
    m.dispose()


@pytest.mark.parametrize("P,new", [(64, 256), (480, 40)])
def test_forge98m_released_shape_matches_oracle(fhp, oracle, backend, P, new):
    """The reference's own Forge-98M configuration (V 16257, ctx 512, d 768, 12 layers,
    12 heads: MODEL_CARD.md:16-17, ModelPresets.cs:40-41) with trained-like parameters
    on the fused decode step.  The second case fills the 512-token context after 32
    cached steps; the rest re-prefill the slid window."""
    shape = (16257, 512, 768, 12, 12)
    m, oc, w = make_model(fhp, oracle, backend, shape, 98)
    prompt = fhp.TrainingRandom(42).ids(16257, P)
    fast = fhp.Sampler.generate(m, prompt, new, 0.0, 0, None)
    assert route(fhp) == fhp._native.FH_ROUTE_FUSED_STEP
    ids, lg = fhp.Sampler.generate(m, prompt, new, 0.0, 0, None, return_logits=True)
    t = fhp.Sampler.last_timing
    assert t["cached_steps"] == min(new - 1, 512 - P) and t["reprefill_steps"] == new - 1 - t["cached_steps"]
    oracle.set_threads(8)
    rids, rlg = oracle.generate(oc, w, prompt, new, return_logits=True)
    np.testing.assert_array_equal(ids, rids)
    np.testing.assert_array_equal(fast, rids)
    assert rel_err(lg, rlg) <= TOL_F32
    m.dispose()


def test_forward_last_batch_matches_oracle(fhp, oracle, backend):
    shape = (16384, 1024, 768, 12, 12)
    m, oc, w = make_model(fhp, oracle, backend, shape, 77, batch=2)
    r = fhp.TrainingRandom(5)
    ids = np.stack([r.ids(16384, 40), r.ids(16384, 40)])
    out = m.forward_last(ids)
    for b in range(2):
        assert rel_err(out[b], oracle.forward(oc, w, ids[b])[-1]) <= TOL_F32
    m.dispose()


def test_sampler_exact_on_same_logits(fhp, oracle, backend):
    """Given the same logits, history and uniform, the device sampler returns the
    oracle's id (Sampler.cs:29-69, 111-165), including top-k ties and bans."""
    rng = np.random.default_rng(11)
    cases = 0
    for trial in range(60):
        # V > 16384 takes the block-per-row sampler kernel instead of the register-resident one
        V = int(rng.choice([7, 100, 2256, 16384, 30000, 65536]))
        lg = (rng.standard_normal(V) * 2).astype(np.float32)
        if trial % 3 == 0:
            lg = np.round(lg, 1).astype(np.float32)  # ties
        hist = rng.integers(0, min(V, 50), size=int(rng.integers(0, 80))).astype(np.int32)
        T = float(rng.choice([0.0, 0.7, 1.0]))
        k = int(rng.choice([0, 1, 30, V - 1, V + 3]))
        pen = float(rng.choice([1.0, 1.1, 2.0]))
        ng = int(rng.choice([0, 1, 2, 4]))
        u = float(rng.random())
        dev = fhp.DeviceBuffer.from_array(backend, lg.astype(np.float32))
        got = fhp.Sampler.sample_device_logits(backend, dev.ptr, V, hist, T, k, u, pen, ng)
        dev.free()
        adj = oracle.apply_repetition_controls(lg, hist, pen, ng) if (pen != 1.0 or ng > 0) else lg
        want = oracle.sample(adj, T, k, u)
        assert got == want, (trial, V, T, k, pen, ng)
        cases += 1
    assert cases == 60


@pytest.mark.parametrize("shape", ["narrow", "wide", "ties"])
@pytest.mark.parametrize("k", [1, 30, 700, 5000])
def test_sampler_top_k_selection(fhp, oracle, backend, shape, k):
    """Top-k thresholds where every logit shares its top key bits (all in [2, 4)),
    where the largest values are far apart (no narrow window around the maximum
    holds k of them) and with heavy ties, at V = 16384: the device id equals the
    oracle's for several uniforms."""
    rng = np.random.default_rng(k + len(shape))
    V = 16384
    if shape == "narrow":
        lg = (2.0 + 2.0 * rng.random(V)).astype(np.float32)
    elif shape == "wide":
        lg = (rng.standard_normal(V) * 40).astype(np.float32)
    else:
        lg = np.round(rng.standard_normal(V) * 3, 0).astype(np.float32)
    dev = fhp.DeviceBuffer.from_array(backend, lg)
    for u in (0.0, 0.37, 0.999):
        got = fhp.Sampler.sample_device_logits(backend, dev.ptr, V, [], 0.9, k, u)
        assert got == oracle.sample(lg, 0.9, k, u), (shape, k, u)
    dev.free()


def decision_gaps(adj, T, k, u):
    """How far Sampler.Sample's decision (Sampler.cs:29-69) on the adjusted logits
    `adj` is from changing: (top-k gap, CDF gap).  The top-k gap is the distance
    between the k-th and (k+1)-th largest scaled logits (the kept set changes only
    if they cross); the CDF gap is the distance of the draw u * sum from the nearest
    boundary of the chosen interval of the index-ordered cumulative sum, as a
    fraction of the sum."""
    p = np.asarray(adj, np.float64) / T
    V = p.size
    gap_k = np.inf
    if 0 < k < V:
        srt = np.sort(p)
        thr = srt[V - k]
        gap_k = float(thr - srt[V - k - 1])
        p = np.where(p < thr, -np.inf, p)
    e = np.exp(p - p.max())
    cum = np.cumsum(e)
    target = u * cum[-1]
    i = int(np.searchsorted(cum, target, side="right"))
    lo = cum[i - 1] if i > 0 else 0.0
    hi = cum[min(i, V - 1)]
    return gap_k, float(min(hi - target, target - lo) / cum[-1])


@pytest.mark.parametrize("params", ["init", "trained"])
def test_c3_sampling_path(fhp, oracle, backend, params):
    """T 0.7, top-k 30, repetition 1.1, no-repeat-ngram 4, prompt 32 + 512,
    at the initial parameters and at trained-like ones (LayerNorm and bias values away
    from their (1, 0, 0) starting points).

    1. Every step: the oracle's sampler on the GPU's logits, the GPU's window and the
       same uniform returns the GPU's id (the sampler is exact).
    2. Every step: the GPU's logits are within 1e-4 of the oracle's logits for the
       same window: the window never slides (32 + 512 <= 1024), so row 31 + n of one
       oracle forward over the GPU's whole sequence is step n's ForwardLast.
    3. Where the oracle's sampler on the oracle's logits picks another id than the
       GPU's, the GPU's logits are themselves a perturbation within 1e-4 that flips
       the decision (1. and 2.); the decision gap there (top-k threshold or CDF) must
       be within what such a perturbation can move.  The count of agreeing steps is
       in the message.
    4. The free-running oracle trajectory agrees with the GPU's up to its first
       differing step, which must be such a flip.
    """
    shape = (16384, 1024, 768, 12, 12)
    T, K, PEN, NG = 0.7, 30, 1.1, 4
    m, oc, w = make_model(fhp, oracle, backend, shape, 1234, trained=params == "trained")
    prompt = fhp.TrainingRandom(42).ids(16384, 32)
    u = fhp.Random(1).next_doubles(512)
    ids, lg = fhp.Sampler.generate(m, prompt, 512, T, K, fhp.Random(1), repetition_penalty=PEN,
                                   no_repeat_ngram_size=NG, return_logits=True)
    assert len(ids) == 512
    seq = np.concatenate([prompt, ids]).astype(np.int32)
    oracle.set_threads(8)
    tf = oracle.forward(oc, w, seq[:-1])[31:]  # [512, V]: step n's logits on the GPU's window
    flips = []
    for n in range(512):
        window = seq[:32 + n]
        assert rel_err(lg[n], tf[n]) <= TOL_F32, f"step {n}"
        adj = oracle.apply_repetition_controls(lg[n], window, PEN, NG)
        assert oracle.sample(adj, T, K, float(u[n])) == ids[n], f"step {n}"
        adj_ref = oracle.apply_repetition_controls(tf[n], window, PEN, NG)
        if oracle.sample(adj_ref, T, K, float(u[n])) != ids[n]:
            # a perturbation of at most tol * max(1, |l|) per logit moves a scaled logit by
            # at most d = 1.1 tol max(1, max|l|) / T (the penalty scales by 1.1), each
            # exp term by a factor within exp(+-2d), so the CDF by about 4d of the sum
            d = PEN * TOL_F32 * max(1.0, float(np.max(np.abs(tf[n])))) / T
            gk, gc = decision_gaps(adj_ref, T, K, float(u[n]))
            assert gk <= 2 * d or gc <= 4 * d, (n, gk, gc, d)
            flips.append(n)
    agree = 512 - len(flips)
    print(f"C3 ({params}): the oracle's decision on its own logits equals the GPU's id at {agree}/512 steps "
          f"(flips within the fp32 tolerance at {flips})", flush=True)
    assert agree >= 504, f"only {agree}/512 steps agree; flips at {flips}"
    # the same generation without the logits dump draws inside the persistent kernel:
    # the same logits and the reference's arithmetic give the same ids
    fused = fhp.Sampler.generate(m, prompt, 512, T, K, fhp.Random(1), repetition_penalty=PEN,
                                 no_repeat_ngram_size=NG)
    assert route(fhp) & fhp._native.FH_ROUTE_FUSED_SAMPLER and not route(fhp) & fhp._native.FH_ROUTE_RETRIED
    np.testing.assert_array_equal(fused, ids)
    rids, rlg = oracle.generate(oc, w, prompt, 512, temperature=T, top_k=K, uniforms=u, penalty=PEN, ngram=NG,
                                return_logits=True)
    same = int(np.argmax(ids != rids)) if np.any(ids != rids) else 512
    print(f"C3 ({params}): free-running GPU and oracle trajectories agree for {same}/512 steps", flush=True)
    assert same == 512 or same in flips, f"the trajectories part at step {same}, not at a tolerance flip {flips}"
    m.dispose()


def test_batched_decode_matches_single_sequences(fhp, oracle, backend):
    shape = (2256, 128, 128, 4, 4)
    B = 6
    m, oc, w = make_model(fhp, oracle, backend, shape, 21, batch=B)
    r = fhp.TrainingRandom(3)
    prompts = np.stack([r.ids(2256, 20) for _ in range(B)])
    ids, lg = fhp.Sampler.generate(m, prompts, 40, 0.0, 0, None, return_logits=True)
    for b in range(B):
        rids, rlg = oracle.generate(oc, w, prompts[b], 40, return_logits=True)
        np.testing.assert_array_equal(ids[b], rids)
        assert rel_err(lg[b], rlg) <= TOL_F32
    m.dispose()


def test_eos_stops_each_sequence(fhp, oracle, backend):
    m, oc, w = make_model(fhp, oracle, backend, (32, 8, 16, 2, 2), 10)
    first = int(fhp.Sampler.generate(m, [3, 1], 1, 0.0, 0, None)[0])
    out = fhp.Sampler.generate(m, [3, 1], 10, 0.0, 0, None, eos_id=first)
    assert list(out) == [first]
    m.dispose()


# ---- MFMA GEMM (ITensorBackend.MatMulNN through fh_matmul_nn) --------------------------------

def bf16_round(x):
    """float32 -> nearest-even bfloat16, returned as float32 values and raw uint16 bits."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    u32 = u.astype(np.uint32)
    return u32.view(np.float32), (u32 >> 16).astype(np.uint16)


@pytest.mark.parametrize("M,K,N", [(64, 768, 2304), (32, 3072, 768), (300, 1024, 1000), (5, 64, 96),
                                   (130, 96, 257), (7, 40, 33), (1, 32, 130)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_matmul_nn_matches_oracle(fhp, oracle, backend, M, K, N, dtype):
    r = np.random.default_rng(M * 1000 + K + N)
    a = r.standard_normal((M, K)).astype(np.float32)
    b = (r.standard_normal((K, N)) * 0.05).astype(np.float32)
    y0 = r.standard_normal((M, N)).astype(np.float32)
    if dtype == "bf16":
        a_used, _ = bf16_round(a) if K % 32 == 0 else (a, None)  # the MFMA path rounds a; the tiled one does not
        b_used, b_bits = bf16_round(b)
        b_dev_data = b_bits
    else:
        a_used, b_used, b_dev_data = a, b, b
    bufa = fhp.DeviceBuffer.from_array(backend, a)
    bufb = fhp.DeviceBuffer.from_array(backend, b_dev_data)
    bufy = fhp.DeviceBuffer.from_array(backend, y0)
    backend.matmul_nn(bufa, bufb, bufy, M, K, N, accumulate=True, dtype=dtype)
    got = bufy.read(np.float32, M * N).reshape(M, N)
    ref = y0.astype(np.float64) + a_used.astype(np.float64) @ b_used.astype(np.float64)
    # fp32 accumulation in another order than the reference's sequential k: bound
    # the difference by the magnitude of the terms (|a| @ |b|)
    scale = np.abs(a_used).astype(np.float64) @ np.abs(b_used).astype(np.float64) + np.abs(y0)
    assert np.all(np.abs(got - ref) <= 1e-5 * scale + 1e-6), float(np.max(np.abs(got - ref) / (scale + 1e-6)))
    # and against the oracle's own sequential fp32 MatMulNN (CpuBackend.cs:49-57)
    if dtype == "f32":
        exp = oracle.matmul_nn(a, b) + y0
        assert np.all(np.abs(got - exp) <= 1e-5 * scale + 1e-6)
    # without accumulate, y is overwritten
    backend.matmul_nn(bufa, bufb, bufy, M, K, N, accumulate=False, dtype=dtype)
    got2 = bufy.read(np.float32, M * N).reshape(M, N)
    assert np.all(np.abs(got2 - (ref - y0)) <= 1e-5 * scale + 1e-6)
    for buf in (bufa, bufb, bufy):
        buf.free()


def test_bf16_operand_rounding_is_nearest_even_bit_for_bit(fhp, backend):
    """The device rounds a to bf16 before the bf16 GEMM (hardware convert); with an
    identity weight the product returns the rounded operand, which must equal the
    software round-to-nearest-even bit for bit, halfway cases and signs included
    (normal values only: the MFMA treats denormal operands as zero)."""
    M, K, N = 256, 64, 64
    r = np.random.default_rng(7)
    hi = r.integers(0x0080, 0x7F00, size=(M, K)).astype(np.uint32)  # normal exponents, either sign below
    lo = r.integers(0, 0x10000, size=(M, K)).astype(np.uint32)
    lo[:, 0::4] = 0x8000  # exact halfway: ties to even
    lo[:, 1::4] = 0x7FFF
    lo[:, 2::8] = 0x8001
    sign = (r.integers(0, 2, size=(M, K)).astype(np.uint32) << 31)
    a = ((hi << 16) | lo | sign).view(np.float32)
    a[0, :8] = [0.0, -0.0, 1.0, -1.0, 3.0e38, -3.0e38, 1.5, 65504.0]
    eye = np.eye(K, N, dtype=np.float32)
    _, eye_bits = bf16_round(eye)
    bufa = fhp.DeviceBuffer.from_array(backend, a)
    bufb = fhp.DeviceBuffer.from_array(backend, eye_bits)
    bufy = fhp.DeviceBuffer.from_array(backend, np.zeros((M, N), np.float32))
    backend.matmul_nn(bufa, bufb, bufy, M, K, N, accumulate=False, dtype="bf16")
    got = bufy.read(np.float32, M * N).reshape(M, N)
    want, _ = bf16_round(a)
    assert np.array_equal(got, want), int(np.sum(got != want))
    for buf in (bufa, bufb, bufy):
        buf.free()


@pytest.mark.parametrize("nbytes", [4, 60, 4096, 1 << 20, (64 << 20) + 52])
def test_buffer_checksum(fhp, backend, nbytes):
    # fh_buffer_checksum: the sum of the buffer's 32-bit words mod 2^64 (tail words
    # past the last 16-byte unit included), against numpy
    r = np.random.default_rng(nbytes)
    words = r.integers(0, 2**32, size=nbytes // 4, dtype=np.uint64).astype(np.uint32)
    buf = fhp.DeviceBuffer.from_array(backend, words)
    got, ms = buf.checksum(nbytes)
    assert got == int(np.sum(words, dtype=np.uint64))  # numpy's uint64 sum wraps mod 2^64
    assert ms >= 0
    buf.free()


@pytest.mark.parametrize("M,K,N", [(2000, 512, 4000), (256, 4096, 1024), (8192, 1024, 256)])
def test_matmul_nn_bf16_large_tiles(fhp, backend, M, K, N):
    # bf16 products of 256 rows or more run on the bf16-operand GEMM of the window
    # path: 256 x 128 tiles once there are as many tiles as CUs (the first and last
    # cases, ragged in M and N in the first), 128 x 128 below that
    r = np.random.default_rng(M + K + N)
    a = r.standard_normal((M, K)).astype(np.float32)
    b = (r.standard_normal((K, N)) * 0.05).astype(np.float32)
    y0 = r.standard_normal((M, N)).astype(np.float32)
    a_used, _ = bf16_round(a)
    b_used, b_bits = bf16_round(b)
    bufa = fhp.DeviceBuffer.from_array(backend, a)
    bufb = fhp.DeviceBuffer.from_array(backend, b_bits)
    bufy = fhp.DeviceBuffer.from_array(backend, y0)
    backend.matmul_nn(bufa, bufb, bufy, M, K, N, accumulate=True, dtype="bf16")
    got = bufy.read(np.float32, M * N).reshape(M, N)
    ref = y0.astype(np.float64) + a_used.astype(np.float64) @ b_used.astype(np.float64)
    scale = np.abs(a_used).astype(np.float64) @ np.abs(b_used).astype(np.float64) + np.abs(y0)
    assert np.all(np.abs(got - ref) <= 1e-5 * scale + 1e-6), float(np.max(np.abs(got - ref) / (scale + 1e-6)))
    for buf in (bufa, bufb, bufy):
        buf.free()


@pytest.mark.parametrize("M,K,N", [(2000, 512, 4000), (4100, 1024, 4100), (8192, 1024, 3072)])
def test_matmul_nn_bf16_pingpong_tiles(fhp, backend, M, K, N):
    # bf16 products without accumulation over many rows run on the 8-wave
    # ping-pong kernel: 128-row tiles (first case, ragged in M and N: rows and
    # columns past the ends dropped by the store bounds), 256-row tiles looping
    # over several tiles per block (second case ragged, third the C5 qkv shape)
    r = np.random.default_rng(M + K + N + 1)
    a = r.standard_normal((M, K)).astype(np.float32)
    b = (r.standard_normal((K, N)) * 0.05).astype(np.float32)
    a_used, _ = bf16_round(a)
    b_used, b_bits = bf16_round(b)
    bufa = fhp.DeviceBuffer.from_array(backend, a)
    bufb = fhp.DeviceBuffer.from_array(backend, b_bits)
    # a sentinel past the last row checks that nothing is stored beyond the output
    bufy = fhp.DeviceBuffer.from_array(backend, np.full((M + 64, N), 7.0, np.float32))
    backend.matmul_nn(bufa, bufb, bufy, M, K, N, accumulate=False, dtype="bf16")
    full = bufy.read(np.float32, (M + 64) * N).reshape(M + 64, N)
    got = full[:M]
    ref = a_used.astype(np.float64) @ b_used.astype(np.float64)
    scale = np.abs(a_used).astype(np.float64) @ np.abs(b_used).astype(np.float64)
    assert np.all(np.abs(got - ref) <= 1e-5 * scale + 1e-6), float(np.max(np.abs(got - ref) / (scale + 1e-6)))
    assert np.all(full[M:] == 7.0)
    for buf in (bufa, bufb, bufy):
        buf.free()


@pytest.mark.parametrize("M,K,N", [(8192, 4096, 1024), (8100, 2048, 1000), (4096, 4096, 2048), (8704, 2048, 1024),
                                   (8448, 4096, 1024), (11264, 1024, 768)])
def test_matmul_nn_bf16_split_k_accumulate(fhp, backend, M, K, N):
    # accumulating bf16 products whose 256 x 256 tiles cover half the CUs or more
    # but not all split K in two over separate blocks (C5's mlp.proj is the first
    # case; the second is ragged in M and N; the third has 16 x 8 tiles; the fourth
    # 34 x 4 tiles, XCD runs of 34 items): the second half to finish adds the first's
    # sums, the bias and the old y.  The last two have 33 x 4 and 44 x 3 tiles,
    # whose XCD runs of 33 items would put a tile's two halves on different XCDs,
    # so they must run unsplit.  Run twice: the tile counters must be left at zero
    # for the next product (and the split's error word at zero: matmul_nn raises
    # otherwise).
    r = np.random.default_rng(M + K + N + 2)
    a = r.standard_normal((M, K)).astype(np.float32)
    b = (r.standard_normal((K, N)) * 0.05).astype(np.float32)
    y0 = r.standard_normal((M, N)).astype(np.float32)
    a_used, _ = bf16_round(a)
    b_used, b_bits = bf16_round(b)
    prod = a_used.astype(np.float64) @ b_used.astype(np.float64)
    scale = np.abs(a_used).astype(np.float64) @ np.abs(b_used).astype(np.float64)
    bufa = fhp.DeviceBuffer.from_array(backend, a)
    bufb = fhp.DeviceBuffer.from_array(backend, b_bits)
    bufy = fhp.DeviceBuffer.from_array(backend, y0)
    backend.matmul_nn(bufa, bufb, bufy, M, K, N, accumulate=True, dtype="bf16")
    got1 = bufy.read(np.float32, M * N).reshape(M, N)
    ref1 = y0.astype(np.float64) + prod
    tol1 = 1e-5 * (scale + np.abs(y0)) + 1e-6
    assert np.all(np.abs(got1 - ref1) <= tol1), float(np.max(np.abs(got1 - ref1) / tol1))
    backend.matmul_nn(bufa, bufb, bufy, M, K, N, accumulate=True, dtype="bf16")
    got2 = bufy.read(np.float32, M * N).reshape(M, N)
    ref2 = got1.astype(np.float64) + prod
    tol2 = 1e-5 * (scale + np.abs(got1)) + 1e-6
    assert np.all(np.abs(got2 - ref2) <= tol2), float(np.max(np.abs(got2 - ref2) / tol2))
    for buf in (bufa, bufb, bufy):
        buf.free()


def test_c5_shape_bf16_generate_matches_oracle(fhp, oracle, backend):
    # Forge-220M shape with bf16 weights, reduced to a 64-token
    # prompt and 3 steps per sequence so the CPU oracle stays quick; the oracle runs
    # fp32 math on the same bf16-rounded parameters (north star: logits within 2e-2)
    shape = (16384, 1024, 1024, 16, 16)
    B, P, NEW = 2, 64, 3
    ocfg = oracle.Config(*shape)
    w = oracle.trained_like(ocfg, oracle.init_weights(ocfg, 1234), 2234)
    wr = bf16_round(w)[0]  # every parameter carries bf16 precision in a bf16 session
    m = fhp.GptModel(fhp.ModelConfig(*shape), backend, batch=B, dtype="bf16")
    m.load_weights(w)
    r = fhp.TrainingRandom(42)
    prompts = np.stack([r.ids(shape[0], P) for _ in range(B)])
    ids, lg = fhp.Sampler.generate(m, prompts, NEW, 0.0, 0, None, return_logits=True)
    oracle.set_threads(8)
    for b in range(B):
        rids, rlg = oracle.generate(ocfg, wr, prompts[b], NEW, return_logits=True)
        assert rel_err(lg[b][0], rlg[0]) <= 2e-2
        top2 = np.sort(rlg, axis=1)[:, -2:]
        for n in range(NEW):
            if top2[n, 1] - top2[n, 0] > 4e-2:  # ids must agree wherever the margin exceeds the tolerance
                assert ids[b][n] == rids[n]
            else:
                break
    m.dispose()


@pytest.mark.parametrize("B,P", [(4, 64), (8, 1024)])
def test_c5_shape_bf16_window_path_matches_oracle(fhp, oracle, backend, B, P):
    # 256 window rows or more in a bf16 session: LayerNorm, attention and GELU write
    # bf16 operands for the bf16 GEMM (B*P = 256 uses 128-row tiles, 8192 the
    # 256-row tiles of the full C5 prefill; P = 1024 fills the window, so every token
    # after the first re-prefills it: 4 steps there).  Checked against the oracle on
    # bf16-rounded parameters (2e-2) at every step for the first and last sequence,
    # and against the fp32-operand path
    shape = (16384, 1024, 1024, 16, 16)
    NEW = 4 if P == 1024 else 2
    ocfg = oracle.Config(*shape)
    w = oracle.trained_like(ocfg, oracle.init_weights(ocfg, 1234), 2234)
    wr = bf16_round(w)[0]
    prompts = np.stack([fhp.TrainingRandom(42 + b).ids(shape[0], P) for b in range(B)])
    m = fhp.GptModel(fhp.ModelConfig(*shape), backend, batch=B, dtype="bf16")
    m.load_weights(w)
    ids, lg = fhp.Sampler.generate(m, prompts, NEW, 0.0, 0, None, return_logits=True)
    m.dispose()
    os.environ["FORGE_HIP_BF16_ACT"] = "0"
    try:
        m2 = fhp.GptModel(fhp.ModelConfig(*shape), backend, batch=B, dtype="bf16")
    finally:
        del os.environ["FORGE_HIP_BF16_ACT"]
    m2.load_weights(w)
    ids2, lg2 = fhp.Sampler.generate(m2, prompts, NEW, 0.0, 0, None, return_logits=True)
    m2.dispose()
    oracle.set_threads(16)
    C = shape[1]
    for b in (0, B - 1):
        # the two paths round the same operands to bf16 but sum in different orders
        # (split K in the fp32-operand GEMM); 16 layers of bf16 rounding carry that
        # to about 1e-2 of the logits, inside the bf16 bar
        assert rel_err(lg[b][0], lg2[b][0]) <= 2e-2
        # every step teacher-forced on the GPU's own window (after the first step the
        # window slides: the last C ids of prompt + ids so far, positions from 0),
        # so a step after a near tie is still compared on the same input
        for n in range(NEW):
            window = np.concatenate([prompts[b], ids[b][:n]]).astype(np.int32)[-C:]
            ref = oracle.forward(ocfg, wr, window)[-1]
            assert rel_err(lg[b][n], ref) <= 2e-2, (b, n)
            top2 = np.sort(ref)[-2:]
            if top2[1] - top2[0] > 4e-2:
                assert ids[b][n] == int(np.argmax(ref)), (b, n)


@pytest.mark.parametrize("dtype,shape,B,P", [
    ("bf16", (4096, 128, 256, 3, 4), 4, 64),   # bf16 window of 256 rows: the bf16-operand GEMMs
    ("f32", (4096, 128, 256, 3, 4), 4, 64),    # fp32, 256 rows: split-K reductions fused with LN / KV store
    ("f32", (4096, 128, 256, 3, 4), 8, 100),   # fp32, 800 rows: one kernel per op
    ("f32", (64, 16, 16, 2, 2), 2, 8),         # head_dim 8: the generic decode attention in the tail
])
def test_window_last_layer_tail_matches_full_layer(fhp, oracle, backend, dtype, shape, B, P):
    # A window forward runs its last layer past the qkv projection and KV store
    # (which fill the caches for every row) on the last row of each sequence only;
    # FORGE_HIP_LAST_LAYER_TAIL=0 at session creation runs it on every row.  Both
    # against the oracle (on bf16-rounded parameters at 2e-2 for bf16, TOL_F32 for
    # fp32) at every step: step 0 is the window forward, the next steps cached decode
    # steps that read the caches the last layer wrote; and the two sessions against
    # each other
    NEW = 4
    ocfg = oracle.Config(*shape)
    w = oracle.trained_like(ocfg, oracle.init_weights(ocfg, 1234), 2234)
    wr = bf16_round(w)[0] if dtype == "bf16" else w
    tol = 2e-2 if dtype == "bf16" else TOL_F32
    prompts = np.stack([fhp.TrainingRandom(42 + b).ids(shape[0], P) for b in range(B)])
    got = {}
    for tail in ("1", "0"):
        os.environ["FORGE_HIP_LAST_LAYER_TAIL"] = tail
        try:
            m = fhp.GptModel(fhp.ModelConfig(*shape), backend, batch=B, dtype=dtype)
        finally:
            del os.environ["FORGE_HIP_LAST_LAYER_TAIL"]
        m.load_weights(w)
        got[tail] = fhp.Sampler.generate(m, prompts, NEW, 0.0, 0, None, return_logits=True)
        m.dispose()
    (ids, lg), (ids0, lg0) = got["1"], got["0"]
    for b in range(B):
        assert rel_err(lg[b][0], lg0[b][0]) <= tol, b
        same = True  # the two sessions' windows agree until a near tie
        for n in range(NEW):
            window = np.concatenate([prompts[b], ids[b][:n]]).astype(np.int32)[-shape[1]:]
            ref = oracle.forward(ocfg, wr, window)[-1]
            assert rel_err(lg[b][n], ref) <= tol, (b, n)
            top2 = np.sort(ref)[-2:]
            same = same and top2[1] - top2[0] > 2 * tol
            if same:
                assert ids[b][n] == int(np.argmax(ref)) == ids0[b][n], (b, n)


@pytest.mark.parametrize("case", ["greedy_c2", "sampled", "slides", "eos"])
def test_generate_stream_matches_one_shot(fhp, oracle, backend, case):
    # Sampler.Generate as an iterator: any chunking of fh_generate_next yields the ids
    # of one fh_generate call (the fused greedy kernel runs a launch per chunk)
    if case == "greedy_c2":
        m = fhp.GptModel(fhp.ModelConfig(16384, 1024, 768, 12, 12), backend, seed=1234)
        prompt, new, kw = fhp.TrainingRandom(42).ids(16384, 64), 40, {}
    elif case == "sampled":
        m = fhp.GptModel(fhp.ModelConfig(2256, 128, 128, 4, 4), backend, seed=1234)
        prompt, new = fhp.TrainingRandom(42).ids(2256, 16), 30
        kw = dict(temperature=0.7, top_k=30, repetition_penalty=1.1, no_repeat_ngram_size=4)
    elif case == "slides":
        m, oc, w = make_model(fhp, oracle, backend, (32, 8, 16, 2, 2), 8)
        prompt, new, kw = [1, 2, 3, 4, 5], 12, {}
    else:
        m = fhp.GptModel(fhp.ModelConfig(2256, 128, 128, 4, 4), backend, seed=1234)
        prompt, new = fhp.TrainingRandom(42).ids(2256, 16), 30
        first = list(fhp.Sampler.generate(m, prompt, new, 0.0, 0, None))
        kw = dict(eos_id=int(first[9]))
    T, k = kw.get("temperature", 0.0), kw.get("top_k", 0)
    extra = {x: kw[x] for x in ("eos_id", "repetition_penalty", "no_repeat_ngram_size") if x in kw}
    rng = fhp.Random(1) if T > 0 else None
    want = list(fhp.Sampler.generate(m, prompt, new, T, k, rng, **extra))
    for chunk in (1, 7, 64):
        rng = fhp.Random(1) if T > 0 else None
        got = list(fhp.Sampler.generate_stream(m, prompt, new, T, k, rng, chunk=chunk, **extra))
        assert got == want, (case, chunk)
    if case == "eos":
        assert len(want) <= 10 and want[-1] == kw["eos_id"]
    m.dispose()


def _session_route(fhp, m):
    import ctypes
    r = ctypes.c_int32()
    fhp._native.check(fhp._native.lib().fh_last_route(m.handle, ctypes.byref(r)))
    return r.value


def _stream_deferred(fhp, m, prompt, new, opts, u, chunk):
    """fh_generate_begin without uniforms, then fh_generate_next calls of `chunk` steps,
    each bringing its steps' uniforms (as the C# binding draws them); stops at EOS."""
    import ctypes
    N = fhp._native
    prompt = np.ascontiguousarray(prompt, np.int32)
    N.check(N.lib().fh_generate_begin(m.handle, prompt.ctypes.data, 1, prompt.size, new, ctypes.byref(opts), None))
    out = np.zeros(new, np.int32)
    counts = np.zeros(1, np.int32)
    produced = ctypes.c_int32()
    done = 0
    while done < new:
        buf = np.zeros(chunk, np.float64)
        part = u[done:done + chunk]
        buf[:part.size] = part
        N.check(N.lib().fh_generate_next(m.handle, chunk, buf.ctypes.data, out.ctypes.data, counts.ctypes.data,
                                         ctypes.byref(produced)))
        done = produced.value
        if counts[0] < done:  # EOS
            break
    return list(out[:counts[0]])


@pytest.mark.parametrize("chunk", [1, 16])
def test_sampled_stream_runs_the_in_kernel_sampler(fhp, oracle, backend, chunk):
    """The CLI's defaults (T 0.8, top-k 40, an EOS id set, Program.cs:642-644) streamed
    through fh_generate_next with each call's uniforms: on the fused path every call's
    steps run as one launch of the persistent sampled kernel (one step per call with
    chunk 1), and the ids equal one fh_generate call's, EOS included."""
    N = fhp._native
    shape = (16384, 1024, 768, 2, 12)
    m, oc, w = make_model(fhp, oracle, backend, shape, 81)
    prompt = fhp.TrainingRandom(19).ids(shape[0], 40)
    new = 70
    u = fhp.Random(1).next_doubles(new)
    full = list(fhp.Sampler.generate(m, prompt, new, 0.8, 40, fhp.Random(1)))
    eos = int(full[50])  # stops the stream at its first occurrence
    want = list(fhp.Sampler.generate(m, prompt, new, 0.8, 40, fhp.Random(1), eos_id=eos))
    assert route(fhp) & N.FH_ROUTE_FUSED_SAMPLER
    assert want[-1] == eos and len(want) <= 51
    got = _stream_deferred(fhp, m, prompt, new, N.Sampling(0.8, 40, 1.0, 0, eos, 0), u, chunk)
    assert _session_route(fhp, m) & N.FH_ROUTE_FUSED_SAMPLER
    assert got == want
    m.dispose()


def test_sampled_stream_resumes_per_step_after_a_tie(fhp, oracle, backend):
    """An all-ties model (tok_emb zero: every logit is 0) makes the in-kernel sampler
    meet an exact tie at its top-k threshold in a stream: the stream re-runs its steps
    on the per-step sampler and goes on (FH_ROUTE_RETRIED); ids equal fh_generate's."""
    N = fhp._native
    shape = (16384, 1024, 768, 2, 12)
    oc = oracle.Config(*shape)
    w = oracle.trained_like(oc, oracle.init_weights(oc, 3), 4)
    oracle.params(oc, w)["tok_emb"][...] = 0
    m = fhp.GptModel(fhp.ModelConfig(*shape), backend)
    m.load_weights(w)
    prompt = fhp.TrainingRandom(2).ids(shape[0], 20)
    want = list(fhp.Sampler.generate(m, prompt, 30, 0.9, 20, fhp.Random(8), repetition_penalty=1.3))
    u = fhp.Random(8).next_doubles(30)
    got = _stream_deferred(fhp, m, prompt, 30, N.Sampling(0.9, 20, 1.3, 0, -1, 0), u, 7)
    assert _session_route(fhp, m) & N.FH_ROUTE_RETRIED
    assert got == want
    m.dispose()


def test_stream_with_uniforms_per_call(fhp, backend):
    # fh_generate_begin without uniforms: each fh_generate_next brings its chunk's
    # uniforms, as a caller drawing NextDouble per step would (C3 options)
    import ctypes
    N = fhp._native
    m = fhp.GptModel(fhp.ModelConfig(2256, 128, 128, 4, 4), backend, seed=1234)
    prompt = np.ascontiguousarray(fhp.TrainingRandom(42).ids(2256, 16), np.int32)
    new = 23
    want = list(fhp.Sampler.generate(m, prompt, new, 0.7, 30, fhp.Random(1), repetition_penalty=1.1,
                                     no_repeat_ngram_size=4))
    u = fhp.Random(1).next_doubles(new)
    opts = N.Sampling(0.7, 30, 1.1, 4, -1, 0)
    N.check(N.lib().fh_generate_begin(m.handle, prompt.ctypes.data, 1, prompt.size, new, ctypes.byref(opts), None))
    out = np.zeros(new, np.int32)
    counts = np.zeros(1, np.int32)
    produced = ctypes.c_int32()
    done = 0
    while done < new:
        chunk = np.ascontiguousarray(u[done:done + 5])
        buf = np.zeros(5, np.float64)
        buf[:chunk.size] = chunk
        N.check(N.lib().fh_generate_next(m.handle, 5, buf.ctypes.data, out.ctypes.data, counts.ctypes.data,
                                         ctypes.byref(produced)))
        done = produced.value
    assert list(out[:counts[0]]) == want
    with pytest.raises(fhp.HipError):
        N.check(N.lib().fh_generate_next(m.handle, 1, None, out.ctypes.data, counts.ctypes.data,
                                         ctypes.byref(produced)))  # the stream has ended
    m.dispose()


def test_chat_rolling_context(fhp, oracle, backend):
    # Program.cs:736-768 on the C1 shape: 6 greedy turns of 60 ids grow the history
    # past ContextLength (every later turn slides the window) and past 2 x ContextLength
    # (the history is trimmed); each turn equals the oracle's Generate on the same history
    shape = (2256, 128, 128, 4, 4)
    m, oc, w = make_model(fhp, oracle, backend, shape, 1234)
    eos = 2255
    chat = fhp.Chat(m, eos, tokens_per_turn=60, temperature=0.0, chunk=16)
    hist = [eos]
    r = fhp.TrainingRandom(5)
    for turn in range(6):
        user = [int(t) for t in r.ids(2254, 7)]
        hist += user
        hist = hist[-256:]
        got = list(chat.turn(user))
        want = [int(t) for t in oracle.generate(oc, w, np.array(hist, np.int32), 60, eos=eos)]
        assert got == want, turn
        hist += want
        assert chat.history == hist
    chat.reset()
    assert chat.history == [eos]
    m.dispose()


def test_sampled_generation_consumes_one_uniform_per_step(fhp, backend):
    # a sampled generation that stops at eos draws one NextDouble per step it ran, so
    # the next generation on the same Random continues where the reference's would
    m = fhp.GptModel(fhp.ModelConfig(2256, 128, 128, 4, 4), backend, seed=1234)
    prompt = fhp.TrainingRandom(42).ids(2256, 16)
    probe = list(fhp.Sampler.generate(m, prompt, 20, 0.7, 30, fhp.Random(3)))
    eos = probe[4]
    n = probe.index(eos) + 1
    rng = fhp.Random(3)
    first = list(fhp.Sampler.generate(m, prompt, 20, 0.7, 30, rng, eos_id=eos))
    assert len(first) == n and rng._pos == n
    second = list(fhp.Sampler.generate_stream(m, prompt, 20, 0.7, 30, rng, chunk=5))
    ref = fhp.Random(3)
    ref.skip(n)
    assert second == list(fhp.Sampler.generate(m, prompt, 20, 0.7, 30, ref))
    assert rng._pos == n + 20
    m.dispose()


def test_c4_shape_batched_decode_matches_oracle(fhp, oracle, backend):
    # Forge-98M shape, 8 sequences decoded together (the batch-32 workload of
    # BASELINE config 4 at a CPU-checkable size): every decode GEMM has M = 8
    shape = (16384, 1024, 768, 12, 12)
    B = 8
    m, oc, w = make_model(fhp, oracle, backend, shape, 1234, batch=B)
    r = fhp.TrainingRandom(7)
    prompts = np.stack([r.ids(shape[0], 24) for _ in range(B)])
    ids, lg = fhp.Sampler.generate(m, prompts, 6, 0.0, 0, None, return_logits=True)
    oracle.set_threads(8)
    for b in range(B):
        rids, rlg = oracle.generate(oc, w, prompts[b], 6, return_logits=True)
        np.testing.assert_array_equal(ids[b], rids)
        assert rel_err(lg[b], rlg) <= TOL_F32
    m.dispose()


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_head_dim_64_window_prefill_matches_oracle(fhp, oracle, backend, dtype):
    # head_dim 64 runs prefill attention on MFMA tiles of 128 queries x 64 keys:
    # windows of 1, 64, 127, 129 and 200 rows cover single, partial and ragged
    # tiles; a 200-row window past a 160-token context re-prefills every step
    shape = (512, 160, 128, 2, 2)
    ocfg = oracle.Config(*shape)
    w = oracle.trained_like(ocfg, oracle.init_weights(ocfg, 99), 1099)
    wref = bf16_round(w)[0] if dtype == "bf16" else w
    tol = 2e-2 if dtype == "bf16" else TOL_F32
    m = fhp.GptModel(fhp.ModelConfig(*shape), backend, batch=2, dtype=dtype)
    m.load_weights(w)
    r = fhp.TrainingRandom(3)
    for T in (1, 64, 127, 129, 160):
        ids = np.stack([r.ids(shape[0], T), r.ids(shape[0], T)])
        out = m.forward_last(ids)
        for b in range(2):
            assert rel_err(out[b], oracle.forward(ocfg, wref, ids[b])[-1]) <= tol, (T, b)
    prompts = np.stack([r.ids(shape[0], 150), r.ids(shape[0], 150)])
    ids, lg = fhp.Sampler.generate(m, prompts, 20, 0.0, 0, None, return_logits=True)
    for b in range(2):
        rids, rlg = oracle.generate(ocfg, wref, prompts[b], 20, return_logits=True)
        top2 = np.sort(rlg, axis=1)[:, -2:]
        for n in range(20):
            assert rel_err(lg[b][n], rlg[n]) <= tol, (b, n)
            if top2[n, 1] - top2[n, 0] <= 2 * tol:  # a near tie may flip; later steps then differ
                break
            assert ids[b][n] == rids[n], (b, n)
    m.dispose()


def test_batched_decode_attention_over_several_chunks(fhp, oracle, backend):
    # batched decode attention reads 256-key chunks: a 500-token prompt decoded
    # to position 529 crosses the second chunk boundary with a ragged last chunk
    shape = (512, 640, 128, 2, 2)
    B, P, NEW = 3, 500, 30
    m, oc, w = make_model(fhp, oracle, backend, shape, 31, batch=B)
    r = fhp.TrainingRandom(11)
    prompts = np.stack([r.ids(shape[0], P) for _ in range(B)])
    ids, lg = fhp.Sampler.generate(m, prompts, NEW, 0.0, 0, None, return_logits=True)
    for b in range(B):
        rids, rlg = oracle.generate(oc, w, prompts[b], NEW, return_logits=True)
        np.testing.assert_array_equal(ids[b], rids)
        assert rel_err(lg[b], rlg) <= TOL_F32
    m.dispose()


@pytest.mark.parametrize("B,dtype", [(33, "f32"), (70, "f32"), (12, "bf16")])
def test_batched_decode_fused_epilogues(fhp, oracle, backend, B, dtype):
    # batched decode sums the split-K partials in kernels that also do the next
    # step (qkv + KV store, proj + LN2, mlp.proj + the next LayerNorm or LN_f):
    # 33 and 70 rows take the GEMM's 64- and 128-row tiles
    shape = (512, 64, 128, 2, 2)
    ocfg = oracle.Config(*shape)
    w = oracle.trained_like(ocfg, oracle.init_weights(ocfg, 5), 1005)
    wref = bf16_round(w)[0] if dtype == "bf16" else w
    tol = 2e-2 if dtype == "bf16" else TOL_F32
    m = fhp.GptModel(fhp.ModelConfig(*shape), backend, batch=B, dtype=dtype)
    m.load_weights(w)
    r = fhp.TrainingRandom(17)
    prompts = np.stack([r.ids(shape[0], 10) for _ in range(B)])
    ids, lg = fhp.Sampler.generate(m, prompts, 8, 0.0, 0, None, return_logits=True)
    for b in range(B):
        rids, rlg = oracle.generate(ocfg, wref, prompts[b], 8, return_logits=True)
        top2 = np.sort(rlg, axis=1)[:, -2:]
        for n in range(8):
            assert rel_err(lg[b][n], rlg[n]) <= tol, (b, n)
            if top2[n, 1] - top2[n, 0] <= 2 * tol:  # a near tie may flip; later steps then differ
                break
            assert ids[b][n] == rids[n], (b, n)
    m.dispose()


def test_batched_decode_past_four_attention_chunks(fhp, oracle, backend):
    # more than 4 rows and a context above 1024 positions: the attention chunks
    # are combined by their own kernel (the attn.proj operand load combines at
    # most 4) while the split-K reductions stay fused with the KV store and the
    # LayerNorms; positions 1030..1049 span five 256-key chunks
    shape = (512, 1100, 128, 2, 2)
    B, P, NEW = 6, 1030, 20
    m, oc, w = make_model(fhp, oracle, backend, shape, 41, batch=B)
    r = fhp.TrainingRandom(19)
    prompts = np.stack([r.ids(shape[0], P) for _ in range(B)])
    ids, lg = fhp.Sampler.generate(m, prompts, NEW, 0.0, 0, None, return_logits=True)
    oracle.set_threads(8)
    for b in range(B):
        rids, rlg = oracle.generate(oc, w, prompts[b], NEW, return_logits=True)
        np.testing.assert_array_equal(ids[b], rids)
        assert rel_err(lg[b], rlg) <= TOL_F32
    m.dispose()


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_batched_decode_attention_in_proj_over_four_chunks(fhp, oracle, backend, dtype):
    # more than 4 rows and ctx <= 1024: the qkv split-K sum and the K/V store run inside
    # the decode attention and the 256-key chunks are combined in attn.proj's operand
    # load (FH_ROUTE_ATTN_IN_PROJ).  A 500-token prompt decoded for 300 steps attends
    # over 501..800 keys: 2, 3 and 4 chunks, K/V rows stored into chunks 1, 2 and 3
    shape = (512, 1024, 128, 2, 2)
    B, P, NEW = 6, 500, 300
    ocfg = oracle.Config(*shape)
    w = oracle.trained_like(ocfg, oracle.init_weights(ocfg, 51), 1051)
    wref = bf16_round(w)[0] if dtype == "bf16" else w
    tol = 2e-2 if dtype == "bf16" else TOL_F32
    m = fhp.GptModel(fhp.ModelConfig(*shape), backend, batch=B, dtype=dtype)
    m.load_weights(w)
    r = fhp.TrainingRandom(23)
    prompts = np.stack([r.ids(shape[0], P) for _ in range(B)])
    ids, lg = fhp.Sampler.generate(m, prompts, NEW, 0.0, 0, None, return_logits=True)
    assert route(fhp) & fhp._native.FH_ROUTE_ATTN_IN_PROJ
    for b in range(B):
        # teacher-forced: the oracle's logits for each step's own window (row P - 1 + n
        # of one forward over the GPU's sequence), so every step is compared even after
        # a near tie; each greedy id is the oracle's argmax up to such a tie
        seq = np.concatenate([prompts[b], ids[b]]).astype(np.int32)
        tf = oracle.forward(ocfg, wref, seq[:-1])[P - 1:]
        assert rel_err(lg[b], tf) <= tol, (dtype, b)
        for n in range(NEW):
            top = float(tf[n].max())
            assert top - float(tf[n][ids[b][n]]) <= 2 * tol * max(1.0, abs(top)), (dtype, b, n)
    m.dispose()


@pytest.mark.parametrize("params", ["init", "trained"])
def test_c4_config_batch32_long_context(fhp, oracle, backend, params):
    """BASELINE config 4 at its full size: 32 sequences of 512 PCG32 prompt ids (seeds
    42 + b), 512 greedy steps each, so the windows run from 513 to 1023 keys; at the
    initial parameters and at trained-like ones.

    * every sequence's ids equal the same prompt decoded alone (batch 1, the fused
      step), up to a step where the two runs part at a near tie of the batched run's
      logits (within 2e-4 of each other);
    * for sequences 0 and 31 the batched logits match the oracle at every one of the
      512 steps (one teacher-forced oracle forward over the batched run's sequence;
      no slide happens, so row 511 + n is step n's ForwardLast), and each id is the
      oracle's argmax up to a near tie.
    """
    shape = (16384, 1024, 768, 12, 12)
    B, P, NEW = 32, 512, 512
    m, oc, w = make_model(fhp, oracle, backend, shape, 1234, batch=B, trained=params == "trained")
    prompts = np.stack([fhp.TrainingRandom(42 + b).ids(shape[0], P) for b in range(B)])
    ids, lg = fhp.Sampler.generate(m, prompts, NEW, 0.0, 0, None, return_logits=True)
    assert route(fhp) & fhp._native.FH_ROUTE_ATTN_IN_PROJ
    m.dispose()
    single = fhp.GptModel(fhp.ModelConfig(*shape), backend)
    single.load_weights(w)
    parted = []
    for b in range(B):
        one = fhp.Sampler.generate(single, prompts[b], NEW, 0.0, 0, None)
        d = np.nonzero(one != ids[b])[0]
        if d.size:
            n = int(d[0])
            row = lg[b][n].astype(np.float64)
            gap = abs(row[one[n]] - row[ids[b][n]])
            assert gap <= 2 * TOL_F32 * max(1.0, float(row.max())), (b, n, gap)
            parted.append((b, n))
    single.dispose()
    print(f"C4 ({params}): {B - len(parted)}/{B} sequences equal their batch-1 decode over all 512 steps; "
          f"near-tie partings at {parted}", flush=True)
    oracle.set_threads(16)
    for b in (0, B - 1):
        seq = np.concatenate([prompts[b], ids[b]]).astype(np.int32)
        tf = oracle.forward(oc, w, seq[:-1])[P - 1:]
        assert rel_err(lg[b], tf) <= TOL_F32, b
        for n in range(NEW):
            top = float(tf[n].max())
            assert top - float(tf[n][ids[b][n]]) <= 2 * TOL_F32 * max(1.0, abs(top)), (b, n)


@pytest.mark.parametrize("T,k,pen,ng", [(0.7, 30, 1.1, 4), (1.0, 1, 1.0, 0), (0.8, 63, 2.0, 1), (1.3, 5, 1.0, 2),
                                        (0.5, 40, 1.5, 0), (2.0, 12, 1.2, 3)])
def test_in_kernel_sampler_matches_per_step_sampler(fhp, oracle, backend, T, k, pen, ng):
    """Top-k sampling inside the persistent decode kernel (every cached step of one
    launch draws its id from the launch's own logits) against the per-step path (the
    fused step writes the logits, the sampler kernel draws): same ids at every step,
    for greedy-like k = 1, the largest in-kernel k (63), penalties, n-gram bans of
    sizes 1-4; the per-step path's ids are in turn the oracle sampler's on its logits."""
    shape = (16384, 1024, 768, 2, 12)
    m, oc, w = make_model(fhp, oracle, backend, shape, 61)
    prompt = fhp.TrainingRandom(13).ids(shape[0], 40)
    n = 150
    fused = fhp.Sampler.generate(m, prompt, n, T, k, fhp.Random(5), repetition_penalty=pen, no_repeat_ngram_size=ng)
    rt = route(fhp)
    assert rt & fhp._native.FH_ROUTE_FUSED_SAMPLER and not rt & fhp._native.FH_ROUTE_RETRIED, rt
    ids, lg = fhp.Sampler.generate(m, prompt, n, T, k, fhp.Random(5), repetition_penalty=pen,
                                   no_repeat_ngram_size=ng, return_logits=True)
    assert not route(fhp) & fhp._native.FH_ROUTE_FUSED_SAMPLER
    np.testing.assert_array_equal(fused, ids)
    u = fhp.Random(5).next_doubles(n)
    seq = list(prompt)
    for i in range(n):
        adj = oracle.apply_repetition_controls(lg[i], seq, pen, ng) if (pen != 1.0 or ng > 0) else lg[i]
        assert oracle.sample(adj, T, k, float(u[i])) == ids[i], i
        seq.append(int(ids[i]))
    m.dispose()


@pytest.mark.parametrize("mode", ["greedy", "sampled"])
def test_fused_launch_failure_falls_back_to_generic_kernels(fhp, oracle, backend, monkeypatch, mode):
    """FORGE_HIP_INJECT_FUSED_FAILURE=1 (read at session creation) starts every fused
    launch with its error word set, as after a hand-off wait past its spin limit: every
    wait of the launch gives up at once and every block runs to its end.  fh_generate
    then repeats the whole generation on the generic kernels (FH_ROUTE_FALLBACK), whose
    ids equal a session built for the generic kernels and, greedy, the oracle's.  A
    stream (fh_generate_next) has handed out earlier chunks, so it reports the error."""
    N = fhp._native
    shape = (16384, 1024, 768, 2, 12)
    monkeypatch.setenv("FORGE_HIP_INJECT_FUSED_FAILURE", "1")
    m, oc, w = make_model(fhp, oracle, backend, shape, 71)
    monkeypatch.delenv("FORGE_HIP_INJECT_FUSED_FAILURE")
    monkeypatch.setenv("FORGE_HIP_FUSED_DECODE", "0")
    g, _, _ = make_model(fhp, oracle, backend, shape, 71)
    monkeypatch.delenv("FORGE_HIP_FUSED_DECODE")
    prompt = fhp.TrainingRandom(17).ids(shape[0], 40)
    n = 60
    if mode == "greedy":
        args = (0.0, 0, None)
        kw = {}
    else:
        kw = dict(repetition_penalty=1.1, no_repeat_ngram_size=4)
    def run(model):
        a = args if mode == "greedy" else (0.7, 30, fhp.Random(3))
        return fhp.Sampler.generate(model, prompt, n, *a, **kw)
    ids = run(m)
    rt = route(fhp)
    assert rt & N.FH_ROUTE_FALLBACK and not rt & (N.FH_ROUTE_FUSED_STEP | N.FH_ROUTE_FUSED_SAMPLER), rt
    want = run(g)
    assert not route(fhp) & N.FH_ROUTE_FALLBACK
    np.testing.assert_array_equal(ids, want)
    if mode == "greedy":
        np.testing.assert_array_equal(ids, oracle.generate(oc, w, prompt, n))
        with pytest.raises(fhp.HipError, match="spin limit"):
            list(fhp.Sampler.generate_stream(m, prompt, n, 0.0, 0, None, chunk=16))
    # a later generation on the same session fails over again, from a clean state
    np.testing.assert_array_equal(run(m), want)
    m.dispose()
    g.dispose()


def test_in_kernel_sampler_ties_repeat_the_generation_per_step(fhp, oracle, backend):
    """A model whose logits all tie (tok_emb zero: every logit is 0) makes the in-kernel
    sampler meet an exact tie at its top-k threshold; fh_generate then repeats the
    generation with the per-step sampler, which keeps every tied value as the
    reference does: the ids equal the per-step path's."""
    shape = (16384, 1024, 768, 2, 12)
    oc = oracle.Config(*shape)
    w = oracle.trained_like(oc, oracle.init_weights(oc, 3), 4)
    oracle.params(oc, w)["tok_emb"][...] = 0
    m = fhp.GptModel(fhp.ModelConfig(*shape), backend)
    m.load_weights(w)
    prompt = fhp.TrainingRandom(2).ids(shape[0], 20)
    fused = fhp.Sampler.generate(m, prompt, 30, 0.9, 20, fhp.Random(8), repetition_penalty=1.3)
    assert route(fhp) & fhp._native.FH_ROUTE_RETRIED
    ids = fhp.Sampler.generate(m, prompt, 30, 0.9, 20, fhp.Random(8), repetition_penalty=1.3, return_logits=True)[0]
    np.testing.assert_array_equal(fused, ids)
    m.dispose()


@pytest.mark.parametrize("path", ["fused_greedy", "fused_sampled", "batched_fp32", "window_bf16"])
def test_each_path_gives_the_same_bits_run_to_run(fhp, oracle, backend, path):
    """Same inputs, same bits (the reference's same-seed determinism,
    tests/LLM.Core.Tests/ModelTests.cs:45-56): every reduction on the device runs in a
    fixed order (DPP trees, split-K partials summed in split order, the two K halves
    of a bf16 tile added as ((own + other) + bias) + residual whichever half arrives
    first, the fused step's hand-offs gathered by slot), so two runs on one session and
    a run on a second session with the same weights return the same ids and, where
    the path returns them, the same logits bit for bit.  Paths: the persistent batch-1
    kernel (greedy, and sampled with top-k, penalty and n-gram bans), the batched fp32
    decode graph (attention combined in attn.proj's operand load) and bf16 windows of
    8 x 1024 rows (every step re-prefills; mlp.proj with its K split in two)."""
    N = fhp._native
    if path in ("fused_greedy", "fused_sampled"):
        shape, B, P, NEW, dtype = (16384, 1024, 768, 2, 12), 1, 40, 200, "f32"
        want = N.FH_ROUTE_FUSED_STEP | (N.FH_ROUTE_FUSED_SAMPLER if path == "fused_sampled" else 0)
    elif path == "batched_fp32":
        shape, B, P, NEW, dtype = (16384, 1024, 768, 2, 12), 8, 300, 16, "f32"
        want = N.FH_ROUTE_ATTN_IN_PROJ
    else:
        shape, B, P, NEW, dtype = (16384, 1024, 1024, 2, 16), 8, 1024, 2, "bf16"
        want = 0
    ocfg = oracle.Config(*shape)
    w = oracle.trained_like(ocfg, oracle.init_weights(ocfg, 77), 1077)
    r = fhp.TrainingRandom(5)
    prompts = np.stack([r.ids(shape[0], P) for _ in range(B)])
    if B == 1:
        prompts = prompts[0]

    def run(model):
        if path == "fused_sampled":
            return fhp.Sampler.generate(model, prompts, NEW, 0.7, 30, fhp.Random(9), repetition_penalty=1.1,
                                        no_repeat_ngram_size=4), None
        if path == "fused_greedy":
            return fhp.Sampler.generate(model, prompts, NEW, 0.0, 0, None), None
        return fhp.Sampler.generate(model, prompts, NEW, 0.0, 0, None, return_logits=True)

    models = []
    for _ in range(2):
        m = fhp.GptModel(fhp.ModelConfig(*shape), backend, batch=B, dtype=dtype)
        m.load_weights(w)
        models.append(m)
    first = run(models[0])
    assert route(fhp) & want == want, (path, route(fhp))
    for again in (run(models[0]), run(models[1])):
        np.testing.assert_array_equal(again[0], first[0])
        if first[1] is not None:
            assert np.array_equal(np.asarray(again[1], np.float32).view(np.uint32),
                                  np.asarray(first[1], np.float32).view(np.uint32)), path
    for m in models:
        m.dispose()
