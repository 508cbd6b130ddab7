"""The CPU oracle against the reference's own known answers, closed forms and
brute force, plus the committed golden vectors.

Known answers are the literals of the reference tests (paths relative to the
reference checkout): tests/LLM.Core.Tests/CpuBackendTests.cs, InferenceTests.cs,
ModelTests.cs, ModelPresetTests.cs.
"""
import os

import numpy as np
import pytest

from conftest import GOLDEN

SMALL = dict(vocab_size=32, context_length=8, d_model=16, n_layers=2, n_heads=2)  # InferenceTests.cs:17


def cfg(O, **kw):
    return O.Config(kw["vocab_size"], kw["context_length"], kw["d_model"], kw["n_layers"], kw["n_heads"])


# ---- elementwise kernels (CpuBackendTests.cs) ----------------------------------------------

def test_gelu_known_values(oracle):
    # CpuBackendTests.Gelu_KnownValues :211-218
    y = oracle.gelu(np.array([0, 1, -1, 2, -2], np.float32))
    np.testing.assert_allclose(y, [0, 0.841192, -0.158808, 1.954598, -0.045402], atol=1e-4)


def test_gelu_matches_float64_formula(oracle):
    x = np.linspace(-6, 6, 2001, dtype=np.float32)
    c = np.sqrt(2 / np.pi)
    ref = 0.5 * x.astype(np.float64) * (1 + np.tanh(c * (x + 0.044715 * x.astype(np.float64) ** 3)))
    np.testing.assert_allclose(oracle.gelu(x), ref, atol=2e-6, rtol=2e-6)


def test_softmax_rows_sum_to_one(oracle):
    # CpuBackendTests.Softmax_RowsSumToOne :186-208 (incl. the 1000-logit row)
    rng = np.random.default_rng(6)
    x = (rng.random((3, 6)) * 20 - 10).astype(np.float32)
    raw = x.copy()
    x[0, 0] = 1000
    y = oracle.softmax(x)
    np.testing.assert_allclose(y.sum(1), 1, atol=1e-5)
    e = np.exp(raw[2].astype(np.float64))
    np.testing.assert_allclose(y[2], e / e.sum(), atol=1e-5)
    assert y[0, 0] > 0.99


def test_layernorm_normalizes_rows(oracle):
    # CpuBackendTests.LayerNorm_NormalizesRows :252-295
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((3, 8)) * 3).astype(np.float32)
    w = rng.standard_normal(8).astype(np.float32)
    b = rng.standard_normal(8).astype(np.float32)
    y = oracle.layernorm(x, w, b)
    mu = x.astype(np.float64).mean(1, keepdims=True)
    var = x.astype(np.float64).var(1, keepdims=True)
    np.testing.assert_allclose(y, (x - mu) / np.sqrt(var + 1e-5) * w + b, atol=1e-3)
    y1 = oracle.layernorm(x, np.ones(8, np.float32), np.zeros(8, np.float32))
    np.testing.assert_allclose(y1.mean(1), 0, atol=1e-4)
    np.testing.assert_allclose(y1.var(1), 1, atol=1e-3)


# ---- matmuls ---------------------------------------------------------------------------------

def test_matmul_nn_brute_force(oracle):
    # CpuBackendTests.MatMulNN_Forward :85-100 against a float64 triple loop
    rng = np.random.default_rng(1)
    for (M, K, N) in [(3, 5, 4), (7, 33, 19), (1, 768, 40)]:
        a = rng.standard_normal((M, K)).astype(np.float32)
        b = rng.standard_normal((K, N)).astype(np.float32)
        np.testing.assert_allclose(oracle.matmul_nn(a, b), a.astype(np.float64) @ b, atol=1e-4, rtol=1e-5)


def test_matmul_nn_is_sequential_in_k(oracle):
    # CpuBackend.MatMulRowKernel accumulates y += a[m,k]*b[k,:] in ascending k,
    # multiply then add (two roundings); float32 numpy replays that order exactly.
    rng = np.random.default_rng(2)
    a = rng.standard_normal((4, 64)).astype(np.float32)
    b = rng.standard_normal((64, 24)).astype(np.float32)
    y = np.zeros((4, 24), np.float32)
    for k in range(64):
        y = (y + (a[:, k:k + 1] * b[k:k + 1, :]).astype(np.float32)).astype(np.float32)
    np.testing.assert_array_equal(oracle.matmul_nn(a, b), y)


def test_matmul_nt_and_dot(oracle):
    rng = np.random.default_rng(3)
    a = rng.standard_normal((5, 37)).astype(np.float32)
    b = rng.standard_normal((9, 37)).astype(np.float32)
    np.testing.assert_allclose(oracle.matmul_nt(a, b), a.astype(np.float64) @ b.T.astype(np.float64),
                               atol=1e-4, rtol=1e-5)
    # below one 8-lane vector the dot is the plain sequential sum
    x, y = a[0, :7], b[0, :7]
    s = np.float32(0)
    for i in range(7):
        s = np.float32(s + np.float32(x[i] * y[i]))
    assert oracle.dot(x, y) == s
    # 8 lanes, then the lane reduction, then the tail: a single set lane passes through exactly
    x = np.zeros(9, np.float32); y = np.zeros(9, np.float32)
    x[5], y[5], x[8], y[8] = 3, 0.5, 2, 0.25
    assert oracle.dot(x, y) == np.float32(2.0)


# ---- sampler (InferenceTests.cs) --------------------------------------------------------------

def test_greedy_and_zero_temperature(oracle):
    lg = np.array([0.1, 2.5, -1, 2.4], np.float32)  # :20-28
    assert oracle.greedy(lg) == 1
    for u in (0.0, 0.3, 0.999):
        assert oracle.sample(lg, 0.0, 0, u) == 1
    assert oracle.greedy(np.array([1, 3, 3, 2], np.float32)) == 1  # ties keep the first


def test_topk1_is_argmax(oracle):
    lg = np.array([-3, 0.5, 0.4, 0.6], np.float32)  # :30-37
    for u in np.linspace(0, 0.999, 20):
        assert oracle.sample(lg, 1.0, 1, float(u)) == 3


def test_repetition_penalty_literal(oracle):
    out = oracle.apply_repetition_controls([4, -2, 3, 1], [0, 1, 0], 2.0, 0)  # :115-124
    np.testing.assert_array_equal(out, [2, -4, 3, 1])


def test_no_repeat_ngram_literal(oracle):
    out = oracle.apply_repetition_controls([0, 1, 2, 9, 4], [1, 2, 3, 1, 2], 1.0, 3)  # :126-134
    assert np.isneginf(out[3]) and out[4] == 4 and out[0] == 0 and out[1] == 1 and out[2] == 2


def test_no_repeat_ngram_restores_when_all_banned(oracle):
    out = oracle.apply_repetition_controls([2, 1], [0, 1], 1.0, 1)  # :136-144
    np.testing.assert_array_equal(out, [2, 1])


def test_sampling_distribution_matches_softmax(oracle):
    # InferenceTests.Sample_DistributionMatchesSoftmax :51-66 with a seeded uniform stream
    lg = np.array([1, 2, 3], np.float32)
    e = np.exp(lg.astype(np.float64)); e /= e.sum()
    u = oracle.net_random_doubles(4, 20000)
    counts = np.bincount([oracle.sample(lg, 1.0, 0, float(x)) for x in u], minlength=3) / 20000
    np.testing.assert_allclose(counts, e, atol=0.03)


def test_sample_inverse_cdf_brute_force(oracle):
    # Sample = first i with u*sum < prefix_i over exp(l/T - max), top-k keeping ties
    rng = np.random.default_rng(5)
    for trial in range(200):
        V = int(rng.integers(2, 40))
        lg = np.round(rng.standard_normal(V) * 2, 1).astype(np.float32)  # rounding creates ties
        T = float(rng.choice([0.5, 0.7, 1.0, 1.3]))
        k = int(rng.integers(0, V + 2))
        u = float(rng.random())
        p = (lg / np.float32(T)).astype(np.float32)
        if 0 < k < V:
            thr = np.sort(p)[V - k]
            p = np.where(p < thr, -np.inf, p).astype(np.float32)
        e = np.exp((p - p.max()).astype(np.float32)).astype(np.float32)
        s = np.float32(0)
        cs = []
        for v in e:
            s = np.float32(s + v)
            cs.append(s)
        uu = np.float32(np.float32(u) * s)
        want = next((i for i, c in enumerate(cs) if uu < c), V - 1)
        assert oracle.sample(lg, T, k, u) == want


def test_sample_top_k_keeps_ties(oracle):
    lg = np.array([1, 5, 5, 5, 0], np.float32)
    picks = {oracle.sample(lg, 1.0, 2, float(u)) for u in np.linspace(0, 0.999, 50)}
    assert picks == {1, 2, 3}


# ---- model ------------------------------------------------------------------------------------

def test_parameter_counts(oracle):
    assert oracle.param_count(cfg(oracle, **SMALL)) == 7232  # ModelTests.cs:39
    # ModelPresetTests.CandidateCounts_AreStable :34-42
    assert oracle.param_count(oracle.Config(16257, 512, 768, 12, 12)) == 97_934_592
    assert oracle.param_count(oracle.Config(16257, 1024, 1024, 16, 16)) == 219_237_376
    assert oracle.param_count(oracle.Config(16257, 1024, 1024, 24, 16)) == 320_007_168


def test_init_statistics(oracle):
    # ModelTests.Init_ResidualProjectionsUseScaledStd :58-80
    c = oracle.Config(2256, 128, 128, 4, 4)
    w = oracle.init_weights(c, 7)
    d, L = 128, 4
    o = 2256 * d + 128 * d
    blk = 12 * d * d + 13 * d
    ln1w = w[o:o + d]
    qkv = w[o + 2 * d:o + 2 * d + 3 * d * d]
    proj = w[o + 2 * d + 3 * d * d + 3 * d:o + 2 * d + 4 * d * d + 3 * d]
    assert np.all(ln1w == 1) and np.all(w[o + d:o + 2 * d] == 0)
    assert abs(qkv.std() - 0.02) < 0.02 * 0.05
    assert abs(proj.std() - 0.02 / np.sqrt(2 * L)) < 0.02 / np.sqrt(2 * L) * 0.05
    assert np.all(w[-2 * d:-d] == 1) and np.all(w[-d:] == 0)
    assert w.size == o + L * blk + 2 * d


def test_forward_deterministic_per_seed(oracle):
    # ModelTests.Forward_DeterministicPerSeed :45-56
    c = cfg(oracle, **SMALL)
    ids = [3, 1, 4, 1, 5]
    a = oracle.forward(c, oracle.init_weights(c, 42), ids)
    b = oracle.forward(c, oracle.init_weights(c, 42), ids)
    d = oracle.forward(c, oracle.init_weights(c, 43), ids)
    np.testing.assert_array_equal(a, b)
    assert np.any(a != d)


def test_forward_last_equals_last_row(oracle):
    # ModelTests.Forward_OutputShape :24-41: ForwardLast == last row of Forward, exactly
    c = cfg(oracle, **SMALL)
    w = oracle.init_weights(c, 1)
    ids = [1, 2, 3, 4]
    full = oracle.forward(c, w, ids)
    gen_ids, lg = oracle.generate(c, w, ids, 1, kv_cached=False, return_logits=True)
    np.testing.assert_array_equal(lg[0], full[-1])
    assert full.shape == (4, 32)


@pytest.mark.parametrize("shape,prompt_len,steps", [
    ((32, 8, 16, 2, 2), 2, 12),        # slides after 6 steps
    ((32, 8, 16, 2, 2), 12, 6),        # prompt longer than the context
    ((2256, 128, 128, 4, 4), 16, 130),  # config 1 through its slide at step 113
])
def test_kv_cached_equals_full_recompute_bitwise(oracle, shape, prompt_len, steps):
    c = oracle.Config(*shape)
    w = oracle.init_weights(c, 8)
    prompt = oracle.pcg32_ids(9, c.vocab_size, prompt_len)
    a_ids, a_lg = oracle.generate(c, w, prompt, steps, kv_cached=False, return_logits=True)
    b_ids, b_lg = oracle.generate(c, w, prompt, steps, kv_cached=True, return_logits=True)
    np.testing.assert_array_equal(a_ids, b_ids)
    np.testing.assert_array_equal(a_lg, b_lg)


def test_generate_count_window_and_eos(oracle):
    # InferenceTests.Generate_* :81-113
    c = cfg(oracle, **SMALL)
    w = oracle.init_weights(c, 10)
    u = oracle.net_random_doubles(7, 5)
    ids = oracle.generate(c, w, [1, 2], 5, temperature=1.0, uniforms=u)
    assert len(ids) == 5 and all(0 <= t < 32 for t in ids)
    long_prompt = np.arange(12) % 32
    assert len(oracle.generate(c, w, long_prompt, 6)) == 6
    first = oracle.generate(c, w, [3, 1], 1)[0]
    stopped = oracle.generate(c, w, [3, 1], 10, eos=int(first))
    assert list(stopped) == [first]


def test_pcg32_matches_independent_restatement(oracle, fhp):
    # PCG-XSH-RR (O'Neill 2014) with TrainingRandom's seeding; the C++ oracle and
    # the package's big-int Python version are separate implementations.
    for seed in (0, 1, 42, -5, 2**31 - 1):
        want = fhp.TrainingRandom(seed).ids(16384, 64)
        np.testing.assert_array_equal(oracle.pcg32_ids(seed, 16384, 64), want)
    # the rejection rule keeps the draw unbiased: bound 3 rejects values below 2^32 mod 3 == 1
    r = fhp.TrainingRandom(3)
    assert all(0 <= r.next(3) < 3 for _ in range(1000))


def test_net_random_stream_statistics(oracle):
    u = oracle.net_random_doubles(1, 200000)
    assert u.min() >= 0 and u.max() < 1
    assert abs(u.mean() - 0.5) < 0.005 and abs(u.var() - 1 / 12) < 0.002
    # different seeds give different streams; the same seed repeats
    np.testing.assert_array_equal(u[:100], oracle.net_random_doubles(1, 100))
    assert np.any(oracle.net_random_doubles(2, 100) != u[:100])


def test_net_random_published_values(oracle):
    # published outputs of .NET's seeded System.Random: new Random(1).Next() x3
    # (Next() is the raw sample, NextDouble() = sample / int.MaxValue) and
    # new Random(0).NextDouble(); a wrong seed constant, tap or sign fails these
    r1 = oracle.net_random_doubles(1, 3)
    assert [int(round(x * 2147483647)) for x in r1] == [534011718, 237820880, 1002897798]
    assert abs(oracle.net_random_doubles(0, 1)[0] - 0.7262432699679598) < 1e-15


# Published output of the pcg-c demo (pcg32-demo.c, M. O'Neill): pcg32_srandom_r(&rng, 42, 54)
# is TrainingRandom's seeding procedure (state 0, one step, state += seed, one step;
# TrainingRandom.cs:13-20) with the increment (54 << 1) | 1.  Its "Round 1" prints six raw
# outputs, 65 coin flips (pcg32_boundedrand_r(&rng, 2) ? 'H' : 'T') and 33 dice rolls
# (pcg32_boundedrand_r(&rng, 6) + 1); the bounded draw rejects values below -bound % bound,
# the rule of TrainingRandom.Next (:33-46).
PCG_DEMO_U32 = [0xA15C02B7, 0x7B47F409, 0xBA1D3330, 0x83D2F293, 0xBFA4784B, 0xCBED606E]
PCG_DEMO_COINS = "HHTTTHTHHHTHTTTHHHHHTTTHHHTHTHTHTTHTTTHHHHHHTTTTHHTTTTTHTTTTTTTHT"
PCG_DEMO_ROLLS = [3, 4, 1, 1, 2, 2, 3, 2, 4, 3, 2, 4, 3, 3, 5, 2, 3, 1, 3, 1, 5, 1, 4, 1, 5, 6, 4, 6, 6, 2, 6,
                  3, 3]


def _pcg_u32_variant(seed, inc, n, seed_first=False):
    """A deliberately different seeding (the seed added before the first step), to show
    the published vector tells it apart from TrainingRandom's."""
    m = (1 << 64) - 1
    st = [0]

    def step():
        old = st[0]
        st[0] = (old * 6364136223846793005 + inc) & m
        xs = (((old >> 18) ^ old) >> 27) & 0xFFFFFFFF
        rot = old >> 59
        return ((xs >> rot) | (xs << ((-rot) & 31))) & 0xFFFFFFFF

    if seed_first:
        st[0] = (st[0] + seed) & m
        step()
        step()
    return [step() for _ in range(n)]


def test_pcg32_published_demo_stream(oracle):
    inc = (54 << 1) | 1
    out = oracle.pcg32_stream(42, inc, [0] * 6 + [2] * 65 + [6] * 33)
    assert [int(v) for v in out[:6]] == PCG_DEMO_U32
    assert "".join("H" if v else "T" for v in out[6:71]) == PCG_DEMO_COINS
    assert [int(v) + 1 for v in out[71:]] == PCG_DEMO_ROLLS
    # the vector discriminates: adding the seed before the first step gives another stream
    assert _pcg_u32_variant(42, inc, 6, seed_first=True) != PCG_DEMO_U32
    # and the oracle's default increment is TrainingRandom's (:16)
    np.testing.assert_array_equal(oracle.pcg32_stream(7, 0xDA3E39CB94B95BDB, [16384] * 32),
                                  oracle.pcg32_ids(7, 16384, 32).astype(np.uint32))


def test_fill_normal_first_pairs_exact(oracle):
    # Tensor.FillNormal (Tensor.cs:79-91) from new Random(1), whose first three samples are
    # published (534011718, 237820880, 1002897798; NextDouble = sample / int.MaxValue):
    # tok_emb[0..1] are the first Box-Muller pair, computed in double, times the float std
    # widened to double, then cast to float.
    import math
    c = oracle.Config(32, 8, 16, 1, 2)
    w = oracle.init_weights(c, 1)
    n1, n2, n3 = (v / 2147483647 for v in (534011718, 237820880, 1002897798))
    std = float(np.float32(0.02))

    def pair(u1, u2):
        r = math.sqrt(-2.0 * math.log(u1))
        return (np.float32(r * math.cos(2 * math.pi * u2) * std), np.float32(r * math.sin(2 * math.pi * u2) * std))

    want = pair(1.0 - n1, n2)
    assert (w[0], w[1]) == want  # bit for bit
    # planted mistakes move these values: cos/sin swapped, u1 = NextDouble(), the draws taken
    # in the other order, one member duplicated
    assert (want[1], want[0]) != want
    assert pair(n1, n2) != want and pair(1.0 - n2, n1) != want and want[0] != want[1]
    # the second pair's radius is fixed by the third sample alone: u1 = 1 - NextDouble()
    radius = math.hypot(float(w[2]), float(w[3])) / std
    assert abs(radius - math.sqrt(-2.0 * math.log(1.0 - n3))) < 2e-6 * radius


# ---- golden vectors --------------------------------------------------------------------------

def test_golden_c1_greedy(oracle):
    g = np.load(os.path.join(GOLDEN, "c1_greedy.npz"))
    c = oracle.Config(2256, 128, 128, 4, 4)
    w = oracle.init_weights(c, 1234)
    prompt = oracle.pcg32_ids(42, 2256, 16)
    np.testing.assert_array_equal(prompt, g["prompt"])
    ids, lg = oracle.generate(c, w, prompt, 200, kv_cached=True, return_logits=True)
    np.testing.assert_array_equal(ids, g["ids"])
    np.testing.assert_array_equal(lg[g["full_steps"]], g["full_logits"])


def test_golden_tiny_forward(oracle):
    g = np.load(os.path.join(GOLDEN, "tiny_forward.npz"))
    c = cfg(oracle, **SMALL)
    np.testing.assert_array_equal(oracle.forward(c, oracle.init_weights(c, 6), g["ids"]), g["logits"])


def test_golden_net_random(oracle):
    g = np.load(os.path.join(GOLDEN, "net_random.npz"))
    for s in (0, 1, 42):
        np.testing.assert_array_equal(oracle.net_random_doubles(s, 1000), g[f"seed{s}"])


# ---- the forward's composition (Layers.cs:384-392, GptModel.cs:212-222) ---------------------
# The ops above are pinned one by one; these pin how the oracle composes them: block
# order, residual placement, head layout, the causal mask and LN_f before the tied head.
# Parameters are "trained-like" (LayerNorm affine and biases away from 1/0), so every
# LayerNorm and bias term contributes.

import gpt_f64  # noqa: E402

COMP = (97, 24, 32, 3, 4)  # V, ctx, d, L, H: small enough for float64 numpy


def _comp_weights(oracle, seed=3):
    # qkv weights scaled up 8x: at the initial std the scores are so small that the
    # softmax is nearly uniform, and a wrong head layout would hardly show
    c = oracle.Config(*COMP)
    w = oracle.trained_like(c, oracle.init_weights(c, seed), seed + 100)
    for n, v in oracle.params(c, w).items():
        if n.endswith("attn.qkv.w"):
            v *= 8
    return c, w


def _rel(a, e):
    return float(np.max(np.abs(np.asarray(a, np.float64) - e) / np.maximum(1.0, np.abs(e))))


def test_forward_single_token_closed_form(oracle):
    # T = 1: the causal softmax over one key is exactly 1, so attention returns v
    # itself; every block is then a closed form in x alone (no score, no softmax)
    c, w = _comp_weights(oracle)
    P = {n: v.astype(np.float64) for n, v in oracle.params(c, w).items()}
    V, ctx, d, L, H = COMP

    def ln(x, a, b):
        mu = x.mean()
        return (x - mu) / np.sqrt(((x - mu) ** 2).mean() + 1e-5) * a + b

    for tok in (0, 41, 96):
        x = P["tok_emb"][tok] + P["pos_emb"][0]
        for i in range(L):
            g = lambda k: P[f"blocks.{i}.{k}"]  # noqa: E731
            v = (ln(x, g("ln1.w"), g("ln1.b")) @ g("attn.qkv.w") + g("attn.qkv.b"))[2 * d:]
            a = v @ g("attn.proj.w") + g("attn.proj.b") + x
            f = ln(a, g("ln2.w"), g("ln2.b")) @ g("mlp.fc.w") + g("mlp.fc.b")
            x = 0.5 * f * (1 + np.tanh(np.sqrt(2 / np.pi) * (f + 0.044715 * f ** 3))) @ g("mlp.proj.w") \
                + g("mlp.proj.b") + a
        want = ln(x, P["ln_f.w"], P["ln_f.b"]) @ P["tok_emb"].T
        assert _rel(oracle.forward(c, w, [tok])[0], want) <= 1e-5


def test_forward_with_zero_blocks_is_ln_f_of_embeddings(oracle):
    # every block matrix and bias zero: v = 0 so attention adds 0, fc = 0 so GELU(0) = 0
    # and the MLP adds 0; each row's logits are LN_f(tok + pos) tok_emb^T, exactly
    # the embedding path and the tied head
    c, w = _comp_weights(oracle)
    P = oracle.params(c, w)
    for n, v in P.items():
        if n.startswith("blocks.") and not n.endswith(("ln1.w", "ln1.b", "ln2.w", "ln2.b")):
            v[...] = 0
    ids = [5, 17, 5, 90, 0, 33, 62]
    x = P["tok_emb"][ids].astype(np.float64) + P["pos_emb"][:len(ids)]
    mu = x.mean(1, keepdims=True)
    xn = (x - mu) / np.sqrt(((x - mu) ** 2).mean(1, keepdims=True) + 1e-5) * P["ln_f.w"] + P["ln_f.b"]
    assert _rel(oracle.forward(c, w, ids), xn @ P["tok_emb"].T.astype(np.float64)) <= 1e-5


@pytest.mark.parametrize("which", ["attn.proj.b", "mlp.proj.b"])
def test_forward_with_only_output_biases_adds_them(oracle, which):
    # only the output bias of one sub-block non-zero: each block adds exactly that bias
    # to the residual stream (attention of v = 0 and an MLP of fc = 0 contribute
    # nothing else), so the final x is tok + pos + sum over blocks of the bias
    c, w = _comp_weights(oracle)
    P = oracle.params(c, w)
    total = np.zeros(COMP[2])
    for n, v in P.items():
        if n.startswith("blocks.") and not n.endswith(("ln1.w", "ln1.b", "ln2.w", "ln2.b", which)):
            v[...] = 0
        if n.endswith(which):
            total += v
    ids = [7, 3, 3, 80]
    x = P["tok_emb"][ids].astype(np.float64) + P["pos_emb"][:len(ids)] + total
    mu = x.mean(1, keepdims=True)
    xn = (x - mu) / np.sqrt(((x - mu) ** 2).mean(1, keepdims=True) + 1e-5) * P["ln_f.w"] + P["ln_f.b"]
    assert _rel(oracle.forward(c, w, ids), xn @ P["tok_emb"].T.astype(np.float64)) <= 1e-5


def test_forward_matches_float64_restatement(oracle):
    # the whole window (every row, causal attention over 4 heads, 3 blocks) against an
    # independent float64 statement of the reference forward
    c, w = _comp_weights(oracle)
    ids = oracle.pcg32_ids(9, COMP[0], COMP[1])
    want = gpt_f64.forward(oracle.param_layout(c), w, COMP[4], ids)
    assert _rel(oracle.forward(c, w, ids), want) <= 1e-5


@pytest.mark.parametrize("mutation", gpt_f64.MUTATIONS)
def test_composition_checks_catch_mutations(oracle, mutation):
    # each plausible composition mistake (post-LN blocks, a dropped residual, no causal
    # mask, no LN_f, K and V swapped, heads taken as interleaved columns, LN1's
    # parameters reused for LN2) moves the logits far outside the 1e-5 bar the oracle
    # meets above, so the comparison would catch it in the oracle
    c, w = _comp_weights(oracle)
    ids = oracle.pcg32_ids(9, COMP[0], COMP[1])
    good = gpt_f64.forward(oracle.param_layout(c), w, COMP[4], ids)
    bad = gpt_f64.forward(oracle.param_layout(c), w, COMP[4], ids, mutate=mutation)
    assert _rel(bad, good) > 1e-3, mutation
