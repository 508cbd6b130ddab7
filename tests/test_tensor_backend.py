"""The op-level ITensorBackend of the hip backend (fh_op_*, forge_hip.tensor_backend).

CPU tests pin the oracle's restatement of the rest of CpuBackend (training ops) the
way the reference's own CpuBackendTests do: brute-force matmuls, the cross-entropy
hand literal, the AdamW first-step closed form, and finite-difference gradient checks
of every backward kernel against the oracle's forward (CpuBackendTests.cs:86-540,
TrainingTests.cs:40-51).  GPU tests are the reference's device-backend contract
(GpuBackendTests.cs:110-600, CudaBackendTests.cs:274-335) run through the C ABI: each
kernel against the oracle on the same inputs, with the reference's tolerances
(1e-4 forward, 1e-2 backward, exact for copies, gathers and masks), plus the
residency contract and the error paths.  Inputs come from the restated seeded
System.Random with the reference tests' seeds and Box-Muller helper (the stream
itself is parity unpinned vs .NET); index arrays use numpy generators.
"""
import numpy as np
import pytest

FWD, BWD = 1e-4, 1e-2


class NetRng:
    """Sequential NextDouble draws of new Random(seed) (restated generator)."""

    def __init__(self, oracle, seed, n=1 << 16):
        self.d = oracle.net_random_doubles(seed, n)
        self.i = 0

    def next_double(self):
        v = self.d[self.i]
        self.i += 1
        return v

    def rand(self, n, std=1.0):
        """GpuBackendTests.Rand: Box-Muller pairs (cos, sin) in double."""
        out = np.empty(n, np.float32)
        for i in range(0, n, 2):
            u1 = 1.0 - self.next_double()
            u2 = self.next_double()
            r = np.sqrt(-2.0 * np.log(u1))
            out[i] = np.float32(r * np.cos(2 * np.pi * u2) * std)
            if i + 1 < n:
                out[i + 1] = np.float32(r * np.sin(2 * np.pi * u2) * std)
        return out


def near_rel(actual, expected, tol):
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    assert a.shape == e.shape
    if tol == 0:
        np.testing.assert_array_equal(np.asarray(actual), np.asarray(expected))
        return
    err = np.abs(a - e) / np.maximum(1.0, np.abs(e))
    assert not np.any(np.isnan(err)), "NaN"
    assert err.max(initial=0.0) <= tol, f"max rel/abs diff {err.max():.3g} > {tol}"


def naive_matmul(a, b, M, K, N, ta, tb):
    A = np.asarray(a, np.float64).reshape((K, M) if ta else (M, K))
    B = np.asarray(b, np.float64).reshape((N, K) if tb else (K, N))
    return ((A.T if ta else A) @ (B.T if tb else B)).reshape(-1)


def check_grad(analytic, param, loss, eps=1e-2, tol=2e-2):
    """Central differences of a float32 loss against the analytic gradient."""
    for i in range(param.size):
        old = param[i]
        param[i] = old + eps
        lp = loss()
        param[i] = old - eps
        lm = loss()
        param[i] = old
        num = (lp - lm) / (2 * eps)
        assert abs(num - analytic[i]) <= tol * max(1.0, abs(num)), (i, num, analytic[i])


# ---- CPU: the oracle's restatement pinned ----------------------------------------------

@pytest.mark.parametrize("mode,seed", [("nn", 1), ("nt", 2), ("tn", 3)])
def test_oracle_matmuls_match_naive(oracle, mode, seed):
    # CpuBackendTests.MatMulNN/NT/TN_Forward, plain and accumulating
    rng = NetRng(oracle, seed)
    M, K, N = 3, 5, 4
    a = rng.rand(M * K)
    b = rng.rand(K * N)
    y = np.zeros(M * N, np.float32)
    oracle.op_matmul(mode, a, b, y, M, K, N)
    ref = naive_matmul(a, b, M, K, N, mode == "tn", mode == "nt")
    near_rel(y, ref, 1e-4)
    y[:] = -1.5
    oracle.op_matmul(mode, a, b, y, M, K, N, accumulate=True)
    near_rel(y, ref - 1.5, 1e-4)
    # batched: slot s is the plain product of slot s's operands
    S = 3
    a3, b3 = rng.rand(S * M * K), rng.rand(S * K * N)
    y3 = np.zeros(S * M * N, np.float32)
    oracle.op_matmul(mode, a3, b3, y3, M, K, N, slots=S)
    for s in range(S):
        near_rel(y3[s * M * N:(s + 1) * M * N],
                 naive_matmul(a3[s * M * K:(s + 1) * M * K], b3[s * K * N:(s + 1) * K * N], M, K, N, mode == "tn",
                              mode == "nt"), 1e-4)


def test_oracle_rows_and_elementwise(oracle):
    # CpuBackendTests.Transpose_MatchesNaive, AddBiasSumRowsScaleAddInPlace
    rng = NetRng(oracle, 5)
    rows, cols = 3, 4
    y, bias = rng.rand(rows * cols), rng.rand(cols)
    want = y.reshape(rows, cols) + bias
    oracle.op_add_bias(y, bias, rows, cols)
    np.testing.assert_allclose(y.reshape(rows, cols), want, atol=1e-6)
    db = rng.rand(cols)
    prior = db.copy()
    oracle.op_sum_rows(y, db, rows, cols)
    np.testing.assert_allclose(db, prior + y.reshape(rows, cols).sum(0), atol=1e-5)
    z = rng.rand(rows * cols)
    zc = z.copy()
    oracle.op_scale(z, 2.5)
    np.testing.assert_allclose(z, zc * 2.5, atol=1e-5)
    oracle.op_add_in_place(z, zc)
    np.testing.assert_allclose(z, zc * 3.5, atol=1e-5)
    x = rng.rand(15)
    out = np.zeros(15, np.float32)
    oracle.op_transpose(x, out, 3, 5)
    np.testing.assert_array_equal(out.reshape(5, 3), x.reshape(3, 5).T)


def test_oracle_heads_block_mask_embedding(oracle):
    batch, T, H, hd = 3, 7, 2, 5
    D = H * hd
    src = np.arange(batch * T * 3 * D, dtype=np.float32)
    q = np.zeros(batch * H * T * hd, np.float32)
    oracle.op_pack_heads(src, 3 * D, q, batch, T, H, hd, D)
    s3 = src.reshape(batch, T, 3, H, hd)[:, :, 1]  # the K block: [batch, T, H, hd]
    np.testing.assert_array_equal(q.reshape(batch, H, T, hd), s3.transpose(0, 2, 1, 3))
    back = np.zeros_like(src)
    oracle.op_unpack_heads(q, back, 3 * D, batch, T, H, hd, D)
    np.testing.assert_array_equal(back.reshape(batch, T, 3, D)[:, :, 1], src.reshape(batch, T, 3, D)[:, :, 1])
    assert not back.reshape(batch, T, 3, D)[:, :, [0, 2]].any()
    # CopyBlock extract: a 7x23 block at (5, 11) of a [33, 65] into (3, 7) of a zeroed [12, 40]
    y = np.arange(33 * 65, dtype=np.float32)
    blk = np.zeros(12 * 40, np.float32)
    oracle.op_copy_block(y, 65, blk, 40, 5, 11, 3, 7, 7, 23)
    want = np.zeros((12, 40), np.float32)
    want[3:10, 7:30] = y.reshape(33, 65)[5:12, 11:34]
    np.testing.assert_array_equal(blk.reshape(12, 40), want)
    # CausalMask_SetsUpperTriangle over two packed blocks
    T = 4
    sc = np.ones(2 * T * T, np.float32)
    oracle.op_causal_mask(sc, T)
    tri = np.triu(np.ones((T, T), bool), 1)
    for blkn in range(2):
        m = sc[blkn * T * T:(blkn + 1) * T * T].reshape(T, T)
        assert np.all(np.isneginf(m[tri])) and np.all(m[~tri] == 1)
    # Embedding_Lookup
    table = np.arange(5 * 3, dtype=np.float32)
    out = np.zeros(4 * 3, np.float32)
    oracle.op_embedding_forward(table, [0, 2, 2, 4], out, 3)
    np.testing.assert_array_equal(out.reshape(4, 3), table.reshape(5, 3)[[0, 2, 2, 4]])


def test_oracle_layernorm_forward_statistics(oracle):
    # LayerNormForward with its cached statistics: out equals the inference
    # restatement bit for bit, mean and rstd are the row's mean and 1/sqrt(var+eps)
    rng = NetRng(oracle, 104)
    rows, cols, eps = 5, 48, 1e-5
    x, w, b = rng.rand(rows * cols), rng.rand(cols), rng.rand(cols)
    out, mean, rstd = np.zeros(rows * cols, np.float32), np.zeros(rows, np.float32), np.zeros(rows, np.float32)
    oracle.op_layernorm_forward(x, w, b, out, mean, rstd, rows, cols, eps)
    ref = oracle.layernorm(x.reshape(rows, cols), w, b, eps)
    np.testing.assert_array_equal(out.reshape(rows, cols), ref)
    X = x.reshape(rows, cols).astype(np.float64)
    np.testing.assert_allclose(mean, X.mean(1), atol=1e-6)
    np.testing.assert_allclose(rstd, 1 / np.sqrt(X.var(1) + eps), rtol=1e-5)


def test_oracle_cross_entropy_hand_literal(oracle):
    # CpuBackendTests.CrossEntropy_MatchesLogSoftmax
    T, V = 3, 4
    logits = np.array([1, 2, 0.5, -1, 0, 0, 0, 0, -2, 3, 1, 0], np.float32)
    targets = [1, 99, 0]
    probs = np.zeros(T * V, np.float32)
    loss = oracle.op_cross_entropy_forward(logits, targets, probs, T, V, 99)
    exp = 0.0
    for t in range(T):
        if targets[t] == 99:
            continue
        row = logits[t * V:(t + 1) * V].astype(np.float64)
        mx = row.max()
        exp += np.log(np.exp(row - mx).sum()) + mx - row[targets[t]]
    assert abs(loss - exp / 2) <= 1e-4
    np.testing.assert_allclose(probs.reshape(T, V).sum(1), 1.0, atol=1e-5)
    np.testing.assert_allclose(probs[V:2 * V], 0.25, atol=1e-6)


def test_oracle_cross_entropy_aliased_equals_separate(oracle):
    # CpuBackendTests.CrossEntropy_AliasedInPlaceMatchesSeparate
    rng = NetRng(oracle, 42)
    T, V = 3, 5
    logits = np.array([rng.next_double() * 4 - 2 for _ in range(T * V)], np.float32)
    targets = [2, 99, 0]
    pr = np.zeros_like(logits)
    lr_ = oracle.op_cross_entropy_forward(logits.copy(), targets, pr, T, V, 99)
    dr = np.zeros_like(logits)
    oracle.op_cross_entropy_backward(pr, targets, dr, T, V, 99)
    buf = logits.copy()
    l2 = oracle.op_cross_entropy_forward(buf, targets, buf, T, V, 99)
    assert l2 == lr_
    np.testing.assert_array_equal(buf, pr)
    oracle.op_cross_entropy_backward(buf, targets, buf, T, V, 99)
    np.testing.assert_array_equal(buf, dr)


def test_oracle_gradient_checks(oracle):
    # CpuBackendTests.*Backward_GradCheck: every backward kernel against central
    # differences of the oracle's own forward
    rng = NetRng(oracle, 42)
    M, K, N = 3, 4, 2
    a, b, dY = rng.rand(M * K), rng.rand(K * N), rng.rand(M * N)

    def mm_loss():
        y = np.zeros(M * N, np.float32)
        oracle.op_matmul("nn", a, b, y, M, K, N)
        return float(np.dot(y.astype(np.float64), dY))

    dA = np.zeros(M * K, np.float32)
    dB = np.zeros(K * N, np.float32)
    oracle.op_matmul("nt", dY, b, dA, M, N, K)
    oracle.op_matmul("tn", a, dY, dB, K, M, N)
    check_grad(dA, a, mm_loss)
    check_grad(dB, b, mm_loss)

    rows, cols = 3, 4
    x, w, bb, dO = rng.rand(rows * cols), rng.rand(cols), rng.rand(cols), rng.rand(rows * cols)
    mean, rstd = np.zeros(rows, np.float32), np.zeros(rows, np.float32)

    def ln_loss():
        out = np.zeros(rows * cols, np.float32)
        oracle.op_layernorm_forward(x, w, bb, out, mean, rstd, rows, cols, 1e-5)
        return float(np.dot(out.astype(np.float64), dO))

    ln_loss()
    dX, dW, dBb = np.zeros(rows * cols, np.float32), np.zeros(cols, np.float32), np.zeros(cols, np.float32)
    oracle.op_layernorm_backward(dO, x, w, mean, rstd, dX, dW, dBb, rows, cols)
    check_grad(dX, x, ln_loss)
    check_grad(dW, w, ln_loss)
    check_grad(dBb, bb, ln_loss)

    xs, dOs = rng.rand(rows * cols), rng.rand(rows * cols)

    def sm_loss():
        s = xs.copy()
        oracle.op_softmax_forward(s, rows, cols)
        return float(np.dot(s.astype(np.float64), dOs))

    s = xs.copy()
    oracle.op_softmax_forward(s, rows, cols)
    dXs = np.zeros_like(s)
    oracle.op_softmax_backward(dOs, s, dXs, rows, cols)
    check_grad(dXs, xs, sm_loss)

    xg, dOg = rng.rand(12), rng.rand(12)

    def gelu_loss():
        yv = np.zeros(12, np.float32)
        oracle.op_gelu_forward(xg, yv)
        return float(np.dot(yv.astype(np.float64), dOg))

    dXg = np.zeros(12, np.float32)
    oracle.op_gelu_backward(dOg, xg, dXg)
    check_grad(dXg, xg, gelu_loss)

    V, D = 5, 3
    table = rng.rand(V * D)
    idx = [0, 2, 2, 4]
    dOe = rng.rand(len(idx) * D)

    def emb_loss():
        out = np.zeros(len(idx) * D, np.float32)
        oracle.op_embedding_forward(table, idx, out, D)
        return float(np.dot(out.astype(np.float64), dOe))

    dT = np.zeros(V * D, np.float32)
    oracle.op_embedding_backward(dOe, idx, dT, D)
    check_grad(dT, table, emb_loss)
    np.testing.assert_allclose(dT[2 * D:3 * D], dOe[D:2 * D] + dOe[2 * D:3 * D], atol=1e-6)
    assert not dT[D:2 * D].any()

    T, Vc = 3, 4
    lg = rng.rand(T * Vc)
    tg = [1, 99, 0]

    def ce_loss():
        return oracle.op_cross_entropy_forward(lg, tg, np.zeros(T * Vc, np.float32), T, Vc, 99)

    pr = np.zeros(T * Vc, np.float32)
    oracle.op_cross_entropy_forward(lg, tg, pr, T, Vc, 99)
    dl = np.zeros(T * Vc, np.float32)
    oracle.op_cross_entropy_backward(pr, tg, dl, T, Vc, 99)
    check_grad(dl, lg, ce_loss)
    assert not dl[Vc:2 * Vc].any()


def test_oracle_adamw_first_step_and_decay(oracle):
    # TrainingTests.AdamW_FirstStepMovesByAboutLr: mhat = vhat = g after the bias
    # correction, so the first step moves w by lr * g / (|g| + eps) ~ lr
    w, g = np.array([1.0], np.float32), np.array([1.0], np.float32)
    m, v = np.zeros(1, np.float32), np.zeros(1, np.float32)
    oracle.op_adamw(w, g, m, v, 0.1, 0.9, 0.999, 1e-8, 0.0, 1, True)
    assert abs(w[0] - 0.9) <= 1e-4
    # the moments are (1 - beta) * g in float32: (1 - 0.9f) = 0.100000024f
    assert m[0] == np.float32(1) - np.float32(0.9) and v[0] == np.float32(1) - np.float32(0.999)
    # decoupled decay only for matrices: w -= lr*wd*w before the Adam step
    for matrix in (True, False):
        w2, m2, v2 = np.array([2.0], np.float32), np.zeros(1, np.float32), np.zeros(1, np.float32)
        oracle.op_adamw(w2, np.array([0.5], np.float32), m2, v2, 0.01, 0.9, 0.95, 1e-8, 0.1, 1, matrix)
        dec = 2.0 - (0.01 * 0.1 * 2.0 if matrix else 0.0)
        assert abs(w2[0] - (dec - 0.01 * 0.5 / (0.5 + 1e-8))) <= 1e-6


def test_oracle_sum_squares(oracle):
    x = np.random.default_rng(0).standard_normal(100003).astype(np.float32)
    assert abs(oracle.op_sum_squares(x) - float(np.dot(x.astype(np.float64), x))) <= 1e-9 * x.size


def test_python_tensor_mirror(fhp):
    # Tensor.cs: shape ctor zero-fills, data ctor checks the element count
    t = fhp.Tensor(2, 3)
    assert t.Shape == (2, 3) and t.Rank == 2 and t.Length == 6 and t.Cols == 3 and t.Rows == 2
    assert not t.Data.any()
    u = fhp.Tensor(np.arange(6), 3, 2)
    assert u.Data.dtype == np.float32 and u.Cols == 2
    with pytest.raises(ValueError):
        fhp.Tensor(np.arange(5), 3, 2)


# ---- GPU: the device-backend contract ------------------------------------------------------

@pytest.fixture(scope="module")
def tb(fhp):
    b = fhp.HipTensorBackend(0)
    yield b
    b.Dispose()


def dup(fhp, data, *shape):
    return fhp.Tensor(np.array(data, np.float32, copy=True), *shape)


@pytest.mark.gpu
def test_matmul_matches_cpu(fhp, oracle, tb):
    # GpuBackendTests.MatMul_MatchesCpu, plus a size that takes the MFMA GEMM
    rng = NetRng(oracle, 101, 1 << 20)
    for M, K, N in [(37, 53, 29), (128, 256, 192), (256, 512, 384)]:
        a, bN, bT, prior = rng.rand(M * K), rng.rand(K * N), rng.rand(N * K), rng.rand(M * N)
        for acc in (False, True):
            for mode, bb in (("nn", bN), ("nt", bT), ("tn", bN)):
                yc = prior.copy()
                oracle.op_matmul(mode, a, bb, yc, M, K, N, accumulate=acc)
                yg = dup(fhp, prior, M, N)
                fn = {"nn": tb.MatMulNN, "nt": tb.MatMulNT, "tn": tb.MatMulTN}[mode]
                ashape = (K, M) if mode == "tn" else (M, K)
                bshape = (N, K) if mode == "nt" else (K, N)
                fn(dup(fhp, a, *ashape), dup(fhp, bb, *bshape), yg, M, K, N, acc)
                tb.EnsureHostCurrent(yg)
                near_rel(yg.Data, yc, FWD)


@pytest.mark.gpu
def test_elementwise_matches_cpu(fhp, oracle, tb):
    # GpuBackendTests.Elementwise_MatchesCpu
    rng = NetRng(oracle, 102)
    rows, cols = 33, 65
    y, bias = rng.rand(rows * cols), rng.rand(cols)
    yc, yg = y.copy(), dup(fhp, y, rows, cols)
    oracle.op_add_bias(yc, bias, rows, cols)
    tb.AddBias(yg, dup(fhp, bias, cols), rows, cols)
    tb.EnsureHostCurrent(yg)
    near_rel(yg.Data, yc, FWD)
    db0 = rng.rand(cols)
    dbc, dbg = db0.copy(), dup(fhp, db0, cols)
    oracle.op_sum_rows(y, dbc, rows, cols)
    tb.SumRows(dup(fhp, y, rows, cols), dbg, rows, cols)
    tb.EnsureHostCurrent(dbg)
    near_rel(dbg.Data, dbc, BWD)
    src = rng.rand(rows * cols)
    yc, yg = y.copy(), dup(fhp, y, rows, cols)
    oracle.op_add_in_place(yc, src)
    tb.AddInPlace(yg, dup(fhp, src, rows, cols))
    tb.EnsureHostCurrent(yg)
    near_rel(yg.Data, yc, FWD)
    yc, yg = y.copy(), dup(fhp, y, rows, cols)
    oracle.op_scale(yc, -1.75)
    tb.Scale(yg, -1.75)
    tb.EnsureHostCurrent(yg)
    near_rel(yg.Data, yc, FWD)
    trc, trg = np.zeros(cols * rows, np.float32), fhp.Tensor(cols, rows)
    oracle.op_transpose(y, trc, rows, cols)
    tb.Transpose(dup(fhp, y, rows, cols), trg, rows, cols)
    tb.EnsureHostCurrent(trg)
    near_rel(trg.Data, trc, 0)
    cpg = fhp.Tensor(rows, cols)
    tb.Copy(dup(fhp, y, rows, cols), cpg)
    tb.EnsureHostCurrent(cpg)
    near_rel(cpg.Data, y, 0)
    blkc, blkg = np.zeros(12 * 40, np.float32), fhp.Tensor(12, 40)
    oracle.op_copy_block(y, cols, blkc, 40, 5, 11, 3, 7, 7, 23)
    tb.CopyBlock(dup(fhp, y, rows, cols), blkg, 5, 11, 3, 7, 7, 23)
    tb.EnsureHostCurrent(blkg)
    near_rel(blkg.Data, blkc, 0)
    intoc, intog = y.copy(), dup(fhp, y, rows, cols)
    oracle.op_copy_block(blkc, 40, intoc, cols, 3, 7, 9, 30, 7, 23)
    tb.CopyBlock(dup(fhp, blkc, 12, 40), intog, 3, 7, 9, 30, 7, 23)
    tb.EnsureHostCurrent(intog)
    near_rel(intog.Data, intoc, 0)  # the partial write keeps the rest


@pytest.mark.gpu
def test_flat_dispatch_beyond_one_dimension(fhp, tb):
    # GpuBackendTests.FlatDispatch_BeyondOneDimensionalLimit: 5,000,123 elements
    n = 5_000_123
    r = np.random.default_rng(103)
    a, b = r.standard_normal(n).astype(np.float32), r.standard_normal(n).astype(np.float32)
    ag = dup(fhp, a, n)
    tb.AddInPlace(ag, dup(fhp, b, n))
    tb.EnsureHostCurrent(ag)
    near_rel(ag.Data, a + b, FWD)


@pytest.mark.gpu
@pytest.mark.parametrize("rows,cols", [(33, 64), (300, 768)])
def test_layernorm_matches_cpu(fhp, oracle, tb, rows, cols):
    # GpuBackendTests.LayerNorm_MatchesCpu (and a 300-row case: column sums over chunks)
    rng = NetRng(oracle, 104, 1 << 20)
    eps = 1e-5
    x, w, b = rng.rand(rows * cols), rng.rand(cols), rng.rand(cols)
    oc, mc, rc = np.zeros(rows * cols, np.float32), np.zeros(rows, np.float32), np.zeros(rows, np.float32)
    oracle.op_layernorm_forward(x, w, b, oc, mc, rc, rows, cols, eps)
    og, mg, rg = fhp.Tensor(rows, cols), fhp.Tensor(rows), fhp.Tensor(rows)
    tb.LayerNormForward(dup(fhp, x, rows, cols), dup(fhp, w, cols), dup(fhp, b, cols), og, mg, rg, rows, cols, eps)
    for t in (og, mg, rg):
        tb.EnsureHostCurrent(t)
    near_rel(og.Data, oc, FWD)
    near_rel(mg.Data, mc, FWD)
    near_rel(rg.Data, rc, FWD)
    dO, dw0, db0 = rng.rand(rows * cols), rng.rand(cols), rng.rand(cols)
    dxc, dwc, dbc = np.zeros(rows * cols, np.float32), dw0.copy(), db0.copy()
    oracle.op_layernorm_backward(dO, x, w, mc, rc, dxc, dwc, dbc, rows, cols)
    dxg, dwg, dbg = fhp.Tensor(rows, cols), dup(fhp, dw0, cols), dup(fhp, db0, cols)
    tb.LayerNormBackward(dup(fhp, dO, rows, cols), dup(fhp, x, rows, cols), dup(fhp, w, cols), dup(fhp, mc, rows),
                         dup(fhp, rc, rows), dxg, dwg, dbg, rows, cols)
    for t in (dxg, dwg, dbg):
        tb.EnsureHostCurrent(t)
    near_rel(dxg.Data, dxc, BWD)
    near_rel(dwg.Data, dwc, BWD)
    near_rel(dbg.Data, dbc, BWD)


@pytest.mark.gpu
def test_softmax_and_gelu_match_cpu(fhp, oracle, tb):
    # GpuBackendTests.Softmax_MatchesCpu, Gelu_MatchesCpu
    rng = NetRng(oracle, 105, 1 << 17)
    rows, cols = 29, 257
    x = rng.rand(rows * cols, 3.0)
    xc, xg = x.copy(), dup(fhp, x, rows, cols)
    oracle.op_softmax_forward(xc, rows, cols)
    tb.SoftmaxForward(xg, rows, cols)
    tb.EnsureHostCurrent(xg)
    near_rel(xg.Data, xc, FWD)
    dO = rng.rand(rows * cols)
    dxc, dxg = np.zeros(rows * cols, np.float32), fhp.Tensor(rows, cols)
    oracle.op_softmax_backward(dO, xc, dxc, rows, cols)
    tb.SoftmaxBackward(dup(fhp, dO, rows, cols), dup(fhp, xc, rows, cols), dxg, rows, cols)
    tb.EnsureHostCurrent(dxg)
    near_rel(dxg.Data, dxc, BWD)
    rng = NetRng(oracle, 106, 1 << 16)
    n = 10_003
    x = rng.rand(n, 2.0)
    oc, og = np.zeros(n, np.float32), fhp.Tensor(n)
    oracle.op_gelu_forward(x, oc)
    tb.GeluForward(dup(fhp, x, n), og)
    tb.EnsureHostCurrent(og)
    near_rel(og.Data, oc, FWD)
    dO = rng.rand(n)
    dc, dg = np.zeros(n, np.float32), fhp.Tensor(n)
    oracle.op_gelu_backward(dO, x, dc)
    tb.GeluBackward(dup(fhp, dO, n), dup(fhp, x, n), dg)
    tb.EnsureHostCurrent(dg)
    near_rel(dg.Data, dc, FWD)


@pytest.mark.gpu
def test_embedding_and_mask_match_cpu(fhp, oracle, tb):
    # GpuBackendTests.Embedding_MatchesCpu (heavy duplication) and CausalMask_MatchesCpu;
    # the scatter-add adds each id's rows in position order, so it equals the CPU loop
    rng = NetRng(oracle, 107)
    V, D, Tn = 51, 37, 96
    table = rng.rand(V * D)
    idx = np.random.default_rng(107).integers(0, V // 3, Tn).astype(np.int32)
    oc, og = np.zeros(Tn * D, np.float32), fhp.Tensor(Tn, D)
    oracle.op_embedding_forward(table, idx, oc, D)
    tb.EmbeddingForward(dup(fhp, table, V, D), idx, og, D)
    tb.EnsureHostCurrent(og)
    near_rel(og.Data, oc, 0)
    dO, dt0 = rng.rand(Tn * D), rng.rand(V * D)
    dtc, dtg = dt0.copy(), dup(fhp, dt0, V, D)
    oracle.op_embedding_backward(dO, idx, dtc, D)
    tb.EmbeddingBackward(dup(fhp, dO, Tn, D), idx, dtg, D)
    tb.EnsureHostCurrent(dtg)
    near_rel(dtg.Data, dtc, 0)
    rng = NetRng(oracle, 108)
    T = 47
    s = rng.rand(T * T * 3)
    sc, sg = s.copy(), dup(fhp, s, 3 * T, T)
    oracle.op_causal_mask(sc, T)
    tb.CausalMask(sg, T)
    tb.EnsureHostCurrent(sg)
    near_rel(sg.Data, sc, 0)
    with pytest.raises(fhp.ArgumentError, match="outside the table"):
        tb.EmbeddingForward(dup(fhp, table, V, D), [0, V], fhp.Tensor(2, D), D)


@pytest.mark.gpu
@pytest.mark.parametrize("aliased", [False, True])
def test_cross_entropy_matches_cpu(fhp, oracle, tb, aliased):
    # GpuBackendTests.CrossEntropy_MatchesCpu / CrossEntropy_AliasedInPlaceMatchesCpu
    rng = NetRng(oracle, 110 if aliased else 109, 1 << 17)
    T, V, ignore = 61, 389, -1
    logits = rng.rand(T * V, 2.0)
    targets = np.random.default_rng(109).integers(0, V, T).astype(np.int32)
    targets[7] = targets[58] = ignore
    pc = np.zeros(T * V, np.float32)
    lc = oracle.op_cross_entropy_forward(logits, targets, pc, T, V, ignore)
    dlc = np.zeros(T * V, np.float32)
    oracle.op_cross_entropy_backward(pc, targets, dlc, T, V, ignore)
    if aliased:
        buf = dup(fhp, logits, T, V)
        lg = tb.CrossEntropyForward(buf, targets, buf, T, V, ignore)
        tb.EnsureHostCurrent(buf)
        near_rel(buf.Data, pc, FWD)
        tb.CrossEntropyBackward(buf, targets, buf, T, V, ignore)
        tb.EnsureHostCurrent(buf)
        near_rel(buf.Data, dlc, BWD)
    else:
        pg = fhp.Tensor(T, V)
        lg = tb.CrossEntropyForward(dup(fhp, logits, T, V), targets, pg, T, V, ignore)
        tb.EnsureHostCurrent(pg)
        near_rel(pg.Data, pc, FWD)
        dlg = fhp.Tensor(T, V)
        tb.CrossEntropyBackward(dup(fhp, pc, T, V), targets, dlg, T, V, ignore)
        tb.EnsureHostCurrent(dlg)
        near_rel(dlg.Data, dlc, BWD)
        # all ignored: zero loss, zero gradient
        allign = np.full(T, ignore, np.int32)
        assert tb.CrossEntropyForward(dup(fhp, logits, T, V), allign, fhp.Tensor(T, V), T, V, ignore) == 0.0
        dz = dup(fhp, np.ones(T * V), T, V)
        tb.CrossEntropyBackward(dup(fhp, logits, T, V), allign, dz, T, V, ignore)
        tb.EnsureHostCurrent(dz)
        assert not dz.Data.any()
    near_rel(lg, lc, FWD)


@pytest.mark.gpu
def test_loss_accumulation_returns_combined_mean(fhp, tb):
    # CpuBackendTests.CrossEntropy_LossAccumulationReturnsCombinedMean on the device
    f = dup(fhp, [2, 0, -1, 0, 1, 2], 2, 3)
    s = dup(fhp, [-1, 3, 0], 1, 3)
    first = tb.CrossEntropyForward(f, [0, 2], fhp.Tensor(2, 3), 2, 3, -1)
    second = tb.CrossEntropyForward(s, [1], fhp.Tensor(1, 3), 1, 3, -1)
    tb.BeginLossAccumulation()
    assert tb.CrossEntropyForward(f, [0, 2], fhp.Tensor(2, 3), 2, 3, -1) == 0.0  # stays on the device
    tb.CrossEntropyForward(s, [1], fhp.Tensor(1, 3), 1, 3, -1)
    acc = tb.EndLossAccumulation()
    assert abs(acc - (first * 2 + second) / 3) <= 1e-6
    with pytest.raises(fhp.InvalidOperationError, match="not active"):
        tb.EndLossAccumulation()
    tb.BeginLossAccumulation()
    with pytest.raises(fhp.InvalidOperationError, match="already active"):
        tb.BeginLossAccumulation()
    assert tb.EndLossAccumulation() == 0.0


@pytest.mark.gpu
def test_batched_attention_kernels_match_cpu(fhp, oracle, tb):
    # GpuBackendTests.BatchedAttentionKernels_MatchCpu
    rng = NetRng(oracle, 113)
    batch, T, H, hd = 3, 7, 2, 5
    D = H * hd
    src = rng.rand(batch * T * 3 * D)
    pkc = np.zeros(batch * H * T * hd, np.float32)
    oracle.op_pack_heads(src, 3 * D, pkc, batch, T, H, hd, D)
    pkg = fhp.Tensor(batch * H * T, hd)
    tb.PackHeads(dup(fhp, src, batch * T, 3 * D), pkg, batch, T, H, hd, D)
    tb.EnsureHostCurrent(pkg)
    near_rel(pkg.Data, pkc, 0)
    unc = np.zeros(batch * T * 3 * D, np.float32)
    oracle.op_unpack_heads(pkc, unc, 3 * D, batch, T, H, hd, 2 * D)
    ung = fhp.Tensor(batch * T, 3 * D)
    tb.UnpackHeads(dup(fhp, pkc, batch * H * T, hd), ung, batch, T, H, hd, 2 * D)
    tb.EnsureHostCurrent(ung)
    near_rel(ung.Data, unc, 0)
    qkv = [np.zeros(batch * H * T * hd, np.float32) for _ in range(3)]
    for i in range(3):
        oracle.op_pack_heads(src, 3 * D, qkv[i], batch, T, H, hd, i * D)
    qg, kg, vg = (fhp.Tensor(batch * H * T, hd) for _ in range(3))
    tb.PackQkvHeads(dup(fhp, src, batch * T, 3 * D), qg, kg, vg, batch, T, H, hd)
    for t, want in zip((qg, kg, vg), qkv):
        tb.EnsureHostCurrent(t)
        near_rel(t.Data, want, 0)
    back = fhp.Tensor(batch * T, 3 * D)
    tb.UnpackQkvHeads(qg, kg, vg, back, batch, T, H, hd)
    tb.EnsureHostCurrent(back)
    near_rel(back.Data, src, 0)
    rows = batch * H * T
    scores, dO = rng.rand(rows * T), rng.rand(rows * T)
    scale = 0.375
    pc = scores.copy()
    oracle.op_scaled_causal_softmax_forward(pc, rows, T, scale)
    pg = dup(fhp, scores, rows, T)
    tb.ScaledCausalSoftmaxForward(pg, rows, T, scale)
    tb.EnsureHostCurrent(pg)
    near_rel(pg.Data, pc, FWD)
    dsc = np.zeros(rows * T, np.float32)
    oracle.op_scaled_softmax_backward(dO, pc, dsc, rows, T, scale)
    dsg = fhp.Tensor(rows, T)
    tb.ScaledSoftmaxBackward(dup(fhp, dO, rows, T), pg, dsg, rows, T, scale)
    tb.EnsureHostCurrent(dsg)
    near_rel(dsg.Data, dsc, BWD)
    slots, M, K, N = batch * H, T, hd, T
    a, bN, bT, prior = rng.rand(slots * M * K), rng.rand(slots * K * N), rng.rand(slots * N * K), rng.rand(slots * M * N)
    for acc in (False, True):
        for mode, bb, fn in (("nn", bN, tb.BatchedMatMulNN), ("nt", bT, tb.BatchedMatMulNT),
                             ("tn", bN, tb.BatchedMatMulTN)):
            yc = prior.copy()
            oracle.op_matmul(mode, a, bb, yc, M, K, N, accumulate=acc, slots=slots)
            yg = dup(fhp, prior, slots * M, N)
            fn(dup(fhp, a, slots * M, K), dup(fhp, bb, slots * K, N), yg, slots, M, K, N, acc)
            tb.EnsureHostCurrent(yg)
            near_rel(yg.Data, yc, FWD)


@pytest.mark.gpu
def test_residency_contract(fhp, tb):
    # GpuBackendTests.Residency_*, EnsureHostCurrent_RoundTripsDeviceResults
    x = dup(fhp, np.ones(8), 8)
    y = fhp.Tensor(8)
    tb.Copy(x, y)                 # x now has a device copy
    x.Data[:] = 5.0               # host write without InvalidateDeviceCache
    tb.Copy(x, y)
    tb.EnsureHostCurrent(y)
    assert np.all(y.Data == 1.0)  # the kernel saw the stale device copy
    tb.InvalidateDeviceCache(x)
    tb.Copy(x, y)
    assert np.all(y.Data == 1.0)  # no download yet: host copy of y is stale
    tb.EnsureHostCurrent(y)
    assert np.all(y.Data == 5.0)
    tb.Scale(y, 2.0)
    tb.EnsureHostCurrent(y)
    tb.EnsureHostCurrent(y)       # idempotent
    assert np.all(y.Data == 10.0)
    tb.Zero(y)
    assert not y.Data.any()
    tb.AddInPlace(y, x)
    tb.EnsureHostCurrent(y)
    assert np.all(y.Data == 5.0)


@pytest.mark.gpu
def test_adamw_and_sum_squares_match_cpu(fhp, oracle, tb):
    # CudaBackendTests.AdamWAndSumSquares_MatchCpu, GlobalSumSquares_MatchesCpuWithOneReadback
    rng = NetRng(oracle, 912)
    rows, cols = 17, 19

    def vals():
        return np.array([rng.next_double() * 2 - 1 for _ in range(rows * cols)], np.float32)

    w, g, m = vals(), vals(), vals()
    v = np.abs(vals())
    wc, mc, vc = w.copy(), m.copy(), v.copy()
    oracle.op_adamw(wc, g, mc, vc, 3e-4, 0.9, 0.95, 1e-8, 0.1, 37, True)
    wg, gg, mg, vg = (dup(fhp, a, rows, cols) for a in (w, g, m, v))
    tb.AdamWStep(wg, gg, mg, vg, 3e-4, 0.9, 0.95, 1e-8, 0.1, 37)
    for t in (wg, mg, vg):
        tb.EnsureHostCurrent(t)
    np.testing.assert_allclose(wg.Data, wc, atol=2e-5)
    np.testing.assert_allclose(mg.Data, mc, atol=2e-5)
    np.testing.assert_allclose(vg.Data, vc, atol=2e-5)
    # a vector (rank 1) gets no weight decay
    b0 = vals()[:cols]
    bc = b0.copy()
    oracle.op_adamw(bc, g[:cols].copy(), np.zeros(cols, np.float32), np.zeros(cols, np.float32), 1e-2, 0.9, 0.95,
                    1e-8, 0.5, 1, False)
    bg = dup(fhp, b0, cols)
    tb.AdamWStep(bg, dup(fhp, g[:cols], cols), fhp.Tensor(cols), fhp.Tensor(cols), 1e-2, 0.9, 0.95, 1e-8, 0.5, 1)
    tb.EnsureHostCurrent(bg)
    np.testing.assert_allclose(bg.Data, bc, atol=2e-6)
    assert abs(tb.SumSquares(gg) - oracle.op_sum_squares(g)) <= 2e-4 * max(1.0, oracle.op_sum_squares(g))
    r2 = NetRng(oracle, 914, 1 << 21)
    ts, expected = [], 0.0
    for n in (1, 257, 4097, 1_000_003):
        a = np.array(r2.d[r2.i:r2.i + n] * 2 - 1, np.float64) * 0.1
        r2.i += n
        a = a.astype(np.float32)
        expected += float(np.dot(a.astype(np.float64), a))
        ts.append(dup(fhp, a, n))
    actual = tb.GlobalSumSquares(ts)
    assert abs(actual - expected) / max(1.0, expected) < 2e-5
    assert tb.GlobalSumSquares([]) == 0.0
