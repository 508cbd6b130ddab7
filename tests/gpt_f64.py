"""An independent float64 numpy statement of the reference GPT forward, used only to
pin the oracle's composition of its (separately pinned) ops.

It follows the reference's structure, not the oracle's code:
  x = tok_emb[ids] + pos_emb[0..T)                         GptModel.cs:217-218
  per block (TransformerBlock.Forward, Layers.cs:384-392):
    a = Attn(LN1(x)); a += x; m = Mlp(LN2(a)); m += a
  Attn (Layers.cs:191-229): qkv = h W + b; heads are column blocks of width hd in
    the q, k and v thirds (PackQkvHeads, ITensorBackend.cs:58-65); causal softmax of
    q k^T / sqrt(hd); o = p v; concat heads; proj
  Mlp (Layers.cs:306-313): proj(GELU_tanh(fc(h)))
  logits = LN_f(x) tok_emb^T                                GptModel.cs:221, Layers.cs:80-86
in float64 with numpy's own matrix products and exp/tanh, so it shares no
arithmetic with the C++ oracle.  `mutate` plants one plausible composition
mistake so a test can show that the comparison catches it.
"""
import numpy as np

MUTATIONS = ("post_ln", "drop_attn_residual", "drop_mlp_residual", "no_causal_mask", "no_final_ln",
             "swap_k_v", "heads_interleaved", "ln_shared")


def _ln(x, w, b, eps=1e-5):
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * w + b


def _gelu(v):
    return 0.5 * v * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (v + 0.044715 * v ** 3)))


def forward(layout, weights, n_heads, ids, mutate=None):
    """logits [T, V] (float64).  `layout` is oracle.param_layout(cfg)."""
    assert mutate is None or mutate in MUTATIONS
    P = {n: np.asarray(weights[o:o + int(np.prod(s))], np.float64).reshape(s) for n, o, s in layout}
    ids = np.asarray(ids)
    T = ids.size
    tok = P["tok_emb"]
    d = tok.shape[1]
    hd = d // n_heads
    L = sum(1 for n, _, _ in layout if n.endswith("ln1.w"))
    x = tok[ids] + P["pos_emb"][:T]
    causal = np.tril(np.ones((T, T), bool))
    for i in range(L):
        p = lambda k: P[f"blocks.{i}.{k}"]  # noqa: E731
        ln2w, ln2b = (p("ln1.w"), p("ln1.b")) if mutate == "ln_shared" else (p("ln2.w"), p("ln2.b"))
        h = x if mutate == "post_ln" else _ln(x, p("ln1.w"), p("ln1.b"))
        qkv = h @ p("attn.qkv.w") + p("attn.qkv.b")
        q, k, v = qkv[:, :d], qkv[:, d:2 * d], qkv[:, 2 * d:]
        if mutate == "swap_k_v":
            k, v = v, k
        o = np.empty((T, d))
        for hh in range(n_heads):
            cols = (np.arange(hh, d, n_heads) if mutate == "heads_interleaved" else
                    np.arange(hh * hd, (hh + 1) * hd))
            s = q[:, cols] @ k[:, cols].T / np.sqrt(hd)
            if mutate != "no_causal_mask":
                s = np.where(causal, s, -np.inf)
            s = np.exp(s - s.max(axis=1, keepdims=True))
            o[:, cols] = (s / s.sum(axis=1, keepdims=True)) @ v[:, cols]
        a = o @ p("attn.proj.w") + p("attn.proj.b")
        if mutate != "drop_attn_residual":
            a = a + x
        if mutate == "post_ln":
            a = _ln(a, p("ln1.w"), p("ln1.b"))
        h2 = a if mutate == "post_ln" else _ln(a, ln2w, ln2b)
        m = _gelu(h2 @ p("mlp.fc.w") + p("mlp.fc.b")) @ p("mlp.proj.w") + p("mlp.proj.b")
        if mutate != "drop_mlp_residual":
            m = m + a
        if mutate == "post_ln":
            m = _ln(m, ln2w, ln2b)
        x = m
    xf = x if mutate == "no_final_ln" else _ln(x, P["ln_f.w"], P["ln_f.b"])
    return xf @ tok.T
