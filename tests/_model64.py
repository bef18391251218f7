"""Exact (float64) evaluation of the small test models, for model-level logit
checks: a causal forward over a token list, with the weights dequantized by
the pinned oracle and every other step (RMSNorm, RoPE from the f32 tables,
GQA softmax attention, SiLU) in float64. The last position's logits are the
exact value that both the CPU oracle and the GPU approximate in f32.
"""
import numpy as np

from oracle import oracle as O

GGUF_ORDER = (0, 1, 10, 11)  # F32, F16, Q2_K, Q3_K: kept as [k][n] by load_quant


def _deq(dtype, raw, n, k):
    f = O.dequant(dtype, raw, n * k).astype(np.float64)
    return f.reshape(k, n).T if dtype in GGUF_ORDER else f.reshape(n, k)


def logits64(c, emb, layers, dtypes, norms, final, lm, lm_dtype, tokens):
    """c: config dict (TINY form; an optional sliding_window w > 0 lets query i
    see keys i-w+1 ..= i only); layers[l][j] raw bytes of q,k,v,o,gate,up,down;
    dtypes: 7 formats (or one per layer as a list of lists); tokens at
    positions 0..len-1 (positions past the RoPE table clamp to its last row).
    Returns float64 logits of the last position."""
    d, nh, nkv, hd, dff = c["d_model"], c["num_heads"], c["num_kv_heads"], c["head_dim"], c["d_ff"]
    ms, eps = c["max_seq_len"], c["rms_norm_eps"]
    shapes = [(nh * hd, d), (nkv * hd, d), (nkv * hd, d), (d, nh * hd), (dff, d), (dff, d), (d, dff)]
    s, co = O.precompute_rope(ms, hd, c["rope_base"])
    S = s.reshape(ms, hd // 2).astype(np.float64)
    C = co.reshape(ms, hd // 2).astype(np.float64)
    n = len(tokens)

    def rms(v, w):
        return v / np.sqrt((v * v).sum(-1, keepdims=True) / v.shape[-1] + eps) * w.astype(np.float64)

    rows = np.minimum(np.arange(n), ms - 1)
    w = c.get("sliding_window", 0)
    i_, j_ = np.arange(n)[:, None], np.arange(n)[None, :]
    visible = (j_ <= i_) & ((j_ > i_ - w) if w > 0 else True)

    def rope(v):  # v [n][heads][hd], position = row
        a, b = v[..., :hd // 2].copy(), v[..., hd // 2:].copy()
        cc, ss = C[rows][:, None, :], S[rows][:, None, :]
        return np.concatenate([a * cc - b * ss, a * ss + b * cc], axis=-1)

    x = np.asarray(emb, dtype=np.float64)[np.asarray(tokens)]
    for l, L in enumerate(layers):
        dts = dtypes[l] if isinstance(dtypes[0], (list, tuple)) else dtypes
        W = [_deq(dt, w, a, b) for dt, w, (a, b) in zip(dts, L, shapes)]
        h = rms(x, norms[l][0])
        q = rope((h @ W[0].T).reshape(n, nh, hd))
        k = rope((h @ W[1].T).reshape(n, nkv, hd))
        v = (h @ W[2].T).reshape(n, nkv, hd)
        att = np.zeros((n, nh, hd))
        g = nh // nkv
        for hh in range(nh):
            sc = q[:, hh] @ k[:, hh // g].T / np.sqrt(hd)
            sc = np.where(visible, sc, -np.inf)
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            att[:, hh] = (p / p.sum(axis=1, keepdims=True)) @ v[:, hh // g]
        x = x + att.reshape(n, -1) @ W[3].T
        h = rms(x, norms[l][1])
        gt, up = h @ W[4].T, h @ W[5].T
        with np.errstate(over="ignore"):
            x = x + (gt / (1 + np.exp(-gt)) * up) @ W[6].T
    return _deq(lm_dtype, lm, c["vocab_size"], d) @ rms(x[-1], final)
