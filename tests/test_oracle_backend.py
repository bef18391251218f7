"""Pins the oracle's restatement of the two Backend ops (oracle/oracle_backend.c)
to checks that do not retype its formula: Op::RmsNorm equals the runner's
rmsnorm_inplace (pinned in tests/test_oracle.py) bit for bit and a constant row
has a closed form; Op::CausalAttention is checked against special cases that
fix it (one position, a zero query's running mean, one dominant key) and an
f64 brute force of the textbook masked softmax, including the zero columns a
d that num_heads does not divide leaves."""
import numpy as np
import pytest

from oracle import oracle as O


def test_backend_rms_norm_equals_runner_rmsnorm_rows():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((5, 300)) * 4).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(300)).astype(np.float32)
    got = O.backend_rms_norm(x, w, 1e-5)
    for r in range(5):
        assert np.array_equal(got[r], O.rmsnorm(x[r], w, 1e-5))


def test_backend_rms_norm_constant_row():
    x = np.full((2, 64), 3.0, np.float32)
    w = np.full(64, 2.0, np.float32)
    got = O.backend_rms_norm(x, w, 0.0)
    assert np.array_equal(got, np.full((2, 64), 2.0, np.float32))  # 3 / sqrt(9) · 2


def f64_causal(q, k, v, heads, scale):
    b, s, d = q.shape
    hd = d // heads
    out = np.zeros((b, s, d))
    for bi in range(b):
        for h in range(heads):
            cols = slice(h * hd, (h + 1) * hd)
            sc = q[bi, :, cols].astype(np.float64) @ k[bi, :, cols].astype(np.float64).T * scale
            sc[np.triu_indices(s, 1)] = -np.inf
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            out[bi, :, cols] = (p / p.sum(axis=1, keepdims=True)) @ v[bi, :, cols].astype(np.float64)
    return out


@pytest.mark.parametrize("b,s,d,heads", [(1, 7, 64, 2), (2, 33, 96, 3), (1, 20, 70, 4)])
def test_causal_attention_vs_f64(b, s, d, heads):
    rng = np.random.default_rng(s + d)
    q, k, v = (rng.standard_normal((b, s, d)).astype(np.float32) for _ in range(3))
    scale = 1.0 / np.sqrt(d // heads)
    got = O.causal_attention(q, k, v, heads, scale)
    ref = f64_causal(q, k, v, heads, scale)
    np.testing.assert_allclose(got, ref, rtol=2e-5, atol=2e-6)
    hd = d // heads
    assert not got[:, :, heads * hd:].any()  # columns no head owns stay 0


def test_causal_attention_special_cases():
    rng = np.random.default_rng(9)
    q, k, v = (rng.standard_normal((1, 12, 32)).astype(np.float32) for _ in range(3))
    # position 0 sees only itself: out = v_0
    out = O.causal_attention(q, k, v, 2, 0.3)
    assert np.array_equal(out[0, 0], v[0, 0])
    # a zero query weighs keys 0..i equally: out_i = mean of v_0..v_i
    z = np.zeros_like(q)
    out = O.causal_attention(z, k, v, 2, 0.3)
    ref = np.cumsum(v[0].astype(np.float64), axis=0) / np.arange(1, 13)[:, None]
    np.testing.assert_allclose(out[0], ref, rtol=1e-6, atol=1e-6)
    # one key far above the rest takes all the weight
    k2 = np.zeros_like(k)
    k2[0, 3] = 50.0
    q2 = np.ones_like(q)
    out = O.causal_attention(q2, k2, v, 1, 1.0)
    np.testing.assert_allclose(out[0, 3:], np.broadcast_to(v[0, 3], (9, 32)), rtol=0, atol=1e-6)
    with pytest.raises(ValueError):
        O.causal_attention(q, k, v, 0, 1.0)
