"""GPU parity of the Backend trait ops through the C ABI (host slices, as an
`impl Backend for HipBackend` would call them): Op::RmsNorm (cpu.rs:514-545)
and Op::CausalAttention (cpu.rs:1660-1727) against the oracle's restatement
(oracle/oracle_backend.c), plus the argument errors the reference raises or
panics on."""
import ctypes

import numpy as np
import pytest

import aether_amd as A
from oracle import oracle as O
from tests._util import assert_close

pytestmark = pytest.mark.gpu


def ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


@pytest.mark.parametrize("rows,last", [(1, 4096), (7, 300), (3, 1024), (0, 64)])
def test_backend_rms_norm(gpu, rows, last):
    rng = np.random.default_rng(rows * 7 + last)
    x = (rng.standard_normal((rows, last)) * 3).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(last)).astype(np.float32)
    out = np.full((rows, last), np.nan, np.float32)
    A.check(A.lib().aeth_backend_rms_norm(ptr(x), ptr(w), rows, last, 1e-5, ptr(out)), "backend_rms_norm")
    if rows:
        assert_close(out, O.backend_rms_norm(x, w, 1e-5), tol=1e-5, what="rms_norm")


# head_dim 128 (float4 path), 64, 80, 256 (the limit), 5 (scalar path), a d that
# 3 heads do not divide (zero tail columns), batches, and seq past one 64-key chunk
@pytest.mark.parametrize("b,s,d,heads", [(1, 1, 128, 1), (2, 37, 256, 2), (1, 130, 512, 4), (1, 65, 160, 2),
                                         (3, 20, 256, 1), (1, 9, 15, 3), (2, 70, 100, 3)])
def test_backend_causal_attention(gpu, b, s, d, heads):
    rng = np.random.default_rng(b * 1000 + s + d)
    q, k, v = (rng.standard_normal((b, s, d)).astype(np.float32) for _ in range(3))
    scale = float(1.0 / np.sqrt(max(1, d // heads)))
    out = np.full((b, s, d), np.nan, np.float32)
    A.check(A.lib().aeth_backend_causal_attention(ptr(q), ptr(k), ptr(v), b, s, d, heads, scale, ptr(out)),
            "backend_causal_attention")
    ref = O.causal_attention(q, k, v, heads, scale)
    assert_close(out.reshape(b * s, d), ref.reshape(b * s, d), tol=1e-4, what="causal_attention")


def test_backend_causal_attention_nonfinite_scores(gpu):
    """Scores of -inf (q·k overflowing in f32) carry no weight, as the
    reference's `row[j] != -inf` skip (cpu.rs:1705-1721) gives them: a query
    whose early keys all overflow to -inf — a whole 64-key chunk of them, then
    finite keys — still gets a finite row; one whose every key overflows gets
    0; +inf scores give NaN rows on both sides."""
    b, s, d, heads = 1, 150, 128, 1
    rng = np.random.default_rng(9)
    q, k, v = (rng.standard_normal((b, s, d)).astype(np.float32) for _ in range(3))
    q[0, :, :] = np.abs(q[0]) + 1.0
    k[0, :70, :] = -3e37   # every dot with these keys is -inf in f32 (q > 0)
    k[0, 120, :] = 3e37    # +inf for queries 120 and later
    scale = float(1.0 / np.sqrt(d))
    out = np.full((b, s, d), 7.0, np.float32)
    A.check(A.lib().aeth_backend_causal_attention(ptr(q), ptr(k), ptr(v), b, s, d, heads, scale, ptr(out)),
            "backend_causal_attention")
    ref = O.causal_attention(q, k, v, heads, scale)
    assert (ref[0, :70] == 0).all() and np.isfinite(ref[0, 70:120]).all() and np.isnan(ref[0, 120:]).all()
    assert np.array_equal(np.isnan(out), np.isnan(ref))
    fin = np.isfinite(ref)
    assert_close(out[fin][None, :], ref[fin][None, :], tol=1e-4, what="causal_attention with -inf scores")


def test_backend_causal_attention_errors(gpu):
    L = A.lib()
    q = np.zeros((1, 4, 8), np.float32)
    out = np.zeros_like(q)
    assert L.aeth_backend_causal_attention(ptr(q), ptr(q), ptr(q), 1, 4, 8, 0, 1.0, ptr(out)) == A.AETH_EINVAL
    big = np.zeros((1, 2, 514), np.float32)
    ob = np.zeros_like(big)
    assert L.aeth_backend_causal_attention(ptr(big), ptr(big), ptr(big), 1, 2, 514, 2, 1.0,
                                           ptr(ob)) == A.AETH_EUNSUPPORTED
    assert L.aeth_backend_causal_attention(None, None, None, 1, 4, 8, 2, 1.0, None) == A.AETH_EINVAL
    assert L.aeth_backend_rms_norm(ptr(q), ptr(q), 4, 0, 1e-5, ptr(out)) == A.AETH_EINVAL
