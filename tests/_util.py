"""Shared helpers for the parity tests: seeded synthetic GGUF blocks (numpy)
and the tolerance rule of the north star."""
import numpy as np

F32, F16, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 0, 1, 8, 10, 11, 12, 13, 14
GEOM = {F32: (1, 4), F16: (1, 2), Q8_0: (32, 34), Q2_K: (256, 84), Q3_K: (256, 110), Q4_K: (256, 144),
        Q5_K: (256, 176), Q6_K: (256, 210)}


def f16_bytes(v):
    return np.asarray(v, dtype=np.float32).astype(np.float16).view(np.uint8).reshape(-1, 2)


def synth_blocks(dtype, n_blocks, seed):
    """Raw GGUF blocks as BASELINE.json describes the benchmark weights."""
    rng = np.random.default_rng(seed)
    be, bb = GEOM[dtype]
    if dtype == F16:
        return (rng.standard_normal(n_blocks) * 0.05).astype(np.float16).view(np.uint8)
    if dtype == F32:
        return (rng.standard_normal(n_blocks) * 0.05).astype(np.float32).view(np.uint8)
    raw = rng.integers(0, 256, size=(n_blocks, bb), dtype=np.uint8)
    scale = lambda: f16_bytes(np.abs(rng.standard_normal(n_blocks)) * 0.01)
    if dtype == Q8_0:
        raw[:, 0:2] = scale()
        raw[:, 2:] = rng.integers(-127, 128, size=(n_blocks, 32)).astype(np.int8).view(np.uint8)
    elif dtype in (Q4_K, Q5_K, Q2_K):  # d, dmin lead the block
        raw[:, 0:2] = scale()
        raw[:, 2:4] = scale()
    elif dtype == Q3_K:
        raw[:, 108:110] = scale()
    else:
        raw[:, 192:208] = rng.integers(-64, 64, size=(n_blocks, 16)).astype(np.int8).view(np.uint8)
        raw[:, 208:210] = scale()
    return raw.reshape(-1)


def weight(dtype, n, k, seed):
    be, bb = GEOM[dtype]
    nb = (k + 31) // 32 if dtype == Q8_0 else k if be == 1 else k // 256
    return synth_blocks(dtype, n * nb, seed)


def close_mask(g, r, tol=1e-3):
    g = np.asarray(g, dtype=np.float64)
    r = np.asarray(r, dtype=np.float64)
    diff = np.abs(g - r)
    return (diff <= tol) | (diff / np.maximum(1.0, np.abs(r)) <= tol)


def assert_close(g, r, tol=1e-3, cos_min=0.9999, what=""):
    """Per element |g-r| <= tol or |g-r|/max(1,|r|) <= tol (the reference's own
    relative form, src/quant/matmul/tests.rs:406), and per-row cosine > cos_min."""
    g = np.atleast_2d(np.asarray(g, dtype=np.float64))
    r = np.atleast_2d(np.asarray(r, dtype=np.float64))
    assert g.shape == r.shape, (g.shape, r.shape)
    ok = close_mask(g, r, tol)
    if not ok.all():
        i = np.argwhere(~ok)[0]
        raise AssertionError("%s: %d/%d elements out of tolerance; first at %s: got %r ref %r" %
                             (what, (~ok).sum(), ok.size, tuple(i), g[tuple(i)], r[tuple(i)]))
    num = (g * r).sum(axis=1)
    den = np.sqrt((g * g).sum(axis=1) * (r * r).sum(axis=1))
    cos = np.where(den > 0, num / np.where(den > 0, den, 1), 1.0)
    assert (cos > cos_min).all(), "%s: row cosine %r <= %r" % (what, cos.min(), cos_min)


def assert_close_logits(g, r, tol=1e-3, floor=0.0, cos_min=0.9999, what="", exact=None):
    """Whole-model logits (a decode step or a prefill through every layer): the
    element-wise bar of assert_close and per-row cosine > cos_min. Two
    widenings, each used only where a test passes it:
      * `exact` (the float64 logits of the same model, tests/_model64.py): an
        element also passes when its distance from the exact value is at most
        twice the largest distance the reference's own f32 result shows on that
        row (plus 1e-6·max|row|). A logit is an f32 sum whose rounding scales
        with the row's largest terms: on some test models (the GGUF-order Q2_K /
        Q3_K model, logits to ±572) the reference's own f32 result misses the
        plain bar against the exact logits (test_oracle.py,
        test_reference_f32_logits_miss_the_plain_bar_on_a_test_model), so no
        other f32 order can be held to it against the reference there;
      * `floor`: an element also passes within floor·max|r_row| of the
        reference (0 unless given).
    Kernel-level outputs keep the plain element-wise bar, except where the
    reference's own f32 sums miss it (the Q6_K and Q8_0 GEMMs' long rows of
    magnitude in the thousands: exact = the float64 product)."""
    g = np.atleast_2d(np.asarray(g, dtype=np.float64))
    r = np.atleast_2d(np.asarray(r, dtype=np.float64))
    assert g.shape == r.shape, (g.shape, r.shape)
    ok = close_mask(g, r, tol) | (np.abs(g - r) <= floor * np.abs(r).max(axis=1, keepdims=True))
    if exact is not None:
        x = np.atleast_2d(np.asarray(exact, dtype=np.float64))
        band = 2.0 * np.abs(r - x).max(axis=1, keepdims=True) + 1e-6 * np.abs(x).max(axis=1, keepdims=True)
        ok |= np.abs(g - x) <= band
    if not ok.all():
        i = np.argwhere(~ok)[0]
        raise AssertionError("%s: %d/%d logits out of tolerance; first at %s: got %r ref %r (row max %r)" %
                             (what, (~ok).sum(), ok.size, tuple(i), g[tuple(i)], r[tuple(i)], np.abs(r[i[0]]).max()))
    num = (g * r).sum(axis=1)
    den = np.sqrt((g * g).sum(axis=1) * (r * r).sum(axis=1))
    cos = np.where(den > 0, num / np.where(den > 0, den, 1), 1.0)
    assert (cos > cos_min).all(), "%s: row cosine %r <= %r" % (what, cos.min(), cos_min)


def assert_close_rows(g, r, tol=1e-3, what=""):
    """For intermediate state (the KV cache): per row, |g-r| <= tol·max(1, max|r_row|).
    An entry's float error scales with the magnitudes summed into it, i.e. with
    its row, so small entries of large rows get the row's absolute bar; the
    element-wise output bar (assert_close) stays on logits."""
    g = np.atleast_2d(np.asarray(g, dtype=np.float64))
    r = np.atleast_2d(np.asarray(r, dtype=np.float64))
    assert g.shape == r.shape, (g.shape, r.shape)
    scale = np.maximum(1.0, np.abs(r).max(axis=1, keepdims=True))
    bad = np.abs(g - r) > tol * scale
    if bad.any():
        i = tuple(np.argwhere(bad)[0])
        raise AssertionError("%s: %d/%d elements out of row tolerance; first at %s: got %r ref %r (row scale %r)" %
                             (what, bad.sum(), bad.size, i, g[i], r[i], scale[i[0], 0]))
