"""Pins the oracle's restatement of the remaining weight formats
(oracle/oracle_formats.c): Q5_K, Q2_K, Q3_K, F16 and F32, their matmuls,
the Q5_K re-quantizer, the Q5_K / Q6_K int8 dot-product references and the
dequantize → GGUF-order f32 route of quantized_matmul_impl. Each check sets
the function against something other than itself: the pinned Q4_K / Q8_0
pieces, hand-built blocks with exact closed-form values, numpy float16, the
reference's own cross-kernel tolerances (src/quant/matmul/tests.rs:510-826)
and its round-trip bound (tests/correctness.rs:1309), and f64 brute force."""
import numpy as np
import pytest

from oracle import oracle as O
from tests._util import F16, F32, GEOM, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0, synth_blocks

GGUF_ORDER = (F32, F16, Q2_K, Q3_K)


def pack_k4(sc, m):
    """The 12 scale bytes of requantize_q4_k's packing (dispatch.rs:248-256)."""
    out = np.zeros(12, np.uint8)
    for q in range(4):
        out[q] = (sc[q] & 63) | ((sc[q + 4] >> 4) << 6)
        out[4 + q] = (m[q] & 63) | ((m[q + 4] >> 4) << 6)
        out[8 + q] = (sc[q + 4] & 15) | ((m[q + 4] & 15) << 4)
    return out


# ── Q5_K ─────────────────────────────────────────────────────────────────

def test_dequant_q5_k_without_high_bits_is_q4_k():
    """Q5_K = Q4_K's header and nibbles plus a fifth bit per element: with qh
    zero every element equals the (pinned) Q4_K dequant of the same fields."""
    q4 = synth_blocks(Q4_K, 12, 3).reshape(12, 144)
    q5 = np.zeros((12, 176), np.uint8)
    q5[:, :16] = q4[:, :16]
    q5[:, 48:] = q4[:, 16:]
    assert np.array_equal(O.dequant(Q5_K, q5, 12 * 256).view(np.uint32), O.dequant(Q4_K, q4, 12 * 256).view(np.uint32))


def test_dequant_q5_k_hand_block_high_bit_order():
    """d = 1, dmin = 0.5, small integer scales: every value is exact. Element
    e's fifth bit is bit e % 8 of qh[e / 8] (dequant.rs:260-266): a random
    qh pattern moves exactly the elements whose bit is set, by 16·sc."""
    rng = np.random.default_rng(4)
    sc = [s + 1 for s in range(8)]
    m = [7 - s for s in range(8)]
    blk = np.zeros(176, np.uint8)
    blk[0:2] = np.array([1.0], np.float16).view(np.uint8)
    blk[2:4] = np.array([0.5], np.float16).view(np.uint8)
    blk[4:16] = pack_k4(sc, m)
    nib = rng.integers(0, 16, 256)
    for j in range(4):
        for l in range(32):
            blk[48 + 32 * j + l] = nib[64 * j + l] | (nib[64 * j + 32 + l] << 4)
    hbits = rng.integers(0, 2, 256)
    blk[16:48] = np.packbits(hbits.astype(np.uint8), bitorder="little")
    out = O.dequant(Q5_K, blk, 256)
    for e in range(256):
        s = e // 32
        assert out[e] == sc[s] * (nib[e] + 16 * hbits[e]) - 0.5 * m[s], e


def test_requantize_q5_k_round_trip_reference_bound():
    """tests/correctness.rs:1309: gaussian σ = 0.5 clamped to ±1.5, 4×256,
    requantize → dequantize within 0.15."""
    rng = np.random.default_rng(42)
    data = np.clip(rng.standard_normal(4 * 256) * 0.5, -1.5, 1.5).astype(np.float32)
    q = O.requantize(Q5_K, data, 4, 256)
    assert q.size == 4 * 176
    assert np.abs(O.dequant(Q5_K, q, 4 * 256) - data).max() <= 0.15


def test_requantize_q5_k_levels_and_ragged_rows():
    """Every sub-block on the same 32-level grid q/8 (q = 0..31) quantizes
    to sc = 63, m = 0 and q itself, so the values come back up to the f16
    rounding of d (relative 2^-11); a ragged row (cols % 256 ≠ 0) zero-pads
    its last block (dispatch.rs:309-313)."""
    v = np.array([(e % 32) / 8.0 for e in range(256)], np.float32)
    q = O.requantize(Q5_K, v, 1, 256)
    assert list(q[4:8]) == [63 | (3 << 6)] * 4 and list(q[8:12]) == [0] * 4
    back = O.dequant(Q5_K, q, 256)
    np.testing.assert_allclose(back, v, rtol=2 ** -10, atol=0)
    rng = np.random.default_rng(8)
    x = rng.standard_normal(3 * 300).astype(np.float32)
    q = O.requantize(Q5_K, x, 3, 300).reshape(3, 2, 176)
    assert q.shape == (3, 2, 176)
    back = O.dequant(Q5_K, q.reshape(-1), 3 * 512).reshape(3, 512)
    assert np.abs(back[:, :300] - x.reshape(3, 300)).max() < 0.3


# ── Q2_K / Q3_K ──────────────────────────────────────────────────────────

def test_dequant_q2_k_hand_block():
    """d = 1, dmin = 0.5, sub-block s scale byte (s % 16) | ((15 − s) << 4);
    element e = 128·half + 32·t + 16·u + l is bits 2t of qs[32·half + 16u + l]
    in sub-block 8·half + 2t + u (dequant.rs:368-395): out = sc·q − 0.5·m."""
    rng = np.random.default_rng(2)
    q = rng.integers(0, 4, 256)
    blk = np.zeros(84, np.uint8)
    blk[0:2] = np.array([1.0], np.float16).view(np.uint8)
    blk[2:4] = np.array([0.5], np.float16).view(np.uint8)
    blk[4:20] = [(s % 16) | ((15 - s) << 4) for s in range(16)]
    expect = np.zeros(256)
    for half in range(2):
        for t in range(4):
            for u in range(2):
                for l in range(16):
                    e = 128 * half + 32 * t + 16 * u + l
                    blk[20 + 32 * half + 16 * u + l] |= q[e] << (2 * t)
                    s = 8 * half + 2 * t + u
                    expect[e] = (s % 16) * q[e] - 0.5 * (15 - s)
    out = O.dequant(Q2_K, blk, 256)
    assert np.array_equal(out, expect.astype(np.float32))


def pack_q3k_scales(sc6):
    """Inverse of the 6-bit scale unpack (dequant.rs:412-425)."""
    sr = np.zeros(12, np.uint8)
    for i in range(8):
        sr[i] = (sc6[i] & 15) | ((sc6[i + 8] & 15) << 4)
    for i in range(4):
        sr[8 + i] = (sc6[i] >> 4) | ((sc6[i + 4] >> 4) << 2) | ((sc6[i + 8] >> 4) << 4) | ((sc6[i + 12] >> 4) << 6)
    return sr


def test_dequant_q3_k_hand_block():
    """d = 0.5; 16 six-bit scales (stored biased by 32); q ∈ [−4, 3] split as
    low two bits in qs and a high-mask bit that is SET for q ≥ 0 (q = ql)
    and clear for q < 0 (q = ql − 4): out = 0.5·(sc − 32)·q exactly."""
    rng = np.random.default_rng(6)
    sc6 = rng.integers(0, 64, 16)
    q = rng.integers(-4, 4, 256)
    blk = np.zeros(110, np.uint8)
    blk[96:108] = pack_q3k_scales(sc6)
    blk[108:110] = np.array([0.5], np.float16).view(np.uint8)
    for e in range(256):
        s, i = divmod(e, 16)
        ql, hb = (q[e], 1) if q[e] >= 0 else (q[e] + 4, 0)
        blk[32 + 32 * (s // 8) + 16 * (s % 2) + i] |= ql << (2 * ((s // 2) % 4))
        blk[16 * (s % 2) + i] |= hb << (s // 2)
    out = O.dequant(Q3_K, blk, 256)
    expect = np.array([0.5 * (sc6[e // 16] - 32) * q[e] for e in range(256)], np.float32)
    assert np.array_equal(out, expect)


def test_dequant_f16_f32_vs_numpy():
    rng = np.random.default_rng(1)
    h = rng.standard_normal(1000).astype(np.float16)
    assert np.array_equal(O.dequant(F16, h.view(np.uint8), 1000), h.astype(np.float32))
    f = rng.standard_normal(1000).astype(np.float32)
    assert np.array_equal(O.dequant(F32, f.view(np.uint8), 1000), f)


# ── matmuls on [n][k] row-major weights ──────────────────────────────────

def ref_generators(m, k, nbytes):
    """src/quant/matmul/tests.rs:3-17."""
    a = (((np.arange(m * k) * 17) % 100) / 50.0 - 1.0).astype(np.float32)
    b = ((np.arange(nbytes) * 31) % 256).astype(np.uint8)
    return a, b


def f16_weight_bytes(n, k):
    """generate_f16_weight_bytes, tests.rs:573-579."""
    w = (((np.arange(n * k) * 17 + 5) % 200) / 50.0 - 2.0).astype(np.float32)
    return w.astype(np.float16).view(np.uint8)


def within(x, r, abs_tol, rel_tol):
    diff = np.abs(np.asarray(x, np.float64) - np.asarray(r, np.float64))
    return ((diff < abs_tol) | (diff / np.maximum(1.0, np.abs(r)) < rel_tol)).all()


@pytest.mark.parametrize("dtype", [Q5_K, Q2_K, Q3_K])
def test_kquant_matmul_reference_cross_checks(dtype):
    """tests.rs:510-570 (Q5_K), 638-702 (Q2_K), 761-826 (Q3_K): dequantize +
    f32 matmul vs the scalar kernel vs the x86 dispatch (AVX2 order), m in
    {1, 3}, k = 256, n = 8, the reference's own generators; batched vs
    per-row sums within 1e-5."""
    n, k = 8, 256
    for m in (1, 3):
        a, b = ref_generators(m, k, n * (k // 256) * GEOM[dtype][1])
        w = O.dequant(dtype, b, n * k).reshape(n, k)
        ref = (a.reshape(m, k) @ w.T).astype(np.float32)
        s = O.scalar_matmul(dtype, a, b, m, n, k)
        assert within(s, ref, 1e-2, 1e-4)
        assert within(O.avx2_matmul(dtype, a, b, m, n, k), s, 1e-2, 1e-4)
        if m > 1:
            rows = np.stack([O.scalar_matmul(dtype, a[r * k:(r + 1) * k], b, 1, n, k)[0] for r in range(m)])
            assert np.abs(rows - s).max() < 1e-5 * max(1.0, np.abs(s).max())


def test_f16_matmul_reference_cross_checks():
    """tests.rs:581-636: k in {32, 128, 256}, n = 8, m in {1, 3}: dequantize +
    f32 matmul vs scalar vs dispatch within 1e-4 / 1e-5."""
    n = 8
    for k in (32, 128, 256):
        b = f16_weight_bytes(n, k)
        w = O.dequant(F16, b, n * k).reshape(n, k)
        for m in (1, 3):
            a = (((np.arange(m * k) * 17) % 100) / 50.0 - 1.0).astype(np.float32)
            ref = (a.reshape(m, k) @ w.T).astype(np.float32)
            assert within(O.scalar_matmul(F16, a, b, m, n, k), ref, 1e-4, 1e-5)
            assert within(O.avx2_matmul(F16, a, b, m, n, k), ref, 1e-4, 1e-5)


def test_q5_k_avx2_intrinsics_equal_scalar_operation_order():
    rng = np.random.default_rng(13)
    m, n, k = 2, 37, 1024
    b = synth_blocks(Q5_K, n * k // 256, 3)
    a = rng.standard_normal(m * k).astype(np.float32)
    x = O.avx2_matmul(Q5_K, a, b, m, n, k)
    y = O.avx2order_scalar_matmul(Q5_K, a, b, m, n, k)
    assert np.array_equal(x.view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("dtype", [Q5_K, Q2_K, Q3_K, F16])
def test_matmul_vs_f64_brute_force(dtype):
    rng = np.random.default_rng(30 + dtype)
    m, n, k = 2, 48, 1024
    be, bb = GEOM[dtype]
    b = synth_blocks(dtype, n * k // be, 5)
    a = rng.standard_normal(m * k).astype(np.float32)
    w = O.dequant(dtype, b, n * k).reshape(n, k).astype(np.float64)
    exact = a.reshape(m, k).astype(np.float64) @ w.T
    scale = np.abs(a.reshape(m, k)).astype(np.float64) @ np.abs(w).T
    for got in (O.reference_matmul(dtype, a, b, m, n, k), O.scalar_matmul(dtype, a, b, m, n, k)):
        assert (np.abs(got - exact) <= 1e-6 * scale + 1e-6).all()


def test_q5_k_constant_weights_closed_form():
    """W = requantize(1.0), a = 0.5 (the form of benches/quant_matmul.rs:11-14):
    every dequantized weight is equal and every output is K·0.5·w."""
    n, k = 16, 1024
    w = O.requantize(Q5_K, np.ones(n * k, np.float32), n, k)
    v = O.dequant(Q5_K, w, n * k)
    assert np.all(v == v[0])
    c = O.reference_matmul(Q5_K, np.full(k, 0.5, np.float32), w, 1, n, k)
    assert np.all(c == c[0, 0])
    assert abs(c[0, 0] - k * 0.5 * float(v[0])) <= 1e-6 * k


# ── quantized_matmul_impl's GGUF-order route ─────────────────────────────

def test_asymmetric_gguf_order_f16():
    """tests.rs:704-760: F16 weights in GGUF [k, n] order through
    quantized_matmul_impl's fallback (dequantize [k, n] + matmul_f32_gguf)
    equal the f32 matmul of the transposed weights within 1e-4 / 1e-5."""
    k, n = 256, 32
    b = f16_weight_bytes(k, n)
    wg = O.dequant(F16, b, k * n).reshape(k, n)
    for m in (1, 3):
        a = (((np.arange(m * k) * 17) % 100) / 50.0 - 1.0).astype(np.float32)
        ref = (a.reshape(m, k) @ wg).astype(np.float32)
        assert within(O.gguf_order_matmul(F16, a, b, m, n, k), ref, 1e-4, 1e-5)


@pytest.mark.parametrize("dtype", GGUF_ORDER)
def test_gguf_order_route_fma_order_and_zero_rows(dtype):
    """matmul_f32_gguf is a sequential FMA over i, skipping a_i = 0
    (dispatch.rs:541-557): against an f64 product within f32 error, and rows
    whose activation is zero (including one whose weights hold an infinity)
    contribute nothing."""
    rng = np.random.default_rng(dtype + 3)
    m, n, k = 3, 512, 96
    be, bb = GEOM[dtype]
    b = synth_blocks(dtype, k * n // be, 4)
    a = rng.standard_normal((m, k)).astype(np.float32)
    a[:, 5] = 0.0
    wg = O.dequant(dtype, b, k * n).reshape(k, n).astype(np.float64)
    got = O.gguf_order_matmul(dtype, a, b, m, n, k)
    exact = a.astype(np.float64) @ wg
    scale = np.abs(a).astype(np.float64) @ np.abs(wg)
    assert (np.abs(got - exact) <= 1e-6 * scale + 1e-6).all()
    if dtype in (F16, F32):
        bi = b.copy()
        row5 = bi.view(np.float16 if dtype == F16 else np.float32).reshape(k, n)[5]
        row5[:] = np.inf
        assert np.array_equal(O.gguf_order_matmul(dtype, a, bi, m, n, k), got)


# ── int8 dot-product references ──────────────────────────────────────────

@pytest.mark.parametrize("dtype", [Q5_K, Q6_K])
def test_dotprod_reference_is_integer_exact(dtype):
    """matmul_q5_k / q6_k_dotprod_reference (tests.rs:136-330): exact i32 dots
    of the weight quants with the Q8_0 activation quants, so the result equals
    the f64 product of the dequantized activations and weights within f32
    rounding of the per-block terms."""
    rng = np.random.default_rng(23 + dtype)
    m, n, k = 2, 16, 768
    a = rng.standard_normal(m * k).astype(np.float32)
    aq = O.quantize_activations_q8_0(a, m, k)
    b = synth_blocks(dtype, n * k // 256, 2)
    got = O.dotprod_ref(dtype, aq, b, m, n, k)
    ad = O.dequant(Q8_0, aq, m * k).reshape(m, k).astype(np.float64)
    w = O.dequant(dtype, b, n * k).reshape(n, k).astype(np.float64)
    exact = ad @ w.T
    scale = np.abs(ad) @ np.abs(w).T
    assert (np.abs(got - exact) <= 1e-5 * scale + 1e-6).all()


# ── the decode step with every format ────────────────────────────────────

@pytest.mark.parametrize("dts", [[Q5_K] * 7, [F16, Q2_K, Q3_K, F32, Q5_K, Q2_K, Q3_K]])
def test_decode_step_new_formats_match_f64_composition(dts):
    """One decode step of a 1-layer toy model whose weights use the new
    formats (F32/F16/Q2_K/Q3_K in GGUF [in][out] order, Q5_K row-major), and
    the batched prefill of 5 tokens, against a float64 composition of the
    pinned dequantized weights."""
    rng = np.random.default_rng(5)
    vocab, d, nh, nkv, hd, dff, ms = 64, 256, 4, 2, 64, 512, 16
    cfg = O.LlamaCfg(vocab, d, 1, nh, nkv, hd, dff, ms, 10000.0, 1e-5)
    shapes = [(nh * hd, d), (nkv * hd, d), (nkv * hd, d), (d, nh * hd), (dff, d), (dff, d), (d, dff)]
    W = [synth_blocks(dt, n * k // GEOM[dt][0], 40 + j) for j, (dt, (n, k)) in enumerate(zip(dts, shapes))]
    deq = []
    for dt, w, (n, k) in zip(dts, W, shapes):
        f = O.dequant(dt, w, n * k).astype(np.float64)
        deq.append(f.reshape(k, n).T if dt in GGUF_ORDER else f.reshape(n, k))
    norms = [(1 + 0.02 * rng.standard_normal(d)).astype(np.float32) for _ in range(2)]
    final = (1 + 0.02 * rng.standard_normal(d)).astype(np.float32)
    lm = synth_blocks(Q6_K, vocab * d // 256, 99)
    lmw = O.dequant(Q6_K, lm, vocab * d).reshape(vocab, d).astype(np.float64)
    s, c = O.precompute_rope(ms, hd, 10000.0)
    X = rng.standard_normal((5, d)).astype(np.float32)

    def rms(v, w):
        return v / np.sqrt((v * v).sum() / v.size + 1e-5) * w

    def rope(v, nheads, pos):
        v = v.reshape(nheads, hd).copy()
        ss, cc = s.reshape(ms, hd // 2)[pos].astype(np.float64), c.reshape(ms, hd // 2)[pos].astype(np.float64)
        a, b = v[:, :hd // 2].copy(), v[:, hd // 2:].copy()
        v[:, :hd // 2], v[:, hd // 2:] = a * cc - b * ss, a * ss + b * cc
        return v

    K = np.zeros((nkv, ms, hd))
    V = np.zeros((nkv, ms, hd))
    kv = np.zeros((1, 2, nkv, ms, hd), np.float32)
    fill = 0
    for pos in range(5):
        logits, fill = O.decode_step(cfg, X[pos], pos, [W], dts, [norms], final, lm, Q6_K, s, c, kv, fill)
        x = X[pos].astype(np.float64)
        h = rms(x, norms[0])
        q, k_ = rope(deq[0] @ h, nh, pos), rope(deq[1] @ h, nkv, pos)
        K[:, pos], V[:, pos] = k_, (deq[2] @ h).reshape(nkv, hd)
        att = np.zeros((nh, hd))
        for hh in range(nh):
            g = hh // (nh // nkv)
            sc = K[g, :pos + 1] @ q[hh] / np.sqrt(hd)
            p = np.exp(sc - sc.max())
            att[hh] = (p / p.sum()) @ V[g, :pos + 1]
        x = x + deq[3] @ att.reshape(-1)
        h = rms(x, norms[1])
        gt, up = deq[4] @ h, deq[5] @ h
        x = x + deq[6] @ (gt / (1 + np.exp(-gt)) * up)
        ref = lmw @ rms(x, final)
        np.testing.assert_allclose(logits, ref, rtol=1e-4, atol=1e-3 * np.abs(ref).max())
    kvb = np.zeros_like(kv)
    lb = O.forward_batch(cfg, X, [W], dts, [norms], final, lm, Q6_K, s, c, kvb)
    np.testing.assert_allclose(lb, logits, rtol=1e-4, atol=1e-4 * np.abs(logits).max())
    np.testing.assert_allclose(kvb, kv, rtol=1e-4, atol=1e-4)
