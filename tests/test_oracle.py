"""Pins the CPU oracle (oracle/oracle.c) to checks that do not restate its own
formulas: the reference's known-answer tests, exhaustive comparison with
independent f16 conversions, packing round trips, closed forms, f64 brute
force and the reference's own cross-kernel tolerances."""
import os

import numpy as np
import pytest

from oracle import oracle as O
from tests._util import GEOM, Q4_K, Q6_K, Q8_0, synth_blocks

HERE = os.path.dirname(os.path.abspath(__file__))


# ── f16 (third-party `half` 2.7.1 semantics) ─────────────────────────────

def test_f16_to_f32_exhaustive_vs_numpy():
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([O.f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_round_nearest_even_vs_numpy():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(200000) * np.float64(10.0) ** rng.integers(-9, 6, 200000)).astype(np.float32)
    special = np.array([0.0, -0.0, np.inf, -np.inf, 65504.0, 65520.0, 65519.99, 6.1035156e-05, 5.9604645e-08,
                        2.9802322e-08, 2.9802326e-08, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, 1.0 + 2 ** -11 + 2 ** -20,
                        -(1.0 + 2 ** -11), 2049.0, 2051.0], dtype=np.float32)
    x = np.concatenate([x, special])
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    got = np.array([O.f32_to_f16(float(v)) for v in x], dtype=np.uint16)
    assert np.array_equal(got, ref)


def test_decode_d_nan_inf_fallback_all_patterns():
    """decode_f16_scale (common.rs:19-27): finite → the f16 value; NaN/Inf
    patterns (exponent 31) → bits / 65536."""
    for b in range(65536):
        v = O.decode_d(b)
        if (b & 0x7C00) == 0x7C00:
            assert v == np.float32(b / 65536.0), b
        else:
            f = np.uint16(b).view(np.float16).astype(np.float32)
            assert v == f or (v == 0 and f == 0), b


# ── scale packing (get_scale_min_k4 vs requantize_q4_k's packing) ────────

def pack_k4(sc, m):
    """Packing of requantize_q4_k (src/quant/matmul/dispatch.rs:248-256)."""
    out = np.zeros(12, dtype=np.uint8)
    for k in range(4):
        out[k] = (sc[k] & 63) | ((sc[k + 4] >> 4) << 6)
        out[4 + k] = (m[k] & 63) | ((m[k + 4] >> 4) << 6)
        out[8 + k] = (sc[k + 4] & 0x0F) | ((m[k + 4] & 0x0F) << 4)
    return out


def test_get_scale_min_k4_round_trip_all_values():
    vals = np.arange(64)
    for j in range(8):
        for s_ in vals:
            sc = [(s_ + 7 * i) % 64 for i in range(8)]
            m = [(63 - s_ + 5 * i) % 64 for i in range(8)]
            sc[j] = int(s_)
            packed = pack_k4(sc, m)
            for jj in range(8):
                assert O.get_scale_min_k4(jj, packed) == (sc[jj], m[jj])


# ── dequant: reference KATs and closed forms ─────────────────────────────

def test_dequant_q8_0_kat_single_block():
    """tests/gguf_loader.rs:180-195: d = f16(0.5), q = i → 0.5·i."""
    blk = np.zeros(34, dtype=np.uint8)
    blk[0:2] = np.array([0.5], np.float16).view(np.uint8)
    blk[2:] = np.arange(32, dtype=np.int8).view(np.uint8)
    assert np.array_equal(O.dequant(Q8_0, blk, 32), np.arange(32, dtype=np.float32) * 0.5)


def test_dequant_q8_0_kat_two_blocks():
    """tests/gguf_loader.rs:197-221: scales 1 and 2, quants i and i+10."""
    b = np.zeros(68, dtype=np.uint8)
    b[0:2] = np.array([1.0], np.float16).view(np.uint8)
    b[2:34] = np.arange(32, dtype=np.int8).view(np.uint8)
    b[34:36] = np.array([2.0], np.float16).view(np.uint8)
    b[36:68] = (np.arange(32) + 10).astype(np.int8).view(np.uint8)
    out = O.dequant(Q8_0, b, 64)
    assert np.array_equal(out[:32], np.arange(32, dtype=np.float32))
    assert np.array_equal(out[32:], (np.arange(32, dtype=np.float32) + 10) * 2)


def test_dequant_q4_k_hand_block():
    """d = 1, dmin = 0.5, sub-block s has scale s+1 and min s; quant q(l) = l
    % 16 (low) and 15 - l % 16 (high): every value is d·sc·q − dmin·m exactly."""
    sc = [s + 1 for s in range(8)]
    m = list(range(8))
    blk = np.zeros(144, dtype=np.uint8)
    blk[0:2] = np.array([1.0], np.float16).view(np.uint8)
    blk[2:4] = np.array([0.5], np.float16).view(np.uint8)
    blk[4:16] = pack_k4(sc, m)
    for j in range(4):
        for l in range(32):
            blk[16 + 32 * j + l] = (l % 16) | ((15 - l % 16) << 4)
    out = O.dequant(Q4_K, blk, 256)
    for j in range(4):
        for l in range(32):
            assert out[64 * j + l] == sc[2 * j] * (l % 16) - 0.5 * m[2 * j]
            assert out[64 * j + 32 + l] == sc[2 * j + 1] * (15 - l % 16) - 0.5 * m[2 * j + 1]


def test_dequant_q6_k_hand_block():
    """d = 0.25; 6-bit quant of element e is e % 64 (q - 32 in [-32, 31]);
    sub-block scales alternate sign: every value is 0.25·s·(q−32) exactly."""
    q = np.arange(256) % 64
    s = np.array([(i + 1) * (-1) ** i for i in range(16)], dtype=np.int8)
    blk = np.zeros(210, dtype=np.uint8)
    for h in range(2):
        for l in range(32):
            q1, q2, q3, q4 = (q[h * 128 + l + 32 * t] for t in range(4))
            blk[h * 64 + l] = (q1 & 15) | ((q3 & 15) << 4)
            blk[h * 64 + l + 32] = (q2 & 15) | ((q4 & 15) << 4)
            blk[128 + h * 32 + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    blk[192:208] = s.view(np.uint8)
    blk[208:210] = np.array([0.25], np.float16).view(np.uint8)
    out = O.dequant(Q6_K, blk, 256)
    for e in range(256):
        h, r = divmod(e, 128)
        t, l = divmod(r, 32)
        sub = h * 8 + l // 16 + 2 * t
        assert out[e] == 0.25 * float(s[sub]) * float(q[e] - 32), e


@pytest.mark.parametrize("dtype,bound", [(Q4_K, 0.3), (Q6_K, 0.08)])
def test_requantize_round_trip_reference_bounds(dtype, bound):
    """tests/correctness.rs:1272-1316: gaussian σ=0.5 clamped to ±1.5, 4×256,
    requantize → dequantize within 0.3 (Q4_K) / 0.08 (Q6_K)."""
    rng = np.random.default_rng(42)
    data = np.clip(rng.standard_normal(4 * 256) * 0.5, -1.5, 1.5).astype(np.float32)
    q = O.requantize(dtype, data, 4, 256)
    assert q.size == 4 * GEOM[dtype][1]
    back = O.dequant(dtype, q, 4 * 256)
    assert np.abs(back - data).max() <= bound


def test_requantize_q8_0_round_trip_reference_bound():
    """tests/correctness.rs:1253-1264: values in [-1, 1), abs error ≤ 0.01."""
    rng = np.random.default_rng(7)
    for n in (128, 256, 384):
        data = rng.uniform(-1, 1, n).astype(np.float32)
        back = O.dequant(Q8_0, O.requantize(Q8_0, data, 1, n), n)
        assert np.abs(back - data).max() <= 0.01


# ── matmuls ──────────────────────────────────────────────────────────────

def ref_generators(m, k, n, bb):
    """src/quant/matmul/tests.rs:3-17."""
    a = (((np.arange(m * k) * 17) % 100) / 50.0 - 1.0).astype(np.float32)
    b = ((np.arange(n * (k // 256) * bb) * 31) % 256).astype(np.uint8)
    return a, b


@pytest.mark.parametrize("dtype", [Q4_K, Q6_K])
def test_avx2_vs_scalar_reference_tolerance(dtype):
    """tests.rs:386-508 on x86: AVX2 vs scalar kernels, m in {1,3}, k=256,
    n=8: diff < 1e-2 or diff/max(1,|ref|) < 1e-4."""
    for m in (1, 3):
        a, b = ref_generators(m, 256, 8, GEOM[dtype][1])
        s = O.scalar_matmul(dtype, a, b, m, 8, 256)
        v = O.avx2_matmul(dtype, a, b, m, 8, 256)
        diff = np.abs(s - v)
        assert ((diff < 1e-2) | (diff / np.maximum(1.0, np.abs(s)) < 1e-4)).all()


@pytest.mark.parametrize("dtype", [Q4_K, Q6_K])
def test_avx2_intrinsics_equal_scalar_operation_order(dtype):
    """The AVX2-intrinsic build and the scalar restatement of the same
    operation order (hsum_f32x8, avx2.rs:13-20) agree bit for bit."""
    rng = np.random.default_rng(dtype)
    m, n, k = 2, 37, 1024
    b = synth_blocks(dtype, n * k // 256, 3)
    a = rng.standard_normal(m * k).astype(np.float32)
    x = O.avx2_matmul(dtype, a, b, m, n, k)
    y = O.avx2order_scalar_matmul(dtype, a, b, m, n, k)
    assert np.array_equal(x.view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("dtype", [Q8_0, Q4_K, Q6_K])
def test_matmul_vs_f64_brute_force(dtype):
    """Every output equals the f64 dot of the (pinned) dequantized row within
    f32 summation error."""
    rng = np.random.default_rng(11 + dtype)
    m, n, k = 2, 64, 2048
    be, bb = GEOM[dtype]
    b = synth_blocks(dtype, n * (k // be), 5)
    a = rng.standard_normal(m * k).astype(np.float32)
    w = O.dequant(dtype, b, n * k).reshape(n, k).astype(np.float64)
    exact = a.reshape(m, k).astype(np.float64) @ w.T
    got = O.reference_matmul(dtype, a, b, m, n, k)
    scale = np.abs(a.reshape(m, k)).astype(np.float64) @ np.abs(w).T
    assert (np.abs(got - exact) <= 1e-6 * scale + 1e-6).all()


@pytest.mark.parametrize("dtype", [Q8_0, Q4_K, Q6_K])
def test_bench_closed_form_constant_weights(dtype):
    """benches/quant_matmul.rs:11-14: W = requantize(1.0), a = 0.5 → every
    output is K·0.5·dequant(1.0)."""
    n, k = 16, 1024
    w = O.requantize(dtype, np.ones(n * k, np.float32), n, k)
    v = O.dequant(dtype, w, n * k)
    assert np.all(v == v[0])
    c = O.reference_matmul(dtype, np.full(k, 0.5, np.float32), w, 1, n, k)
    assert np.all(c == c[0, 0])
    assert abs(c[0, 0] - k * 0.5 * float(v[0])) <= 1e-6 * k


def test_avx2_q8_0_defect_is_documented():
    """avx2::matmul_q8_0 (avx2.rs:134-207) addresses its second 8 quants at
    +16 bytes: on random blocks it disagrees with the scalar kernel (which
    matches the f64 brute force above), so the HIP path follows the scalar."""
    rng = np.random.default_rng(3)
    n, k = 8, 256
    b = synth_blocks(Q8_0, n * k // 32, 9)
    a = rng.standard_normal(k).astype(np.float32)
    s = O.scalar_matmul(Q8_0, a, b, 1, n, k)
    v = O.avx2_matmul(Q8_0, a, b, 1, n, k)
    assert np.abs(s - v).max() > 1e-2
    # a single block (the last of its buffer: bytes past it read as 0) with
    # q[8:16] == q[16:24] and q[24:32] == 0 makes the mis-addressed reads
    # coincide with the right ones
    blk = np.zeros(34, dtype=np.uint8)
    blk[0:2] = np.array([0.5], np.float16).view(np.uint8)
    qv = rng.integers(-127, 128, 32).astype(np.int8)
    qv[8:16] = qv[16:24]
    qv[24:32] = 0
    blk[2:] = qv.view(np.uint8)
    a2 = rng.standard_normal(32).astype(np.float32)
    np.testing.assert_allclose(O.avx2_matmul(Q8_0, a2, blk, 1, 1, 32), O.scalar_matmul(Q8_0, a2, blk, 1, 1, 32),
                               rtol=1e-6, atol=1e-6)


# ── Q8_0 activation scheme (neon.rs:45-155) and dotprod references ──────

def test_quantize_q8_0_block_hand_cases():
    x = np.zeros(32, np.float32)
    q = O.quantize_activations_q8_0(x, 1, 32)
    assert np.all(q[2:] == 0) and q[0] == 0 and q[1] == 0  # d = 0 → zero quants
    x = np.zeros(32, np.float32)
    x[0] = 127.0  # d = 1 exactly
    x[1:6] = [2.5, 3.5, -2.5, 0.5, 1.5]  # ties to even: 2, 4, -2, 0, 2
    q = O.quantize_activations_q8_0(x, 1, 32)
    assert int(q[0]) | (int(q[1]) << 8) == int(np.array([1.0], np.float16).view(np.uint16)[0])
    assert list(q[2:8].view(np.int8)) == [127, 2, 4, -2, 0, 2]


def test_dotprod_reference_is_integer_exact():
    """matmul_q4_k_dotprod_reference (tests.rs:62-134) against an f64 dot of the
    dequantized activation blocks and weights."""
    rng = np.random.default_rng(21)
    m, n, k = 2, 16, 512
    a = rng.standard_normal(m * k).astype(np.float32)
    aq = O.quantize_activations_q8_0(a, m, k)
    b = synth_blocks(Q4_K, n * k // 256, 2)
    got = O.dotprod_ref(Q4_K, aq, b, m, n, k)
    ad = O.dequant(Q8_0, aq, m * k).reshape(m, k).astype(np.float64)
    w = O.dequant(Q4_K, b, n * k).reshape(n, k).astype(np.float64)
    exact = ad @ w.T
    scale = np.abs(ad) @ np.abs(w).T
    assert (np.abs(got - exact) <= 1e-5 * scale + 1e-6).all()


def test_dotprod_q8_0_reference_is_integer_exact():
    """matmul_q8_0_dotprod_reference (tests.rs:28-60) against the float64 product
    of the dequantized Q8_0 activation blocks and weights: per block an exact i32
    sum times d_a·d_b, so only f32 rounding separates them. k = 200 is ragged
    (blocks_per_row = div_ceil(k, 32) = 7, the last activation block zero-padded
    by the quantizer)."""
    rng = np.random.default_rng(23)
    for m, n, k in ((3, 24, 512), (2, 8, 200)):
        nb = (k + 31) // 32
        a = rng.standard_normal(m * k).astype(np.float32) * 3
        aq = O.quantize_activations_q8_0(a, m, k)
        b = synth_blocks(Q8_0, n * nb, 3)
        got = O.dotprod_ref(Q8_0, aq, b, m, n, k)
        ad = O.dequant(Q8_0, aq, m * nb * 32).reshape(m, nb * 32).astype(np.float64)
        w = O.dequant(Q8_0, b, n * nb * 32).reshape(n, nb * 32).astype(np.float64)
        assert not ad[:, k:].any()  # the padded tail of the last block holds zeros
        exact = ad @ w.T
        scale = np.abs(ad) @ np.abs(w).T
        assert (np.abs(got - exact) <= 1e-6 * scale + 1e-7).all()


def _q8_block(d, q):
    return np.concatenate([np.array([d], np.float32).astype(np.float16).view(np.uint8),
                           np.asarray(q, np.int8).view(np.uint8)])


def test_dotprod_q8_0_reference_hand_blocks():
    """Two blocks per row with distinct scales on both sides, exact in f32:
    block 0 contributes (Σ i·1)·(d_a·d_b) and block 1 (Σ 2·q_b)·(d_a·d_b). A
    block index off by one, a scale paired with the wrong block or a wrong row
    of activations changes the sums (140, 316, ... instead of 252 and 318)."""
    i = np.arange(32)
    qb1 = np.where(i < 16, 3, -1)
    a = np.concatenate([_q8_block(1.0, i), _q8_block(0.5, np.full(32, 2)),    # row 0
                        _q8_block(0.5, i), _q8_block(1.0, np.full(32, 2))])   # row 1: scales swapped
    b = np.concatenate([_q8_block(0.25, np.ones(32)), _q8_block(4.0, qb1)])
    got = O.dotprod_ref(Q8_0, a, b, 2, 1, 64)
    # row 0: 496·(1·0.25) + 64·(0.5·4) = 124 + 128; row 1: 496·(0.5·0.25) + 64·(1·4) = 62 + 256
    assert got.ravel().tolist() == [252.0, 318.0]


# ── decode-step math ─────────────────────────────────────────────────────

def test_rmsnorm_constant_vector():
    n, c, eps = 4096, 3.0, 1e-5
    w = np.linspace(0.5, 1.5, n).astype(np.float32)
    out = O.rmsnorm(np.full(n, c, np.float32), w, eps)
    np.testing.assert_allclose(out, c / np.sqrt(c * c + eps) * w, rtol=2e-6)


def test_rope_identity_and_rotation():
    ms, hd, base = 64, 128, 500000.0
    s, c = O.precompute_rope(ms, hd, base)
    rng = np.random.default_rng(1)
    x = rng.standard_normal(4 * hd).astype(np.float32)
    assert np.array_equal(O.apply_rope(x, 4, hd, 0, s, c, ms), x)
    for pos in (1, 37, 63, 500):  # 500 clamps to 63
        y = O.apply_rope(x, 4, hd, pos, s, c, ms).reshape(4, hd).astype(np.float64)
        xr = x.reshape(4, hd).astype(np.float64)
        p = min(pos, ms - 1)
        th = p * base ** (-2.0 * np.arange(hd // 2) / hd)
        e0 = xr[:, :64] * np.cos(th) - xr[:, 64:] * np.sin(th)
        e1 = xr[:, :64] * np.sin(th) + xr[:, 64:] * np.cos(th)
        np.testing.assert_allclose(y, np.concatenate([e0, e1], 1), atol=2e-4)
        np.testing.assert_allclose(np.hypot(y[:, :64], y[:, 64:]), np.hypot(xr[:, :64], xr[:, 64:]), rtol=1e-5)


def test_attention_one_hot_and_uniform():
    hd, seq = 128, 50
    rng = np.random.default_rng(2)
    v = rng.standard_normal((seq, hd)).astype(np.float32)
    k = np.zeros((seq, hd), np.float32)
    q = np.zeros(hd, np.float32)
    np.testing.assert_allclose(O.attn_direct(q, k, v, seq, hd), v.mean(0), atol=1e-6)  # uniform scores
    k[17] = 1.0
    q[:] = 10.0
    np.testing.assert_allclose(O.attn_direct(q, k, v, seq, hd), v[17], atol=1e-6)


def test_argmax_last_of_ties():
    x = np.array([1, 5, 2, 5, 5, 0], np.float32)
    assert O.argmax(x) == 4


def test_decode_step_matches_f64_composition():
    """One decode step of a 1-layer toy model against a float64 composition of
    the pinned pieces (dequantized weights, rope table): catches wiring errors
    (GQA head mapping, cache slot, residuals, SiLU glue)."""
    rng = np.random.default_rng(5)
    vocab, d, nh, nkv, hd, dff, ms = 64, 256, 4, 2, 64, 512, 16
    cfg = O.LlamaCfg(vocab, d, 1, nh, nkv, hd, dff, ms, 10000.0, 1e-5)
    shapes = [(nh * hd, d), (nkv * hd, d), (nkv * hd, d), (d, nh * hd), (dff, d), (dff, d), (d, dff)]
    W = [synth_blocks(Q4_K, n * k // 256, 40 + j) for j, (n, k) in enumerate(shapes)]
    norms = [(1 + 0.02 * rng.standard_normal(d)).astype(np.float32) for _ in range(2)]
    final = (1 + 0.02 * rng.standard_normal(d)).astype(np.float32)
    lm = synth_blocks(Q6_K, vocab * d // 256, 99)
    x0 = rng.standard_normal(d).astype(np.float32)
    s, c = O.precompute_rope(ms, hd, 10000.0)
    kv = np.zeros((1, 2, nkv, ms, hd), np.float32)
    kv[0, :, :, :3] = rng.standard_normal((2, nkv, 3, hd))  # 3 cached positions
    kv0 = kv.copy()
    pos, fill = 3, 3
    logits, fill2 = O.decode_step(cfg, x0, pos, [W], [Q4_K] * 7, [norms], final, lm, Q6_K, s, c, kv, fill)
    assert fill2 == 4
    # f64 composition
    deq = [O.dequant(Q4_K, w, n * k).reshape(n, k).astype(np.float64) for w, (n, k) in zip(W, shapes)]
    lmw = O.dequant(Q6_K, lm, vocab * d).reshape(vocab, d).astype(np.float64)

    def rms(v, w):
        return v / np.sqrt((v * v).sum() / v.size + 1e-5) * w

    def rope(v, nheads):
        v = v.reshape(nheads, hd).copy()
        ss, cc = s.reshape(ms, hd // 2)[pos].astype(np.float64), c.reshape(ms, hd // 2)[pos].astype(np.float64)
        a, b = v[:, :hd // 2].copy(), v[:, hd // 2:].copy()
        v[:, :hd // 2], v[:, hd // 2:] = a * cc - b * ss, a * ss + b * cc
        return v

    x = x0.astype(np.float64)
    h = rms(x, norms[0])
    q, k_, v_ = rope(deq[0] @ h, nh), rope(deq[1] @ h, nkv), (deq[2] @ h).reshape(nkv, hd)
    K = kv0[0, 0].astype(np.float64).copy()
    V = kv0[0, 1].astype(np.float64).copy()
    K[:, fill], V[:, fill] = k_, v_
    att = np.zeros((nh, hd))
    for hh in range(nh):
        g = hh // (nh // nkv)
        sc = K[g, :fill + 1] @ q[hh] / np.sqrt(hd)
        p = np.exp(sc - sc.max())
        att[hh] = (p / p.sum()) @ V[g, :fill + 1]
    x = x + deq[3] @ att.reshape(-1)
    h = rms(x, norms[1])
    gt, up = deq[4] @ h, deq[5] @ h
    x = x + deq[6] @ (gt / (1 + np.exp(-gt)) * up)
    ref = lmw @ rms(x, final)
    np.testing.assert_allclose(logits, ref, rtol=1e-4, atol=1e-3 * np.abs(ref).max())
    np.testing.assert_allclose(kv[0, 0, :, fill], k_, rtol=1e-4, atol=1e-4)


def _toy_model(nl, seed, dts=None):
    rng = np.random.default_rng(seed)
    vocab, d, nh, nkv, hd, dff, ms = 64, 256, 4, 2, 64, 512, 16
    shapes = [(nh * hd, d), (nkv * hd, d), (nkv * hd, d), (d, nh * hd), (dff, d), (dff, d), (d, dff)]
    dts = dts or [Q4_K] * 7
    W = [[synth_blocks(dts[j], n * k // GEOM[dts[j]][0], seed * 1000 + 10 * l + j) for j, (n, k) in enumerate(shapes)]
         for l in range(nl)]
    norms = [[(1 + 0.02 * rng.standard_normal(d)).astype(np.float32) for _ in range(2)] for _ in range(nl)]
    final = (1 + 0.02 * rng.standard_normal(d)).astype(np.float32)
    lm = synth_blocks(Q6_K, vocab * d // 256, seed + 99)
    return dict(vocab=vocab, d=d, nh=nh, nkv=nkv, hd=hd, dff=dff, ms=ms, W=W, norms=norms, final=final, lm=lm,
                dts=dts, rng=rng)


def test_decode_step_resume_at_the_last_layer_is_the_head():
    """orc_decode_step_from entered at start_layer = n_layers (a budgeted decode
    whose every layer completed, runner.rs:1201-1217) runs no layer: its logits
    are the final RMSNorm and the LM head of x — bit for bit the pinned rmsnorm
    and LM-head matmul, and the float64 composition — the cache is not written
    and its fill still advances (StaticKVCache::advance)."""
    t = _toy_model(2, 31)
    cfg = O.LlamaCfg(t["vocab"], t["d"], 2, t["nh"], t["nkv"], t["hd"], t["dff"], t["ms"], 10000.0, 1e-5)
    s, c = O.precompute_rope(t["ms"], t["hd"], 10000.0)
    x = (t["rng"].standard_normal(t["d"]) * 4).astype(np.float32)
    kv = t["rng"].standard_normal((2, 2, t["nkv"], t["ms"], t["hd"])).astype(np.float32)
    kv0 = kv.copy()
    logits, fill = O.decode_step(cfg, x, 5, t["W"], t["dts"], t["norms"], t["final"], t["lm"], Q6_K, s, c, kv, 5,
                                 start_layer=2)
    assert fill == 6 and np.array_equal(kv, kv0)
    head = O.reference_matmul(Q6_K, O.rmsnorm(x, t["final"], 1e-5), t["lm"], 1, t["vocab"], t["d"])[0]
    assert np.array_equal(logits.view(np.uint32), head.view(np.uint32))
    x64 = x.astype(np.float64)
    h = x64 / np.sqrt((x64 * x64).mean() + 1e-5) * t["final"]
    lmw = O.dequant(Q6_K, t["lm"], t["vocab"] * t["d"]).reshape(t["vocab"], t["d"]).astype(np.float64)
    ref = lmw @ h
    np.testing.assert_allclose(logits, ref, rtol=1e-5, atol=1e-5 * np.abs(ref).max())


def test_decode_step_resume_at_layer_one():
    """Entered at layer 1 of a 2-layer model with x as the residual stream after
    layer 0, the step equals a 1-layer model made of layer 1 alone (its
    weights, norms and cache layer) — logits and written K/V bit for bit —
    whatever layer 0's weights and cache hold, and it leaves layer 0's cache
    untouched. Resuming one layer early or late, or indexing the weights,
    norms or cache by the wrong layer, changes the result."""
    t = _toy_model(2, 37)
    cfg2 = O.LlamaCfg(t["vocab"], t["d"], 2, t["nh"], t["nkv"], t["hd"], t["dff"], t["ms"], 10000.0, 1e-5)
    cfg1 = O.LlamaCfg(t["vocab"], t["d"], 1, t["nh"], t["nkv"], t["hd"], t["dff"], t["ms"], 10000.0, 1e-5)
    s, c = O.precompute_rope(t["ms"], t["hd"], 10000.0)
    x = (t["rng"].standard_normal(t["d"]) * 2).astype(np.float32)
    kv = np.zeros((2, 2, t["nkv"], t["ms"], t["hd"]), np.float32)
    kv[:, :, :, :4] = t["rng"].standard_normal((2, 2, t["nkv"], 4, t["hd"]))
    pos, fill = 4, 4
    runs = []
    for garbage_seed in (1, 2):
        g = _toy_model(1, 500 + garbage_seed)  # layer 0 replaced by unrelated weights, norms and cache
        W = [g["W"][0], t["W"][1]]
        norms = [g["norms"][0], t["norms"][1]]
        k2 = kv.copy()
        k2[0] = g["rng"].standard_normal(k2[0].shape)
        k2_l0 = k2[0].copy()
        lg, f2 = O.decode_step(cfg2, x, pos, W, t["dts"], norms, t["final"], t["lm"], Q6_K, s, c, k2, fill,
                               start_layer=1)
        assert f2 == fill + 1 and np.array_equal(k2[0], k2_l0)
        runs.append((lg, k2[1].copy()))
    assert np.array_equal(runs[0][0], runs[1][0]) and np.array_equal(runs[0][1], runs[1][1])
    k1 = kv[1:2].copy()
    l1, f1 = O.decode_step(cfg1, x, pos, [t["W"][1]], t["dts"], [t["norms"][1]], t["final"], t["lm"], Q6_K, s, c, k1,
                           fill)
    assert f1 == fill + 1
    assert np.array_equal(runs[0][0].view(np.uint32), l1.view(np.uint32))
    assert np.array_equal(runs[0][1], k1[0])
    assert not np.array_equal(k1[0], kv[1])  # the step wrote slot 4 of layer 1
    # entering at layer 0 (the whole step) or at layer 2 (the head alone) gives other logits
    for other in (0, 2):
        lo, _ = O.decode_step(cfg2, x, pos, [t["W"][0], t["W"][1]], t["dts"], t["norms"], t["final"], t["lm"], Q6_K, s,
                              c, kv.copy(), fill, start_layer=other)
        assert np.abs(lo - l1).max() > 1e-2 * np.abs(l1).max()


def test_attn_direct_sliding_window_is_attention_over_the_last_w_keys():
    """attn_direct with sliding_window w < seq (runner.rs:1768-1777) masks the
    keys before seq - w: the result equals plain attention over the last w
    positions (float64 as well); w >= seq is no window at all."""
    hd, seq = 128, 45
    rng = np.random.default_rng(9)
    q = rng.standard_normal(hd).astype(np.float32)
    k = rng.standard_normal((seq, hd)).astype(np.float32)
    v = rng.standard_normal((seq, hd)).astype(np.float32)
    full = O.attn_direct(q, k, v, seq, hd)
    for w in (1, 7, 44):
        got = O.attn_direct(q, k, v, seq, hd, window=w)
        tail = O.attn_direct(q, k[seq - w:], v[seq - w:], w, hd)
        np.testing.assert_allclose(got, tail, rtol=1e-6, atol=1e-6)
        sc = k[seq - w:].astype(np.float64) @ q / np.sqrt(hd)
        p = np.exp(sc - sc.max())
        np.testing.assert_allclose(got, (p / p.sum()) @ v[seq - w:], rtol=1e-5, atol=1e-5)
        assert np.abs(got - full).max() > 1e-3
    assert np.array_equal(O.attn_direct(q, k, v, seq, hd, window=seq), full)
    assert np.array_equal(O.attn_direct(q, k, v, seq, hd, window=1000), full)
    np.testing.assert_allclose(O.attn_direct(q, k, v, seq, hd, window=1), v[seq - 1], rtol=1e-6, atol=1e-6)


def test_sliding_window_prefill_and_decode():
    """The window in both CPU paths: forward_batch's attention_batch (query i
    sees keys max(0, i - w + 1) ..= i, runner.rs:1825-1845) and the decode
    step's attn_direct (keys seq - w .. seq) agree token by token, match the
    float64 model with the same mask, differ from the unwindowed model, and a
    window at least the prompt length changes nothing."""
    from tests._model64 import logits64

    t = _toy_model(2, 41, dts=[Q4_K, Q8_0, Q6_K, Q4_K, Q4_K, Q8_0, Q6_K])
    n, ms = 13, 16
    emb = t["rng"].standard_normal((t["vocab"], t["d"])).astype(np.float32)
    toks = t["rng"].integers(0, t["vocab"], n)
    s, c = O.precompute_rope(ms, t["hd"], 10000.0)
    res = {}
    for w in (0, 5, 13):
        cfg = O.LlamaCfg(t["vocab"], t["d"], 2, t["nh"], t["nkv"], t["hd"], t["dff"], ms, 10000.0, 1e-5, w)
        kvb = np.zeros((2, 2, t["nkv"], ms, t["hd"]), np.float32)
        lb = O.forward_batch(cfg, emb[toks], t["W"], t["dts"], t["norms"], t["final"], t["lm"], Q6_K, s, c, kvb)
        kvs = np.zeros_like(kvb)
        fill = 0
        for i in range(n):
            ls, fill = O.decode_step(cfg, emb[toks[i]], i, t["W"], t["dts"], t["norms"], t["final"], t["lm"], Q6_K, s,
                                     c, kvs, fill)
        np.testing.assert_allclose(lb, ls, rtol=1e-4, atol=1e-4 * np.abs(ls).max())
        np.testing.assert_allclose(kvb, kvs, rtol=1e-4, atol=1e-4)
        cd = dict(vocab_size=t["vocab"], d_model=t["d"], num_heads=t["nh"], num_kv_heads=t["nkv"], head_dim=t["hd"],
                  d_ff=t["dff"], max_seq_len=ms, rope_base=10000.0, rms_norm_eps=1e-5, sliding_window=w)
        ex = logits64(cd, emb, t["W"], t["dts"], t["norms"], t["final"], t["lm"], Q6_K, list(toks))
        np.testing.assert_allclose(lb, ex, rtol=1e-4, atol=1e-4 * np.abs(ex).max())
        res[w] = lb
    assert np.abs(res[5] - res[0]).max() > 1e-2 * np.abs(res[0]).max()
    assert np.array_equal(res[13], res[0])


def test_reference_f32_logits_miss_the_plain_bar_on_a_test_model():
    """Why model-level logits are anchored on the float64 model: on the
    GGUF-order test model (Q3_K / Q2_K layers, an F16 down projection, Q6_K
    head; 19-token prompt, logits up to ±572) the reference's own f32 result —
    batched prefill and token-by-token decode alike — sits more than
    1e-3·max(1, |r|) from the exact logits on some entries (e.g. 3.2e-3 on a
    logit of -1.8). No other f32 evaluation order can be held to the plain
    element-wise bar against it there; the GPU tests of such models measure
    both against the float64 value instead (assert_close_logits' `exact`)."""
    from tests._model64 import logits64
    from tests._models import TINY, build_tiny, oracle_cfg
    from tests._util import F16, Q2_K, Q3_K, close_mask

    dts = [Q3_K, Q3_K, Q3_K, Q2_K, Q2_K, Q2_K, F16]
    c = dict(TINY, max_seq_len=64)
    m = build_tiny(seed=22, layer_dtype=dts, c=c)
    s, co = O.precompute_rope(64, c["head_dim"], c["rope_base"])
    toks = np.random.default_rng(1).integers(0, c["vocab_size"], 19)
    kv = np.zeros((2, 2, c["num_kv_heads"], 64, c["head_dim"]), np.float32)
    ref = O.forward_batch(oracle_cfg(c), m["emb"][toks], m["layers"], dts, m["norms"], m["final"], m["lm"], Q6_K, s,
                          co, kv)
    ex = logits64(c, m["emb"], m["layers"], dts, m["norms"], m["final"], m["lm"], Q6_K, list(toks))
    bad = ~close_mask(ref, ex)
    assert bad.sum() >= 2 and np.abs(ex).max() > 500
    assert (np.abs(ex[bad]) < 10).all()  # moderate logits, far below the row's maximum
    assert np.abs(ref - ex).max() <= 2.5e-5 * np.abs(ex).max()


def test_forward_batch_matches_sequential_decode_steps():
    """Batched prefill (forward_batch + attention_batch) of a 2-layer toy model
    with mixed dtypes equals the prompt fed through the pinned decode step one
    token at a time from an empty cache: same logits of the last token (up to
    f32 summation order) and the same K/V in slots 0..n-1. Also a prompt of
    one token, and the empty prompt is refused."""
    rng = np.random.default_rng(11)
    vocab, d, nh, nkv, hd, dff, ms = 96, 256, 4, 2, 64, 512, 24
    nl = 2
    cfg = O.LlamaCfg(vocab, d, nl, nh, nkv, hd, dff, ms, 10000.0, 1e-5)
    shapes = [(nh * hd, d), (nkv * hd, d), (nkv * hd, d), (d, nh * hd), (dff, d), (dff, d), (d, dff)]
    dts = [[Q4_K] * 7, [Q8_0, Q8_0, Q8_0, Q6_K, Q4_K, Q4_K, Q6_K]]
    W = []
    for l in range(nl):
        row = []
        for j, (n, k) in enumerate(shapes):
            be, _ = GEOM[dts[l][j]]
            row.append(synth_blocks(dts[l][j], n * k // be, 100 * l + j))
        W.append(row)
    norms = [[(1 + 0.02 * rng.standard_normal(d)).astype(np.float32) for _ in range(2)] for _ in range(nl)]
    final = (1 + 0.02 * rng.standard_normal(d)).astype(np.float32)
    lm = synth_blocks(Q6_K, vocab * d // 256, 99)
    s, c = O.precompute_rope(ms, hd, 10000.0)
    for n in (9, 1):
        X = rng.standard_normal((n, d)).astype(np.float32)
        kvb = np.zeros((nl, 2, nkv, ms, hd), np.float32)
        lb = O.forward_batch(cfg, X, W, dts, norms, final, lm, Q6_K, s, c, kvb)
        kvs = np.zeros_like(kvb)
        fill = 0
        for i in range(n):
            ls, fill = O.decode_step(cfg, X[i], i, W, dts, norms, final, lm, Q6_K, s, c, kvs, fill)
        assert fill == n
        np.testing.assert_allclose(lb, ls, rtol=1e-4, atol=1e-4 * np.abs(ls).max())
        np.testing.assert_allclose(kvb[:, :, :, :n], kvs[:, :, :, :n], rtol=1e-4, atol=1e-4)
        assert not kvb[:, :, :, n:].any()
    with pytest.raises(RuntimeError):
        O.forward_batch(cfg, np.zeros((0, d), np.float32), W, dts, norms, final, lm, Q6_K, s, c, kvb)


# ── frozen oracle vectors ────────────────────────────────────────────────

def test_golden_fixture():
    """tests/golden/oracle_vectors.npz (tests/golden/make_golden.py): seeded
    inputs with the oracle outputs frozen when it was pinned."""
    g = np.load(os.path.join(HERE, "golden", "oracle_vectors.npz"))
    for dt, name in ((Q8_0, "q8_0"), (Q4_K, "q4_k"), (Q6_K, "q6_k")):
        raw = g[name + "_raw"]
        n, k = g[name + "_shape"]
        assert np.array_equal(O.dequant(dt, raw, n * k).view(np.uint32), g[name + "_deq"].view(np.uint32))
        out = O.reference_matmul(dt, g["a"][:k], raw, 1, n, k)
        assert np.array_equal(out.view(np.uint32), g[name + "_mm"].view(np.uint32))


# ── re-quantizer rounding, pinned by hand blocks (tests/requant_hand_cases.py) ──

def test_requantize_hand_blocks_round_half_away_with_f32_scale():
    from tests import requant_hand_cases as H

    for make in (H.q8_0_ties, H.q8_0_f32_scale):
        x, expect = make()
        H.check_bytes(O.requantize(Q8_0, x, 1, 32), expect, make.__name__)
    for make in (H.q4_k_ties, H.q4_k_f32_scale):
        x, expect = make()
        H.check_bytes(O.requantize(Q4_K, x, 1, 256), expect, make.__name__)
    for x, dbits, sc0, deq in H.q6_k_cases():
        b = O.requantize(Q6_K, x, 1, 256)
        assert int(b[208]) | (int(b[209]) << 8) == dbits
        assert int(b[192]) == sc0
        assert list(O.dequant(Q6_K, b, 256)[:len(deq)]) == deq
