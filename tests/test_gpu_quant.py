"""GPU parity of the quantized-matmul kernels against the CPU oracle.

Bars (north star): dequantized weights bit-exact; matmul outputs within
|g-r| <= 1e-3 or |g-r|/max(1,|r|) <= 1e-3 per element and per-row cosine
> 0.9999 against the reference's x86 path (AVX2 for Q4_K/Q6_K, the scalar
kernel for Q8_0 — see oracle/oracle.c on the AVX2 Q8_0 defect).
"""
import ctypes

import numpy as np
import pytest

import aether_amd as A
from oracle import oracle as O
from tests._util import (F16, F32, GEOM, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0, assert_close, assert_close_logits,
                         assert_close_rows, synth_blocks, weight)

pytestmark = pytest.mark.gpu
DTYPES = [Q8_0, Q4_K, Q5_K, Q6_K]           # the formats with a fused kernel (row-major [n][k] blocks)
DEQ_DTYPES = DTYPES + [Q2_K, Q3_K, F16, F32]


def dev(torch, arr):
    t = torch.from_numpy(np.ascontiguousarray(arr)).cuda()
    return t


def make_weight(torch, dtype, n, k, raw):
    w = ctypes.c_void_p()
    A.check(A.lib().aeth_weight_create(dtype, n, k, raw.ctypes.data, 0, None, ctypes.byref(w)), "weight_create")
    return w


def gemv(torch, w, x, n, m=1, flags=0, y0=None):
    L = A.lib()
    xd = dev(torch, x.astype(np.float32))
    yd = torch.zeros(m * n, dtype=torch.float32, device="cuda") if y0 is None else dev(torch, y0.astype(np.float32))
    A.check(L.aeth_qmatmul(w, xd.data_ptr(), m, yd.data_ptr(), flags, None), "qmatmul")
    torch.cuda.synchronize()
    return yd.cpu().numpy().reshape(m, n)


# ── dequant: bit-exact ────────────────────────────────────────────────────

@pytest.mark.parametrize("dtype", DEQ_DTYPES)
def test_dequant_bit_exact_random_bytes(gpu, dtype):
    """Fully random bytes: f16 scales hit subnormals, NaN and Inf patterns
    (the bits/65536 rule of decode_d, dequant.rs:161-168)."""
    torch = gpu
    be, bb = GEOM[dtype]
    nblk = 4096
    rng = np.random.default_rng(dtype)
    raw = rng.integers(0, 256, nblk * bb, dtype=np.uint8)
    if dtype == Q8_0:  # the plain-f16 path: keep finite scales so NaN != NaN does not matter
        rb = raw.reshape(nblk, bb)
        rb[:, 1] &= 0x7B
    if dtype == F16:
        raw.reshape(-1, 2)[:, 1] &= 0x7B
    if dtype == F32:
        raw.reshape(-1, 4)[:, 3] &= 0x7F
    n = nblk * be
    ref = O.dequant(dtype, raw, n)
    out = torch.full((n,), float("nan"), dtype=torch.float32, device="cuda")
    rd = dev(torch, raw)
    A.check(A.lib().aeth_dequant(dtype, rd.data_ptr(), n, out.data_ptr(), None), "dequant")
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("dtype", DEQ_DTYPES)
def test_dequant_bit_exact_benchmark_blocks(gpu, dtype):
    torch = gpu
    be, bb = GEOM[dtype]
    nblk = 20000
    raw = synth_blocks(dtype, nblk, 7)
    n = nblk * be
    ref = O.dequant(dtype, raw, n)
    out = torch.empty(n, dtype=torch.float32, device="cuda")
    rd = dev(torch, raw)
    A.check(A.lib().aeth_dequant(dtype, rd.data_ptr(), n, out.data_ptr(), None), "dequant")
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("dtype", DTYPES)
def test_weight_relayout_round_trip(gpu, dtype):
    """Planar device layout reproduces the GGUF bytes exactly."""
    n, k = 97, 512
    raw = weight(dtype, n, k, 3)
    w = make_weight(gpu, dtype, n, k, raw)
    back = np.zeros_like(raw)
    A.check(A.lib().aeth_weight_export_raw(w, back.ctypes.data, 0, None), "export")
    assert A.lib().aeth_weight_bytes(w) == raw.size
    A.lib().aeth_weight_free(w)
    assert np.array_equal(back, raw)


# ── GEMV / GEMM parity ────────────────────────────────────────────────────

SHAPES = [(1, 64, 256), (1, 300, 512), (1, 1000, 4096), (1, 333, 14336), (3, 8, 256), (4, 129, 1024),
          (1, 16, 768), (2, 48, 2048), (1, 5000, 8192)]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m,n,k", SHAPES)
def test_matmul_parity(gpu, dtype, m, n, k):
    rng = np.random.default_rng(m * 1000 + n + k)
    raw = weight(dtype, n, k, n + k)
    x = rng.standard_normal(m * k).astype(np.float32)
    w = make_weight(gpu, dtype, n, k, raw)
    got = gemv(gpu, w, x, n, m)
    A.lib().aeth_weight_free(w)
    ref = O.reference_matmul(dtype, x, raw, m, n, k)
    assert_close(got, ref, what="%d m=%d n=%d k=%d" % (dtype, m, n, k))


# Q8_0 rows hold ceil(k/32) blocks (q8_0.rs:16); the last block's quants past k
# are ignored. k = 200 pads the device layout with a zero block (groups of 4),
# k = 100 / 1000 are not multiples of 8 (element-wise activation loads).
@pytest.mark.parametrize("m,n,k", [(1, 70, 200), (1, 45, 100), (2, 33, 1000), (1, 17, 32), (3, 40, 4128)])
def test_matmul_parity_q8_0_ragged_k(gpu, m, n, k):
    rng = np.random.default_rng(n * 7 + k)
    raw = weight(Q8_0, n, k, n + 3 * k)
    x = rng.standard_normal(m * k).astype(np.float32)
    w = make_weight(gpu, Q8_0, n, k, raw)
    back = np.zeros_like(raw)
    A.check(A.lib().aeth_weight_export_raw(w, back.ctypes.data, 0, None), "export")
    assert np.array_equal(back, raw)
    got = gemv(gpu, w, x, n, m)
    A.lib().aeth_weight_free(w)
    ref = O.reference_matmul(Q8_0, x, raw, m, n, k)
    assert_close(got, ref, what="q8_0 m=%d n=%d k=%d" % (m, n, k))


@pytest.mark.parametrize("dtype", DTYPES)
def test_matmul_nonfinite_activation_gives_nan_rows(gpu, dtype):
    """A NaN activation makes every output NaN, as NaN·w does in every row of the
    reference's sums (an infinity also yields NaN rows here, see DESIGN)."""
    n, k = 40, 512
    raw = weight(dtype, n, k, 5)
    x = np.random.default_rng(1).standard_normal(k).astype(np.float32)
    x[300] = np.nan
    w = make_weight(gpu, dtype, n, k, raw)
    got = gemv(gpu, w, x, n, 1)
    A.lib().aeth_weight_free(w)
    ref = O.reference_matmul(dtype, x, raw, 1, n, k)
    assert np.isnan(ref).all() and np.isnan(got).all()


@pytest.mark.parametrize("dtype", [Q4_K, Q5_K, Q6_K])
def test_matmul_reference_generators(gpu, dtype):
    """The reference's own test inputs (src/quant/matmul/tests.rs:3-17,
    :386-508): a[i] = ((i*17)%100)/50 - 1, b[i] = (i*31)%256 — f16 scales hit
    NaN/Inf patterns, so outputs reach ~1e7. m = 20 takes the Q4_K and Q6_K GEMMs."""
    for m in (1, 3, 20):
        k, n = 256, 8
        bb = GEOM[dtype][1]
        b = ((np.arange(n * (k // 256) * bb) * 31) % 256).astype(np.uint8)
        a = (((np.arange(m * k) * 17) % 100) / 50.0 - 1.0).astype(np.float32)
        w = make_weight(gpu, dtype, n, k, b)
        got = gemv(gpu, w, a, n, m)
        A.lib().aeth_weight_free(w)
        assert_close(got, O.avx2_matmul(dtype, a, b, m, n, k), what="ref generators m=%d" % m)


def test_matmul_accumulate_epilogue(gpu):
    """c += A·Wᵀ (the fused residual add of runner.rs:1609-1611)."""
    n, k = 256, 4096
    rng = np.random.default_rng(11)
    raw = weight(Q4_K, n, k, 5)
    x = rng.standard_normal(k).astype(np.float32)
    y0 = rng.standard_normal(n).astype(np.float32)
    w = make_weight(gpu, Q4_K, n, k, raw)
    got = gemv(gpu, w, x, n, 1, A.MM_ACCUMULATE, y0)
    A.lib().aeth_weight_free(w)
    ref = O.reference_matmul(Q4_K, x, raw, 1, n, k)[0]
    assert_close(got[0], y0 + ref)


@pytest.mark.parametrize("dtype,n,k", [(Q8_0, 4096, 4096), (Q4_K, 14336, 4096), (Q6_K, 128256, 4096),
                                       (Q5_K, 14336, 4096)])
def test_benchmark_config_parity(gpu, dtype, n, k):
    """BASELINE configs 1-3 at full size, weights from the device generator
    copied back so oracle and GPU see identical bytes."""
    torch = gpu
    L = A.lib()
    be, bb = GEOM[dtype]
    nb = k // be
    raw_d = torch.empty(n * nb * bb, dtype=torch.uint8, device="cuda")
    A.check(L.aeth_fill_synthetic_raw(dtype, 0xAE7E40 + dtype, raw_d.data_ptr(), n * nb, None), "fill")
    xd = torch.empty(k, dtype=torch.float32, device="cuda")
    A.check(L.aeth_fill_normal_f32(0x5EED + dtype, xd.data_ptr(), k, 0.0, 1.0, None), "fill x")
    w = ctypes.c_void_p()
    A.check(L.aeth_weight_create(dtype, n, k, raw_d.data_ptr(), 1, None, ctypes.byref(w)), "create")
    yd = torch.empty(n, dtype=torch.float32, device="cuda")
    A.check(L.aeth_qmatmul(w, xd.data_ptr(), 1, yd.data_ptr(), 0, None), "qmatmul")
    torch.cuda.synchronize()
    L.aeth_weight_free(w)
    raw = raw_d.cpu().numpy()
    x = xd.cpu().numpy()
    ref = O.reference_matmul(dtype, x, raw, 1, n, k)
    assert_close(yd.cpu().numpy(), ref, what="config dtype %d" % dtype)


@pytest.mark.parametrize("dtype,n,k", [(Q4_K, 50000, 4096), (Q8_0, 50000, 1024), (Q6_K, 33000, 512),
                                       (Q4_K, 20000, 4096), (Q5_K, 28700, 2048), (Q8_0, 30000, 512)])
def test_gemv_tall_ragged_parity(gpu, dtype, n, k):
    """Tall matrices take the refilling ring of tiles (4 to 8 tiles per CU: one
    workgroup per CU, 5 to 8 tiles each); these row counts leave the last
    workgroup fewer tiles than the others (and fewer than the ring holds), so
    its surplus loads and the past-the-end refills are exercised."""
    torch = gpu
    L = A.lib()
    be, bb = GEOM[dtype]
    nb = k // be
    raw_d = torch.empty(n * nb * bb, dtype=torch.uint8, device="cuda")
    A.check(L.aeth_fill_synthetic_raw(dtype, 0x7A11 + dtype, raw_d.data_ptr(), n * nb, None), "fill")
    xd = torch.empty(k, dtype=torch.float32, device="cuda")
    A.check(L.aeth_fill_normal_f32(0x5EED + n, xd.data_ptr(), k, 0.0, 1.0, None), "fill x")
    w = ctypes.c_void_p()
    A.check(L.aeth_weight_create(dtype, n, k, raw_d.data_ptr(), 1, None, ctypes.byref(w)), "create")
    yd = torch.empty(n, dtype=torch.float32, device="cuda")
    A.check(L.aeth_qmatmul(w, xd.data_ptr(), 1, yd.data_ptr(), 0, None), "qmatmul")
    torch.cuda.synchronize()
    L.aeth_weight_free(w)
    ref = O.reference_matmul(dtype, xd.cpu().numpy(), raw_d.cpu().numpy(), 1, n, k)
    assert_close(yd.cpu().numpy(), ref, what="tall dtype %d n=%d" % (dtype, n))


# ── host-slice boundary: quantized_matmul_impl / QuantKernel registry ────

def test_quantized_matmul_impl_host_slices(gpu):
    L = A.lib()
    A.check(L.aeth_weight_cache_clear())
    n, k, m = 40, 512, 2
    rng = np.random.default_rng(5)
    for dtype in DTYPES:
        raw = weight(dtype, n, k, dtype)
        a = rng.standard_normal(m * k).astype(np.float32)
        c = np.full(m * n, np.nan, dtype=np.float32)
        A.check(L.aeth_quantized_matmul_impl(a.ctypes.data, m, raw.ctypes.data, raw.size, n, k, dtype,
                                             c.ctypes.data), "quantized_matmul_impl")
        assert_close(c.reshape(m, n), O.reference_matmul(dtype, a, raw, m, n, k))
        c2 = np.full(m * n, np.nan, dtype=np.float32)
        fn = {Q8_0: L.aeth_matmul_q8_0, Q4_K: L.aeth_matmul_q4_k, Q5_K: L.aeth_matmul_q5_k,
              Q6_K: L.aeth_matmul_q6_k}[dtype]
        A.check(fn(a.ctypes.data, raw.ctypes.data, raw.size, m, n, k, c2.ctypes.data), "matmul_q*")
        assert np.array_equal(c, c2)
    A.check(L.aeth_weight_cache_clear())


def test_registry_dispatch(gpu):
    """register_kernel / dispatch_matmul (registry.rs:33-63): duplicate
    registration is refused; dispatch reports whether a kernel ran."""
    L = A.lib()
    buf = ctypes.create_string_buffer(64)
    first = L.aeth_registered_kernel_name(Q4_K, buf, 64) == 0
    if first:
        A.check(L.aeth_register_hip_kernels(), "register")
    assert L.aeth_register_hip_kernels() == -5  # AETH_ESTATE: already registered
    assert L.aeth_registered_kernel_name(Q4_K, buf, 64) == 1 and b"Q4_K" in buf.value
    n, k = 16, 256
    raw = weight(Q4_K, n, k, 1)
    a = np.random.default_rng(1).standard_normal(k).astype(np.float32)
    c = np.zeros(n, dtype=np.float32)
    assert L.aeth_dispatch_matmul(a.ctypes.data, 1, raw.ctypes.data, raw.size, n, k, Q4_K, c.ctypes.data) == 1
    assert_close(c[None], O.reference_matmul(Q4_K, a, raw, 1, n, k))
    assert L.aeth_dispatch_matmul(a.ctypes.data, 1, raw.ctypes.data, raw.size, n, k, 2, c.ctypes.data) == 0  # Q4_0
    A.check(L.aeth_weight_cache_clear())


def test_bad_arguments_are_errors(gpu):
    L = A.lib()
    raw = weight(Q4_K, 4, 256, 1)
    a = np.zeros(256, dtype=np.float32)
    c = np.zeros(4, dtype=np.float32)
    # too few weight bytes for the shape
    assert L.aeth_quantized_matmul_impl(a.ctypes.data, 1, raw.ctypes.data, raw.size - 1, 4, 256, Q4_K,
                                        c.ctypes.data) == -1
    assert L.aeth_quantized_matmul_impl(a.ctypes.data, 1, raw.ctypes.data, raw.size, 4, 256, 2, c.ctypes.data) == -4
    assert "bytes" in A.last_error() or "dtype" in A.last_error()


def test_synthetic_generator_deterministic(gpu):
    torch = gpu
    L = A.lib()
    outs = []
    for _ in range(2):
        t = torch.empty(1000 * 144, dtype=torch.uint8, device="cuda")
        A.check(L.aeth_fill_synthetic_raw(Q4_K, 1234, t.data_ptr(), 1000, None))
        outs.append(t.cpu().numpy())
    assert np.array_equal(outs[0], outs[1])
    blk = outs[0].reshape(1000, 144)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float32).ravel()
    assert (d >= 0).all() and 0.004 < d.mean() < 0.012  # |N(0,1)|*0.01 has mean 0.008
    q = blk[:, 16:]
    assert abs(q.mean() - 127.5) < 2.0


# The Q4_K GEMM (m > 1): the K-split kernel with super-block counts that split
# unevenly over its 8 waves (3, 4, 10, 64, 80; fewer super-blocks than waves
# leaves waves idle); m and n off the 64 × 128 tile grid.
# Row magnitudes span 2^-12 .. 2^20 (the per-block fp16 exponent), with an
# all-zero row, and the accumulate epilogue is checked on top.
@pytest.mark.parametrize("m,n,k", [(70, 130, 768), (65, 300, 1024), (130, 40, 2560), (16, 16, 512), (45, 48, 16384),
                                   (34, 64, 20480), (37, 96, 8192)])
def test_gemm_q4k_tiles_exponents_accumulate(gpu, m, n, k):
    """Ragged tiles, per-row exponents (2^20, 2^-12, zero rows, a block past
    fp16 range) and accumulate, up to rows of 16384 and 20480 elements (the
    prep holds 1, 2, 4 or 8 steps of a row per wave, 20480 in two chunks); K
    split over 8, 10 and 4 workgroups for the last three shapes."""
    check_q4k_gemm(gpu, m, n, k)


def check_q4k_gemm(gpu, m, n, k):
    rng = np.random.default_rng(m * 31 + n * 7 + k)
    raw = weight(Q4_K, n, k, 3 * n + k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    scale = np.ones(m, dtype=np.float32)
    scale[m // 3] = 2.0 ** 20
    scale[m // 2] = 2.0 ** -12
    scale[(2 * m) // 3] = 0.0
    if m > 40:
        scale[33:40] = 2.0 ** 15  # a block with values past fp16 range next to ordinary rows
    x *= scale[:, None]
    w = make_weight(gpu, Q4_K, n, k, raw)
    y0 = rng.standard_normal((m, n)).astype(np.float32)
    got = gemv(gpu, w, x.ravel(), n, m)
    got_acc = gemv(gpu, w, x.ravel(), n, m, flags=A.MM_ACCUMULATE, y0=y0)
    A.lib().aeth_weight_free(w)
    ref = O.reference_matmul(Q4_K, x.ravel(), raw, m, n, k).reshape(m, n)
    # rows of magnitude 1 take the element-wise bar; the scaled rows a bar
    # relative to their own magnitude (an f32 sum's error scales with its terms)
    plain = scale == 1.0
    assert_close(got[plain], ref[plain], what="gemm m=%d n=%d k=%d" % (m, n, k))
    assert_close_rows(got, ref, what="gemm (scaled rows) m=%d n=%d k=%d" % (m, n, k))
    assert_close(got_acc[plain], (ref + y0)[plain], what="gemm accumulate m=%d n=%d k=%d" % (m, n, k))
    assert np.all(got[(2 * m) // 3] == 0.0)


# Small batches of Q4_K rows: the row-batched GEMV below 16 rows unless m · (weight
# bytes) reaches 150 MB from 5 rows, else the GEMM (aeth_q4k_gemm_rows; its K split over
# up to 8 workgroups at these m); both sides of each boundary, plain, accumulate and the
# dot-product mode (a14 activation blocks).
@pytest.mark.parametrize("m,n,k", [(2, 4096, 4096), (15, 4096, 4096), (16, 4096, 4096), (10, 6144, 4096),
                                   (11, 6144, 4096), (4, 14336, 4096), (5, 14336, 4096), (4, 4096, 14336),
                                   (5, 4096, 14336), (4, 28672, 4096), (5, 28672, 4096)])
def test_q4k_small_batches(gpu, m, n, k):
    rng = np.random.default_rng(m * 101 + n + k)
    raw = weight(Q4_K, n, k, 5 * n + m)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = make_weight(gpu, Q4_K, n, k, raw)
    y0 = rng.standard_normal((m, n)).astype(np.float32)
    got = gemv(gpu, w, x.ravel(), n, m)
    got_acc = gemv(gpu, w, x.ravel(), n, m, flags=A.MM_ACCUMULATE, y0=y0)
    got_q8 = gemv(gpu, w, x.ravel(), n, m, flags=A.MM_Q8_ACTIVATIONS)
    A.lib().aeth_weight_free(w)
    ref = O.reference_matmul(Q4_K, x.ravel(), raw, m, n, k).reshape(m, n)
    assert_close(got, ref, what="q4_k m=%d n=%d k=%d" % (m, n, k))
    assert_close(got_acc, ref + y0, what="q4_k accumulate m=%d n=%d k=%d" % (m, n, k))
    ref_q8 = O.dotprod_ref(Q4_K, O.quantize_activations_q8_0(x.ravel(), m, k), raw, m, n, k).reshape(m, n)
    assert_close(got_q8, ref_q8, what="q4_k dot-product mode m=%d n=%d k=%d" % (m, n, k))


# Small batches of Q8_0 rows (aeth_q80_gemm_rows): the row-batched GEMV until m · (weight bytes)
# reaches 380 MB for weights up to 32 MiB and 180 MB above (from 3 rows), else the GEMM; both sides
# of the switch at the measured crossovers, plain, accumulate and the dot-product mode.
@pytest.mark.parametrize("m,n,k", [(21, 4096, 4096), (22, 4096, 4096), (2, 4096, 14336), (3, 4096, 14336),
                                   (2, 14336, 4096), (3, 14336, 4096)])
def test_q80_small_batches(gpu, m, n, k):
    rng = np.random.default_rng(m * 103 + n + k)
    raw = weight(Q8_0, n, k, 7 * n + m)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = make_weight(gpu, Q8_0, n, k, raw)
    y0 = rng.standard_normal((m, n)).astype(np.float32)
    got = gemv(gpu, w, x.ravel(), n, m)
    got_acc = gemv(gpu, w, x.ravel(), n, m, flags=A.MM_ACCUMULATE, y0=y0)
    got_q8 = gemv(gpu, w, x.ravel(), n, m, flags=A.MM_Q8_ACTIVATIONS)
    A.lib().aeth_weight_free(w)
    ref = O.reference_matmul(Q8_0, x.ravel(), raw, m, n, k).reshape(m, n)
    assert_close(got, ref, what="q8_0 m=%d n=%d k=%d" % (m, n, k))
    assert_close(got_acc, ref + y0, what="q8_0 accumulate m=%d n=%d k=%d" % (m, n, k))
    ref_q8 = O.dotprod_ref(Q8_0, O.quantize_activations_q8_0(x.ravel(), m, k), raw, m, n, k).reshape(m, n)
    assert_close(got_q8, ref_q8, what="q8_0 dot-product mode m=%d n=%d k=%d" % (m, n, k))


def check_q5k_gemm(torch, m, n, k):
    """Q5_K product of m rows against the oracle (avx2::matmul_q5_k with m rows), as
    check_q4k_gemm: per-row exponents (2^20, 2^-12, a zero row, a block of 2^15 rows past
    fp16 range), plain, accumulate and the dot-product mode. The fifth bits are random, so
    quants reach 31 and rows of magnitude 1 are anchored on the float64 product of the same
    operands too (as check_q6k_gemm explains)."""
    rng = np.random.default_rng(m * 43 + n * 13 + k)
    raw = weight(Q5_K, n, k, 11 * n + k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    scale = np.ones(m, dtype=np.float32)
    scale[m // 3] = 2.0 ** 20
    scale[m // 2] = 2.0 ** -12
    scale[(2 * m) // 3] = 0.0
    if m > 40:
        scale[33:40] = 2.0 ** 15
    x *= scale[:, None]
    w = make_weight(torch, Q5_K, n, k, raw)
    y0 = rng.standard_normal((m, n)).astype(np.float32)
    got = gemv(torch, w, x.ravel(), n, m)
    got_acc = gemv(torch, w, x.ravel(), n, m, flags=A.MM_ACCUMULATE, y0=y0)
    got_q8 = gemv(torch, w, x.ravel(), n, m, flags=A.MM_Q8_ACTIVATIONS)
    A.lib().aeth_weight_free(w)
    ref = O.reference_matmul(Q5_K, x.ravel(), raw, m, n, k).reshape(m, n)
    plain = scale == 1.0
    w64 = O.dequant(Q5_K, raw, n * k).reshape(n, k).astype(np.float64)
    ex = x[plain].astype(np.float64) @ w64.T
    what = "q5_k m=%d n=%d k=%d" % (m, n, k)
    assert_close_logits(got[plain], ref[plain], floor=0.0, exact=ex, what=what)
    assert_close_rows(got, ref, what=what + " (scaled rows)")
    assert_close_logits(got_acc[plain], (ref + y0)[plain], floor=0.0, exact=ex + y0[plain], what=what + " accumulate")
    assert np.all(got[(2 * m) // 3] == 0.0)
    aq = O.quantize_activations_q8_0(x.ravel(), m, k)
    ref_q8 = O.dotprod_ref(Q5_K, aq, raw, m, n, k).reshape(m, n)
    ex_q8 = O.dequant(Q8_0, aq, m * k).reshape(m, k)[plain].astype(np.float64) @ w64.T
    assert_close_rows(got_q8, ref_q8, what=what + " dot-product mode")
    assert_close_logits(got_q8[plain], ref_q8[plain], floor=0.0, exact=ex_q8, what=what + " dot-product mode")


# The Q5_K GEMM (the K-split kernel's Q5_K form: planar Q5_K, whole super-blocks, from 16
# rows): super-block counts that split unevenly over its 8 waves, K split over workgroups
# where the tiles are fewer than the CUs (the last four shapes), m and n off the 64 × 128 grid.
@pytest.mark.parametrize("m,n,k", [(70, 130, 768), (65, 300, 1024), (130, 40, 2560), (16, 16, 512), (45, 48, 16384),
                                   (34, 64, 20480), (37, 96, 8192), (200, 100, 14336)])
def test_gemm_q5k_tiles_exponents_accumulate(gpu, m, n, k):
    check_q5k_gemm(gpu, m, n, k)


def test_gemm_q5k_without_fifth_bits_is_the_q4k_gemm(gpu):
    """A Q5_K weight whose qh bytes are all zero is the Q4_K weight with the same d, dmin,
    scales and qs (q5_k.rs:49-56 adds 16 per set bit): the Q5_K GEMM's result equals the Q4_K
    GEMM's bit for bit (same kernel frame, same K split, every operand exact), and setting
    every fifth bit moves each output by 16·Σ d·sc·x, the product of a weight whose q are all
    16 and whose mins are zero (anchored on float64)."""
    m, n, k = 70, 200, 2048
    rng = np.random.default_rng(5)
    q4 = weight(Q4_K, n, k, 77).reshape(-1, 144)
    q5 = np.zeros((q4.shape[0], 176), np.uint8)
    q5[:, 0:16] = q4[:, 0:16]
    q5[:, 48:176] = q4[:, 16:144]
    x = rng.standard_normal((m, k)).astype(np.float32)
    outs = []
    for dt, raw in ((Q4_K, q4.reshape(-1)), (Q5_K, q5.reshape(-1))):
        w = make_weight(gpu, dt, n, k, raw)
        outs.append(gemv(gpu, w, x.ravel(), n, m))
        A.lib().aeth_weight_free(w)
    assert np.array_equal(outs[0], outs[1])
    q5[:, 16:48] = 0xFF
    w = make_weight(gpu, Q5_K, n, k, q5.reshape(-1))
    got = gemv(gpu, w, x.ravel(), n, m)
    A.lib().aeth_weight_free(w)
    w64 = O.dequant(Q5_K, q5.reshape(-1), n * k).reshape(n, k).astype(np.float64)
    w64_4 = O.dequant(Q4_K, q4.reshape(-1), n * k).reshape(n, k).astype(np.float64)
    ex = x.astype(np.float64) @ w64.T
    assert np.abs(w64 - w64_4).max() > 0  # the bits matter
    ref = O.reference_matmul(Q5_K, x.ravel(), q5.reshape(-1), m, n, k).reshape(m, n)
    assert_close_logits(got, ref, floor=0.0, exact=ex, what="q5_k, every fifth bit set")


# Small batches of Q5_K rows: the row-batched GEMV below 16 rows unless m · (weight bytes)
# reaches 150 MB from 5 rows, else the GEMM (aeth_q5k_gemm_rows); both sides of each boundary.
@pytest.mark.parametrize("m,n,k", [(15, 4096, 4096), (16, 4096, 4096), (4, 14336, 4096), (5, 14336, 4096),
                                   (4, 4096, 14336), (5, 4096, 14336)])
def test_q5k_small_batches(gpu, m, n, k):
    rng = np.random.default_rng(m * 103 + n + k)
    raw = weight(Q5_K, n, k, 7 * n + m)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = make_weight(gpu, Q5_K, n, k, raw)
    y0 = rng.standard_normal((m, n)).astype(np.float32)
    got = gemv(gpu, w, x.ravel(), n, m)
    got_acc = gemv(gpu, w, x.ravel(), n, m, flags=A.MM_ACCUMULATE, y0=y0)
    got_q8 = gemv(gpu, w, x.ravel(), n, m, flags=A.MM_Q8_ACTIVATIONS)
    A.lib().aeth_weight_free(w)
    ref = O.reference_matmul(Q5_K, x.ravel(), raw, m, n, k).reshape(m, n)
    w64 = O.dequant(Q5_K, raw, n * k).reshape(n, k).astype(np.float64)
    ex = x.astype(np.float64) @ w64.T
    what = "q5_k m=%d n=%d k=%d" % (m, n, k)
    assert_close_logits(got, ref, floor=0.0, exact=ex, what=what)
    assert_close_logits(got_acc, ref + y0, floor=0.0, exact=ex + y0, what=what + " accumulate")
    aq = O.quantize_activations_q8_0(x.ravel(), m, k)
    ref_q8 = O.dotprod_ref(Q5_K, aq, raw, m, n, k).reshape(m, n)
    ex_q8 = O.dequant(Q8_0, aq, m * k).reshape(m, k).astype(np.float64) @ w64.T
    assert_close_logits(got_q8, ref_q8, floor=0.0, exact=ex_q8, what=what + " dot-product mode")


def check_q6k_gemm(torch, m, n, k):
    """Q6_K product of m rows against the oracle: per-row exponents (2^20, 2^-12, a zero
    row, a block of 2^15 rows past fp16 range when m > 40), plain, accumulate and the
    dot-product mode; the weights carry the scale extremes -128 and 127 (16·hi + lo with
    hi = -8 and 7) and super-blocks whose d is zero.

    With those scales and k up to 20480 a row's outputs reach several thousand, and the
    reference's own f32 sums then sit up to 7e-3 from the float64 product of the same
    operands (k = 16384: median 2.8e-4, max 6.9e-3), past the element-wise bar on small
    entries. Rows of magnitude 1 are therefore also anchored on that float64 product: an
    element passes the element-wise bar against the reference, or sits within twice the
    reference's largest distance from the float64 product on its row (assert_close_logits
    with exact, no floor)."""
    rng = np.random.default_rng(m * 37 + n * 11 + k)
    raw = weight(Q6_K, n, k, 9 * n + k).reshape(-1, 210)
    nblk = raw.shape[0]
    pick = rng.integers(0, nblk, max(2, nblk // 16))
    raw[pick[0::2], 192:208] = np.int8(-128).view(np.uint8)
    raw[pick[1::2], 192:208] = np.int8(127).view(np.uint8)
    raw[rng.integers(0, nblk, max(1, nblk // 20)), 208:210] = 0
    raw = raw.reshape(-1)
    x = rng.standard_normal((m, k)).astype(np.float32)
    scale = np.ones(m, dtype=np.float32)
    scale[m // 3] = 2.0 ** 20
    scale[m // 2] = 2.0 ** -12
    scale[(2 * m) // 3] = 0.0
    if m > 40:
        scale[33:40] = 2.0 ** 15
    x *= scale[:, None]
    w = make_weight(torch, Q6_K, n, k, raw)
    y0 = rng.standard_normal((m, n)).astype(np.float32)
    got = gemv(torch, w, x.ravel(), n, m)
    got_acc = gemv(torch, w, x.ravel(), n, m, flags=A.MM_ACCUMULATE, y0=y0)
    got_q8 = gemv(torch, w, x.ravel(), n, m, flags=A.MM_Q8_ACTIVATIONS)
    A.lib().aeth_weight_free(w)
    ref = O.reference_matmul(Q6_K, x.ravel(), raw, m, n, k).reshape(m, n)
    plain = scale == 1.0
    w64 = O.dequant(Q6_K, raw, n * k).reshape(n, k).astype(np.float64)
    ex = x[plain].astype(np.float64) @ w64.T
    what = "q6_k m=%d n=%d k=%d" % (m, n, k)
    assert_close_logits(got[plain], ref[plain], floor=0.0, exact=ex, what=what)
    assert_close_rows(got, ref, what=what + " (scaled rows)")
    assert_close_logits(got_acc[plain], (ref + y0)[plain], floor=0.0, exact=ex + y0[plain], what=what + " accumulate")
    assert np.all(got[(2 * m) // 3] == 0.0)
    aq = O.quantize_activations_q8_0(x.ravel(), m, k)
    ref_q8 = O.dotprod_ref(Q6_K, aq, raw, m, n, k).reshape(m, n)
    ex_q8 = O.dequant(Q8_0, aq, m * k).reshape(m, k)[plain].astype(np.float64) @ w64.T
    assert_close_rows(got_q8, ref_q8, what=what + " dot-product mode")
    assert_close_logits(got_q8[plain], ref_q8[plain], floor=0.0, exact=ex_q8, what=what + " dot-product mode")


# The Q6_K GEMM (planar Q6_K, whole super-blocks, m · weight bytes >= 200 MB): super-block
# counts that split unevenly over its 8 waves (2, 3, 4, 8, 10, 16, 24, 32, 56, 64, 80), K
# also split over 2, 3, 4, 7, 8 and 10 workgroups per tile where the tiles are fewer than
# the CUs, m and n off the 64 × 128 tile grid.
@pytest.mark.parametrize("m,n,k", [(70, 4600, 768), (16, 30000, 512), (65, 3700, 1024), (130, 1900, 2560),
                                   (45, 2200, 16384), (37, 1100, 8192), (200, 100, 14336), (34, 400, 20480),
                                   (17, 7100, 2048), (30, 2000, 4096), (25, 1700, 6144)])
def test_gemm_q6k_tiles_exponents_accumulate(gpu, m, n, k):
    check_q6k_gemm(gpu, m, n, k)


def check_q80_gemm(torch, m, n, k):
    """Q8_0 product of m rows against the oracle, as check_q6k_gemm: per-row exponents, plain,
    accumulate and the dot-product mode; the weights carry quants −128 and 127 and blocks whose
    d is zero. Rows of magnitude 1 are anchored on the float64 product of the same operands."""
    rng = np.random.default_rng(m * 41 + n * 13 + k)
    raw = weight(Q8_0, n, k, 11 * n + k).reshape(-1, 34)
    nblk = raw.shape[0]
    pick = rng.integers(0, nblk, max(2, nblk // 16))
    raw[pick[0::2], 2:34] = np.int8(-128).view(np.uint8)
    raw[pick[1::2], 2:34] = np.int8(127).view(np.uint8)
    raw[rng.integers(0, nblk, max(1, nblk // 20)), 0:2] = 0
    raw = raw.reshape(-1)
    x = rng.standard_normal((m, k)).astype(np.float32)
    scale = np.ones(m, dtype=np.float32)
    scale[m // 3] = 2.0 ** 20
    scale[m // 2] = 2.0 ** -12
    scale[(2 * m) // 3] = 0.0
    if m > 40:
        scale[33:40] = 2.0 ** 15
    x *= scale[:, None]
    w = make_weight(torch, Q8_0, n, k, raw)
    y0 = rng.standard_normal((m, n)).astype(np.float32)
    got = gemv(torch, w, x.ravel(), n, m)
    got_acc = gemv(torch, w, x.ravel(), n, m, flags=A.MM_ACCUMULATE, y0=y0)
    got_q8 = gemv(torch, w, x.ravel(), n, m, flags=A.MM_Q8_ACTIVATIONS)
    A.lib().aeth_weight_free(w)
    ref = O.reference_matmul(Q8_0, x.ravel(), raw, m, n, k).reshape(m, n)
    plain = scale == 1.0
    w64 = O.dequant(Q8_0, raw, n * k).reshape(n, k).astype(np.float64)
    ex = x[plain].astype(np.float64) @ w64.T
    what = "q8_0 m=%d n=%d k=%d" % (m, n, k)
    assert_close_logits(got[plain], ref[plain], floor=0.0, exact=ex, what=what)
    assert_close_rows(got, ref, what=what + " (scaled rows)")
    assert_close_logits(got_acc[plain], (ref + y0)[plain], floor=0.0, exact=ex + y0[plain], what=what + " accumulate")
    assert np.all(got[(2 * m) // 3] == 0.0)
    aq = O.quantize_activations_q8_0(x.ravel(), m, k)
    ref_q8 = O.dotprod_ref(Q8_0, aq, raw, m, n, k).reshape(m, n)
    ex_q8 = O.dequant(Q8_0, aq, m * k).reshape(m, k)[plain].astype(np.float64) @ w64.T
    assert_close_rows(got_q8, ref_q8, what=what + " dot-product mode")
    assert_close_logits(got_q8[plain], ref_q8[plain], floor=0.0, exact=ex_q8, what=what + " dot-product mode")


# The Q8_0 GEMM (planar Q8_0, k a multiple of 32, from 16 rows): block counts that split
# unevenly over the 8 waves or leave waves idle (4, 25 — not whole groups of 4 — 40, 64, 128,
# 448), K split over 2 and 7 workgroups, m and n off the tile grid.
@pytest.mark.parametrize("m,n,k", [(70, 130, 128), (16, 16, 800), (65, 300, 1280), (130, 40, 4096),
                                   (45, 48, 14336), (200, 64, 4096), (17, 700, 2048), (512, 256, 4096)])
def test_gemm_q80_tiles_exponents_accumulate(gpu, m, n, k):
    check_q80_gemm(gpu, m, n, k)


# Q4_K / Q5_K / Q6_K scales with the f16 exponent 31 (decode_d's rule, dequant.rs:161-168: such
# bits are read as bits / 65536): a weight holding a few of them takes the GEMV instance with the
# rule, the same weight without them the one with a plain f16 conversion; both against the oracle.
@pytest.mark.parametrize("dtype", [Q4_K, Q5_K, Q6_K])
@pytest.mark.parametrize("special", [False, True])
def test_gemv_exponent31_scales(gpu, dtype, special):
    n, k = 300, 1024
    raw = weight(dtype, n, k, 91).reshape(n * k // 256, -1)
    if special:
        pats = np.array([0x7C00, 0xFC00, 0x7E01, 0x7FFF], np.uint16).view(np.uint8).reshape(4, 2)
        rows = [3, 77, 150, 299]
        for i, r in enumerate(rows):
            blk = r * (k // 256) + i % (k // 256)
            if dtype == Q6_K:
                raw[blk, 208:210] = pats[i]
            else:
                raw[blk, 2 * (i & 1):2 * (i & 1) + 2] = pats[i]  # d, then dmin
    raw = raw.reshape(-1)
    x = np.random.default_rng(5).standard_normal(k).astype(np.float32)
    w = make_weight(gpu, dtype, n, k, raw)
    got = gemv(gpu, w, x, n)
    A.lib().aeth_weight_free(w)
    ref = O.reference_matmul(dtype, x, raw, 1, n, k)
    assert np.isfinite(ref).all()
    assert_close(got, ref, what="dtype %d special scales %s" % (dtype, special))


# Q8_0 block scales that are NaN or infinite (q8_0.rs decodes d as a plain f16 and adds d·Σ per
# block): +Inf, −Inf and NaN scales in several blocks of some rows, at batch sizes that would
# otherwise take the Q8_0 GEMM (20, 64 rows) or the dequantized DGEMM (150 rows), and one row:
# every element equals the scalar reference's class (NaN, ±Inf) and the finite rows stay
# within the bar.
@pytest.mark.parametrize("m", [1, 20, 64, 150])
def test_q80_nonfinite_block_scales(gpu, m):
    n, k = 96, 1024
    rng = np.random.default_rng(m + 5)
    raw = weight(Q8_0, n, k, 77).reshape(n, k // 32, 34)
    h = lambda bits: np.array([bits], np.uint16).view(np.uint8)
    raw[3, 5, 0:2] = h(0x7C00)                                  # +Inf
    raw[3, 20, 0:2] = h(0x7C00)                                 # two in one row (the rescale's Inf·0 case)
    raw[7, 1, 0:2] = h(0xFC00)                                  # −Inf
    raw[7, 30, 0:2] = h(0x7C00)                                 # mixed signs
    raw[11, 9, 0:2] = h(0x7E00)                                 # NaN
    raw[40, 2, 0:2], raw[40, 3, 0:2], raw[40, 31, 0:2] = h(0x7C00), h(0x7C00), h(0xFC00)
    raw = raw.reshape(-1)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = make_weight(gpu, Q8_0, n, k, raw)
    got = gemv(gpu, w, x.ravel(), n, m)
    A.lib().aeth_weight_free(w)
    ref = O.reference_matmul(Q8_0, x.ravel(), raw, m, n, k).reshape(m, n)
    assert np.array_equal(np.isnan(got), np.isnan(ref)), "NaN pattern m=%d" % m
    assert np.array_equal(np.isposinf(got), np.isposinf(ref)) and np.array_equal(np.isneginf(got), np.isneginf(ref))
    assert np.isnan(ref).any() and np.isinf(ref).any()  # the cases occur
    fin = np.isfinite(ref)
    assert_close(got[fin], ref[fin], what="finite entries m=%d" % m)


# Small batches of Q6_K rows: the row-batched GEMV until m · (weight bytes) reaches 200 MB,
# then the GEMM (aeth_q6k_gemm_rows); both sides of the boundary at three weight sizes, plain,
# accumulate and the dot-product mode.
@pytest.mark.parametrize("m,n,k", [(4, 4096, 14336), (5, 4096, 14336), (14, 4096, 4096), (15, 4096, 4096),
                                   (58, 1024, 4096), (59, 1024, 4096)])
def test_q6k_small_batches(gpu, m, n, k):
    rng = np.random.default_rng(m * 103 + n + k)
    raw = weight(Q6_K, n, k, 3 * n + m)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = make_weight(gpu, Q6_K, n, k, raw)
    y0 = rng.standard_normal((m, n)).astype(np.float32)
    got = gemv(gpu, w, x.ravel(), n, m)
    got_acc = gemv(gpu, w, x.ravel(), n, m, flags=A.MM_ACCUMULATE, y0=y0)
    got_q8 = gemv(gpu, w, x.ravel(), n, m, flags=A.MM_Q8_ACTIVATIONS)
    A.lib().aeth_weight_free(w)
    ref = O.reference_matmul(Q6_K, x.ravel(), raw, m, n, k).reshape(m, n)
    assert_close(got, ref, what="q6_k m=%d n=%d k=%d" % (m, n, k))
    assert_close(got_acc, ref + y0, what="q6_k accumulate m=%d n=%d k=%d" % (m, n, k))
    ref_q8 = O.dotprod_ref(Q6_K, O.quantize_activations_q8_0(x.ravel(), m, k), raw, m, n, k).reshape(m, n)
    assert_close(got_q8, ref_q8, what="q6_k dot-product mode m=%d n=%d k=%d" % (m, n, k))


@pytest.mark.parametrize("n", [4096, 14336])
def test_prefill_gemm_config_parity(gpu, n):
    """BASELINE config 4 (M = 512, K = 4096, Q4_K weights as config 2): the
    full GEMM on the GPU; the oracle (AVX2 path, m = 512) is evaluated on 96
    sampled weight rows (output columns)."""
    torch = gpu
    L = A.lib()
    m, k = 512, 4096
    nb = k // 256
    raw_d = torch.empty(n * nb * 144, dtype=torch.uint8, device="cuda")
    A.check(L.aeth_fill_synthetic_raw(Q4_K, 0xAE7E43 + n, raw_d.data_ptr(), n * nb, None), "fill")
    ad = torch.empty(m * k, dtype=torch.float32, device="cuda")
    A.check(L.aeth_fill_normal_f32(0x77 + n, ad.data_ptr(), m * k, 0.0, 1.0, None), "fill a")
    w = ctypes.c_void_p()
    A.check(L.aeth_weight_create(Q4_K, n, k, raw_d.data_ptr(), 1, None, ctypes.byref(w)), "create")
    cd = torch.empty(m * n, dtype=torch.float32, device="cuda")
    A.check(L.aeth_qmatmul(w, ad.data_ptr(), m, cd.data_ptr(), 0, None), "gemm")
    torch.cuda.synchronize()
    L.aeth_weight_free(w)
    got = cd.cpu().numpy().reshape(m, n)
    raw = raw_d.cpu().numpy().reshape(n, nb * 144)
    cols = np.sort(np.random.default_rng(n).choice(n, 96, replace=False))
    cols[0], cols[-1] = 0, n - 1
    ref = O.reference_matmul(Q4_K, ad.cpu().numpy(), raw[cols].reshape(-1), m, len(cols), k)
    assert_close(got[:, cols], ref, what="prefill GEMM n=%d" % n)


def g2_tile(i, gm, gn):
    """The K-split GEMM's workgroup → 64 × 128 tile order (g2_tile, aeth_gemm_common.hpp):
    tile ids dealt round-robin over the 8 XCDs when their count is a multiple of 8, then
    column-major within groups of 4 row-tiles."""
    T = gm * gn
    if T % 8 == 0:
        i = (i & 7) * (T >> 3) + (i >> 3)
    grp = i // (4 * gn)
    rows = min(4, gm - 4 * grp)
    j = i - grp * 4 * gn
    return 4 * grp + j % rows, j // rows


# More 64 × 128 tiles than CUs with the last round at most half full: the GEMM splits the K
# range of those last tiles over the idle CUs and a second kernel sums them. n is chosen from the
# device's CU count so that the tiles are one round plus `tail` (19 split in 2, 69 in 3, 4 in 8,
# 119 in 2 at 256 CUs), its last column tile `nrag` columns short. Up to 8 of the tail tiles (the
# first and last among them) and three whole tiles are checked against the oracle, for each of the
# four GEMMs (Q4_K, Q5_K, Q6_K, Q8_0), plain and accumulate; Q6_K and Q8_0 with the float64 anchor
# of their own GEMM tests (check_q6k_gemm), since the reference's f32 sums of their rows drift past
# the element-wise bar.
@pytest.mark.parametrize("dtype,m,k,tail,nrag", [(Q4_K, 300, 4096, 19, 40), (Q4_K, 260, 16384, 69, 0),
                                                 (Q4_K, 100, 16384, 4, 40), (Q5_K, 130, 8192, 119, 0),
                                                 (Q6_K, 260, 16384, 69, 0), (Q6_K, 300, 4096, 19, 40),
                                                 (Q8_0, 300, 4096, 19, 40), (Q8_0, 100, 16384, 4, 40)])
def test_gemm_tail_round_split(gpu, dtype, m, k, tail, nrag):
    torch = gpu
    L = A.lib()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    gm = -(-m // 64)
    gn = -(-(cus + tail) // gm)
    n = 128 * gn - nrag
    be, bb = GEOM[dtype]
    nb = k // be
    raw_d = torch.empty(n * nb * bb, dtype=torch.uint8, device="cuda")
    A.check(L.aeth_fill_synthetic_raw(dtype, 0x7A11 + n, raw_d.data_ptr(), n * nb, None), "fill")
    rng = np.random.default_rng(m + n)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y0 = rng.standard_normal((m, n)).astype(np.float32)
    w = ctypes.c_void_p()
    A.check(L.aeth_weight_create(dtype, n, k, raw_d.data_ptr(), 1, None, ctypes.byref(w)), "create")
    try:
        got = gemv(torch, w, x.ravel(), n, m)
        got_acc = gemv(torch, w, x.ravel(), n, m, flags=A.MM_ACCUMULATE, y0=y0)
    finally:
        L.aeth_weight_free(w)
    raw = raw_d.cpu().numpy().reshape(n, nb * bb)
    T = gm * gn
    tail = T % cus
    assert T > cus and 0 < 2 * tail <= cus, "shape %d x %d does not leave a short last round on %d CUs" % (m, n, cus)
    print("tiles %d, tail %d split %d ways" % (T, tail, min(cus // tail, k // 2048)), flush=True)
    tails = sorted(set(np.linspace(T - tail, T - 1, min(tail, 8)).round().astype(int).tolist()))
    for t in tails + [0, T // 2, T - tail - 1]:
        tm, tn = g2_tile(t, gm, gn)
        r0, r1, c0, c1 = 64 * tm, min(m, 64 * tm + 64), 128 * tn, min(n, 128 * tn + 128)
        ref = O.reference_matmul(dtype, x[r0:r1].ravel(), raw[c0:c1].ravel(), r1 - r0, c1 - c0, k).reshape(r1 - r0, -1)
        what = "tile %d (%d, %d) of %d x %d x %d" % (t, tm, tn, m, n, k)
        if dtype in (Q6_K, Q8_0):  # rows in the hundreds: also anchored on the float64 product (check_q6k_gemm)
            w64 = O.dequant(dtype, raw[c0:c1].ravel(), (c1 - c0) * k).reshape(c1 - c0, k).astype(np.float64)
            ex = x[r0:r1].astype(np.float64) @ w64.T
            assert_close_logits(got[r0:r1, c0:c1], ref, floor=0.0, exact=ex, what=what)
            assert_close_logits(got_acc[r0:r1, c0:c1], ref + y0[r0:r1, c0:c1], floor=0.0, exact=ex + y0[r0:r1, c0:c1],
                                what=what + " accumulate")
        else:
            assert_close(got[r0:r1, c0:c1], ref, what=what)
            assert_close(got_acc[r0:r1, c0:c1], ref + y0[r0:r1, c0:c1], what=what + " accumulate")


# ── F32 / F16 / Q2_K / Q3_K: GGUF-order and row kernels ───────────────────
# quantized_matmul_impl keeps these formats in GGUF [k][n] order and multiplies
# by dequantize + matmul_f32_gguf (dispatch.rs:126-133, 541-574); the
# standalone matmul_f16 / _q2_k / _q3_k take [n][k] rows (x86: avx2.rs:210-389).
GGUF_DTYPES = [F32, F16, Q2_K, Q3_K]
# n = 300 / 128: K-quant blocks straddle the rows of W; k = 37: blocks span rows
GGUF_SHAPES = [(1, 256, 256), (1, 4096, 1024), (3, 512, 300), (17, 768, 512), (1, 14336, 4096), (9, 256, 37),
               (2, 300, 512), (1, 128, 1024)]


@pytest.mark.parametrize("dtype", GGUF_DTYPES)
@pytest.mark.parametrize("m,n,k", GGUF_SHAPES)
def test_gguf_order_matmul_parity(gpu, dtype, m, n, k):
    torch = gpu
    L = A.lib()
    be, bb = GEOM[dtype]
    rng = np.random.default_rng(n + k + m)
    raw = synth_blocks(dtype, n * k // be, n + 7 * k + dtype)
    x = rng.standard_normal(m * k).astype(np.float32)
    x[rng.integers(0, m * k, 5)] = 0.0  # skipped rows of W (matmul_f32_gguf's a_i == 0 test)
    w = make_weight(torch, dtype, n, k, raw)
    back = np.zeros_like(raw)
    A.check(L.aeth_weight_export_raw(w, back.ctypes.data, 0, None), "export")
    assert np.array_equal(back, raw) and L.aeth_weight_bytes(w) == raw.size
    got = gemv(torch, w, x, n, m)
    y0 = rng.standard_normal(m * n).astype(np.float32)
    got_acc = gemv(torch, w, x, n, m, flags=A.MM_ACCUMULATE, y0=y0)
    L.aeth_weight_free(w)
    ref = O.gguf_order_matmul(dtype, x, raw, m, n, k)
    assert_close(got, ref, what="gguf-order dtype %d m=%d n=%d k=%d" % (dtype, m, n, k))
    assert_close(got_acc, ref + y0.reshape(m, n), what="gguf-order accumulate")


def test_gguf_order_zero_activation_skips_infinite_weights(gpu):
    """A zero activation skips its weight row even when that row holds an
    infinity (0·inf would be NaN): matmul_f32_gguf's `if scale != 0.0`."""
    n, k = 512, 64
    w16 = (np.random.default_rng(1).standard_normal((k, n)) * 0.1).astype(np.float16)
    w16[7] = np.inf
    x = np.random.default_rng(2).standard_normal(k).astype(np.float32)
    x[7] = 0.0
    raw = w16.view(np.uint8).ravel()
    w = make_weight(gpu, F16, n, k, raw)
    got = gemv(gpu, w, x, n, 1)
    A.lib().aeth_weight_free(w)
    ref = O.gguf_order_matmul(F16, x, raw, 1, n, k)
    assert np.isfinite(ref).all() and np.isfinite(got).all()
    assert_close(got, ref)


def test_gguf_order_shape_rules(gpu):
    """GGUF-order weights: lanes read 4 consecutive outputs (n % 4 == 0) and
    K-quant tensors are whole blocks (n·k % 256 == 0)."""
    raw = synth_blocks(Q2_K, 302 * 128 // 256, 1)
    w = ctypes.c_void_p()
    assert A.lib().aeth_weight_create(Q2_K, 302, 128, raw.ctypes.data, 0, None, ctypes.byref(w)) == A.AETH_EUNSUPPORTED
    assert "% 4" in A.last_error()
    assert A.lib().aeth_weight_create(Q3_K, 4, 100, raw.ctypes.data, 0, None, ctypes.byref(w)) == A.AETH_EINVAL
    assert "whole blocks" in A.last_error()


@pytest.mark.parametrize("dtype,m,n,k", [(Q2_K, 1, 40, 512), (Q2_K, 3, 8, 256), (Q3_K, 1, 300, 4096), (Q3_K, 5, 33, 768),
                                         (F16, 1, 8, 32), (F16, 3, 8, 128), (F16, 2, 70, 100), (F16, 1, 1000, 4096),
                                         (Q2_K, 20, 64, 512), (Q3_K, 40, 48, 1024), (F16, 24, 64, 256)])
def test_row_kernels_standalone(gpu, dtype, m, n, k):
    """matmul_q2_k / matmul_q3_k / matmul_f16 on [n][k] rows against the x86
    dispatch (AVX2 order) — for F16 also the reference's own k = 32 / 128
    cases (tests.rs:581-636)."""
    L = A.lib()
    be, bb = GEOM[dtype]
    rng = np.random.default_rng(k * 3 + n)
    raw = synth_blocks(dtype, n * (k // be), n + k)
    a = rng.standard_normal(m * k).astype(np.float32)
    c = np.full(m * n, np.nan, dtype=np.float32)
    fn = {Q2_K: L.aeth_matmul_q2_k, Q3_K: L.aeth_matmul_q3_k, F16: L.aeth_matmul_f16}[dtype]
    A.check(fn(a.ctypes.data, raw.ctypes.data, raw.size, m, n, k, c.ctypes.data), "matmul rows")
    ref = O.reference_matmul(dtype, a, raw, m, n, k)
    assert_close(c.reshape(m, n), ref, what="rows dtype %d" % dtype)
    A.check(L.aeth_weight_cache_clear())


def test_row_kernels_reference_generators(gpu):
    """tests.rs:638-826: the reference's own Q2_K / Q3_K inputs (k = 256, n = 8,
    m in {1, 3}) through the standalone kernels, against its scalar kernels."""
    L = A.lib()
    for dtype, fn in ((Q2_K, L.aeth_matmul_q2_k), (Q3_K, L.aeth_matmul_q3_k)):
        for m in (1, 3):
            k, n = 256, 8
            b = ((np.arange(n * GEOM[dtype][1]) * 31) % 256).astype(np.uint8)
            a = (((np.arange(m * k) * 17) % 100) / 50.0 - 1.0).astype(np.float32)
            c = np.zeros(m * n, dtype=np.float32)
            A.check(fn(a.ctypes.data, b.ctypes.data, b.size, m, n, k, c.ctypes.data), "rows")
            assert_close(c.reshape(m, n), O.scalar_matmul(dtype, a, b, m, n, k), what="ref gen %d m=%d" % (dtype, m))
    A.check(L.aeth_weight_cache_clear())


def test_quantized_matmul_impl_gguf_order_formats(gpu):
    """quantized_matmul_impl with F32 / F16 / Q2_K / Q3_K bytes in GGUF order
    (test_asymmetric_gguf_order_f16, tests.rs:704-760, in general form), and
    the same bytes through a registered kernel."""
    L = A.lib()
    A.check(L.aeth_weight_cache_clear())
    k, n, m = 256, 512, 3
    rng = np.random.default_rng(9)
    buf = ctypes.create_string_buffer(64)
    if L.aeth_registered_kernel_name(Q4_K, buf, 64) == 0:
        A.check(L.aeth_register_hip_kernels(), "register")
    for dtype in GGUF_DTYPES:
        raw = synth_blocks(dtype, k * n // GEOM[dtype][0], 30 + dtype)
        a = rng.standard_normal(m * k).astype(np.float32)
        c = np.full(m * n, np.nan, dtype=np.float32)
        A.check(L.aeth_quantized_matmul_impl(a.ctypes.data, m, raw.ctypes.data, raw.size, n, k, dtype,
                                             c.ctypes.data), "quantized_matmul_impl")
        assert_close(c.reshape(m, n), O.gguf_order_matmul(dtype, a, raw, m, n, k), what="qmi dtype %d" % dtype)
        assert L.aeth_registered_kernel_name(dtype, buf, 64) == 1
        c2 = np.zeros(m * n, dtype=np.float32)
        assert L.aeth_dispatch_matmul(a.ctypes.data, m, raw.ctypes.data, raw.size, n, k, dtype, c2.ctypes.data) == 1
        assert np.array_equal(c, c2)
    A.check(L.aeth_weight_cache_clear())


# ── the int8 dot-product path (aarch64 dotprod hosts) ────────────────────
# AETH_MM_Q8_ACTIVATIONS: activations become Q8_0 blocks exactly as
# quantize_activations_q8_0 makes them (neon.rs:45-155), then exact integer
# dots against the weight quants (matmul_*_dotprod; their references in
# tests.rs:28-330). Only the f32 summation order differs from the references.
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m,n,k", [(1, 64, 256), (1, 1000, 4096), (3, 129, 1024), (1, 333, 14336), (2, 48, 2048)])
def test_dotprod_mode_parity(gpu, dtype, m, n, k):
    rng = np.random.default_rng(m + n + k + dtype)
    raw = weight(dtype, n, k, 3 * n + k)
    x = rng.standard_normal(m * k).astype(np.float32)
    x[: min(64, k)] *= 50.0  # blocks with a large maximum next to ordinary ones
    w = make_weight(gpu, dtype, n, k, raw)
    got = gemv(gpu, w, x, n, m, flags=A.MM_Q8_ACTIVATIONS)
    A.lib().aeth_weight_free(w)
    aq = O.quantize_activations_q8_0(x, m, k)
    ref = O.dotprod_ref(dtype, aq, raw, m, n, k)
    assert_close(got, ref, what="dotprod dtype %d m=%d n=%d k=%d" % (dtype, m, n, k))


@pytest.mark.parametrize("m,n,k", [(1, 40, 100), (2, 33, 1000), (3, 16, 4128)])
def test_dotprod_mode_q8_0_ragged_k(gpu, m, n, k):
    """Q8_0 rows of ceil(k/32) blocks: the last activation block is zero-padded
    (quantize_activations_q8_0, neon.rs:115-126)."""
    rng = np.random.default_rng(k)
    raw = weight(Q8_0, n, k, n + k)
    x = rng.standard_normal(m * k).astype(np.float32)
    w = make_weight(gpu, Q8_0, n, k, raw)
    got = gemv(gpu, w, x, n, m, flags=A.MM_Q8_ACTIVATIONS)
    A.lib().aeth_weight_free(w)
    ref = O.dotprod_ref(Q8_0, O.quantize_activations_q8_0(x, m, k), raw, m, n, k)
    assert_close(got, ref, what="dotprod q8_0 ragged k=%d" % k)


def test_dotprod_mode_reference_generators_and_nan(gpu):
    """The reference's own dotprod inputs (tests.rs:386-570: k = 256, n = 8,
    m in {1, 3}) for Q4_K / Q5_K / Q6_K, and a NaN activation giving NaN rows
    (its block scale is NaN, as vmaxq_f32 propagates it)."""
    for dtype in (Q4_K, Q5_K, Q6_K):
        for m in (1, 3):
            k, n = 256, 8
            b = ((np.arange(n * GEOM[dtype][1]) * 31) % 256).astype(np.uint8)
            a = (((np.arange(m * k) * 17) % 100) / 50.0 - 1.0).astype(np.float32)
            w = make_weight(gpu, dtype, n, k, b)
            got = gemv(gpu, w, a, n, m, flags=A.MM_Q8_ACTIVATIONS)
            A.lib().aeth_weight_free(w)
            ref = O.dotprod_ref(dtype, O.quantize_activations_q8_0(a, m, k), b, m, n, k)
            assert_close(got, ref, what="dotprod ref gen %d m=%d" % (dtype, m))
    raw = weight(Q4_K, 32, 512, 4)
    x = np.random.default_rng(2).standard_normal(512).astype(np.float32)
    x[100] = np.nan
    w = make_weight(gpu, Q4_K, 32, 512, raw)
    got = gemv(gpu, w, x, 32, 1, flags=A.MM_Q8_ACTIVATIONS)
    A.lib().aeth_weight_free(w)
    assert np.isnan(got).all()


def test_quantized_matmul_dotprod_host_slices(gpu):
    L = A.lib()
    A.check(L.aeth_weight_cache_clear())
    n, k, m = 40, 512, 2
    rng = np.random.default_rng(6)
    for dtype in DTYPES + [F16, Q2_K]:
        raw = synth_blocks(dtype, n * k // GEOM[dtype][0], 50 + dtype)
        a = rng.standard_normal(m * k).astype(np.float32)
        c = np.full(m * n, np.nan, dtype=np.float32)
        A.check(L.aeth_quantized_matmul_dotprod(a.ctypes.data, m, raw.ctypes.data, raw.size, n, k, dtype,
                                                c.ctypes.data), "quantized_matmul_dotprod")
        if dtype in DTYPES:
            ref = O.dotprod_ref(dtype, O.quantize_activations_q8_0(a, m, k), raw, m, n, k)
        else:  # no dot-product kernel: the GGUF-order route as on x86
            ref = O.gguf_order_matmul(dtype, a, raw, m, n, k)
        assert_close(c.reshape(m, n), ref, what="dotprod host dtype %d" % dtype)
    A.check(L.aeth_weight_cache_clear())


# The dot-product mode at m > 1 runs the Q4_K prefill GEMM with Q8_0 activation
# blocks (each 32-element block quantised as quantize_q8_0_block, neon.rs:45-104,
# then used as q·d_a): odd super-block counts, ragged
# m, both column extents, and a NaN row among finite ones.
@pytest.mark.parametrize("m,n,k", [(64, 256, 4096), (150, 4096, 4096), (512, 256, 4096), (70, 512, 1280),
                                   (33, 128, 14336)])
def test_dotprod_mode_gemm(gpu, m, n, k):
    rng = np.random.default_rng(m * 7 + n + k)
    raw = weight(Q4_K, n, k, m + n)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[1, :64] *= 300.0      # a block maximum far above its neighbours
    x[2] *= 2.0 ** -12      # tiny blocks (f16 scales near the subnormal range)
    x[3, 5:37] = 0.0        # a straddled zero block: d = 0 → zero quants
    if m > 4:
        x[4, 7] = np.nan
    w = make_weight(gpu, Q4_K, n, k, raw)
    got = gemv(gpu, w, x.ravel(), n, m, flags=A.MM_Q8_ACTIVATIONS)
    A.lib().aeth_weight_free(w)
    aq = O.quantize_activations_q8_0(x.ravel(), m, k)
    ref = O.dotprod_ref(Q4_K, aq, raw, m, n, k)
    if m > 4:
        assert np.isnan(got[4]).all() and np.isnan(ref[4]).all()
        keep = np.arange(m) != 4
        got, ref = got[keep], ref[keep]
    assert np.isfinite(got).all()
    assert_close(got, ref, what="dotprod GEMM m=%d n=%d k=%d" % (m, n, k))


GEMM_KERNEL_SCRIPT = r"""
import sys, numpy as np, torch
sys.path.insert(0, %r)
import aether_amd as A
from oracle import oracle as O
from tests._util import weight, assert_close
A.check(A.lib().aeth_init(0))
for m, n, k in ((130, 200, 1024), (64, 128, 2048), (70, 48, 1280), (33, 96, 14336), (34, 64, 20480)):
    raw = weight(12, n, k, m + n)
    x = np.random.default_rng(m).standard_normal((m, k)).astype(np.float32)
    w = __import__("ctypes").c_void_p()
    rawd = torch.from_numpy(raw).cuda()
    A.check(A.lib().aeth_weight_create(12, n, k, rawd.data_ptr(), 1, None, __import__("ctypes").byref(w)))
    xd = torch.from_numpy(x).cuda()
    y = torch.empty(m * n, dtype=torch.float32, device="cuda")
    A.check(A.lib().aeth_qmatmul(w, xd.data_ptr(), m, y.data_ptr(), 0, None))
    torch.cuda.synchronize()
    assert_close(y.cpu().numpy().reshape(m, n), O.reference_matmul(12, x.ravel(), raw, m, n, k), what="kernel")
    A.lib().aeth_weight_free(w)
# a prefill: the fused RMSNorm / SwiGLU producers and the gate|up GEMM's SwiGLU epilogue on this kernel
from tests.test_gpu_decode import TINY, build_tiny, make_runner, oracle_cfg
from tests._util import Q4_K, assert_close_logits
c = dict(TINY, max_seq_len=192)
md = build_tiny(seed=21, c=c)
r = make_runner(md, c)
s, co = O.precompute_rope(c["max_seq_len"], c["head_dim"], c["rope_base"])
kv = np.zeros((c["num_layers"], 2, c["num_kv_heads"], c["max_seq_len"], c["head_dim"]), dtype=np.float32)
toks = np.random.default_rng(5).integers(0, c["vocab_size"], 150).astype(np.int32)
logits = np.empty(c["vocab_size"], dtype=np.float32)
A.check(A.lib().aeth_runner_prefill(r, toks.ctypes.data, 150, logits.ctypes.data, None), "prefill")
ref = O.forward_batch(oracle_cfg(c), md["emb"][toks], md["layers"], [Q4_K] * 7, md["norms"], md["final"], md["lm"],
                      md["lm_dtype"], s, co, kv)
assert_close_logits(logits, ref, what="prefill")
A.lib().aeth_runner_free(r)
print("ok")
"""


@pytest.mark.parametrize("var,val", [("AETH_GEMM_KERNEL", "2")])
def test_gemm_alternate_kernels(gpu, var, val):
    """The GEMM kernel the default picks only for buffers past 2 GiB:
    AETH_GEMM_KERNEL=2 (the single-K-group ring kernel), read once per process,
    so it runs in a fresh process: plain products, then a runner prefill (its
    fused producers and the gate|up GEMM's SwiGLU epilogue) against the oracle."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, **{var: val})
    r = subprocess.run([sys.executable, "-c", GEMM_KERNEL_SCRIPT % root], env=env, cwd=root, timeout=240,
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stdout[-2000:]


Q6K_GEMM_SCRIPT = r"""
import sys, torch
sys.path.insert(0, %r)
import aether_amd as A
A.check(A.lib().aeth_init(0))
from tests.test_gpu_quant import check_q4k_gemm, check_q6k_gemm, check_q80_gemm
for m, n, k in ((70, 130, 768), (16, 16, 512), (3, 48, 1024), (65, 300, 1024), (33, 96, 14336), (200, 64, 14336),
                (34, 64, 20480)):
    check_q6k_gemm(torch, m, n, k)
for m, n, k in ((3, 48, 1024), (4, 300, 4096), (6, 64, 14336)):  # the Q4_K GEMM below its 16-row floor
    check_q4k_gemm(torch, m, n, k)
for m, n, k in ((3, 48, 1024), (6, 64, 14336)):  # and the Q8_0 GEMM
    check_q80_gemm(torch, m, n, k)
from tests.test_gpu_decode import test_runner_mixed_formats
for mix in (0, 1):
    for n in (23, 150):
        test_runner_mixed_formats(torch, mix, n)
print("ok")
"""


def test_q6k_gemm_small_weights(gpu):
    """The Q6_K GEMM on weights too small for the default to pick it (AETH_Q6K_GEMM_ROWS=2,
    read once per process, so in a fresh process): ragged tiles from 3 rows, K split over up
    to 10 workgroups, and runner prefills of mixed-format layers, where the Q6_K v projection
    writes its columns of q|k|v with the output row stride and the Q6_K down projection adds
    the residual; and the Q4_K and Q8_0 GEMMs at 3 to 6 rows (AETH_Q4K_GEMM_ROWS=2,
    AETH_Q80_GEMM_ROWS=2)."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, AETH_Q6K_GEMM_ROWS="2", AETH_Q4K_GEMM_ROWS="2", AETH_Q80_GEMM_ROWS="2")
    r = subprocess.run([sys.executable, "-c", Q6K_GEMM_SCRIPT % root], env=env, cwd=root, timeout=240,
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stdout[-2000:]


# Batched products of the rows the format's GEMM does not take (k not a whole number of
# blocks / super-blocks): below a per-format row count (Q8_0 112, Q5_K and Q6_K 80) the
# row-batched GEMV, from it the weight dequantized once and one DGEMM — planar Q8_0 /
# Q5_K / Q6_K rows (including Q8_0's ragged k and K-quant rows whose tail past k/256
# blocks the reference ignores), accumulate, and the dot-product mode's Q8_0
# activation blocks, on both paths. With whole blocks the Q8_0, Q5_K and Q6_K GEMMs
# take the product (the Q8_0 150-row, Q5_K 70- and 300-row and Q6_K 150-row cases).
@pytest.mark.parametrize("dtype,m,n,k", [(Q8_0, 16, 300, 1000), (Q8_0, 400, 128, 1000), (Q8_0, 150, 512, 4096),
                                         (Q5_K, 70, 256, 2048), (Q5_K, 300, 64, 2048), (Q6_K, 150, 1024, 4096),
                                         (Q6_K, 260, 96, 4096), (Q6_K, 33, 96, 14336), (Q5_K, 20, 64, 600),
                                         (Q5_K, 100, 64, 600), (Q6_K, 100, 200, 1100), (Q6_K, 40, 64, 1300)])
def test_batched_dequant_gemm(gpu, dtype, m, n, k):
    rng = np.random.default_rng(m + n + k + dtype)
    raw = weight(dtype, n, k, 5 * n + k)
    x = rng.standard_normal(m * k).astype(np.float32)
    w = make_weight(gpu, dtype, n, k, raw)
    got = gemv(gpu, w, x, n, m)
    y0 = rng.standard_normal(m * n).astype(np.float32)
    got_acc = gemv(gpu, w, x, n, m, flags=A.MM_ACCUMULATE, y0=y0)
    got_q8 = gemv(gpu, w, x, n, m, flags=A.MM_Q8_ACTIVATIONS)
    A.lib().aeth_weight_free(w)
    ref = O.reference_matmul(dtype, x, raw, m, n, k)
    assert_close(got, ref, what="batched dtype %d m=%d n=%d k=%d" % (dtype, m, n, k))
    assert_close(got_acc, ref + y0.reshape(m, n), what="batched accumulate")
    ref_q8 = O.dotprod_ref(dtype, O.quantize_activations_q8_0(x, m, k), raw, m, n, k)
    assert_close(got_q8, ref_q8, what="batched dot-product mode")


# GGUF-order Q2_K / Q3_K: the row-batched GEMV, and from 40 / 32 rows the dequantized DGEMM.
@pytest.mark.parametrize("dtype,m,n,k", [(Q2_K, 24, 512, 1024), (Q2_K, 40, 512, 1024), (Q2_K, 260, 64, 1024),
                                         (Q3_K, 16, 768, 512), (Q3_K, 64, 300, 512), (Q3_K, 200, 96, 512)])
def test_batched_dequant_gemm_gguf_order(gpu, dtype, m, n, k):
    rng = np.random.default_rng(n + k + m)
    raw = synth_blocks(dtype, n * k // 256, n + 3 * k + dtype)
    x = rng.standard_normal(m * k).astype(np.float32)
    x[rng.integers(0, m * k, 9)] = 0.0
    w = make_weight(gpu, dtype, n, k, raw)
    got = gemv(gpu, w, x, n, m)
    A.lib().aeth_weight_free(w)
    assert_close(got, O.gguf_order_matmul(dtype, x, raw, m, n, k), what="batched gguf-order %d" % dtype)


@pytest.mark.parametrize("dtype,m,n,k", [(Q4_K, 3, 40, 600), (Q6_K, 2, 48, 1000), (Q5_K, 20, 33, 300),
                                         (Q4_K, 40, 64, 1300)])
def test_dotprod_mode_batched_ragged_k(gpu, dtype, m, n, k):
    """The reference's batched K-quant dotprod kernels read row r's activation
    blocks from r·(k/256)·8 on (neon.rs:517-518, :994) while the quantizer lays
    rows ceil(k/32) blocks apart: for k % 256 != 0 rows past the first see a
    shifted window. The oracle restates that indexing; the device matches it."""
    rng = np.random.default_rng(m + n + k)
    raw = weight(dtype, n, k, 7 * n + k)
    x = rng.standard_normal(m * k).astype(np.float32)
    w = make_weight(gpu, dtype, n, k, raw)
    got = gemv(gpu, w, x, n, m, flags=A.MM_Q8_ACTIVATIONS)
    A.lib().aeth_weight_free(w)
    ref = O.dotprod_ref(dtype, O.quantize_activations_q8_0(x, m, k), raw, m, n, k)
    assert_close(got, ref, what="batched ragged dotprod %d m=%d k=%d" % (dtype, m, k))
