"""GPU re-quantizers, the Q8_0 activation quantizer and the device load path,
byte for byte against the CPU oracle (requantize: dispatch.rs:139-537;
activation scheme: neon.rs:45-155; load_quant: model_loader.rs:330-386).

Inputs mix ordinary values with the blocks the reference's branches single
out: all-zero blocks (d = 1), constant and one-signed blocks, ragged row tails
(partial last blocks), values far apart in magnitude, exact rounding ties,
and NaN / infinity elements (Rust's f32::max/min drop a NaN operand; the
activation scheme's max propagates it).
"""
import ctypes

import numpy as np
import pytest

import aether_amd as A
from oracle import oracle as O
from tests._util import GEOM, Q4_K, Q5_K, Q6_K, Q8_0, assert_close, synth_blocks

pytestmark = pytest.mark.gpu
DTYPES = [Q8_0, Q4_K, Q5_K, Q6_K]


def special_rows(rng, rows, cols, with_nonfinite=True):
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    if rows > 1:
        x[1] *= 1000.0
    if rows > 2:
        x[2, : min(cols, 64)] = 0.0                      # zero blocks / sub-blocks
    if rows > 3:
        x[3] = np.abs(x[3]) + 0.25                        # one-signed (no negative minimum)
    if rows > 4:
        x[4, : min(cols, 40)] = -2.5                      # constant run
    if rows > 5:
        x[5] *= np.float32(2.0 ** -20)                    # tiny scales (f16 subnormal d)
    if rows > 6 and with_nonfinite:
        x[6, 3] = np.nan
        x[6, min(cols - 1, 40)] = np.inf
        x[6, min(cols - 1, 77)] = -np.inf
    if rows > 7:
        x[7] = np.round(x[7] * 8.0) / 8.0                 # many exact ties after scaling
    return x


def to_dev(torch, arr):
    return torch.from_numpy(np.ascontiguousarray(arr)).cuda()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,cols", [(8, 256), (9, 300), (8, 1000), (3, 32), (2, 33), (16, 4096)])
def test_requantize_byte_exact(gpu, dtype, rows, cols):
    torch = gpu
    rng = np.random.default_rng(rows * 131 + cols + dtype)
    x = special_rows(rng, rows, cols)
    be, bb = GEOM[dtype]
    nbytes = rows * ((cols + be - 1) // be) * bb
    out = torch.full((nbytes,), 0xA5, dtype=torch.uint8, device="cuda")
    xd = to_dev(torch, x)  # device copies stay referenced until the kernel has run
    A.check(A.lib().aeth_requantize(dtype, xd.data_ptr(), rows, cols, out.data_ptr(), None), "requantize")
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ref = O.requantize(dtype, x.ravel(), rows, cols)
    bad = np.flatnonzero(got != ref)
    assert bad.size == 0, "dtype %d: %d/%d bytes differ, first at byte %d (block %d): got %d ref %d" % (
        dtype, bad.size, got.size, bad[0], bad[0] // bb, got[bad[0]], ref[bad[0]])


@pytest.mark.parametrize("m,k", [(1, 32), (3, 100), (8, 4096), (9, 1000), (2, 31)])
def test_quantize_activations_q8_0_byte_exact(gpu, m, k):
    torch = gpu
    rng = np.random.default_rng(m * 7 + k)
    a = special_rows(rng, m, k)
    if m > 8:
        # ties: x·(1/d) lands on .5 for d = 1 (max |x| = 127)
        a[8, :] = (np.arange(k) % 7 - 3).astype(np.float32) + 0.5
        a[8, 0] = 127.0
    nbytes = m * ((k + 31) // 32) * 34
    out = torch.full((nbytes,), 0x5A, dtype=torch.uint8, device="cuda")
    ad = to_dev(torch, a)
    A.check(A.lib().aeth_quantize_activations_q8_0(ad.data_ptr(), m, k, out.data_ptr(), None), "quant")
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ref = O.quantize_activations_q8_0(a.ravel(), m, k)
    bad = np.flatnonzero(got != ref)
    assert bad.size == 0, "%d/%d bytes differ, first at byte %d (block %d): got %d ref %d" % (
        bad.size, got.size, bad[0], bad[0] // 34, got[bad[0]], ref[bad[0]])


def test_q8_0_activation_blocks_feed_the_dotprod_reference(gpu):
    """The GPU-quantized activation blocks give the reference's dotprod result
    (tests.rs:28-60 / 62-134) exactly as the oracle's own blocks do."""
    torch = gpu
    rng = np.random.default_rng(3)
    m, n, k = 3, 24, 512
    a = rng.standard_normal((m, k)).astype(np.float32)
    out = torch.empty(m * (k // 32) * 34, dtype=torch.uint8, device="cuda")
    ad = to_dev(torch, a)
    A.check(A.lib().aeth_quantize_activations_q8_0(ad.data_ptr(), m, k, out.data_ptr(), None), "quant")
    torch.cuda.synchronize()
    aq = out.cpu().numpy()
    for dtype in (Q8_0, Q4_K):
        nb = k // 32 if dtype == Q8_0 else k // 256
        b = synth_blocks(dtype, n * nb, 11 + dtype).ravel()
        got = O.dotprod_ref(dtype, aq, b, m, n, k)
        ref = O.dotprod_ref(dtype, O.quantize_activations_q8_0(a.ravel(), m, k), b, m, n, k)
        assert np.array_equal(got, ref)
        # 8-bit activations stay close to the f32 path (per-row cosine only: element
        # errors of a rounded activation scheme are not bounded by the 1e-3 bar)
        f = O.reference_matmul(dtype, a.ravel(), b, m, n, k).astype(np.float64)
        g = got.astype(np.float64)
        cos = (g * f).sum(1) / np.sqrt((g * g).sum(1) * (f * f).sum(1))
        assert (cos > 0.999).all(), cos


@pytest.mark.parametrize("rows,cols", [(1, 1), (33, 70), (256, 129), (1000, 37)])
def test_transpose_f32(gpu, rows, cols):
    torch = gpu
    x = np.random.default_rng(rows + cols).standard_normal((rows, cols)).astype(np.float32)
    out = torch.empty(rows * cols, dtype=torch.float32, device="cuda")
    xd = to_dev(torch, x)
    A.check(A.lib().aeth_transpose_f32(xd.data_ptr(), rows, cols, out.data_ptr(), None), "transpose")
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().reshape(cols, rows), x.T)


def load_quant_oracle(dtype, raw, k, n):
    """transpose_quantized_bytes (model_loader.rs:372-385) on the CPU oracle."""
    flat = O.dequant(dtype, raw, k * n)
    be = GEOM[dtype][0]
    if dtype != Q8_0:
        flat[(k * n) // be * be:] = 0.0  # whole blocks only; the reference's vector starts zeroed
    return O.requantize(dtype, flat.reshape(k, n).T.ravel(), n, k)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("k,n", [(256, 48), (512, 33), (1024, 16)])
def test_load_quant_byte_exact_and_usable(gpu, dtype, k, n):
    torch = gpu
    L = A.lib()
    be, bb = GEOM[dtype]
    raw = synth_blocks(dtype, (k * n + be - 1) // be, 100 + k + n + dtype).ravel()
    ws = torch.empty(L.aeth_load_quant_ws_bytes(k, n), dtype=torch.uint8, device="cuda")
    out = torch.empty(n * ((k + be - 1) // be) * bb, dtype=torch.uint8, device="cuda")
    rawd = to_dev(torch, raw)
    A.check(L.aeth_load_quant(dtype, rawd.data_ptr(), k, n, out.data_ptr(), ws.data_ptr(), None), "load_quant")
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ref = load_quant_oracle(dtype, raw, k, n)
    bad = np.flatnonzero(got != ref)
    assert bad.size == 0, "dtype %d k=%d n=%d: %d bytes differ, first at %d" % (dtype, k, n, bad.size, bad[0])
    # the re-laid weight drops into the matmul path: [n][k] blocks, y = W·x
    w = ctypes.c_void_p()
    A.check(L.aeth_weight_create(dtype, n, k, out.data_ptr(), 1, None, ctypes.byref(w)), "weight_create")
    x = np.random.default_rng(k).standard_normal(k).astype(np.float32)
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    xd = to_dev(torch, x)
    A.check(L.aeth_qmatmul(w, xd.data_ptr(), 1, y.data_ptr(), 0, None), "qmatmul")
    torch.cuda.synchronize()
    L.aeth_weight_free(w)
    assert_close(y.cpu().numpy(), O.reference_matmul(dtype, x, ref, 1, n, k)[0], what="load_quant → GEMV")


def test_requantize_and_load_quant_bad_arguments(gpu):
    L = A.lib()
    assert L.aeth_requantize(3, None, 1, 32, None, None) == A.AETH_EUNSUPPORTED
    assert L.aeth_requantize(Q8_0, None, 1, 32, None, None) == A.AETH_EINVAL
    assert L.aeth_requantize(Q8_0, None, 0, 32, None, None) == A.AETH_OK
    assert L.aeth_quantize_activations_q8_0(None, 1, 0, None, None) == A.AETH_EINVAL
    assert L.aeth_load_quant(Q4_K, None, 256, 4, None, None, None) == A.AETH_EINVAL
    assert L.aeth_load_quant(16, None, 256, 4, None, None, None) == A.AETH_EUNSUPPORTED
    assert L.aeth_load_quant_ws_bytes(256, 4) == 2 * 256 * 4 * 4


def test_requantize_hand_blocks(gpu):
    """The device re-quantizers on the hand blocks of tests/requant_hand_cases.py:
    halves round away from zero and quants divide by the f32 scale, not the
    stored f16 one — literal expected bytes, not the oracle's output."""
    from tests import requant_hand_cases as H

    torch = gpu

    def dev_requant(dtype, x, cols):
        be, bb = GEOM[dtype]
        out = torch.full((bb * (cols // be),), 0xA5, dtype=torch.uint8, device="cuda")
        xd = to_dev(torch, x)
        A.check(A.lib().aeth_requantize(dtype, xd.data_ptr(), 1, cols, out.data_ptr(), None), "requantize")
        torch.cuda.synchronize()
        return out.cpu().numpy()

    for make in (H.q8_0_ties, H.q8_0_f32_scale):
        x, expect = make()
        H.check_bytes(dev_requant(Q8_0, x, 32), expect, make.__name__)
    for make in (H.q4_k_ties, H.q4_k_f32_scale):
        x, expect = make()
        H.check_bytes(dev_requant(Q4_K, x, 256), expect, make.__name__)
    for x, dbits, sc0, deq in H.q6_k_cases():
        b = dev_requant(Q6_K, x, 256)
        assert int(b[208]) | (int(b[209]) << 8) == dbits
        assert int(b[192]) == sc0
        assert list(O.dequant(Q6_K, b, 256)[:len(deq)]) == deq
