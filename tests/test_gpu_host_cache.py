"""The host-slice weight cache (quantized_matmul_impl / matmul_q* over borrowed
slices, dispatch.rs:98-135): a weight rewritten in place at the same address
and length is uploaded again (content fingerprint), the device bytes the cache
holds stay under its limit (LRU), and concurrent host threads get their own
results. The reference reads b_raw on every call, so any stale reuse would be
a parity break."""
import ctypes
import threading

import numpy as np
import pytest

import aether_amd as A
from oracle import oracle as O
from tests._util import Q4_K, Q6_K, Q8_0, assert_close, weight

pytestmark = pytest.mark.gpu


def run(dtype, a, raw, m, n, k):
    c = np.full(m * n, np.nan, np.float32)
    A.check(A.lib().aeth_quantized_matmul_impl(a.ctypes.data, m, raw.ctypes.data, raw.size, n, k, dtype,
                                               c.ctypes.data), "quantized_matmul_impl")
    return c.reshape(m, n)


@pytest.mark.parametrize("dtype,m", [(Q4_K, 1), (Q4_K, 70), (Q6_K, 1), (Q8_0, 3)])
def test_weight_rewritten_in_place_is_reloaded(gpu, dtype, m):
    L = A.lib()
    A.check(L.aeth_weight_cache_clear())
    n, k = 48, 512
    raw = weight(dtype, n, k, 11)
    a = np.random.default_rng(2).standard_normal(m * k).astype(np.float32)
    addr = raw.ctypes.data
    first = run(dtype, a, raw, m, n, k)
    assert_close(first, O.reference_matmul(dtype, a, raw, m, n, k))
    raw[:] = weight(dtype, n, k, 12)  # same buffer, same length, new bytes
    assert raw.ctypes.data == addr
    second = run(dtype, a, raw, m, n, k)
    assert_close(second, O.reference_matmul(dtype, a, raw, m, n, k))
    assert not np.array_equal(first, second)
    raw[7] ^= 0x01  # a single flipped bit is seen too
    third = run(dtype, a, raw, m, n, k)
    assert_close(third, O.reference_matmul(dtype, a, raw, m, n, k))
    A.check(L.aeth_weight_cache_clear())
    assert L.aeth_weight_cache_bytes() == 0


def test_cache_is_bounded_lru(gpu):
    L = A.lib()
    A.check(L.aeth_weight_cache_clear())
    n, k = 64, 1024
    raws = [weight(Q4_K, n, k, 30 + i) for i in range(4)]
    one = raws[0].size
    try:
        A.check(L.aeth_weight_cache_set_limit(2 * one + one // 2))  # room for two weights
        a = np.random.default_rng(4).standard_normal(k).astype(np.float32)
        for r in raws + raws[::-1]:
            assert_close(run(Q4_K, a, r, 1, n, k), O.reference_matmul(Q4_K, a, r, 1, n, k))
            assert L.aeth_weight_cache_bytes() <= 2 * one + one // 2
        assert L.aeth_weight_cache_bytes() == 2 * one
        A.check(L.aeth_weight_cache_set_limit(0))  # nothing is kept, calls still run
        assert L.aeth_weight_cache_bytes() == 0
        assert_close(run(Q4_K, a, raws[1], 1, n, k), O.reference_matmul(Q4_K, a, raws[1], 1, n, k))
        assert L.aeth_weight_cache_bytes() == 0
        assert L.aeth_weight_cache_set_limit(-1) == A.AETH_EINVAL
    finally:
        A.check(L.aeth_weight_cache_set_limit(32 << 30))
        A.check(L.aeth_weight_cache_clear())


def test_concurrent_host_threads(gpu):
    """RunnerPool-style concurrent callers (runner.rs:2099-2175): each thread's
    result matches its own reference."""
    L = A.lib()
    A.check(L.aeth_weight_cache_clear())
    n, k = 256, 2048
    jobs = []
    for t in range(6):
        dt = (Q4_K, Q6_K, Q8_0)[t % 3]
        m = (1, 9, 1)[t % 3]
        raw = weight(dt, n, k, 50 + t)
        a = np.random.default_rng(t).standard_normal(m * k).astype(np.float32)
        jobs.append((dt, a, raw, m))
    out = [None] * len(jobs)
    errs = []

    def work(i):
        try:
            dt, a, raw, m = jobs[i]
            for _ in range(3):
                out[i] = run(dt, a, raw, m, n, k)
        except Exception as e:  # reported after join
            errs.append(e)

    th = [threading.Thread(target=work, args=(i,)) for i in range(len(jobs))]
    for t in th:
        t.start()
    for t in th:
        t.join()
    assert not errs, errs
    for (dt, a, raw, m), got in zip(jobs, out):
        assert_close(got, O.reference_matmul(dt, a, raw, m, n, k), what="thread dtype %d" % dt)
    A.check(L.aeth_weight_cache_clear())


@pytest.mark.parametrize("m", [1, 5])
def test_quantized_matmul_impl_b_f32_cache(gpu, m):
    """quantized_matmul_impl's b_f32_cache branch (dispatch.rs:113-117): the
    cached f32 weight in GGUF [k][n] order is multiplied by matmul_f32_gguf and
    b_raw is ignored; without a cache the raw bytes are used."""
    L = A.lib()
    n, k = 64, 512
    raw = weight(Q4_K, n, k, 77)
    # the cache a LayerCache would hold: the weight dequantized, GGUF [in][out] order
    cache = np.ascontiguousarray(O.dequant(Q4_K, raw, n * k).reshape(n, k).T)
    a = np.random.default_rng(m).standard_normal(m * k).astype(np.float32)
    c = np.full(m * n, np.nan, np.float32)
    junk = np.zeros_like(raw)  # not read when the cache is given
    A.check(L.aeth_quantized_matmul_impl_cached(a.ctypes.data, m, junk.ctypes.data, junk.size, n, k, Q4_K,
                                                c.ctypes.data, cache.ctypes.data), "impl_cached")
    assert_close(c.reshape(m, n), O.matmul_f32_gguf(a, cache, m, n, k))
    c2 = np.full(m * n, np.nan, np.float32)
    A.check(L.aeth_quantized_matmul_impl_cached(a.ctypes.data, m, raw.ctypes.data, raw.size, n, k, Q4_K,
                                                c2.ctypes.data, None), "impl_cached (no cache)")
    assert_close(c2.reshape(m, n), O.reference_matmul(Q4_K, a, raw, m, n, k))
    A.check(L.aeth_weight_cache_clear())


def test_stream_read_arguments(gpu):
    torch = gpu
    L = A.lib()
    src = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(4096, dtype=torch.int32, device="cuda")
    A.check(L.aeth_stream_read(src.data_ptr(), src.numel(), sink.data_ptr(), sink.numel(), None), "stream_read")
    torch.cuda.synchronize()
    assert not sink.any()
    assert L.aeth_stream_read(src.data_ptr(), 15, sink.data_ptr(), sink.numel(), None) == A.AETH_EINVAL
    assert L.aeth_stream_read(src.data_ptr(), src.numel(), sink.data_ptr(), 100, None) == A.AETH_EINVAL
