"""aeth_attn_decode_noalloc (no counterpart in the reference: decode attention
for callers that cannot allocate, with its partials in a static device array)
against aeth_attn_decode, which runs the same kernels on a library allocation:
two calls in a row, the second with a smaller input, must give the existing
entry point's results exactly; sizes beyond the static array are refused."""
import numpy as np
import pytest

import aether_amd as A

pytestmark = pytest.mark.gpu


def test_attn_decode_noalloc_matches_attn_decode(gpu):
    torch = gpu
    L = A.lib()
    nh, nkv, hd = 32, 8, 128
    for ms, seq in ((4096, 2049), (1024, 77)):  # the second call is smaller
        rng = np.random.default_rng(seq)
        kv = torch.from_numpy(rng.standard_normal((2, nkv, ms, hd)).astype(np.float32)).cuda()
        q = torch.from_numpy(rng.standard_normal(nh * hd).astype(np.float32)).cuda()
        ref = torch.full((nh * hd,), float("nan"), device="cuda")
        got = torch.full((nh * hd,), float("nan"), device="cuda")
        A.check(L.aeth_attn_decode(q.data_ptr(), kv.data_ptr(), nh, nkv, hd, ms, seq, ref.data_ptr(), None))
        A.check(L.aeth_attn_decode_noalloc(q.data_ptr(), kv.data_ptr(), nh, nkv, hd, ms, seq, got.data_ptr(), None))
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (ms, seq)
        assert torch.isfinite(got).all()
    # 64 heads over 16384 positions need 64·128·130 floats (chunks of 128 positions) > 2^20
    assert L.aeth_attn_decode_noalloc(q.data_ptr(), kv.data_ptr(), 64, 8, hd, 16384, 10, got.data_ptr(),
                                      None) == A.AETH_EINVAL
    assert "more than" in A.last_error()
