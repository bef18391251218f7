"""GPU parity of the decode-step kernels and the device LlamaRunner against
the CPU oracle's restatement of runner.rs (rmsnorm, RoPE, attention, SiLU,
argmax, one full decode step)."""
import ctypes

import numpy as np
import pytest

import aether_amd as A
from oracle import oracle as O
from tests._model64 import logits64
from tests._models import TINY, build_tiny, oracle_cfg
from tests._util import (F16, F32, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0, assert_close, assert_close_logits,
                         assert_close_rows, weight)

pytestmark = pytest.mark.gpu


def dev(torch, arr):
    return torch.from_numpy(np.ascontiguousarray(arr)).cuda()


@pytest.mark.parametrize("n", [4096, 1024, 8192, 4000, 100])
def test_rmsnorm(gpu, n):
    """Row lengths of the one-pass register kernel (multiples of 1024) and of
    the general loop."""
    torch = gpu
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, n)).astype(np.float32) * 3
    w = (1 + 0.02 * rng.standard_normal(n)).astype(np.float32)
    xd, wd = dev(torch, x), dev(torch, w)
    od = torch.empty_like(xd)
    A.check(A.lib().aeth_rmsnorm(xd.data_ptr(), wd.data_ptr(), 3, n, 1e-5, od.data_ptr(), None))
    torch.cuda.synchronize()
    ref = np.stack([O.rmsnorm(x[i], w, 1e-5) for i in range(3)])
    assert_close(od.cpu().numpy(), ref, tol=1e-5)


@pytest.mark.parametrize("pos", [0, 1, 2047, 5000])
def test_rope(gpu, pos):
    torch = gpu
    nh, hd, ms = 40, 128, 4096
    s, c = O.precompute_rope(ms, hd, 500000.0)
    x = np.random.default_rng(pos).standard_normal(nh * hd).astype(np.float32)
    xd, sd, cd = dev(torch, x), dev(torch, s), dev(torch, c)  # keep the device tensors alive across the call
    A.check(A.lib().aeth_rope(xd.data_ptr(), nh, hd, pos, sd.data_ptr(), cd.data_ptr(), ms, None))
    torch.cuda.synchronize()
    ref = O.apply_rope(x, nh, hd, pos, s, c, ms)
    assert_close(xd.cpu().numpy(), ref, tol=1e-5)
    if pos == 0:
        assert np.array_equal(xd.cpu().numpy(), x)  # θ = 0: identity


@pytest.mark.parametrize("seq", [1, 63, 64, 65, 127, 128, 129, 2049])
def test_attention_and_kv_append(gpu, seq):
    torch = gpu
    L = A.lib()
    nh, nkv, hd, ms = 32, 8, 128, 2304
    rng = np.random.default_rng(seq)
    kv = rng.standard_normal((2, nkv, ms, hd)).astype(np.float32)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k_new = rng.standard_normal(nkv * hd).astype(np.float32)
    v_new = rng.standard_normal(nkv * hd).astype(np.float32)
    kvd, kd, vd, qd = dev(torch, kv), dev(torch, k_new), dev(torch, v_new), dev(torch, q)
    slot = seq - 1
    A.check(L.aeth_kv_append(kvd.data_ptr(), kd.data_ptr(), vd.data_ptr(), nkv, hd, ms, slot, None))
    od = torch.empty(nh * hd, dtype=torch.float32, device="cuda")
    A.check(L.aeth_attn_decode(qd.data_ptr(), kvd.data_ptr(), nh, nkv, hd, ms, seq, od.data_ptr(), None))
    torch.cuda.synchronize()
    kv[0, :, slot, :] = k_new.reshape(nkv, hd)
    kv[1, :, slot, :] = v_new.reshape(nkv, hd)
    assert np.array_equal(kvd.cpu().numpy(), kv)
    ref = np.concatenate([O.attn_direct(q[h * hd:(h + 1) * hd], kv[0, h // (nh // nkv)], kv[1, h // (nh // nkv)], seq,
                                        hd) for h in range(nh)])
    assert_close(od.cpu().numpy(), ref, tol=1e-4)


@pytest.mark.parametrize("seq", [1, 65, 700])
def test_attention_ignores_stale_chunk_partials(gpu, seq):
    """The merge loads every chunk slot of its scratch before it reads the
    sequence length; slots past the live chunks hold what an earlier call left.
    An earlier call over 2049 positions with a NaN query leaves NaN partials in
    every slot: a shorter call after it on the same stream must match the
    oracle with no NaN."""
    torch = gpu
    L = A.lib()
    nh, nkv, hd, ms = 32, 8, 128, 2304
    rng = np.random.default_rng(100 + seq)
    kv = rng.standard_normal((2, nkv, ms, hd)).astype(np.float32)
    kvd = dev(torch, kv)
    od = torch.empty(nh * hd, dtype=torch.float32, device="cuda")
    qnan = dev(torch, np.full(nh * hd, np.nan, dtype=np.float32))
    A.check(L.aeth_attn_decode(qnan.data_ptr(), kvd.data_ptr(), nh, nkv, hd, ms, 2049, od.data_ptr(), None))
    torch.cuda.synchronize()
    assert np.isnan(od.cpu().numpy()).all()
    q = rng.standard_normal(nh * hd).astype(np.float32)
    qd = dev(torch, q)
    A.check(L.aeth_attn_decode(qd.data_ptr(), kvd.data_ptr(), nh, nkv, hd, ms, seq, od.data_ptr(), None))
    torch.cuda.synchronize()
    got = od.cpu().numpy()
    ref = np.concatenate([O.attn_direct(q[h * hd:(h + 1) * hd], kv[0, h // (nh // nkv)], kv[1, h // (nh // nkv)], seq,
                                        hd) for h in range(nh)])
    assert np.isfinite(got).all()
    assert_close(got, ref, tol=1e-4)


def test_attention_one_hot(gpu):
    """A query aligned with one cached key far above the rest attends only to
    that position: out = v_t."""
    torch = gpu
    nh, nkv, hd, ms, seq = 4, 1, 128, 256, 200
    kv = np.zeros((2, nkv, ms, hd), dtype=np.float32)
    rng = np.random.default_rng(3)
    kv[1] = rng.standard_normal((nkv, ms, hd))
    kv[0, 0, 77, :] = 1.0
    q = np.full(nh * hd, 10.0, dtype=np.float32)
    od = torch.empty(nh * hd, dtype=torch.float32, device="cuda")
    qd, kvd = dev(torch, q), dev(torch, kv)
    A.check(A.lib().aeth_attn_decode(qd.data_ptr(), kvd.data_ptr(), nh, nkv, hd, ms, seq, od.data_ptr(), None))
    torch.cuda.synchronize()
    got = od.cpu().numpy().reshape(nh, hd)
    for h in range(nh):
        np.testing.assert_allclose(got[h], kv[1, 0, 77], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("nh,nkv,ms,seq", [(64, 8, 4096, 3000), (8, 8, 512, 300), (16, 2, 8192, 8192),
                                           (32, 8, 2688, 2600), (4, 1, 256, 1)])
def test_attention_shapes(gpu, nh, nkv, ms, seq):
    """Query-head groups of 1, 4 and 8; the longest cache (8192 positions: 64
    chunks of 128, past the 32 the merge loads in one batch); back-to-back calls
    of different shapes share one workspace."""
    torch = gpu
    hd = 128
    rng = np.random.default_rng(seq + nh)
    kv = rng.standard_normal((2, nkv, ms, hd)).astype(np.float32)
    g = nh // nkv
    for rep in range(2):
        q = rng.standard_normal(nh * hd).astype(np.float32)
        s = seq if rep == 0 else max(1, seq // 3)
        od = torch.empty(nh * hd, dtype=torch.float32, device="cuda")
        qd, kvd = dev(torch, q), dev(torch, kv)
        A.check(A.lib().aeth_attn_decode(qd.data_ptr(), kvd.data_ptr(), nh, nkv, hd, ms, s, od.data_ptr(), None))
        torch.cuda.synchronize()
        ref = np.concatenate([O.attn_direct(q[h * hd:(h + 1) * hd], kv[0, h // g], kv[1, h // g], s, hd)
                              for h in range(nh)])
        assert_close(od.cpu().numpy(), ref, tol=1e-4, what="attn nh=%d nkv=%d seq=%d" % (nh, nkv, s))


def test_silu_mul_and_add(gpu):
    torch = gpu
    rng = np.random.default_rng(4)
    n = 14336
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    gd, ud = dev(torch, g), dev(torch, u)
    A.check(A.lib().aeth_silu_mul(gd.data_ptr(), ud.data_ptr(), n, None))
    A.check(A.lib().aeth_add(gd.data_ptr(), ud.data_ptr(), n, None))
    torch.cuda.synchronize()
    ref = (g * (1.0 / (1.0 + np.exp(-g))) * u + u).astype(np.float32)
    assert_close(gd.cpu().numpy(), ref, tol=1e-5)


def test_argmax_last_max_wins(gpu):
    torch = gpu
    n = 128256
    x = np.random.default_rng(5).standard_normal(n).astype(np.float32)
    x[[10, 50000, 128000]] = 9.0  # ties: the last index wins (Iterator::max_by)
    od = torch.empty(1, dtype=torch.int32, device="cuda")
    xd = dev(torch, x)
    A.check(A.lib().aeth_argmax(xd.data_ptr(), n, od.data_ptr(), None))
    torch.cuda.synchronize()
    assert int(od.cpu()[0]) == 128000 == O.argmax(x)


# Prefill attention (attention_batch, runner.rs:1809-1883) against an f64
# restatement of its formula: s_t = (q·k_t)/√hd for t ≤ i, max-subtracted
# softmax, Σ p_t v_t. Group sizes 1, 2, 4, 8 take the f32-MFMA kernel, 3 the
# f32 VALU one; ragged n against the 16-key and query blocks, n = max_seq with
# a partial last key block (the MFMA kernel's range-checked loads read its rows
# past n as zeros), the 8B shape, and sharp softmaxes (scaled q: the running
# max grows by more than the kernel's rescale threshold).
@pytest.mark.parametrize("n,nh,nkv,max_seq,qs", [(1, 4, 4, 8, 1.0), (70, 8, 2, 96, 1.0), (150, 4, 2, 192, 3.0),
                                                 (33, 8, 1, 40, 1.0), (64, 6, 2, 64, 1.0), (512, 32, 8, 512, 1.0),
                                                 (97, 16, 4, 128, 4.0), (37, 16, 2, 37, 2.0), (45, 4, 4, 45, 1.0),
                                                 (130, 8, 2, 160, 12.0)])
def test_attn_prefill_matches_f64(gpu, n, nh, nkv, max_seq, qs):
    torch = gpu
    hd = 128
    rng = np.random.default_rng(n * 13 + nh)
    stride = (nh + 2 * nkv) * hd
    q = (rng.standard_normal((n, stride)) * qs).astype(np.float32)
    kv = np.zeros((2, nkv, max_seq, hd), dtype=np.float32)
    kv[:, :, :n] = rng.standard_normal((2, nkv, n, hd)).astype(np.float32)
    out = torch.empty(n * nh * hd, dtype=torch.float32, device="cuda")
    qd, kvd = torch.from_numpy(q).cuda(), torch.from_numpy(kv).cuda()  # kept alive across the launch
    A.check(A.lib().aeth_attn_prefill(qd.data_ptr(), stride, kvd.data_ptr(), n, nh, nkv, hd, max_seq,
                                      out.data_ptr(), None), "attn_prefill")
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(n, nh, hd)
    G = nh // nkv
    ref = np.empty((n, nh, hd))
    K = kv[0].astype(np.float64)
    V = kv[1].astype(np.float64)
    for h in range(nh):
        qh = q[:, h * hd:(h + 1) * hd].astype(np.float64)
        sc = qh @ K[h // G, :n].T / np.sqrt(hd)
        sc[np.triu_indices(n, 1)] = -np.inf
        p = np.exp(sc - sc.max(axis=1, keepdims=True))
        ref[:, h] = (p / p.sum(axis=1, keepdims=True)) @ V[h // G, :n]
    assert_close(got.reshape(n, -1), ref.reshape(n, -1), what="attn_prefill n=%d nh=%d nkv=%d" % (n, nh, nkv))
    assert np.abs(got - ref).max() < 1e-5


# ── device LlamaRunner vs the oracle's decode step ───────────────────────

def make_runner(m, c=TINY):
    cfg = A.LlamaConfig(**c)
    nl = c["num_layers"]
    wp = (ctypes.c_void_p * (nl * 7))(*[m["layers"][l][j].ctypes.data for l in range(nl) for j in range(7)])
    dt = (ctypes.c_int32 * (nl * 7))(*(m["layer_dtype"] * nl))
    npp = (ctypes.c_void_p * (nl * 2))(*[m["norms"][l][j].ctypes.data for l in range(nl) for j in range(2)])
    r = ctypes.c_void_p()
    A.check(A.lib().aeth_runner_create(ctypes.byref(cfg), wp, dt, npp, m["final"].ctypes.data, m["lm"].ctypes.data,
                                       m["lm_dtype"], m["emb"].ctypes.data, 0, ctypes.byref(r)), "runner_create")
    return r


@pytest.mark.parametrize("layer_dtype", [Q4_K, Q8_0, Q6_K, Q5_K])
def test_runner_decode_matches_oracle(gpu, layer_dtype):
    m = build_tiny(seed=2, layer_dtype=layer_dtype)
    r = make_runner(m)
    L = A.lib()
    c = TINY
    ocfg = oracle_cfg()
    s, co = O.precompute_rope(c["max_seq_len"], c["head_dim"], c["rope_base"])
    kv = np.zeros((c["num_layers"], 2, c["num_kv_heads"], c["max_seq_len"], c["head_dim"]), dtype=np.float32)
    fill = 0
    tok = 1
    try:
        for step in range(6):
            logits = np.empty(c["vocab_size"], dtype=np.float32)
            nxt = ctypes.c_int32()
            A.check(L.aeth_runner_decode(r, tok, step, logits.ctypes.data, ctypes.byref(nxt)), "decode")
            ref, fill = O.decode_step(ocfg, m["emb"][tok], step, m["layers"], [layer_dtype] * 7, m["norms"], m["final"],
                                      m["lm"], m["lm_dtype"], s, co, kv, fill)
            assert_close_logits(logits, ref, what="step %d" % step)
            assert nxt.value == O.argmax(logits)
            tok = O.argmax(ref)  # teacher forcing on the CPU's token
        assert L.aeth_runner_seq_len(r) == 6
        kv_dev = np.empty_like(kv)
        fl = ctypes.c_int32()
        A.check(L.aeth_runner_kv_to_host(r, kv_dev.ctypes.data, ctypes.byref(fl)))
        assert fl.value == 6
        assert_close_rows(kv_dev.reshape(-1, c["head_dim"]), kv.reshape(-1, c["head_dim"]), what="kv")
    finally:
        L.aeth_runner_free(r)


# Batched prefill (forward_batch) against the oracle's restatement: one query /
# key block (37), a full cache (64), a single token, and several ragged blocks
# with the GEMM path (150 of 192); GEMM for Q4_K, Q5_K and Q8_0 from 16 tokens (the fused
# RMSNorm prep and SwiGLU output included), the row-batched GEMV and standalone RMSNorm /
# SwiGLU below that (5, 12) and for the other formats.
@pytest.mark.parametrize("layer_dtype,n,max_seq", [(Q4_K, 37, 64), (Q8_0, 64, 64), (Q6_K, 1, 64), (Q4_K, 150, 192),
                                                   (Q5_K, 40, 64), (Q4_K, 5, 64), (Q4_K, 12, 64), (Q8_0, 150, 192),
                                                   (Q5_K, 150, 192)])
def test_runner_prefill_matches_oracle(gpu, layer_dtype, n, max_seq):
    c = dict(TINY, max_seq_len=max_seq)
    m = build_tiny(seed=7, layer_dtype=layer_dtype)
    r = make_runner(m, c)
    L = A.lib()
    ocfg = oracle_cfg(c)
    s, co = O.precompute_rope(c["max_seq_len"], c["head_dim"], c["rope_base"])
    kv = np.zeros((c["num_layers"], 2, c["num_kv_heads"], c["max_seq_len"], c["head_dim"]), dtype=np.float32)
    toks = np.random.default_rng(n).integers(0, c["vocab_size"], n).astype(np.int32)
    try:
        logits = np.empty(c["vocab_size"], dtype=np.float32)
        nxt = ctypes.c_int32()
        A.check(L.aeth_runner_prefill(r, toks.ctypes.data, n, logits.ctypes.data, ctypes.byref(nxt)), "prefill")
        ref = O.forward_batch(ocfg, m["emb"][toks], m["layers"], [layer_dtype] * 7, m["norms"], m["final"], m["lm"],
                              m["lm_dtype"], s, co, kv)
        assert_close_logits(logits, ref, what="prefill n=%d" % n)
        assert nxt.value == O.argmax(logits)
        assert L.aeth_runner_seq_len(r) == n
        kv_dev = np.empty_like(kv)
        fl = ctypes.c_int32()
        A.check(L.aeth_runner_kv_to_host(r, kv_dev.ctypes.data, ctypes.byref(fl)))
        assert fl.value == n
        assert_close_rows(kv_dev[:, :, :, :n].reshape(-1, c["head_dim"]), kv[:, :, :, :n].reshape(-1, c["head_dim"]),
                          what="kv after prefill")
        assert not kv_dev[:, :, :, n:].any()
        if n < max_seq:  # decoding continues from the prefilled cache
            tok = O.argmax(ref)
            A.check(L.aeth_runner_decode(r, tok, n, logits.ctypes.data, None), "decode after prefill")
            ref2, fill = O.decode_step(ocfg, m["emb"][tok], n, m["layers"], [layer_dtype] * 7, m["norms"], m["final"],
                                       m["lm"], m["lm_dtype"], s, co, kv, n)
            assert fill == n + 1 and L.aeth_runner_seq_len(r) == n + 1
            assert_close_logits(logits, ref2, what="decode after prefill")
    finally:
        L.aeth_runner_free(r)


# GQA group sizes G = query heads per KV head: the MFMA attention packs 16/G
# queries × G heads into its 16 score columns (G = 2 is TINY above); n = 70 is
# ragged against every query block, the 16-key blocks and the block pairs.
@pytest.mark.parametrize("heads,kv_heads", [(4, 4), (8, 2), (8, 1)])
def test_runner_prefill_gqa_groups(gpu, heads, kv_heads):
    c = dict(TINY, num_heads=heads, num_kv_heads=kv_heads, max_seq_len=96)
    n = 70
    m = build_tiny(seed=heads * 10 + kv_heads, c=c)
    r = make_runner(m, c)
    L = A.lib()
    s, co = O.precompute_rope(c["max_seq_len"], c["head_dim"], c["rope_base"])
    kv = np.zeros((c["num_layers"], 2, c["num_kv_heads"], c["max_seq_len"], c["head_dim"]), dtype=np.float32)
    toks = np.random.default_rng(heads).integers(0, c["vocab_size"], n).astype(np.int32)
    try:
        logits = np.empty(c["vocab_size"], dtype=np.float32)
        A.check(L.aeth_runner_prefill(r, toks.ctypes.data, n, logits.ctypes.data, None), "prefill")
        ref = O.forward_batch(oracle_cfg(c), m["emb"][toks], m["layers"], [Q4_K] * 7, m["norms"], m["final"], m["lm"],
                              m["lm_dtype"], s, co, kv)
        assert_close_logits(logits, ref, what="prefill heads=%d kv_heads=%d" % (heads, kv_heads))
    finally:
        L.aeth_runner_free(r)


# Files that mix formats inside a layer (llama.cpp's Q4_K_M keeps attn_v and
# ffn_down in Q6_K): q/k/v and gate/up of different formats are run as separate
# weights (three GEMVs into q|k|v, gate and up GEMVs then SiLU·up; strided GEMM
# columns in prefill). n = 150 takes the Q4_K GEMM with the output row stride.
MIXED = [[Q4_K, Q4_K, Q6_K, Q4_K, Q4_K, Q4_K, Q6_K],     # Q4_K_M
         [Q8_0, Q4_K, Q6_K, Q6_K, Q4_K, Q8_0, Q4_K]]     # every split, GEMV and GEMM columns


@pytest.mark.parametrize("mix", [0, 1])
@pytest.mark.parametrize("n", [1, 23, 150])
def test_runner_mixed_formats(gpu, mix, n):
    c = dict(TINY, max_seq_len=192)
    m = build_tiny(seed=11 + mix, layer_dtype=MIXED[mix], c=c)
    r = make_runner(m, c)
    L = A.lib()
    ocfg = oracle_cfg(c)
    s, co = O.precompute_rope(c["max_seq_len"], c["head_dim"], c["rope_base"])
    kv = np.zeros((c["num_layers"], 2, c["num_kv_heads"], c["max_seq_len"], c["head_dim"]), dtype=np.float32)
    toks = np.random.default_rng(n).integers(0, c["vocab_size"], n).astype(np.int32)
    try:
        logits = np.empty(c["vocab_size"], dtype=np.float32)
        A.check(L.aeth_runner_prefill(r, toks.ctypes.data, n, logits.ctypes.data, None), "prefill")
        ref = O.forward_batch(ocfg, m["emb"][toks], m["layers"], MIXED[mix], m["norms"], m["final"], m["lm"],
                              m["lm_dtype"], s, co, kv)
        # anchored on the float64 evaluation: at n = 150 the reference's own f32 logits
        # drift from it by 1.8e-5·max|row| (9.5e-4 on logits below 1)
        seq = list(toks)
        ex = lambda: logits64(c, m["emb"], m["layers"], MIXED[mix], m["norms"], m["final"], m["lm"], m["lm_dtype"], seq)
        assert_close_logits(logits, ref, what="mixed prefill n=%d" % n, exact=ex())
        fill = n
        tok = O.argmax(ref)
        for step in range(2):
            A.check(L.aeth_runner_decode(r, tok, fill, logits.ctypes.data, None), "mixed decode")
            ref, fill = O.decode_step(ocfg, m["emb"][tok], fill, m["layers"], MIXED[mix], m["norms"], m["final"],
                                      m["lm"], m["lm_dtype"], s, co, kv, fill)
            seq.append(tok)
            assert_close_logits(logits, ref, what="mixed decode step %d" % step, exact=ex())
            tok = O.argmax(ref)
        # separately stored weights export as they were given
        for j in range(7):
            blob = np.empty(m["layers"][1][j].nbytes, dtype=np.uint8)
            A.check(L.aeth_runner_export(r, j, 1, blob.ctypes.data, blob.nbytes), "export %d" % j)
            assert np.array_equal(blob, m["layers"][1][j].view(np.uint8).ravel()), "export %d" % j
    finally:
        L.aeth_runner_free(r)


# Layers and LM heads in the formats the reference keeps in GGUF order (F32 /
# F16 / Q2_K / Q3_K: dequantize + matmul_f32_gguf, dispatch.rs:126-133), mixed
# with fused ones: decode steps (eager and replayed as a HIP graph, whose
# GGUF-order GEMVs use the runner's own scratch) and prefill against the oracle.
GGUF_MIX = [[F16, Q2_K, Q3_K, F32, Q5_K, Q2_K, Q3_K], [Q3_K, Q3_K, Q3_K, Q2_K, Q2_K, Q2_K, F16]]


@pytest.mark.parametrize("mix,lm_dtype", [(0, F16), (1, Q6_K)])
def test_runner_gguf_order_formats(gpu, mix, lm_dtype):
    c = dict(TINY, max_seq_len=64)
    m = build_tiny(seed=21 + mix, layer_dtype=GGUF_MIX[mix], lm_dtype=lm_dtype, c=c)
    L = A.lib()
    ocfg = oracle_cfg(c)
    s, co = O.precompute_rope(c["max_seq_len"], c["head_dim"], c["rope_base"])
    n = 19
    toks = np.random.default_rng(mix).integers(0, c["vocab_size"], n).astype(np.int32)
    r = make_runner(m, c)
    try:
        kv = np.zeros((c["num_layers"], 2, c["num_kv_heads"], c["max_seq_len"], c["head_dim"]), dtype=np.float32)
        logits = np.empty(c["vocab_size"], dtype=np.float32)
        A.check(L.aeth_runner_prefill(r, toks.ctypes.data, n, logits.ctypes.data, None), "prefill")
        ref = O.forward_batch(ocfg, m["emb"][toks], m["layers"], GGUF_MIX[mix], m["norms"], m["final"], m["lm"],
                              lm_dtype, s, co, kv)
        seq = list(toks)
        ex = lambda: logits64(c, m["emb"], m["layers"], GGUF_MIX[mix], m["norms"], m["final"], m["lm"], lm_dtype, seq)
        assert_close_logits(logits, ref, what="gguf-order prefill", exact=ex())
        tok, fill = O.argmax(ref), n
        for step in range(2):
            nxt = ctypes.c_int32()
            A.check(L.aeth_runner_decode(r, tok, fill, logits.ctypes.data, ctypes.byref(nxt)), "decode")
            ref, fill = O.decode_step(ocfg, m["emb"][tok], fill, m["layers"], GGUF_MIX[mix], m["norms"], m["final"],
                                      m["lm"], lm_dtype, s, co, kv, fill)
            seq.append(tok)
            assert_close_logits(logits, ref, what="gguf-order decode %d" % step, exact=ex())
            assert nxt.value == O.argmax(logits)
            tok = O.argmax(ref)
    finally:
        L.aeth_runner_free(r)
    outs = []
    for use_graph in (0, 1):
        r = make_runner(m, c)
        t = (ctypes.c_int32 * 8)()
        A.check(L.aeth_runner_generate(r, 1, 0, 8, t, use_graph), "generate")
        outs.append(list(t))
        L.aeth_runner_free(r)
    assert outs[0] == outs[1]


def test_runner_prefill_bad_arguments(gpu):
    m = build_tiny(seed=8)
    r = make_runner(m)
    L = A.lib()
    try:
        toks = np.zeros(TINY["max_seq_len"] + 1, dtype=np.int32)
        assert L.aeth_runner_prefill(r, toks.ctypes.data, 0, None, None) == -1
        assert L.aeth_runner_prefill(r, toks.ctypes.data, TINY["max_seq_len"] + 1, None, None) == -1
        toks[3] = TINY["vocab_size"]
        assert L.aeth_runner_prefill(r, toks.ctypes.data, 5, None, None) == -1
    finally:
        L.aeth_runner_free(r)


def test_runner_generate_graph_matches_eager(gpu):
    m = build_tiny(seed=3)
    L = A.lib()
    outs = []
    for use_graph in (0, 1, 1):
        r = make_runner(m)
        toks = (ctypes.c_int32 * 10)()
        A.check(L.aeth_runner_generate(r, 1, 0, 10, toks, use_graph), "generate")
        if use_graph:  # a second replay batch continues the sequence
            more = (ctypes.c_int32 * 5)()
            A.check(L.aeth_runner_generate(r, toks[9], 10, 5, more, use_graph), "generate 2")
            outs.append(list(toks) + list(more))
        else:
            more = (ctypes.c_int32 * 5)()
            A.check(L.aeth_runner_generate(r, toks[9], 10, 5, more, 0), "generate 2")
            outs.append(list(toks) + list(more))
        L.aeth_runner_free(r)
    assert outs[0] == outs[1] == outs[2]


def test_c_api_surface(gpu):
    """aether_* over a device runner: queries, decode, argmax, budget."""
    L = A.lib()
    m = build_tiny(seed=4)
    r = make_runner(m)
    model = L.aether_model_from_runner(r)
    assert model
    try:
        assert L.aether_vocab_size(model) == TINY["vocab_size"]
        assert L.aether_num_layers(model) == TINY["num_layers"]
        assert L.aether_d_model(model) == TINY["d_model"]
        assert L.aether_context_len(model) == TINY["max_seq_len"]
        logits = np.empty(TINY["vocab_size"], dtype=np.float32)
        toks = (ctypes.c_int * 3)(1, 5, 9)
        assert L.aether_prefill(model, toks, 3, logits.ctypes.data) == 0
        assert L.aeth_runner_seq_len(r) == 3
        t = L.aether_argmax(model, logits.ctypes.data)
        assert t == O.argmax(logits)
        assert L.aether_sample(model, logits.ctypes.data, 0.0, 1.0) == t
        assert L.aether_decode(model, t, 3, logits.ctypes.data) == 0
        # a generous budget completes like aether_decode
        L.aether_set_frame_budget(model, 10000.0)
        assert abs(L.aether_frame_budget(model) - 10000.0) < 1e-3
        assert L.aether_decode_budgeted(model, 2, 4, logits.ctypes.data) == 0
        assert L.aeth_runner_seq_len(r) == 5
        assert L.aether_load(b"/nonexistent.gguf") is None
    finally:
        L.aether_free(model)


def test_decode_budgeted_timeout_and_resume(gpu):
    """aether_decode_budgeted (c_api.rs:324-355 → decode_step_budgeted,
    runner.rs:1201-1282) forced from the host: a budget of 1e-9 ms has expired
    at the first layer check, so the call returns AETHER_TIMEOUT (-2) without
    logits and records completed_layer = 0 (the reference's
    layer_idx.saturating_sub(1) at layer 0); a retry with the same (token, pos)
    resumes at layer 1 with the saved residual stream — i.e. layer 0 is skipped,
    exactly as the reference does — and, given time, completes. The oracle enters
    its decode step at layer 1 with x = the embedding (orc_decode_step_from). A
    retry with another (token, pos) drops the partial state and runs every layer."""
    L = A.lib()
    m = build_tiny(seed=6)
    r = make_runner(m)
    model = L.aether_model_from_runner(r)
    c = TINY
    ocfg = oracle_cfg()
    s, co = O.precompute_rope(c["max_seq_len"], c["head_dim"], c["rope_base"])
    kv = np.zeros((c["num_layers"], 2, c["num_kv_heads"], c["max_seq_len"], c["head_dim"]), dtype=np.float32)
    try:
        toks = np.array([3, 17, 29], np.int32)
        logits = np.full(c["vocab_size"], np.nan, np.float32)
        assert L.aether_prefill(model, toks.ctypes.data, 3, logits.ctypes.data) == 0
        O.forward_batch(ocfg, m["emb"][toks], m["layers"], [Q4_K] * 7, m["norms"], m["final"], m["lm"],
                        m["lm_dtype"], s, co, kv)
        tok = 41
        L.aether_set_frame_budget(model, 1e-9)
        sentinel = np.full(c["vocab_size"], 7.0, np.float32)
        for _ in range(2):  # expires before layer 0, then again right at the resume layer
            assert L.aether_decode_budgeted(model, tok, 3, sentinel.ctypes.data) == -2
            assert (sentinel == 7.0).all()  # no logits written on a timeout
            assert L.aeth_runner_seq_len(r) == 3
        L.aether_set_frame_budget(model, 1e6)
        assert L.aether_decode_budgeted(model, tok, 3, logits.ctypes.data) == 0
        assert L.aeth_runner_seq_len(r) == 4
        ref, fill = O.decode_step(ocfg, m["emb"][tok], 3, m["layers"], [Q4_K] * 7, m["norms"], m["final"], m["lm"],
                                  m["lm_dtype"], s, co, kv, 3, start_layer=1)
        assert fill == 4
        assert_close_logits(logits, ref, what="resumed at layer 1")
        # a timed-out attempt for (tok2, 4), then a different token at pos 4: fresh step
        L.aether_set_frame_budget(model, 1e-9)
        assert L.aether_decode_budgeted(model, 55, 4, sentinel.ctypes.data) == -2
        L.aether_set_frame_budget(model, 1e6)
        assert L.aether_decode_budgeted(model, 56, 4, logits.ctypes.data) == 0
        ref, fill = O.decode_step(ocfg, m["emb"][56], 4, m["layers"], [Q4_K] * 7, m["norms"], m["final"], m["lm"],
                                  m["lm_dtype"], s, co, kv, 4)
        assert_close_logits(logits, ref, what="fresh step after a dropped partial")
        kv_dev = np.empty_like(kv)
        fl = ctypes.c_int32()
        A.check(L.aeth_runner_kv_to_host(r, kv_dev.ctypes.data, ctypes.byref(fl)))
        assert fl.value == 5
        assert_close_rows(kv_dev[:, :, :, :5].reshape(-1, c["head_dim"]), kv[:, :, :, :5].reshape(-1, c["head_dim"]),
                          what="kv after budgeted steps")
        # budget <= 0: the plain decode
        L.aether_set_frame_budget(model, 0.0)
        assert L.aether_decode_budgeted(model, 57, 5, logits.ctypes.data) == 0
        ref, fill = O.decode_step(ocfg, m["emb"][57], 5, m["layers"], [Q4_K] * 7, m["norms"], m["final"], m["lm"],
                                  m["lm_dtype"], s, co, kv, 5)
        assert_close_logits(logits, ref, what="unbudgeted")
    finally:
        L.aether_free(model)


def test_runners_prefill_concurrently(gpu):
    """Two runners prefilling from two host threads at once (each on its own
    stream, with the GEMM's scratch per stream) give exactly their serial
    results; the Q4_K GEMM runs for n = 150."""
    import threading

    L = A.lib()
    c = dict(TINY, max_seq_len=192)
    models = [build_tiny(seed=40 + i, c=c) for i in range(2)]
    toks = [np.random.default_rng(60 + i).integers(0, c["vocab_size"], 150).astype(np.int32) for i in range(2)]

    def prefill(r, t, out):
        A.check(L.aeth_runner_prefill(r, t.ctypes.data, t.size, out.ctypes.data, None), "prefill")

    serial = []
    for i in range(2):
        r = make_runner(models[i], c)
        out = np.empty(c["vocab_size"], np.float32)
        prefill(r, toks[i], out)
        serial.append(out)
        L.aeth_runner_free(r)
    runners = [make_runner(models[i], c) for i in range(2)]
    try:
        for rep in range(3):
            outs = [np.empty(c["vocab_size"], np.float32) for _ in range(2)]
            th = [threading.Thread(target=prefill, args=(runners[i], toks[i], outs[i])) for i in range(2)]
            for t in th:
                t.start()
            for t in th:
                t.join()
            for i in range(2):
                assert np.array_equal(outs[i], serial[i]), "runner %d rep %d" % (i, rep)
    finally:
        for r in runners:
            L.aeth_runner_free(r)
