"""Context semantics of the device runner against the oracle:
  * sliding-window attention (ArchConfig::sliding_window): attn_direct masks the
    positions before seq - w in decode (runner.rs:1768-1777) and
    attention_batch the keys before i - w + 1 in prefill (:1825-1845);
  * the cache length: LlamaRunner::new / new_streaming hold
    min(max_seq_len, 4096) positions (runner.rs:225, :339) — RoPE rows past
    4095 clamp to the last one (apply_rope_inplace, :1895-1896) and a step
    into a full cache is refused (kv_cache.rs:40-44; the reference's decode
    then indexes past its scores and panics)."""
import ctypes

import numpy as np
import pytest

import aether_amd as A
from oracle import oracle as O
from tests._model64 import logits64
from tests._models import TINY, build_tiny, oracle_cfg
from tests._util import Q4_K, Q8_0, assert_close_logits, assert_close_rows
from tests.test_gpu_decode import make_runner

pytestmark = pytest.mark.gpu


# (query heads, KV heads, window, prompt length, cache length): G = 2, 8, 1 take the
# f32-MFMA prefill attention, G = 3 the VALU one; windows shorter than a 16-key block,
# spanning several, and longer than the prompt; n = 150 and 130 run the GEMM
# projections and make the decode steps skip a whole 128-position chunk (window start
# 131 → chunk 0 left out, chunk 1 partly masked; window 64 at seq 131 → start 67, chunk
# 0 partly masked). The random test models attend sharply (a query's weights past a few keys often
# underflow to 0), so the windows are chosen where masking changes the oracle's
# logits, which the test checks.
CASES = [(4, 2, 4, 37, 64), (4, 2, 20, 150, 192), (8, 1, 33, 70, 96), (4, 4, 6, 45, 64), (6, 2, 9, 70, 96),
         (4, 2, 100, 37, 128), (8, 2, 64, 130, 192)]


@pytest.mark.parametrize("heads,kv_heads,window,n,max_seq", CASES)
def test_runner_sliding_window_matches_oracle(gpu, heads, kv_heads, window, n, max_seq):
    c = dict(TINY, num_heads=heads, num_kv_heads=kv_heads, max_seq_len=max_seq, sliding_window=window)
    dts = [Q4_K, Q4_K, Q8_0, Q4_K, Q4_K, Q4_K, Q4_K]
    m = build_tiny(seed=heads * 7 + window, layer_dtype=dts, c=c)
    r = make_runner(m, c)
    L = A.lib()
    ocfg = oracle_cfg(c)
    s, co = O.precompute_rope(max_seq, c["head_dim"], c["rope_base"])
    kv = np.zeros((c["num_layers"], 2, kv_heads, max_seq, c["head_dim"]), np.float32)
    toks = np.random.default_rng(n + window).integers(0, c["vocab_size"], n).astype(np.int32)
    print("sliding window %d: heads %d / %d, prefill %d tokens" % (window, heads, kv_heads, n), flush=True)
    try:
        logits = np.empty(c["vocab_size"], np.float32)
        A.check(L.aeth_runner_prefill(r, toks.ctypes.data, n, logits.ctypes.data, None), "prefill")
        ref = O.forward_batch(ocfg, m["emb"][toks], m["layers"], dts, m["norms"], m["final"], m["lm"], m["lm_dtype"],
                              s, co, kv)
        seq = list(toks)
        ex = lambda: logits64(c, m["emb"], m["layers"], dts, m["norms"], m["final"], m["lm"], m["lm_dtype"], seq)
        assert_close_logits(logits, ref, what="windowed prefill", exact=ex())
        if window < n:  # the window matters for this model and prompt
            ref0 = O.forward_batch(oracle_cfg(dict(c, sliding_window=0)), m["emb"][toks], m["layers"], dts, m["norms"],
                                   m["final"], m["lm"], m["lm_dtype"], s, co, np.zeros_like(kv))
            assert np.abs(ref0 - ref).max() > 1e-3 * np.abs(ref).max()
        kv_dev = np.empty_like(kv)
        fl = ctypes.c_int32()
        A.check(L.aeth_runner_kv_to_host(r, kv_dev.ctypes.data, ctypes.byref(fl)), "kv_to_host")
        assert fl.value == n
        assert_close_rows(kv_dev[:, :, :, :n].reshape(-1, c["head_dim"]), kv[:, :, :, :n].reshape(-1, c["head_dim"]),
                          what="kv after the windowed prefill")
        tok, fill = O.argmax(ref), n
        for step in range(3):
            nxt = ctypes.c_int32()
            A.check(L.aeth_runner_decode(r, tok, fill, logits.ctypes.data, ctypes.byref(nxt)), "decode")
            ref, fill = O.decode_step(ocfg, m["emb"][tok], fill, m["layers"], dts, m["norms"], m["final"], m["lm"],
                                      m["lm_dtype"], s, co, kv, fill)
            seq.append(tok)
            assert_close_logits(logits, ref, what="windowed decode %d" % step, exact=ex())
            assert nxt.value == O.argmax(logits)
            tok = O.argmax(ref)
    finally:
        L.aeth_runner_free(r)
    # the captured step (HIP graph) windows as the eager one does
    outs = []
    for use_graph in (0, 1):
        r = make_runner(m, c)
        try:
            A.check(L.aeth_runner_prefill(r, toks.ctypes.data, n, None, None), "prefill")
            t = (ctypes.c_int32 * 6)()
            A.check(L.aeth_runner_generate(r, int(toks[-1]), n, 6, t, use_graph), "generate")
            outs.append(list(t))
        finally:
            L.aeth_runner_free(r)
    assert outs[0] == outs[1]


def test_window_reaching_past_the_prompt_changes_nothing(gpu):
    """A window at least the sequence length masks no key: logits equal the
    unwindowed runner's bit for bit (prefill and a decode step)."""
    L = A.lib()
    c0 = dict(TINY, max_seq_len=96)
    n = 40
    toks = np.random.default_rng(4).integers(0, c0["vocab_size"], n).astype(np.int32)
    outs = []
    for w in (0, 41, 1000):
        c = dict(c0, sliding_window=w)
        m = build_tiny(seed=3, c=c)
        r = make_runner(m, c)
        try:
            a = np.empty(c["vocab_size"], np.float32)
            b = np.empty(c["vocab_size"], np.float32)
            A.check(L.aeth_runner_prefill(r, toks.ctypes.data, n, a.ctypes.data, None), "prefill")
            A.check(L.aeth_runner_decode(r, 7, n, b.ctypes.data, None), "decode")
            outs.append((a, b))
        finally:
            L.aeth_runner_free(r)
    for a, b in outs[1:]:
        assert np.array_equal(a, outs[0][0]) and np.array_equal(b, outs[0][1])


def _random_cache(c, fill, seed):
    kv = np.zeros((c["num_layers"], 2, c["num_kv_heads"], c["max_seq_len"], c["head_dim"]), np.float32)
    kv[:, :, :, :fill] = np.random.default_rng(seed).standard_normal(kv[:, :, :, :fill].shape)
    return kv


def test_cache_holds_4096_positions_and_rope_clamps(gpu):
    """max_seq_len 8192 without the opt-in: the cache and the RoPE table hold
    4096 positions (aether_context_len = 4096, the table equals the oracle's of
    4096 rows); with 4094 positions filled, steps at positions 4096 and 4097 use
    RoPE row 4095 and fill slots 4094 and 4095 — logits and K/V against the
    oracle's decode step at those positions — and the next step is refused, as
    the oracle refuses a full cache."""
    L = A.lib()
    c = dict(TINY, max_seq_len=8192)
    m = build_tiny(seed=13, c=c)
    r = make_runner(m, c)
    model = L.aether_model_from_runner(r)
    assert model
    ce = dict(c, max_seq_len=4096)  # what the runner holds
    try:
        assert L.aether_context_len(model) == 4096
        s, co = O.precompute_rope(4096, c["head_dim"], c["rope_base"])
        tab = np.empty(s.size, np.float32)
        A.check(L.aeth_runner_export(r, 12, 0, tab.ctypes.data, tab.nbytes), "export rope")
        assert np.array_equal(tab, s)
        kv = _random_cache(ce, 4094, 77)
        A.check(L.aeth_runner_kv_from_host(r, kv.ctypes.data, 4094), "kv_from_host")
        ocfg = oracle_cfg(ce)
        logits = np.empty(c["vocab_size"], np.float32)
        tok, fill = 5, 4094
        for pos in (4096, 4097):
            print("decode at position %d, cache fill %d" % (pos, fill), flush=True)
            assert L.aether_decode(model, tok, pos, logits.ctypes.data) == 0
            ref, fill = O.decode_step(ocfg, m["emb"][tok], pos, m["layers"], m["layer_dtype"], m["norms"], m["final"],
                                      m["lm"], m["lm_dtype"], s, co, kv, fill)
            assert_close_logits(logits, ref, what="decode at %d" % pos)
            tok = O.argmax(ref)
        assert fill == 4096 and L.aeth_runner_seq_len(r) == 4096
        kv_dev = np.empty_like(kv)
        fl = ctypes.c_int32()
        A.check(L.aeth_runner_kv_to_host(r, kv_dev.ctypes.data, ctypes.byref(fl)), "kv_to_host")
        assert fl.value == 4096
        assert_close_rows(kv_dev[:, :, :, 4094:].reshape(-1, c["head_dim"]), kv[:, :, :, 4094:].reshape(-1, c["head_dim"]),
                          what="slots 4094 and 4095")
        assert np.array_equal(kv_dev[:, :, :, :4094], kv[:, :, :, :4094])
        assert L.aether_decode(model, tok, 4098, logits.ctypes.data) == -1  # full cache: refused
        with pytest.raises(RuntimeError):
            O.decode_step(ocfg, m["emb"][tok], 4098, m["layers"], m["layer_dtype"], m["norms"], m["final"], m["lm"],
                          m["lm_dtype"], s, co, kv, fill)
        toks = np.zeros(4097, np.int32)
        assert L.aether_prefill(model, toks.ctypes.data, 4097, logits.ctypes.data) == -1  # past the cache
    finally:
        L.aether_free(model)


def test_full_context_opt_in(gpu):
    """AETH_CFG_FULL_CONTEXT keeps max_seq_len (8192 here): a step at position
    5000 over a 5000-position cache matches the oracle with the 8192-row table."""
    L = A.lib()
    c = dict(TINY, max_seq_len=8192, flags=A.CFG_FULL_CONTEXT)
    m = build_tiny(seed=14, c=c)
    r = make_runner(m, c)
    model = L.aether_model_from_runner(r)
    try:
        assert L.aether_context_len(model) == 8192
        kv = _random_cache(c, 5000, 78)
        A.check(L.aeth_runner_kv_from_host(r, kv.ctypes.data, 5000), "kv_from_host")
        s, co = O.precompute_rope(8192, c["head_dim"], c["rope_base"])
        logits = np.empty(c["vocab_size"], np.float32)
        assert L.aether_decode(model, 9, 5000, logits.ctypes.data) == 0
        ref, fill = O.decode_step(oracle_cfg(c), m["emb"][9], 5000, m["layers"], m["layer_dtype"], m["norms"],
                                  m["final"], m["lm"], m["lm_dtype"], s, co, kv, 5000)
        assert fill == 5001 and L.aeth_runner_seq_len(r) == 5001
        assert_close_logits(logits, ref, what="decode at 5000")
    finally:
        L.aether_free(model)
    cfg = A.LlamaConfig(**dict(TINY, max_seq_len=8193, flags=A.CFG_FULL_CONTEXT))
    rr = ctypes.c_void_p()
    assert L.aeth_runner_create(ctypes.byref(cfg), None, (ctypes.c_int32 * 14)(*([Q4_K] * 14)), None, None, None, 14,
                                None, 1, ctypes.byref(rr)) != 0  # past the decode attention's 8192
    cfg = A.LlamaConfig(**dict(TINY, sliding_window=-1))
    assert L.aeth_runner_create(ctypes.byref(cfg), None, (ctypes.c_int32 * 14)(*([Q4_K] * 14)), None, None, None, 14,
                                None, 1, ctypes.byref(rr)) != 0
