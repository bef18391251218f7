"""The decode step at the LLaMA-8B widths of BASELINE config 4 (d 4096, 32/8
heads of 128, d_ff 14336, vocab 128256, RoPE θ 500000, KV prefilled to 2048
positions) — the shapes where the fused kernels of the benchmark run:
  * the 6144-row q|k|v GEMV with the attention RMSNorm fused,
  * the 28672-row interleaved gate|up GEMV with RMSNorm and SwiGLU fused,
  * the k = 14336 down GEMV accumulating into the residual,
  * the 128256-row Q6_K LM head on the refilling ring with the final RMSNorm
    and the 64-bit atomicMax greedy argmax fused.
A 2-layer model of those widths is built on the device from a seed, exported
through aeth_runner_export and run teacher-forced against the oracle's decode
step (runner.rs:1557-1646); the full 32-layer model is run teacher-forced
against the oracle for two steps and checked by properties (graph replay =
eager, finite logits, fused argmax = host argmax)."""
import ctypes

import numpy as np
import pytest

import aether_amd as A
from oracle import oracle as O
from tests._util import Q4_K, Q6_K, assert_close_logits, assert_close_rows

pytestmark = pytest.mark.gpu

C8B = dict(vocab_size=128256, d_model=4096, num_layers=2, num_heads=32, num_kv_heads=8, head_dim=128, d_ff=14336,
           max_seq_len=4096, rope_base=500000.0, rms_norm_eps=1e-5)
PREFILLED = 2048


def synthetic_runner(c, seed):
    cfg = A.LlamaConfig(**c)
    nl = c["num_layers"]
    dt = (ctypes.c_int32 * (nl * 7))(*([Q4_K] * (nl * 7)))
    r = ctypes.c_void_p()
    A.check(A.lib().aeth_runner_create(ctypes.byref(cfg), None, dt, None, None, None, Q6_K, None, seed,
                                       ctypes.byref(r)), "runner_create")
    return r


def export(r, which, l, nbytes, dtype=np.uint8):
    buf = np.empty(nbytes // np.dtype(dtype).itemsize, dtype=dtype)
    A.check(A.lib().aeth_runner_export(r, which, l, buf.ctypes.data, nbytes), "export %d/%d" % (which, l))
    return buf


def test_decode_8b_widths_match_oracle(gpu):
    c = C8B
    L = A.lib()
    d, dff, kvd, V = c["d_model"], c["d_ff"], c["num_kv_heads"] * c["head_dim"], c["vocab_size"]
    r = synthetic_runner(c, 0x8B8B8B)
    try:
        A.check(L.aeth_runner_fill_kv(r, 0x4B56, PREFILLED), "fill_kv")
        rowb = lambda k: (k // 256) * 144
        sizes = [d * rowb(d), kvd * rowb(d), kvd * rowb(d), d * rowb(d), dff * rowb(d), dff * rowb(d), d * rowb(dff)]
        layers = [[export(r, j, l, sizes[j]) for j in range(7)] for l in range(c["num_layers"])]
        norms = [[export(r, 7 + j, l, d * 4, np.float32) for j in range(2)] for l in range(c["num_layers"])]
        final = export(r, 9, 0, d * 4, np.float32)
        lm = export(r, 10, 0, V * 16 * 210)
        kv = np.empty((c["num_layers"], 2, c["num_kv_heads"], c["max_seq_len"], c["head_dim"]), np.float32)
        fl = ctypes.c_int32()
        A.check(L.aeth_runner_kv_to_host(r, kv.ctypes.data, ctypes.byref(fl)), "kv_to_host")
        assert fl.value == PREFILLED
        s, co = O.precompute_rope(c["max_seq_len"], c["head_dim"], c["rope_base"])
        assert np.array_equal(export(r, 12, 0, s.nbytes, np.float32), s)  # the runner's RoPE table is the oracle's
        ocfg = O.LlamaCfg(V, d, c["num_layers"], c["num_heads"], c["num_kv_heads"], c["head_dim"], dff,
                          c["max_seq_len"], c["rope_base"], c["rms_norm_eps"])
        tok, fill = 1, PREFILLED
        logits = np.empty(V, np.float32)
        for step in range(3):
            print("8B-width decode step %d (token %d, pos %d)" % (step, tok, fill), flush=True)
            nxt = ctypes.c_int32()
            A.check(L.aeth_runner_decode(r, tok, fill, logits.ctypes.data, ctypes.byref(nxt)), "decode")
            emb = export(r, 11, tok, d * 4, np.float32)
            ref, fill = O.decode_step(ocfg, emb, fill, layers, [Q4_K] * 7, norms, final, lm, Q6_K, s, co, kv, fill)
            assert np.isfinite(logits).all()
            assert_close_logits(logits, ref, what="8B-width step %d" % step)
            assert nxt.value == O.argmax(logits), (nxt.value, O.argmax(logits))  # fused argmax = host argmax
            tok = O.argmax(ref)
        kv_dev = np.empty_like(kv)
        A.check(L.aeth_runner_kv_to_host(r, kv_dev.ctypes.data, ctypes.byref(fl)), "kv_to_host")
        assert fl.value == PREFILLED + 3
        new = slice(PREFILLED, PREFILLED + 3)
        assert_close_rows(kv_dev[:, :, :, new].reshape(-1, c["head_dim"]), kv[:, :, :, new].reshape(-1, c["head_dim"]),
                          what="kv slots written by the steps")
        assert np.array_equal(kv_dev[:, :, :, :PREFILLED], kv[:, :, :, :PREFILLED])
    finally:
        L.aeth_runner_free(r)


# Prefill widths: the Q4_K GEMMs' activation prep holds each wave's share of a row's ⌈k/512⌉ steps
# (4 waves per row) in registers, rounded up to 1, 2, 4 or 8 steps, and instantiates the RMSNorm
# producer at k = d_model and the SwiGLU producer at k = d_ff for each. (overrides of C8B, steps per
# wave for RMSNorm / SwiGLU)
WIDTHS = {
    "8b": (dict(), "2 / 8"),
    "d6144_ff8192": (dict(vocab_size=4096, d_model=6144, num_layers=1, num_heads=48, num_kv_heads=12, d_ff=8192),
                     "4 / 4"),
    "d9216_ff3072": (dict(vocab_size=4096, d_model=9216, num_layers=1, num_heads=72, num_kv_heads=9, d_ff=3072),
                     "8 (18 steps: 5 5 4 4) / 2"),
    # the gate|up GEMM's 2 × 260 = 520 tiles leave a last round of 8, split in two over K, under the SwiGLU
    # epilogue (k_gemm_tail_sum writes h); the down GEMM's plain prep reads k = 16640 in two register chunks
    "d4096_ff16640": (dict(vocab_size=4096, d_model=4096, num_layers=1, num_heads=32, num_kv_heads=8, d_ff=16640),
                      "2 / plain, 33 steps (8 8 8 9) in two chunks"),
    "d2048_ff5632": (dict(vocab_size=4096, d_model=2048, num_layers=1, num_heads=16, num_kv_heads=4, d_ff=5632),
                     "1 / 4 (11 steps: 2 3 3 3)"),
}


@pytest.mark.parametrize("width", list(WIDTHS))
def test_prefill_8b_widths_match_oracle(gpu, width):
    """Batched prefill (forward_batch, runner.rs:833-993) of 70 tokens: the
    Q4_K GEMMs with the RMSNorm (q|k|v, gate|up at k = d_model) and the
    SwiGLU (down, k = d_ff) run inside their activation prep; 70 rows leave
    58 rows of the last 64-row tile empty. The 8B widths and four others
    that reach the prep's other register shares (and, at d_ff 16640, the
    gate|up GEMM's last-round K split under its SwiGLU epilogue)."""
    c = dict(C8B, max_seq_len=256, **WIDTHS[width][0])
    L = A.lib()
    d, dff, V = c["d_model"], c["d_ff"], c["vocab_size"]
    qd, kvd = c["num_heads"] * c["head_dim"], c["num_kv_heads"] * c["head_dim"]
    n = 70
    r = synthetic_runner(c, 0x8B8B8C)
    try:
        rowb = lambda k: (k // 256) * 144
        sizes = [qd * rowb(d), kvd * rowb(d), kvd * rowb(d), d * rowb(qd), dff * rowb(d), dff * rowb(d), d * rowb(dff)]
        layers = [[export(r, j, l, sizes[j]) for j in range(7)] for l in range(c["num_layers"])]
        norms = [[export(r, 7 + j, l, d * 4, np.float32) for j in range(2)] for l in range(c["num_layers"])]
        final = export(r, 9, 0, d * 4, np.float32)
        lm = export(r, 10, 0, V * (d // 256) * 210)
        toks = np.random.default_rng(n).integers(0, V, n).astype(np.int32)
        emb = np.stack([export(r, 11, int(t), d * 4, np.float32) for t in toks])
        s, co = O.precompute_rope(c["max_seq_len"], c["head_dim"], c["rope_base"])
        ocfg = O.LlamaCfg(V, d, c["num_layers"], c["num_heads"], c["num_kv_heads"], c["head_dim"], dff,
                          c["max_seq_len"], c["rope_base"], c["rms_norm_eps"])
        print("prefill of %d tokens, %s (prep steps per wave %s)" % (n, width, WIDTHS[width][1]), flush=True)
        logits = np.empty(V, np.float32)
        nxt = ctypes.c_int32()
        A.check(L.aeth_runner_prefill(r, toks.ctypes.data, n, logits.ctypes.data, ctypes.byref(nxt)), "prefill")
        kv = np.zeros((c["num_layers"], 2, c["num_kv_heads"], c["max_seq_len"], c["head_dim"]), np.float32)
        ref = O.forward_batch(ocfg, emb, layers, [Q4_K] * 7, norms, final, lm, Q6_K, s, co, kv)
        assert np.isfinite(logits).all()
        assert_close_logits(logits, ref, what="%s prefill" % width)
        assert nxt.value == O.argmax(logits)
        kv_dev = np.empty_like(kv)
        fl = ctypes.c_int32()
        A.check(L.aeth_runner_kv_to_host(r, kv_dev.ctypes.data, ctypes.byref(fl)), "kv_to_host")
        assert fl.value == n
        assert_close_rows(kv_dev[:, :, :, :n].reshape(-1, c["head_dim"]), kv[:, :, :, :n].reshape(-1, c["head_dim"]),
                          what="kv after the %s prefill" % width)
    finally:
        L.aeth_runner_free(r)


def test_decode_8b_full_depth_matches_oracle(gpu):
    """BASELINE config 4 itself: all 32 layers, KV prefilled to 2048 positions,
    two teacher-forced steps against the oracle's decode step
    (forward_one_internal, runner.rs:1557-1646) — logits (element-wise bar and
    cosine > 0.9999), the fused greedy argmax, and the K/V slots the steps write.
    About 4 s of single-thread CPU per oracle step."""
    c = dict(C8B, num_layers=32)
    L = A.lib()
    d, dff, kvd, V = c["d_model"], c["d_ff"], c["num_kv_heads"] * c["head_dim"], c["vocab_size"]
    r = synthetic_runner(c, 0x8B8B8B)
    try:
        A.check(L.aeth_runner_fill_kv(r, 0x4B56, PREFILLED), "fill_kv")
        rowb = lambda k: (k // 256) * 144
        sizes = [d * rowb(d), kvd * rowb(d), kvd * rowb(d), d * rowb(d), dff * rowb(d), dff * rowb(d), d * rowb(dff)]
        layers = [[export(r, j, l, sizes[j]) for j in range(7)] for l in range(c["num_layers"])]
        norms = [[export(r, 7 + j, l, d * 4, np.float32) for j in range(2)] for l in range(c["num_layers"])]
        final = export(r, 9, 0, d * 4, np.float32)
        lm = export(r, 10, 0, V * 16 * 210)
        kv = np.empty((c["num_layers"], 2, c["num_kv_heads"], c["max_seq_len"], c["head_dim"]), np.float32)
        fl = ctypes.c_int32()
        A.check(L.aeth_runner_kv_to_host(r, kv.ctypes.data, ctypes.byref(fl)), "kv_to_host")
        assert fl.value == PREFILLED
        s, co = O.precompute_rope(c["max_seq_len"], c["head_dim"], c["rope_base"])
        ocfg = O.LlamaCfg(V, d, c["num_layers"], c["num_heads"], c["num_kv_heads"], c["head_dim"], dff,
                          c["max_seq_len"], c["rope_base"], c["rms_norm_eps"])
        tok, fill = 1, PREFILLED
        logits = np.empty(V, np.float32)
        for step in range(2):
            print("32-layer decode step %d (token %d, pos %d)" % (step, tok, fill), flush=True)
            nxt = ctypes.c_int32()
            A.check(L.aeth_runner_decode(r, tok, fill, logits.ctypes.data, ctypes.byref(nxt)), "decode")
            emb = export(r, 11, tok, d * 4, np.float32)
            ref, fill = O.decode_step(ocfg, emb, fill, layers, [Q4_K] * 7, norms, final, lm, Q6_K, s, co, kv, fill)
            print("  oracle step done; logits span %.1f" % np.abs(ref).max(), flush=True)
            assert_close_logits(logits, ref, what="32-layer step %d" % step)
            assert nxt.value == O.argmax(logits), (nxt.value, O.argmax(logits))
            tok = O.argmax(ref)
        kv_dev = np.empty_like(kv)
        A.check(L.aeth_runner_kv_to_host(r, kv_dev.ctypes.data, ctypes.byref(fl)), "kv_to_host")
        assert fl.value == PREFILLED + 2
        new = slice(PREFILLED, PREFILLED + 2)
        assert_close_rows(kv_dev[:, :, :, new].reshape(-1, c["head_dim"]), kv[:, :, :, new].reshape(-1, c["head_dim"]),
                          what="kv slots written by the 32-layer steps")
        assert np.array_equal(kv_dev[:, :, :, :PREFILLED], kv[:, :, :, :PREFILLED])
    finally:
        L.aeth_runner_free(r)


def test_decode_8b_full_depth_graph_equals_eager(gpu):
    """32 layers: eager steps (logits back each step) and the captured HIP graph
    (greedy on the device) give the same tokens; logits are finite and the
    fused LM-head argmax is the host argmax of the logits returned."""
    c = dict(C8B, num_layers=32)
    L = A.lib()
    r = synthetic_runner(c, 0x8B8B8B)
    n = 8
    try:
        A.check(L.aeth_runner_fill_kv(r, 0x4B56, PREFILLED), "fill_kv")
        eager = []
        tok = 1
        logits = np.empty(c["vocab_size"], np.float32)
        for step in range(n):
            nxt = ctypes.c_int32()
            A.check(L.aeth_runner_decode(r, tok, PREFILLED + step, logits.ctypes.data, ctypes.byref(nxt)), "decode")
            assert np.isfinite(logits).all(), step
            assert nxt.value == O.argmax(logits), step
            eager.append(nxt.value)
            tok = nxt.value
        print("32-layer eager tokens", eager, flush=True)
        for rep in range(2):
            A.check(L.aeth_runner_fill_kv(r, 0x4B56, PREFILLED), "fill_kv")
            toks = (ctypes.c_int32 * n)()
            A.check(L.aeth_runner_generate(r, 1, PREFILLED, n, toks, 1), "generate (graph)")
            assert list(toks) == eager, (rep, list(toks), eager)
            assert L.aeth_runner_seq_len(r) == PREFILLED + n
    finally:
        L.aeth_runner_free(r)
