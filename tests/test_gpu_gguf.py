"""aether_load: a GGUF v3 file → the device runner (gguf.rs:297-397,
model_loader.rs:159-386, c_api.rs:41-102), checked end to end: a small Llama
file with quantized weights in GGUF order ([in, out]) and F32/F16 norms and
embeddings is loaded, then prefill and one decode step are compared with the
oracle run on the tensors the reference's loader would build (load_quant's
dequantize → transpose → requantize, the token-embedding transpose)."""
import ctypes

import numpy as np
import pytest

import aether_amd as A
from oracle import oracle as O
from tests._model64 import logits64
from tests._util import F16, F32, GEOM, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0, assert_close_logits, synth_blocks
from tests.gguf_writer import ARR, F32, STR, U32, write_gguf

pytestmark = pytest.mark.gpu

CFG = dict(vocab_size=512, d_model=256, num_layers=2, num_heads=2, num_kv_heads=1, head_dim=128, d_ff=512,
           max_seq_len=64, rope_base=10000.0, rms_norm_eps=1e-5)


def quant_gguf(dtype, k, n, seed):
    """GGUF bytes of a [k, n] tensor and the QuantWeight bytes load_quant makes of them
    (re-quantized [n][k] rows for Q8_0 / Q4_K / Q5_K / Q6_K, the bytes themselves
    otherwise, model_loader.rs:344-350)."""
    be = GEOM[dtype][0]
    raw = synth_blocks(dtype, (k * n + be - 1) // be, seed).ravel()
    if dtype in (F32, F16, Q2_K, Q3_K):
        return raw, raw
    flat = O.dequant(dtype, raw, k * n)
    return raw, O.requantize(dtype, flat.reshape(k, n).T.ravel(), n, k)


def build_file(path, layer_dtype=Q4_K, lm_dtype=Q6_K, f16_norms=False, context=64, extra_meta=(), drop=None,
               override=None):
    c = CFG
    dts = list(layer_dtype) if isinstance(layer_dtype, (list, tuple)) else [layer_dtype] * 7
    d, dff, v = c["d_model"], c["d_ff"], c["vocab_size"]
    qd, kvd = c["num_heads"] * c["head_dim"], c["num_kv_heads"] * c["head_dim"]
    rng = np.random.default_rng(5)
    tensors, model = [], dict(layers=[], norms=[])
    emb_gguf = rng.standard_normal((d, v)).astype(np.float32)     # read as [d_model][vocab]
    model["emb"] = np.ascontiguousarray(emb_gguf.T)
    tensors.append(("token_embd.weight", [d, v], 0, emb_gguf.view(np.uint8).ravel()))

    def norm(name):
        x = (1 + 0.02 * rng.standard_normal(d)).astype(np.float32)
        if f16_norms:
            h = x.astype(np.float16)
            tensors.append((name, [d], 1, h.view(np.uint8).ravel()))
            return h.astype(np.float32)
        tensors.append((name, [d], 0, x.view(np.uint8).ravel()))
        return x

    names = ["attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"]
    shapes = [(qd, d), (kvd, d), (kvd, d), (d, qd), (dff, d), (dff, d), (d, dff)]   # [out, in]
    for l in range(c["num_layers"]):
        an = norm("blk.%d.attn_norm.weight" % l)
        fn = norm("blk.%d.ffn_norm.weight" % l)
        model["norms"].append([an, fn])
        ws = []
        for j, (n, k) in enumerate(shapes):
            raw, qw = quant_gguf(dts[j], k, n, 1000 + 10 * l + j)
            tensors.append(("blk.%d.%s.weight" % (l, names[j]), [k, n], dts[j], raw))
            ws.append(qw)
        model["layers"].append(ws)
    model["final"] = norm("output_norm.weight")
    raw, model["lm"] = quant_gguf(lm_dtype, d, v, 77)
    tensors.append(("output.weight", [d, v], lm_dtype, raw))
    if drop:
        tensors = [t for t in tensors if t[0] != drop]
    if override:
        tensors = [override if t[0] == override[0] else t for t in tensors]
    meta = [("general.architecture", STR, "llama"),
            ("general.alignment", U32, 32),
            ("llama.embedding_length", U32, d),
            ("llama.block_count", U32, c["num_layers"]),
            ("llama.attention.head_count", U32, c["num_heads"]),
            ("llama.attention.head_count_kv", U32, c["num_kv_heads"]),
            ("llama.feed_forward_length", U32, dff),
            ("llama.context_length", U32, context),
            ("llama.rope.freq_base", F32, c["rope_base"]),
            ("llama.attention.layer_norm_rms_epsilon", F32, c["rms_norm_eps"]),
            ("tokenizer.ggml.tokens", ARR, (STR, ["<unk>", "<s>", "</s>", "a"])),
            ("tokenizer.ggml.bos_token_id", U32, 7),
            ("tokenizer.ggml.eos_token_id", U32, 9)] + list(extra_meta)
    write_gguf(str(path), meta, tensors)
    model["layer_dtype"], model["lm_dtype"] = dts, lm_dtype
    return model


def last_error(L):
    return ctypes.cast(L.aether_last_error(), ctypes.c_char_p).value.decode()


Q4_K_M = [Q4_K, Q4_K, Q6_K, Q4_K, Q4_K, Q4_K, Q6_K]   # llama.cpp's mix: attn_v and ffn_down in Q6_K


Q5_K_M = [Q5_K, Q5_K, Q6_K, Q5_K, Q5_K, Q5_K, Q6_K]


Q3_K_M = [Q3_K, Q3_K, Q5_K, Q4_K, Q3_K, Q3_K, Q5_K]          # llama.cpp's Q3_K_M mix
LOW_BIT = [Q2_K, Q2_K, Q3_K, F16, Q2_K, Q2_K, Q3_K]


@pytest.mark.parametrize("layer_dtype,f16_norms,lm_dtype", [(Q4_K, False, Q6_K), (Q8_0, True, Q6_K),
                                                            (Q6_K, False, Q6_K), (Q4_K_M, False, Q6_K),
                                                            (Q5_K_M, True, Q6_K), (Q3_K_M, False, Q6_K),
                                                            (LOW_BIT, True, F16)])
def test_aether_load_prefill_decode_match_oracle(gpu, tmp_path, layer_dtype, f16_norms, lm_dtype):
    L = A.lib()
    path = tmp_path / "tiny.gguf"
    mdl = build_file(path, layer_dtype=layer_dtype, f16_norms=f16_norms, lm_dtype=lm_dtype)
    m = L.aether_load(str(path).encode())
    assert m, last_error(L)
    try:
        c = CFG
        assert L.aether_vocab_size(m) == c["vocab_size"] and L.aether_d_model(m) == c["d_model"]
        assert L.aether_num_layers(m) == c["num_layers"] and L.aether_context_len(m) == 64
        assert (L.aether_bos_id(m), L.aether_eos_id(m)) == (7, 9)
        ocfg = O.LlamaCfg(c["vocab_size"], c["d_model"], c["num_layers"], c["num_heads"], c["num_kv_heads"],
                          c["head_dim"], c["d_ff"], 64, c["rope_base"], c["rms_norm_eps"])
        s, co = O.precompute_rope(64, c["head_dim"], c["rope_base"])
        kv = np.zeros((c["num_layers"], 2, c["num_kv_heads"], 64, c["head_dim"]), dtype=np.float32)
        toks = np.random.default_rng(3).integers(0, c["vocab_size"], 20).astype(np.int32)
        logits = np.empty(c["vocab_size"], dtype=np.float32)
        assert L.aether_prefill(m, toks.ctypes.data, len(toks), logits.ctypes.data) == 0, last_error(L)
        ref = O.forward_batch(ocfg, mdl["emb"][toks], mdl["layers"], mdl["layer_dtype"], mdl["norms"], mdl["final"],
                              mdl["lm"], mdl["lm_dtype"], s, co, kv)
        ex = lambda seq: logits64(dict(c, max_seq_len=64), mdl["emb"], mdl["layers"], mdl["layer_dtype"], mdl["norms"],
                                  mdl["final"], mdl["lm"], mdl["lm_dtype"], seq)
        assert_close_logits(logits, ref, what="aether_load prefill", exact=ex(list(toks)))
        tok = int(np.argmax(ref))
        assert L.aether_decode(m, tok, len(toks), logits.ctypes.data) == 0, last_error(L)
        ref2, _ = O.decode_step(ocfg, mdl["emb"][tok], len(toks), mdl["layers"], mdl["layer_dtype"], mdl["norms"],
                                mdl["final"], mdl["lm"], mdl["lm_dtype"], s, co, kv, len(toks))
        assert_close_logits(logits, ref2, what="aether_load decode", exact=ex(list(toks) + [tok]))
    finally:
        L.aether_free(m)


def test_aether_load_rejects_bad_files(gpu, tmp_path):
    L = A.lib()
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUX" + b"\0" * 60)
    assert not L.aether_load(str(bad).encode())
    assert "magic" in last_error(L)
    assert not L.aether_load(str(tmp_path / "missing.gguf").encode())
    assert "open" in last_error(L)
    p = tmp_path / "no_v.gguf"
    build_file(p, drop="blk.1.attn_v.weight")
    assert not L.aether_load(str(p).encode())
    assert "blk.1.attn_v.weight" in last_error(L)
    p = tmp_path / "q4_0_weight.gguf"  # Q4_0 (ggml type 2) is not a format of this build
    build_file(p, override=("blk.0.ffn_up.weight", [256, 512], 2, np.zeros(256 * 512 // 32 * 18, dtype=np.uint8)))
    assert not L.aether_load(str(p).encode())
    assert "ffn_up" in last_error(L)
    p = tmp_path / "swa0.gguf"  # a window of 0 would mask every position: refused
    build_file(p, extra_meta=[("llama.attention.sliding_window_length", U32, 0)])
    assert not L.aether_load(str(p).encode())
    assert "sliding_window" in last_error(L)
    p = tmp_path / "long.gguf"
    build_file(p, context=131072)
    m = L.aether_load_streaming(str(p).encode(), 2)
    assert m, last_error(L)
    assert L.aether_context_len(m) == 4096  # min(context_length, 4096), c_api.rs:123-127
    L.aether_free(m)


def test_aether_load_sliding_window_and_context_cap(gpu, tmp_path):
    """A file with attention.sliding_window_length 3 (ArchConfig::sliding_window,
    model_loader.rs:286) and context_length 8192: the runner holds 4096 positions
    (runner.rs:225; aether_context_len 4096), prefill and decode attend over the
    last 3 positions, and a decode at position 5000 takes RoPE row 4095 — each
    against the oracle with the same window and a 4096-row table."""
    L = A.lib()
    path = tmp_path / "swa.gguf"
    mdl = build_file(path, layer_dtype=Q4_K_M, context=8192,
                     extra_meta=[("llama.attention.sliding_window_length", U32, 3)])
    m = L.aether_load(str(path).encode())
    assert m, last_error(L)
    try:
        c = dict(CFG, max_seq_len=4096, sliding_window=3)
        assert L.aether_context_len(m) == 4096
        ocfg = O.LlamaCfg(c["vocab_size"], c["d_model"], c["num_layers"], c["num_heads"], c["num_kv_heads"],
                          c["head_dim"], c["d_ff"], 4096, c["rope_base"], c["rms_norm_eps"], 3)
        s, co = O.precompute_rope(4096, c["head_dim"], c["rope_base"])
        kv = np.zeros((c["num_layers"], 2, c["num_kv_heads"], 4096, c["head_dim"]), dtype=np.float32)
        toks = np.random.default_rng(8).integers(0, c["vocab_size"], 20).astype(np.int32)
        logits = np.empty(c["vocab_size"], dtype=np.float32)
        assert L.aether_prefill(m, toks.ctypes.data, len(toks), logits.ctypes.data) == 0, last_error(L)
        ref = O.forward_batch(ocfg, mdl["emb"][toks], mdl["layers"], mdl["layer_dtype"], mdl["norms"], mdl["final"],
                              mdl["lm"], mdl["lm_dtype"], s, co, kv)
        ex = logits64(c, mdl["emb"], mdl["layers"], mdl["layer_dtype"], mdl["norms"], mdl["final"], mdl["lm"],
                      mdl["lm_dtype"], list(toks))
        assert_close_logits(logits, ref, what="windowed aether_load prefill", exact=ex)
        unwindowed = O.forward_batch(O.LlamaCfg(*[getattr(ocfg, f) for f, _ in ocfg._fields_[:-1]]), mdl["emb"][toks],
                                     mdl["layers"], mdl["layer_dtype"], mdl["norms"], mdl["final"], mdl["lm"],
                                     mdl["lm_dtype"], s, co, np.zeros_like(kv))
        assert np.abs(unwindowed - ref).max() > 1e-2 * np.abs(ref).max()  # the window matters here
        tok = int(np.argmax(ref))
        assert L.aether_decode(m, tok, 5000, logits.ctypes.data) == 0, last_error(L)
        ref2, fill = O.decode_step(ocfg, mdl["emb"][tok], 5000, mdl["layers"], mdl["layer_dtype"], mdl["norms"],
                                   mdl["final"], mdl["lm"], mdl["lm_dtype"], s, co, kv, len(toks))
        assert fill == 21
        assert_close_logits(logits, ref2, what="windowed decode at position 5000")
    finally:
        L.aether_free(m)


def test_aether_load_greedy_generation_is_deterministic(gpu, tmp_path):
    """The reference's end-to-end determinism property (tests/e2e.rs:220-250): a
    GGUF file loaded, prompted and decoded greedily for 16 tokens, then freed and
    loaded again, gives the same tokens. Here the logits of every step must also
    be bit-identical between the two loads, and each step's logits are checked
    against the oracle's decode step fed the same tokens (teacher-forced on the
    device's own greedy path, runner.rs:1557-1646, sample :1964-1973)."""
    L = A.lib()
    c = CFG
    path = tmp_path / "e2e.gguf"
    mdl = build_file(path, layer_dtype=Q4_K_M, lm_dtype=Q6_K)
    prompt = np.random.default_rng(11).integers(0, c["vocab_size"], 6).astype(np.int32)
    n_gen = 16

    def run():
        m = L.aether_load(str(path).encode())
        assert m, last_error(L)
        toks, rows = [], []
        try:
            logits = np.empty(c["vocab_size"], dtype=np.float32)
            assert L.aether_prefill(m, prompt.ctypes.data, len(prompt), logits.ctypes.data) == 0, last_error(L)
            rows.append(logits.copy())
            for i in range(n_gen):
                tok = L.aether_argmax(m, logits.ctypes.data)
                assert 0 <= tok < c["vocab_size"]
                toks.append(tok)
                if i + 1 < n_gen:
                    assert L.aether_decode(m, tok, len(prompt) + i, logits.ctypes.data) == 0, last_error(L)
                    rows.append(logits.copy())
        finally:
            L.aether_free(m)
        return toks, rows

    toks1, rows1 = run()
    toks2, rows2 = run()
    assert toks1 == toks2, "greedy generation differs between two loads of the same file"
    for i, (a, b) in enumerate(zip(rows1, rows2)):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), "step %d logits differ between loads" % i

    # every step against the oracle, on the device's tokens
    ocfg = O.LlamaCfg(c["vocab_size"], c["d_model"], c["num_layers"], c["num_heads"], c["num_kv_heads"],
                      c["head_dim"], c["d_ff"], 64, c["rope_base"], c["rms_norm_eps"])
    s, co = O.precompute_rope(64, c["head_dim"], c["rope_base"])
    kv = np.zeros((c["num_layers"], 2, c["num_kv_heads"], 64, c["head_dim"]), dtype=np.float32)
    ref = O.forward_batch(ocfg, mdl["emb"][prompt], mdl["layers"], mdl["layer_dtype"], mdl["norms"], mdl["final"],
                          mdl["lm"], mdl["lm_dtype"], s, co, kv)
    seq = list(prompt)
    ex = lambda sq: logits64(dict(c, max_seq_len=64), mdl["emb"], mdl["layers"], mdl["layer_dtype"], mdl["norms"],
                             mdl["final"], mdl["lm"], mdl["lm_dtype"], sq)
    assert_close_logits(rows1[0], ref, what="e2e prefill", exact=ex(seq))
    fill = len(prompt)
    for i in range(1, n_gen):
        tok = toks1[i - 1]
        ref, fill = O.decode_step(ocfg, mdl["emb"][tok], len(prompt) + i - 1, mdl["layers"], mdl["layer_dtype"],
                                  mdl["norms"], mdl["final"], mdl["lm"], mdl["lm_dtype"], s, co, kv, fill)
        seq.append(tok)
        assert_close_logits(rows1[i], ref, what="e2e decode step %d" % i, exact=ex(seq))
    # aether_argmax keeps the last maximal index on ties (Iterator::max_by, c_api.rs:384-396)
    for i, row in enumerate(rows1):
        assert toks1[i] == len(row) - 1 - int(np.argmax(row[::-1])), "step %d: argmax" % i
