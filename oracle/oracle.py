"""ctypes front-end for the CPU oracle (liboracle.so built from oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker. The product path
(aether_amd) never imports this module.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

F32, F16, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 0, 1, 8, 10, 11, 12, 13, 14
BLOCK_ELEMS = {F32: 1, F16: 1, Q8_0: 32, Q2_K: 256, Q3_K: 256, Q4_K: 256, Q5_K: 256, Q6_K: 256}
BLOCK_BYTES = {F32: 4, F16: 2, Q8_0: 34, Q2_K: 84, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210}
_SOURCES = ("oracle.c", "oracle_formats.c", "oracle_backend.c", "oracle.h", "Makefile")


def build(force=False):
    """Compile liboracle.so with the committed Makefile (gcc)."""
    if force or not os.path.exists(_LIB_PATH) or (
        os.path.getmtime(_LIB_PATH) < max(os.path.getmtime(os.path.join(_HERE, f)) for f in _SOURCES)
    ):
        subprocess.check_call(["make", "-s", "-B" if force else "-s", "-C", _HERE])
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        f32p = ctypes.POINTER(ctypes.c_float)
        u8p = ctypes.POINTER(ctypes.c_uint8)
        sz = ctypes.c_size_t
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_decode_d.restype = ctypes.c_float
        L.orc_decode_d.argtypes = [ctypes.c_uint16]
        L.orc_argmax.restype = ctypes.c_int32
        L.orc_argmax.argtypes = [f32p, sz]
        L.orc_decode_step.restype = ctypes.c_int
        L.orc_decode_step_from.restype = ctypes.c_int
        L.orc_causal_attention.restype = ctypes.c_int
        L.orc_forward_batch.restype = ctypes.c_int
        _lib = L
    return _lib


def _p(a, ct):
    return a.ctypes.data_as(ctypes.POINTER(ct))


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a):
    return np.ascontiguousarray(a, dtype=np.uint8)


# ── scalars ──────────────────────────────────────────────────────────────

def f16_to_f32(bits):
    return lib().orc_f16_to_f32(int(bits))


def f32_to_f16(x):
    return lib().orc_f32_to_f16(float(x))


def decode_d(bits):
    return lib().orc_decode_d(int(bits))


def get_scale_min_k4(j, scales):
    s = _u8(scales)
    sc, m = ctypes.c_uint8(), ctypes.c_uint8()
    lib().orc_get_scale_min_k4(ctypes.c_int(j), _p(s, ctypes.c_uint8), ctypes.byref(sc), ctypes.byref(m))
    return sc.value, m.value


# ── dequant ──────────────────────────────────────────────────────────────

def dequant(dtype, data, n):
    data = _u8(data)
    out = np.empty(n, dtype=np.float32)
    L = lib()
    if dtype == Q8_0:
        L.orc_dequant_q8_0(_p(data, ctypes.c_uint8), ctypes.c_size_t(data.size), ctypes.c_size_t(n),
                           _p(out, ctypes.c_float))
    elif dtype == Q4_K:
        L.orc_dequant_q4_k(_p(data, ctypes.c_uint8), ctypes.c_size_t(n), _p(out, ctypes.c_float))
    elif dtype == Q6_K:
        L.orc_dequant_q6_k(_p(data, ctypes.c_uint8), ctypes.c_size_t(n), _p(out, ctypes.c_float))
    elif dtype in (F32, F16, Q2_K, Q3_K, Q5_K):
        if L.orc_dequant_any(ctypes.c_int(dtype), _p(data, ctypes.c_uint8), ctypes.c_size_t(n),
                             _p(out, ctypes.c_float)) != 0:
            raise ValueError(dtype)
    else:
        raise ValueError(dtype)
    return out


# ── matmuls: c[m,n] = a[m,k] · W[n,k]^T ─────────────────────────────────

def _mm(fn, a, b, m, n, k, with_len=False):
    a = _f32(a)
    b = _u8(b)
    c = np.empty(m * n, dtype=np.float32)
    args = [_p(a, ctypes.c_float), _p(b, ctypes.c_uint8)]
    if with_len:
        args.append(ctypes.c_size_t(b.size))
    args += [ctypes.c_size_t(m), ctypes.c_size_t(n), ctypes.c_size_t(k), _p(c, ctypes.c_float)]
    fn(*args)
    return c.reshape(m, n)


def avx2_matmul(dtype, a, b, m, n, k):
    """The x86 route of quantized_matmul_impl (AVX2 path for Q4_K/Q6_K)."""
    L = lib()
    if dtype == Q4_K:
        return _mm(L.orc_avx2_matmul_q4_k, a, b, m, n, k)
    if dtype == Q5_K:
        return _mm(L.orc_avx2_matmul_q5_k, a, b, m, n, k)
    if dtype == Q6_K:
        return _mm(L.orc_avx2_matmul_q6_k, a, b, m, n, k)
    if dtype == Q8_0:
        return _mm(L.orc_avx2_matmul_q8_0, a, b, m, n, k, with_len=True)
    if dtype == Q2_K:
        return _mm(L.orc_avx2order_matmul_q2_k, a, b, m, n, k)
    if dtype == Q3_K:
        return _mm(L.orc_avx2order_matmul_q3_k, a, b, m, n, k)
    if dtype == F16:
        return _mm(L.orc_avx2order_matmul_f16, a, b, m, n, k)
    raise ValueError(dtype)


def avx2order_scalar_matmul(dtype, a, b, m, n, k):
    L = lib()
    fn = {Q4_K: L.orc_avx2order_scalar_matmul_q4_k, Q5_K: L.orc_avx2order_scalar_matmul_q5_k,
          Q6_K: L.orc_avx2order_scalar_matmul_q6_k}[dtype]
    return _mm(fn, a, b, m, n, k)


def scalar_matmul(dtype, a, b, m, n, k):
    L = lib()
    if dtype == Q8_0:
        return _mm(L.orc_scalar_matmul_q8_0, a, b, m, n, k, with_len=True)
    if dtype == Q4_K:
        return _mm(L.orc_scalar_matmul_q4_k, a, b, m, n, k)
    if dtype == Q6_K:
        return _mm(L.orc_scalar_matmul_q6_k, a, b, m, n, k)
    fn = {Q5_K: L.orc_scalar_matmul_q5_k, Q2_K: L.orc_scalar_matmul_q2_k, Q3_K: L.orc_scalar_matmul_q3_k,
          F16: L.orc_scalar_matmul_f16}.get(dtype)
    if fn is None:
        raise ValueError(dtype)
    return _mm(fn, a, b, m, n, k)


def reference_matmul(dtype, a, b, m, n, k):
    """What the reference computes on an x86 AVX2 host for this dtype on
    [n][k] row-major weights (matmul_q*, matmul_f16), except Q8_0, whose AVX2
    kernel mis-addresses its quants (see oracle.c); Q8_0 uses the scalar
    kernel, which is the format's stated semantics."""
    if dtype == Q8_0:
        return scalar_matmul(dtype, a, b, m, n, k)
    return avx2_matmul(dtype, a, b, m, n, k)


def matmul_f32_gguf(a, b, m, n, k):
    """matmul_f32_gguf (dispatch.rs:541-574): b is f32 [k][n] (GGUF order)."""
    a, b = _f32(a), _f32(b)
    c = np.empty(m * n, dtype=np.float32)
    lib().orc_matmul_f32_gguf(_p(a, ctypes.c_float), _p(b, ctypes.c_float), ctypes.c_size_t(m),
                              ctypes.c_size_t(n), ctypes.c_size_t(k), _p(c, ctypes.c_float))
    return c.reshape(m, n)


def gguf_order_matmul(dtype, a, b, m, n, k):
    """quantized_matmul_impl's fallback for F32/F16/Q2_K/Q3_K weights kept in
    GGUF [k][n] order: dequantize(b, [k, n]) then matmul_f32_gguf."""
    a, b = _f32(a), _u8(b)
    c = np.empty(m * n, dtype=np.float32)
    rc = lib().orc_gguf_order_matmul(ctypes.c_int(dtype), _p(a, ctypes.c_float), ctypes.c_size_t(m),
                                     _p(b, ctypes.c_uint8), ctypes.c_size_t(n), ctypes.c_size_t(k),
                                     _p(c, ctypes.c_float))
    if rc != 0:
        raise ValueError(dtype)
    return c.reshape(m, n)


# ── requantize / Q8 activations / dotprod references ────────────────────

def requantize(dtype, data, rows, cols):
    data = _f32(data)
    be, bb = BLOCK_ELEMS[dtype], BLOCK_BYTES[dtype]
    out = np.zeros(rows * ((cols + be - 1) // be) * bb, dtype=np.uint8)
    fn = {Q8_0: lib().orc_requantize_q8_0, Q4_K: lib().orc_requantize_q4_k, Q5_K: lib().orc_requantize_q5_k,
          Q6_K: lib().orc_requantize_q6_k}[dtype]
    fn(_p(data, ctypes.c_float), ctypes.c_size_t(rows), ctypes.c_size_t(cols), _p(out, ctypes.c_uint8))
    return out


def quantize_activations_q8_0(a, m, k):
    a = _f32(a)
    out = np.zeros(m * ((k + 31) // 32) * 34, dtype=np.uint8)
    lib().orc_quantize_activations_q8_0(_p(a, ctypes.c_float), ctypes.c_size_t(m), ctypes.c_size_t(k),
                                        _p(out, ctypes.c_uint8))
    return out


def dotprod_ref(dtype, aq, b, m, n, k):
    aq = _u8(aq)
    b = _u8(b)
    c = np.empty(m * n, dtype=np.float32)
    fn = {Q8_0: lib().orc_dotprod_ref_q8_0, Q4_K: lib().orc_dotprod_ref_q4_k, Q5_K: lib().orc_dotprod_ref_q5_k,
          Q6_K: lib().orc_dotprod_ref_q6_k}[dtype]
    fn(_p(aq, ctypes.c_uint8), _p(b, ctypes.c_uint8), ctypes.c_size_t(m), ctypes.c_size_t(n),
       ctypes.c_size_t(k), _p(c, ctypes.c_float))
    return c.reshape(m, n)


# ── decode-step math ─────────────────────────────────────────────────────

def rmsnorm(x, w, eps):
    x = _f32(x)
    w = _f32(w)
    out = np.empty_like(x)
    lib().orc_rmsnorm(_p(x, ctypes.c_float), _p(w, ctypes.c_float), ctypes.c_size_t(x.size),
                      ctypes.c_float(eps), _p(out, ctypes.c_float))
    return out


def precompute_rope(max_seq, head_dim, base):
    half = head_dim // 2
    s = np.empty(max_seq * half, dtype=np.float32)
    c = np.empty(max_seq * half, dtype=np.float32)
    lib().orc_precompute_rope(ctypes.c_size_t(max_seq), ctypes.c_size_t(head_dim), ctypes.c_float(base),
                              _p(s, ctypes.c_float), _p(c, ctypes.c_float))
    return s, c


def apply_rope(x, n_heads, head_dim, pos, sin_t, cos_t, max_seq):
    x = _f32(x).copy()
    lib().orc_apply_rope(_p(x, ctypes.c_float), ctypes.c_size_t(n_heads), ctypes.c_size_t(head_dim),
                         ctypes.c_size_t(pos), _p(_f32(sin_t), ctypes.c_float),
                         _p(_f32(cos_t), ctypes.c_float), ctypes.c_size_t(max_seq))
    return x


def attn_direct(q, k_st, v_st, seq, head_dim, window=0):
    q, k_st, v_st = _f32(q), _f32(k_st), _f32(v_st)
    scores = np.empty(seq, dtype=np.float32)
    out = np.empty(head_dim, dtype=np.float32)
    lib().orc_attn_direct(_p(q, ctypes.c_float), _p(k_st, ctypes.c_float), _p(v_st, ctypes.c_float),
                          ctypes.c_size_t(seq), ctypes.c_size_t(head_dim), ctypes.c_size_t(window),
                          _p(scores, ctypes.c_float), _p(out, ctypes.c_float))
    return out


def argmax(logits):
    lg = _f32(logits)
    return lib().orc_argmax(_p(lg, ctypes.c_float), ctypes.c_size_t(lg.size))


class LlamaCfg(ctypes.Structure):
    _fields_ = [("vocab", ctypes.c_int32), ("d_model", ctypes.c_int32), ("n_layers", ctypes.c_int32),
                ("n_heads", ctypes.c_int32), ("n_kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
                ("d_ff", ctypes.c_int32), ("max_seq", ctypes.c_int32), ("rope_base", ctypes.c_float),
                ("eps", ctypes.c_float), ("sliding_window", ctypes.c_int32)]


def _dtype_of(layer_dtypes, l, j):
    """layer_dtypes: seven formats for every layer, or one list of seven per layer."""
    if isinstance(layer_dtypes[0], (list, tuple)):
        return layer_dtypes[l][j]
    return layer_dtypes[j]


def decode_step(cfg, x_embed, pos, layer_weights, layer_dtypes, norms, final_norm, lm_head, lm_dtype,
                rope_sin, rope_cos, kv, seq_len, start_layer=0):
    """One CPU decode step (runner.rs:1557-1646). layer_weights: list over layers
    of 7 uint8 arrays (q,k,v,o,gate,up,down); norms: list over layers of
    (attn_norm, ffn_norm). kv is updated in place. Returns (logits, seq_len).
    start_layer > 0 enters the step there with x_embed as the residual stream
    (the resume of a budgeted decode, runner.rs:1201-1217)."""
    L = lib()
    nl = cfg.n_layers
    keep = []
    wp = (ctypes.POINTER(ctypes.c_uint8) * (nl * 7))()
    wt = (ctypes.c_int32 * (nl * 7))()
    for l in range(nl):
        for j in range(7):
            arr = _u8(layer_weights[l][j])
            keep.append(arr)
            wp[l * 7 + j] = _p(arr, ctypes.c_uint8)
            wt[l * 7 + j] = _dtype_of(layer_dtypes, l, j)
    npp = (ctypes.POINTER(ctypes.c_float) * (nl * 2))()
    for l in range(nl):
        for j in range(2):
            arr = _f32(norms[l][j])
            keep.append(arr)
            npp[l * 2 + j] = _p(arr, ctypes.c_float)
    x = _f32(x_embed)
    fn_ = _f32(final_norm)
    lm = _u8(lm_head)
    rs, rc = _f32(rope_sin), _f32(rope_cos)
    assert kv.dtype == np.float32 and kv.flags.c_contiguous
    sl = ctypes.c_int32(seq_len)
    logits = np.empty(cfg.vocab, dtype=np.float32)
    rc_ = L.orc_decode_step_from(ctypes.byref(cfg), _p(x, ctypes.c_float), ctypes.c_int32(pos),
                                 ctypes.c_int32(start_layer), wp, wt, npp,
                            _p(fn_, ctypes.c_float), _p(lm, ctypes.c_uint8), ctypes.c_int32(lm_dtype),
                            _p(rs, ctypes.c_float), _p(rc, ctypes.c_float), _p(kv, ctypes.c_float),
                            ctypes.byref(sl), _p(logits, ctypes.c_float))
    if rc_ != 0:
        raise RuntimeError("orc_decode_step failed: %d" % rc_)
    return logits, sl.value


def _model_ptrs(cfg, layer_weights, layer_dtypes, norms):
    nl = cfg.n_layers
    keep = []
    wp = (ctypes.POINTER(ctypes.c_uint8) * (nl * 7))()
    wt = (ctypes.c_int32 * (nl * 7))()
    for l in range(nl):
        for j in range(7):
            arr = _u8(layer_weights[l][j])
            keep.append(arr)
            wp[l * 7 + j] = _p(arr, ctypes.c_uint8)
            wt[l * 7 + j] = _dtype_of(layer_dtypes, l, j)
    npp = (ctypes.POINTER(ctypes.c_float) * (nl * 2))()
    for l in range(nl):
        for j in range(2):
            arr = _f32(norms[l][j])
            keep.append(arr)
            npp[l * 2 + j] = _p(arr, ctypes.c_float)
    return keep, wp, wt, npp


def forward_batch(cfg, x_embeds, layer_weights, layer_dtypes, norms, final_norm, lm_head, lm_dtype,
                  rope_sin, rope_cos, kv):
    """Batched prefill (forward_batch, runner.rs:833-993): x_embeds [n][d] are
    the prompt's embedding rows at positions 0..n-1; kv is written at slots
    0..n-1 in place. Returns the last token's logits."""
    L = lib()
    keep, wp, wt, npp = _model_ptrs(cfg, layer_weights, layer_dtypes, norms)
    x = _f32(x_embeds)
    n = x.size // cfg.d_model
    fn_, lm = _f32(final_norm), _u8(lm_head)
    rs, rc = _f32(rope_sin), _f32(rope_cos)
    assert kv.dtype == np.float32 and kv.flags.c_contiguous
    logits = np.empty(cfg.vocab, dtype=np.float32)
    rc_ = L.orc_forward_batch(ctypes.byref(cfg), _p(x, ctypes.c_float), ctypes.c_int32(n), wp, wt, npp,
                              _p(fn_, ctypes.c_float), _p(lm, ctypes.c_uint8), ctypes.c_int32(lm_dtype),
                              _p(rs, ctypes.c_float), _p(rc, ctypes.c_float), _p(kv, ctypes.c_float),
                              _p(logits, ctypes.c_float))
    if rc_ != 0:
        raise RuntimeError("orc_forward_batch failed: %d" % rc_)
    del keep
    return logits


# ── Backend trait ops (src/backend/cpu.rs) ───────────────────────────────

def backend_rms_norm(x, w, eps):
    """Op::RmsNorm (cpu.rs:514-545) over the rows of x ([..., last_dim])."""
    x, w = _f32(x), _f32(w)
    last = w.size
    out = np.empty_like(x)
    lib().orc_backend_rms_norm(_p(x, ctypes.c_float), _p(w, ctypes.c_float), ctypes.c_size_t(x.size // last),
                               ctypes.c_size_t(last), ctypes.c_float(eps), _p(out, ctypes.c_float))
    return out


def causal_attention(q, k, v, num_heads, scale):
    """Op::CausalAttention (cpu.rs:1660-1727) on [batch][seq][d] arrays."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    b, s, d = q.shape
    out = np.empty_like(q)
    scratch = np.empty(max(1, s), dtype=np.float32)
    rc = lib().orc_causal_attention(_p(q, ctypes.c_float), _p(k, ctypes.c_float), _p(v, ctypes.c_float),
                                    ctypes.c_size_t(b), ctypes.c_size_t(s), ctypes.c_size_t(d),
                                    ctypes.c_size_t(num_heads), ctypes.c_float(scale), _p(scratch, ctypes.c_float),
                                    _p(out, ctypes.c_float))
    if rc != 0:
        raise ValueError("causal_attention: num_heads must be positive")
    return out
