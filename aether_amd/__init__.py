"""aether_amd — MI355X (gfx950) quantized-matmul hot path of Aether.

Python front-end over the C ABI of libaether_hip.so (include/aether_hip.h,
include/aether.h). All compute runs in the HIP library; there is no CPU
path: if the library is missing or no GPU is present, calls raise.
"""
import ctypes
import os

__all__ = ["lib", "check", "AethError", "LIB_PATH", "DTYPE_F32", "DTYPE_F16", "DTYPE_Q8_0", "DTYPE_Q2_K",
           "DTYPE_Q3_K", "DTYPE_Q4_K", "DTYPE_Q5_K", "DTYPE_Q6_K",
           "LlamaConfig", "header_symbols", "MM_ACCUMULATE", "MM_Q8_ACTIVATIONS", "block_geometry", "AETH_OK", "AETH_EINVAL",
           "AETH_EHIP", "AETH_ENOMEM", "AETH_EUNSUPPORTED", "AETH_ESTATE"]

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libaether_hip.so")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")

DTYPE_F32, DTYPE_F16, DTYPE_Q8_0, DTYPE_Q2_K, DTYPE_Q3_K = 0, 1, 8, 10, 11
DTYPE_Q4_K, DTYPE_Q5_K, DTYPE_Q6_K = 12, 13, 14
MM_ACCUMULATE, MM_Q8_ACTIVATIONS = 1, 2
# return codes (include/aether_hip.h)
AETH_OK, AETH_EINVAL, AETH_EHIP, AETH_ENOMEM, AETH_EUNSUPPORTED, AETH_ESTATE = 0, -1, -2, -3, -4, -5
_GEOM = {DTYPE_F32: (1, 4), DTYPE_F16: (1, 2), DTYPE_Q8_0: (32, 34), DTYPE_Q2_K: (256, 84), DTYPE_Q3_K: (256, 110),
         DTYPE_Q4_K: (256, 144), DTYPE_Q5_K: (256, 176), DTYPE_Q6_K: (256, 210)}


class AethError(RuntimeError):
    pass


class LlamaConfig(ctypes.Structure):
    _fields_ = [("vocab_size", ctypes.c_int32), ("d_model", ctypes.c_int32), ("num_layers", ctypes.c_int32),
                ("num_heads", ctypes.c_int32), ("num_kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
                ("d_ff", ctypes.c_int32), ("max_seq_len", ctypes.c_int32), ("rope_base", ctypes.c_float),
                ("rms_norm_eps", ctypes.c_float), ("sliding_window", ctypes.c_int32), ("flags", ctypes.c_int32)]


CFG_FULL_CONTEXT = 1  # aeth_llama_config.flags: keep max_seq_len past 4096 (up to 8192)
RUNNER_MAX_SEQ = 4096  # the cache length cap of LlamaRunner::new (runner.rs:225)


_lib = None
_c = ctypes
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_INT = ctypes.c_int

_SIGS = {
    "aeth_init": (_INT, [_INT]),
    "aeth_last_error": (ctypes.c_char_p, []),
    "aeth_block_geometry": (_INT, [_INT, _P, _P]),
    "aeth_weight_create": (_INT, [_INT, _I64, _I64, _P, _INT, _P, ctypes.POINTER(_P)]),
    "aeth_weight_free": (_INT, [_P]),
    "aeth_weight_bytes": (_I64, [_P]),
    "aeth_weight_export_raw": (_INT, [_P, _P, _INT, _P]),
    "aeth_dequant": (_INT, [_INT, _P, _I64, _P, _P]),
    "aeth_requantize": (_INT, [_INT, _P, _I64, _I64, _P, _P]),
    "aeth_quantize_activations_q8_0": (_INT, [_P, _I64, _I64, _P, _P]),
    "aeth_transpose_f32": (_INT, [_P, _I64, _I64, _P, _P]),
    "aeth_load_quant_ws_bytes": (_I64, [_I64, _I64]),
    "aeth_load_quant": (_INT, [_INT, _P, _I64, _I64, _P, _P, _P]),
    "aeth_qmatmul": (_INT, [_P, _P, _I64, _P, ctypes.c_uint, _P]),
    "aeth_quantized_matmul_impl": (_INT, [_P, _I64, _P, _I64, _I64, _I64, _INT, _P]),
    "aeth_quantized_matmul_dotprod": (_INT, [_P, _I64, _P, _I64, _I64, _I64, _INT, _P]),
    "aeth_quantized_matmul_impl_cached": (_INT, [_P, _I64, _P, _I64, _I64, _I64, _INT, _P, _P]),
    "aeth_stream_read": (_INT, [_P, _I64, _P, _I64, _P]),
    "aeth_mfma_rate": (_INT, [_INT, _INT, _INT, _P, _P]),
    "aeth_matmul_q8_0": (_INT, [_P, _P, _I64, _I64, _I64, _I64, _P]),
    "aeth_matmul_q4_k": (_INT, [_P, _P, _I64, _I64, _I64, _I64, _P]),
    "aeth_matmul_q5_k": (_INT, [_P, _P, _I64, _I64, _I64, _I64, _P]),
    "aeth_matmul_q2_k": (_INT, [_P, _P, _I64, _I64, _I64, _I64, _P]),
    "aeth_matmul_q3_k": (_INT, [_P, _P, _I64, _I64, _I64, _I64, _P]),
    "aeth_matmul_f16": (_INT, [_P, _P, _I64, _I64, _I64, _I64, _P]),
    "aeth_matmul_q6_k": (_INT, [_P, _P, _I64, _I64, _I64, _I64, _P]),
    "aeth_register_hip_kernels": (_INT, []),
    "aeth_registered_kernel_name": (_INT, [_INT, ctypes.c_char_p, _INT]),
    "aeth_dispatch_matmul": (_INT, [_P, _I64, _P, _I64, _I64, _I64, _INT, _P]),
    "aeth_weight_cache_clear": (_INT, []),
    "aeth_weight_cache_set_limit": (_INT, [_I64]),
    "aeth_weight_cache_bytes": (_I64, []),
    "aeth_weight_fingerprint": (_INT, [_P, _I64, _P]),
    "aeth_backend_rms_norm": (_INT, [_P, _P, _I64, _I64, ctypes.c_float, _P]),
    "aeth_backend_causal_attention": (_INT, [_P, _P, _P, _I64, _I64, _I64, _I64, ctypes.c_float, _P]),
    "aeth_causal_attention": (_INT, [_P, _P, _P, _I64, _I64, _I64, _I64, ctypes.c_float, _P, _P]),
    "aeth_rmsnorm": (_INT, [_P, _P, _I64, _I64, ctypes.c_float, _P, _P]),
    "aeth_rope": (_INT, [_P, _I64, _I64, _I64, _P, _P, _I64, _P]),
    "aeth_kv_append": (_INT, [_P, _P, _P, _I64, _I64, _I64, _I64, _P]),
    "aeth_attn_decode": (_INT, [_P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P]),
    "aeth_attn_decode_noalloc": (_INT, [_P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P]),
    "aeth_attn_prefill": (_INT, [_P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _P, _P]),
    "aeth_silu_mul": (_INT, [_P, _P, _I64, _P]),
    "aeth_add": (_INT, [_P, _P, _I64, _P]),
    "aeth_argmax": (_INT, [_P, _I64, _P, _P]),
    "aeth_fill_synthetic_raw": (_INT, [_INT, ctypes.c_uint64, _P, _I64, _P]),
    "aeth_fill_normal_f32": (_INT, [ctypes.c_uint64, _P, _I64, ctypes.c_float, ctypes.c_float, _P]),
    "aeth_runner_create": (_INT, [ctypes.POINTER(LlamaConfig), _P, _P, _P, _P, _P, _I32, _P, ctypes.c_uint64,
                                  ctypes.POINTER(_P)]),
    "aeth_runner_free": (_INT, [_P]),
    "aeth_runner_fill_kv": (_INT, [_P, ctypes.c_uint64, _I32]),
    "aeth_runner_kv_to_host": (_INT, [_P, _P, _P]),
    "aeth_runner_kv_from_host": (_INT, [_P, _P, _I32]),
    "aeth_runner_seq_len": (_INT, [_P]),
    "aeth_runner_decode": (_INT, [_P, _I32, _I32, _P, _P]),
    "aeth_runner_prefill": (_INT, [_P, _P, _I32, _P, _P]),
    "aeth_runner_generate": (_INT, [_P, _I32, _I32, _I32, _P, _INT]),
    "aeth_runner_export": (_INT, [_P, _INT, _I32, _P, _I64]),
    "aeth_runner_stream": (_P, [_P]),
    # aether.h
    "aether_load": (_P, [ctypes.c_char_p]),
    "aether_load_streaming": (_P, [ctypes.c_char_p, _INT]),
    "aether_free": (None, [_P]),
    "aether_model_from_runner": (_P, [_P]),
    "aether_vocab_size": (_INT, [_P]),
    "aether_context_len": (_INT, [_P]),
    "aether_num_layers": (_INT, [_P]),
    "aether_d_model": (_INT, [_P]),
    "aether_eos_id": (_INT, [_P]),
    "aether_bos_id": (_INT, [_P]),
    "aether_num_gpu_layers": (_INT, [_P]),
    "aether_num_cpu_layers": (_INT, [_P]),
    "aether_set_frame_budget": (None, [_P, ctypes.c_float]),
    "aether_frame_budget": (ctypes.c_float, [_P]),
    "aether_encode": (_P, [_P, ctypes.c_char_p, _P]),
    "aether_decode_token": (_P, [_P, _INT]),
    "aether_free_string": (None, [_P]),
    "aether_free_tokens": (None, [_P]),
    "aether_prefill": (_INT, [_P, _P, _INT, _P]),
    "aether_decode": (_INT, [_P, _INT, _INT, _P]),
    "aether_decode_budgeted": (_INT, [_P, _INT, _INT, _P]),
    "aether_sample": (_INT, [_P, _P, ctypes.c_float, ctypes.c_float]),
    "aether_argmax": (_INT, [_P, _P]),
    "aether_last_error": (_P, []),
}


def lib():
    """Loads libaether_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise AethError("libaether_hip.so is not built: run `python -m aether_amd.build` "
                            "(no CPU fallback exists)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def last_error():
    e = lib().aeth_last_error()
    return e.decode() if e else ""


def check(rc, what=""):
    if rc != 0:
        raise AethError("%s failed (%d): %s" % (what or "aether call", rc, last_error()))
    return rc


def block_geometry(dtype):
    return _GEOM[dtype]


def header_symbols():
    """Function names declared in include/*.h."""
    import re
    names = []
    for h in sorted(os.listdir(INCLUDE)):
        if not h.endswith(".h"):
            continue
        txt = open(os.path.join(INCLUDE, h)).read()
        txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
        for m in re.finditer(r"\b(?:AETH_API|AETHER_API)\b[^;(]*?\b((?:aeth|aether)_\w+)\s*\(", txt):
            names.append(m.group(1))
    return names
