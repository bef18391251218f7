// Host side of the quantized-matmul path: the device-pointer entry points,
// the QuantKernel plugin registry (src/quant/matmul/registry.rs:7-63) with its
// HIP kernels, and quantized_matmul_impl / matmul_q* over host slices
// (src/quant/matmul/dispatch.rs:98-135, avx2_dispatch.rs:58-68).
#include <hip/hip_runtime.h>

#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <tuple>

#include "aeth_common.hpp"
#include "aeth_internal.hpp"
#include "aeth_ops_internal.hpp"

// ── per-device scratch for the standalone decode-op entry points ─────────
// One buffer per (device, use); calls that overlap on one device (different
// host threads or streams) share it and race; the runner uses its own.
namespace {
struct Workspace {
    void* ptr = nullptr;
    size_t bytes = 0;
};
std::mutex g_ws_mu;
std::map<std::pair<int, int>, Workspace> g_ws;
enum { WS_ATTN = 0, WS_ARGMAX = 1 };

int workspace(int use, size_t bytes, void** out) {
    int dev = 0;
    AETH_HIP_CHECK(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(g_ws_mu);
    Workspace& w = g_ws[std::make_pair(dev, use)];
    if (w.bytes < bytes) {
        if (w.ptr) AETH_HIP_CHECK(hipFree(w.ptr));
        w.ptr = nullptr;
        w.bytes = 0;
        AETH_HIP_CHECK(hipMalloc(&w.ptr, bytes));
        AETH_HIP_CHECK(hipMemset(w.ptr, 0, bytes));
        w.bytes = bytes;
    }
    *out = w.ptr;
    return AETH_OK;
}
}  // namespace

int aeth_qmatmul_ld(const aeth_weight* w, const float* d_a, int64_t m, float* d_c, int64_t ldc, unsigned flags,
                    hipStream_t s) {
    if (m > 1 && w->dtype == AETH_DTYPE_Q4_K && !(flags & AETH_MM_Q8_ACTIVATIONS))
        return aeth_gemm_q4k_launch(w, d_a, m, d_c, flags, s, ldc);
    GemvEpi e;
    e.flags = flags;
    e.ldc = ldc;
    return aeth_gemv_launch_ex(w, d_a, m, d_c, e, s);
}

extern "C" AETH_API int aeth_qmatmul(const aeth_weight* w, const float* d_a, int64_t m, float* d_c, unsigned flags,
                                     void* stream) {
    if (!w || !d_a || !d_c || m <= 0) return aeth_set_error(AETH_EINVAL, "aeth_qmatmul: bad argument");
    return aeth_qmatmul_ld(w, d_a, m, d_c, 0, flags, (hipStream_t)stream);
}

extern "C" AETH_API int aeth_rmsnorm(const float* d_x, const float* d_w, int64_t rows, int64_t n, float eps,
                                     float* d_out, void* stream) {
    if (!d_x || !d_w || !d_out || rows < 0 || n < 0) return aeth_set_error(AETH_EINVAL, "aeth_rmsnorm: bad argument");
    return aeth_rmsnorm_launch(d_x, d_w, rows, n, eps, d_out, (hipStream_t)stream);
}

extern "C" AETH_API int aeth_rope(float* d_x, int64_t n_heads, int64_t head_dim, int64_t pos, const float* d_sin,
                                  const float* d_cos, int64_t max_seq, void* stream) {
    if (!d_x || !d_sin || !d_cos || max_seq <= 0 || head_dim % 2 || pos < 0)
        return aeth_set_error(AETH_EINVAL, "aeth_rope: bad argument");
    return aeth_rope_launch(d_x, n_heads, head_dim, nullptr, pos, d_sin, d_cos, max_seq, (hipStream_t)stream);
}

extern "C" AETH_API int aeth_kv_append(float* d_layer_kv, const float* d_k, const float* d_v, int64_t kv_heads,
                                       int64_t head_dim, int64_t max_seq, int64_t slot, void* stream) {
    if (!d_layer_kv || !d_k || !d_v || slot < 0) return aeth_set_error(AETH_EINVAL, "aeth_kv_append: bad argument");
    if (slot >= max_seq) return aeth_set_error(AETH_EINVAL, "aeth_kv_append: cache full (slot %lld)", (long long)slot);
    return aeth_kv_append_launch(d_layer_kv, d_k, d_v, kv_heads, head_dim, max_seq, nullptr, slot,
                                 (hipStream_t)stream);
}

extern "C" AETH_API int aeth_attn_decode(const float* d_q, const float* d_layer_kv, int64_t n_heads, int64_t kv_heads,
                                         int64_t head_dim, int64_t max_seq, int64_t seq, float* d_out, void* stream) {
    if (!d_q || !d_layer_kv || !d_out || seq <= 0 || seq > max_seq)
        return aeth_set_error(AETH_EINVAL, "aeth_attn_decode: bad argument (seq %lld, max_seq %lld)", (long long)seq,
                              (long long)max_seq);
    void* ws = nullptr;
    int rc = workspace(WS_ATTN, sizeof(float) * aeth_attn_ws_floats(n_heads, head_dim, max_seq), &ws);
    if (rc) return rc;
    return aeth_attn_launch(d_q, nullptr, (float*)d_layer_kv, nullptr, nullptr, nullptr, seq, n_heads, kv_heads,
                            head_dim, max_seq, (float*)ws, d_out, (hipStream_t)stream);
}

extern "C" AETH_API int aeth_attn_prefill(const float* d_q, int64_t q_stride, const float* d_layer_kv, int64_t n,
                                          int64_t n_heads, int64_t kv_heads, int64_t head_dim, int64_t max_seq,
                                          float* d_out, void* stream) {
    if (!d_q || !d_layer_kv || !d_out || n <= 0 || n > max_seq || kv_heads <= 0 || n_heads <= 0 ||
        n_heads % kv_heads != 0 || q_stride < n_heads * head_dim || (q_stride & 3))
        return aeth_set_error(AETH_EINVAL, "aeth_attn_prefill: bad argument (n %lld, max_seq %lld)", (long long)n,
                              (long long)max_seq);
    return aeth_attn_prefill_launch(d_q, q_stride, d_layer_kv, n, n_heads, kv_heads, head_dim, max_seq, d_out,
                                    (hipStream_t)stream);
}

extern "C" AETH_API int aeth_silu_mul(float* d_gate, const float* d_up, int64_t n, void* stream) {
    if (!d_gate || !d_up || n < 0) return aeth_set_error(AETH_EINVAL, "aeth_silu_mul: bad argument");
    return aeth_silu_mul_launch(d_gate, d_up, n, (hipStream_t)stream);
}

extern "C" AETH_API int aeth_add(float* d_x, const float* d_y, int64_t n, void* stream) {
    if (!d_x || !d_y || n < 0) return aeth_set_error(AETH_EINVAL, "aeth_add: bad argument");
    return aeth_add_launch(d_x, d_y, n, (hipStream_t)stream);
}

extern "C" AETH_API int aeth_argmax(const float* d_logits, int64_t n, int32_t* d_out, void* stream) {
    if (!d_logits || !d_out) return aeth_set_error(AETH_EINVAL, "aeth_argmax: bad argument");
    void* ws = nullptr;
    int rc = workspace(WS_ARGMAX, (size_t)aeth_argmax_ws_bytes(), &ws);
    if (rc) return rc;
    return aeth_argmax_launch(d_logits, n, d_out, nullptr, ws, (hipStream_t)stream);
}

// ── host-slice path: QuantWeight bytes → cached device weight ────────────
namespace {
using WKey = std::tuple<const void*, int64_t, int, int64_t, int64_t, int, int>;  // ptr, len, dtype, n, k, device, order
std::mutex g_wc_mu;
std::map<WKey, aeth_weight*> g_wcache;

int cached_weight(const uint8_t* b_raw, int64_t b_len, int dtype, int order, int64_t n, int64_t k, aeth_weight** out) {
    int be, bb;
    int rc = aeth_block_geometry(dtype, &be, &bb);
    if (rc) return rc;
    int64_t need = aeth_weight_raw_bytes(dtype, order, n, k);
    if (b_len < need)
        return aeth_set_error(AETH_EINVAL, "weight bytes %lld < %lld needed for [%lld, %lld] dtype %d",
                              (long long)b_len, (long long)need, (long long)n, (long long)k, dtype);
    int dev = 0;
    AETH_HIP_CHECK(hipGetDevice(&dev));
    WKey key{b_raw, b_len, dtype, n, k, dev, order};
    std::lock_guard<std::mutex> lk(g_wc_mu);
    auto it = g_wcache.find(key);
    if (it != g_wcache.end()) {
        *out = it->second;
        return AETH_OK;
    }
    aeth_weight* w = nullptr;
    rc = aeth_weight_create_ex(dtype, order, n, k, b_raw, 0, nullptr, &w);
    if (rc) return rc;
    g_wcache[key] = w;
    *out = w;
    return AETH_OK;
}

// One host-slice matmul: H2D a, launch, D2H c (QuantKernel::matmul semantics:
// c is fully written). order: how b_raw is laid out — the QuantWeight form
// (planar for the fused formats, GGUF [k][n] for the others) or [n][k] rows.
int host_matmul(const float* a, int64_t m, const uint8_t* b_raw, int64_t b_len, int64_t n, int64_t k, int dtype,
                float* c, int order = -1, unsigned flags = 0) {
    if (order < 0) order = aeth_dtype_fused(dtype) ? AETH_ORDER_PLANAR : AETH_ORDER_GGUF;
    if (!a || !b_raw || !c || m <= 0 || n <= 0 || k <= 0)
        return aeth_set_error(AETH_EINVAL, "matmul: bad argument (m=%lld n=%lld k=%lld)", (long long)m, (long long)n,
                              (long long)k);
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0)
        return aeth_set_error(AETH_EHIP, "matmul: no HIP device available (no CPU fallback in this library)");
    aeth_weight* w = nullptr;
    int rc = cached_weight(b_raw, b_len, dtype, order, n, k, &w);
    if (rc) return rc;
    float *da = nullptr, *dc = nullptr;
    AETH_HIP_CHECK(hipMalloc((void**)&da, sizeof(float) * m * k));
    hipError_t e = hipMalloc((void**)&dc, sizeof(float) * m * n);
    if (e != hipSuccess) {
        hipFree(da);
        return aeth_set_error(AETH_ENOMEM, "matmul: hipMalloc failed: %s", hipGetErrorString(e));
    }
    e = hipMemcpy(da, a, sizeof(float) * m * k, hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        rc = aeth_qmatmul(w, da, m, dc, flags, nullptr);
        if (rc == AETH_OK) {
            e = hipMemcpy(c, dc, sizeof(float) * m * n, hipMemcpyDeviceToHost);
        }
    }
    hipFree(da);
    hipFree(dc);
    if (rc) return rc;
    if (e != hipSuccess) return aeth_set_error(AETH_EHIP, "matmul: copy failed: %s", hipGetErrorString(e));
    return AETH_OK;
}
}  // namespace

extern "C" AETH_API int aeth_weight_cache_clear(void) {
    std::lock_guard<std::mutex> lk(g_wc_mu);
    for (auto& kv : g_wcache) aeth_weight_free(kv.second);
    g_wcache.clear();
    return AETH_OK;
}

// ── QuantKernel registry (registry.rs:7-63) ──────────────────────────────
namespace aeth {

// trait QuantKernel: Send + Sync { fn matmul(&self, a, m, b_raw, n, k, c);
// fn dtype(&self) -> GGUFDtype; fn name(&self) -> &'static str; }
class QuantKernel {
  public:
    virtual ~QuantKernel() = default;
    virtual int matmul(const float* a, int64_t m, const uint8_t* b_raw, int64_t b_len, int64_t n, int64_t k,
                       float* c) const = 0;
    virtual int dtype() const = 0;
    virtual const char* name() const = 0;
};

class HipQuantKernel final : public QuantKernel {
  public:
    explicit HipQuantKernel(int dtype) : dtype_(dtype) {}
    int matmul(const float* a, int64_t m, const uint8_t* b_raw, int64_t b_len, int64_t n, int64_t k,
               float* c) const override {
        return host_matmul(a, m, b_raw, b_len, n, k, dtype_, c);
    }
    int dtype() const override { return dtype_; }
    const char* name() const override {
        switch (dtype_) {
            case AETH_DTYPE_F32: return "F32 (hip gfx950)";
            case AETH_DTYPE_F16: return "F16 (hip gfx950)";
            case AETH_DTYPE_Q2_K: return "Q2_K (hip gfx950)";
            case AETH_DTYPE_Q3_K: return "Q3_K (hip gfx950)";
            case AETH_DTYPE_Q8_0: return "Q8_0 (hip gfx950)";
            case AETH_DTYPE_Q4_K: return "Q4_K (hip gfx950)";
            case AETH_DTYPE_Q5_K: return "Q5_K (hip gfx950)";
            default: return "Q6_K (hip gfx950)";
        }
    }

  private:
    int dtype_;
};

std::mutex g_reg_mu;  // RwLock in the reference; lookups are short
std::map<int, std::unique_ptr<QuantKernel>> g_registry;

// register_kernel: a duplicate dtype is an error (the reference panics).
int register_kernel(std::unique_ptr<QuantKernel> k) {
    std::lock_guard<std::mutex> lk(g_reg_mu);
    int dt = k->dtype();
    if (g_registry.count(dt))
        return aeth_set_error(AETH_ESTATE, "QuantKernel for dtype %d already registered", dt);
    g_registry[dt] = std::move(k);
    return AETH_OK;
}

// dispatch_matmul: 1 if a registered kernel ran, 0 if none for dtype.
int dispatch_matmul(const float* a, int64_t m, const uint8_t* b_raw, int64_t b_len, int64_t n, int64_t k, int dtype,
                    float* c) {
    const QuantKernel* kern = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_reg_mu);
        auto it = g_registry.find(dtype);
        if (it != g_registry.end()) kern = it->second.get();
    }
    if (!kern) return 0;
    int rc = kern->matmul(a, m, b_raw, b_len, n, k, c);
    return rc ? rc : 1;
}

}  // namespace aeth

extern "C" AETH_API int aeth_register_hip_kernels(void) {
    for (int dt : {AETH_DTYPE_F32, AETH_DTYPE_F16, AETH_DTYPE_Q8_0, AETH_DTYPE_Q2_K, AETH_DTYPE_Q3_K, AETH_DTYPE_Q4_K,
                   AETH_DTYPE_Q5_K, AETH_DTYPE_Q6_K}) {
        int rc = aeth::register_kernel(std::unique_ptr<aeth::QuantKernel>(new aeth::HipQuantKernel(dt)));
        if (rc) return rc;
    }
    return AETH_OK;
}

extern "C" AETH_API int aeth_registered_kernel_name(int dtype, char* buf, int buf_len) {
    std::lock_guard<std::mutex> lk(aeth::g_reg_mu);
    auto it = aeth::g_registry.find(dtype);
    if (it == aeth::g_registry.end()) return 0;
    if (buf && buf_len > 0) snprintf(buf, (size_t)buf_len, "%s", it->second->name());
    return 1;
}

extern "C" AETH_API int aeth_dispatch_matmul(const float* a, int64_t m, const uint8_t* b_raw, int64_t b_len, int64_t n,
                                             int64_t k, int dtype, float* c) {
    return aeth::dispatch_matmul(a, m, b_raw, b_len, n, k, dtype, c);
}

// quantized_matmul_impl (dispatch.rs:98-135): registered kernel first; with
// none registered the supported dtypes still run on the HIP kernels directly
// (this library has no CPU path). F32 / F16 / Q2_K / Q3_K bytes are GGUF
// [k][n], as load_quant leaves them and the reference's dequantize fallback
// reads them (dispatch.rs:126-133).
extern "C" AETH_API int aeth_quantized_matmul_impl(const float* a, int64_t m, const uint8_t* b_raw, int64_t b_len,
                                                   int64_t n, int64_t k, int dtype, float* c) {
    int rc = aeth::dispatch_matmul(a, m, b_raw, b_len, n, k, dtype, c);
    if (rc == 1) return AETH_OK;
    if (rc < 0) return rc;
    int be, bb;
    if (aeth_block_geometry(dtype, &be, &bb) != AETH_OK)
        return aeth_set_error(AETH_EUNSUPPORTED, "quantized_matmul_impl: dtype %d not on the HIP path", dtype);
    return host_matmul(a, m, b_raw, b_len, n, k, dtype, c);
}

// quantized_matmul_impl on an aarch64 host with dotprod: Q8_0 / Q4_K / Q5_K /
// Q6_K through the int8 dot-product kernels, the other formats as on x86.
extern "C" AETH_API int aeth_quantized_matmul_dotprod(const float* a, int64_t m, const uint8_t* b_raw, int64_t b_len,
                                                      int64_t n, int64_t k, int dtype, float* c) {
    int be, bb;
    if (aeth_block_geometry(dtype, &be, &bb) != AETH_OK)
        return aeth_set_error(AETH_EUNSUPPORTED, "quantized_matmul_dotprod: dtype %d not on the HIP path", dtype);
    return host_matmul(a, m, b_raw, b_len, n, k, dtype, c, -1, AETH_MM_Q8_ACTIVATIONS);
}

extern "C" AETH_API int aeth_matmul_q8_0(const float* a, const uint8_t* b, int64_t b_len, int64_t m, int64_t n,
                                         int64_t k, float* c) {
    return host_matmul(a, m, b, b_len, n, k, AETH_DTYPE_Q8_0, c);
}
extern "C" AETH_API int aeth_matmul_q4_k(const float* a, const uint8_t* b, int64_t b_len, int64_t m, int64_t n,
                                         int64_t k, float* c) {
    return host_matmul(a, m, b, b_len, n, k, AETH_DTYPE_Q4_K, c);
}
extern "C" AETH_API int aeth_matmul_q5_k(const float* a, const uint8_t* b, int64_t b_len, int64_t m, int64_t n,
                                         int64_t k, float* c) {
    return host_matmul(a, m, b, b_len, n, k, AETH_DTYPE_Q5_K, c);
}
extern "C" AETH_API int aeth_matmul_q2_k(const float* a, const uint8_t* b, int64_t b_len, int64_t m, int64_t n,
                                         int64_t k, float* c) {
    return host_matmul(a, m, b, b_len, n, k, AETH_DTYPE_Q2_K, c, AETH_ORDER_ROWS);
}
extern "C" AETH_API int aeth_matmul_q3_k(const float* a, const uint8_t* b, int64_t b_len, int64_t m, int64_t n,
                                         int64_t k, float* c) {
    return host_matmul(a, m, b, b_len, n, k, AETH_DTYPE_Q3_K, c, AETH_ORDER_ROWS);
}
extern "C" AETH_API int aeth_matmul_f16(const float* a, const uint8_t* b, int64_t b_len, int64_t m, int64_t n,
                                        int64_t k, float* c) {
    return host_matmul(a, m, b, b_len, n, k, AETH_DTYPE_F16, c, AETH_ORDER_ROWS);
}
extern "C" AETH_API int aeth_matmul_q6_k(const float* a, const uint8_t* b, int64_t b_len, int64_t m, int64_t n,
                                         int64_t k, float* c) {
    return host_matmul(a, m, b, b_len, n, k, AETH_DTYPE_Q6_K, c);
}
