// Batched products (from a few hundred rows, per format: aeth_host.cpp) for the block formats without a matrix-core GEMM
// of their own: Q8_0, Q5_K and Q6_K rows, and Q2_K / Q3_K (GGUF order or
// rows). The weight is dequantized once per call (bit-exact with
// src/loader/dequant.rs), weight and activations are widened to f64, and one
// rocBLAS DGEMM forms every sum on the fp64 matrix cores: products of f32
// values are exact in f64 and the f64 sum of 4096-14336 of them stays within
// a few f64 ulps, so the single rounding to f32 at the end lands within the
// reference's own f32 summation error (matmul_q6_k_batched, q6_k.rs:90-190,
// and the AVX2 kernels sum in f32; an f32 SGEMM in yet another order was
// measured 1.1e-3 away from them on Q6_K outputs near 0.17, past the 1e-3
// bar). Without this, a prefill of m rows would stream such a weight m times
// through the row-batched GEMV.
#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <utility>

#include "aeth_common.hpp"
#include "aeth_internal.hpp"

namespace {
__global__ void k_widen(const float* __restrict__ src, int64_t rows, int64_t cols, int64_t lds,
                        double* __restrict__ dst) {
    const int64_t total = rows * cols;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / cols, c = i - r * cols;
        dst[i] = (double)src[r * lds + c];
    }
}

// c = (float)p, or c + (float)p with accumulate (the reference adds the f32 product); p is
// the sum, in order, of `parts` K-range products m·n apart
__global__ void k_narrow(const double* __restrict__ p, int64_t m, int64_t n, int parts, float* __restrict__ c,
                         int64_t ldc, int accumulate) {
    const int64_t total = m * n;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / n, j = i - r * n;
        double sum = p[i];
        for (int q = 1; q < parts; q++) sum += p[(int64_t)q * total + i];
        const float v = (float)sum;
        float* dst = c + r * ldc + j;
        *dst = accumulate ? *dst + v : v;
    }
}

unsigned grid_for(int64_t total) { return (unsigned)std::min<int64_t>(aeth_cdiv(total, 256), 16384); }

std::mutex g_blas_mu;
std::map<std::pair<int, hipStream_t>, rocblas_handle> g_handles;

int blas_handle(hipStream_t s, rocblas_handle* out) {
    int dev = 0;
    AETH_HIP_CHECK(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(g_blas_mu);
    rocblas_handle& h = g_handles[std::make_pair(dev, s)];
    if (!h) {
        if (rocblas_create_handle(&h) != rocblas_status_success) {
            h = nullptr;
            return aeth_set_error(AETH_EHIP, "rocblas_create_handle failed");
        }
        if (rocblas_set_stream(h, s) != rocblas_status_success)
            return aeth_set_error(AETH_EHIP, "rocblas_set_stream failed");
    }
    *out = h;
    return AETH_OK;
}
}  // namespace

void aeth_blas_release_stream(hipStream_t s) {
    std::lock_guard<std::mutex> lk(g_blas_mu);
    for (auto it = g_handles.begin(); it != g_handles.end();) {
        if (it->first.second == s) {
            rocblas_destroy_handle(it->second);
            it = g_handles.erase(it);
        } else {
            ++it;
        }
    }
}

int aeth_dequant_gemm_launch(const aeth_weight* w, const float* d_a, int64_t m, float* d_c, int64_t ldc,
                             unsigned flags, hipStream_t s) {
    int be, bb;
    int rc = aeth_block_geometry(w->dtype, &be, &bb);
    if (rc) return rc;
    const int64_t n = w->n, k = w->k;
    if (ldc <= 0) ldc = n;
    if (m > INT32_MAX || n > INT32_MAX || k > INT32_MAX || ldc > INT32_MAX)
        return aeth_set_error(AETH_EINVAL, "dequant gemm: shape beyond int32");
    const bool rows = w->order != AETH_ORDER_GGUF;  // [n][k] row blocks, else GGUF [k][n]
    // K covered by the product: Q8_0 rows hold ceil(k/32) blocks of which k elements
    // count; K-quant rows k/256 whole blocks (the reference ignores the tail of x)
    const int64_t kx = rows && w->dtype != AETH_DTYPE_Q8_0 && be > 1 ? (k / be) * be : k;
    const int64_t lda_w = rows ? w->nb * be : n;  // f32 row stride of the dequantized weight
    const int64_t wfloats = rows ? n * lda_w : n * k;
    // scratch: the f32 weight (then its raw bytes for a planar weight), the f64
    // weight, the f64 activations and the f64 product
    const bool planar = w->order == AETH_ORDER_PLANAR;
    const int64_t wf_b = aeth_cdiv(wfloats * 4, 256) * 256, raw_b = planar ? aeth_cdiv(w->bytes, 256) * 256 : 0;
    const int64_t w64_b = aeth_cdiv(n * kx * 8, 256) * 256, a64_b = aeth_cdiv(m * kx * 8, 256) * 256;
    const int64_t kb = aeth_cdiv(k, 32);
    // K split into `parts` ranges, one batch of the DGEMM each, when its 128 × 128 tiles would leave
    // CUs idle (m = 512, n = 4096: 128 tiles): the f64 partial products are summed in order after
    int parts = 1;
    {
        const int64_t tiles = aeth_cdiv(n, 128) * aeth_cdiv(m, 128), cus = aeth_num_cus();
        while (parts < 4 && tiles * parts * 2 <= cus && kx % (parts * 2) == 0 && kx / (parts * 2) >= 512) parts *= 2;
    }
    // the int8 dot-product path exists for Q8_0 / Q4_K / Q5_K / Q6_K only (the flag is ignored otherwise)
    const bool q8 = (flags & AETH_MM_Q8_ACTIVATIONS) && aeth_dtype_fused(w->dtype);
    const int64_t q_b = q8 ? aeth_cdiv(m * kb * 34, 256) * 256 + m * kb * 32 * 4 : 0;
    void* ws = nullptr;
    if ((rc = aeth_stream_scratch(s, AETH_SCRATCH_DEQ,
                                  (size_t)(wf_b + raw_b + w64_b + a64_b + parts * m * n * 8 + q_b + 256), &ws)))
        return rc;
    uint8_t* base = (uint8_t*)ws;
    float* Wf = (float*)base;
    uint8_t* tmp = base + wf_b;
    double* W64 = (double*)(tmp + raw_b);
    double* A64 = (double*)((uint8_t*)W64 + w64_b);
    double* P64 = (double*)((uint8_t*)A64 + a64_b);
    uint8_t* qbuf = (uint8_t*)(P64 + parts * m * n);
    const void* raw = w->base;
    if (planar) {  // back to GGUF row blocks, then dequantize
        if ((rc = aeth_weight_export_raw(w, tmp, 1, s))) return rc;
        raw = tmp;
    }
    if ((rc = aeth_dequant(w->dtype, raw, wfloats, Wf, s))) return rc;
    // W as an f64 (n × kx) row-major matrix for [n][k] rows, (kx × n) for GGUF [k][n]
    if (rows) hipLaunchKernelGGL(k_widen, dim3(grid_for(n * kx)), dim3(256), 0, s, Wf, n, kx, lda_w, W64);
    else hipLaunchKernelGGL(k_widen, dim3(grid_for(n * kx)), dim3(256), 0, s, Wf, kx, n, n, W64);
    AETH_LAUNCH_CHECK();
    const float* Asrc = d_a;
    int64_t lda_a = k;
    if (q8) {  // A → its Q8_0 activation blocks, used as q·d_a
        float* Aq = (float*)(qbuf + aeth_cdiv(m * kb * 34, 256) * 256);
        if ((rc = aeth_quantize_activations_q8_0(d_a, m, k, qbuf, s)) ||
            (rc = aeth_dequant(AETH_DTYPE_Q8_0, qbuf, m * kb * 32, Aq, s)))
            return rc;
        Asrc = Aq;
        // the reference's batched K-quant dotprod kernels find row r's activation
        // blocks at r·(k/256)·8 (neon.rs:517-518, :994) although the quantizer lays
        // rows out ceil(k/32) blocks apart; for k % 256 != 0 rows past the first
        // therefore read a shifted window of the blocks, reproduced here
        lda_a = w->dtype == AETH_DTYPE_Q8_0 ? kb * 32 : (k / 256) * 256;
    }
    hipLaunchKernelGGL(k_widen, dim3(grid_for(m * kx)), dim3(256), 0, s, Asrc, m, kx, lda_a, A64);
    AETH_LAUNCH_CHECK();
    rocblas_handle h = nullptr;
    if ((rc = blas_handle(s, &h))) return rc;
    // column-major view: Pᵀ (n × m, ld n) = Wop (n × kx) · A64ᵀ (kx × m, ld kx); batch q takes the
    // K range [q·kc, (q + 1)·kc): kc columns of A64ᵀ's rows and of Wop's (rows of W64 for [n][k]
    // weights, kc·n elements on for GGUF [k][n]), into its own n × m product
    const double alpha = 1.0, beta = 0.0;
    const int64_t kc = kx / parts;
    const rocblas_status st = rocblas_dgemm_strided_batched(
        h, rows ? rocblas_operation_transpose : rocblas_operation_none, rocblas_operation_none, (int)n, (int)m, (int)kc,
        &alpha, W64, rows ? (int)kx : (int)n, rows ? kc : kc * n, A64, (int)kx, kc, &beta, P64, (int)n, m * n, parts);
    if (st != rocblas_status_success) return aeth_set_error(AETH_EHIP, "rocblas_dgemm failed (status %d)", (int)st);
    hipLaunchKernelGGL(k_narrow, dim3(grid_for(m * n)), dim3(256), 0, s, P64, m, n, parts, d_c, ldc,
                       (flags & AETH_MM_ACCUMULATE) ? 1 : 0);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}
