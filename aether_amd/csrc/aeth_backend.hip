// The two decode-path ops of the reference's device trait Backend
// (src/backend/mod.rs:12-218) on the GPU: Op::RmsNorm (src/backend/cpu.rs:
// 514-545) and Op::CausalAttention (cpu.rs:1660-1727), as host-slice entry
// points a Rust `impl Backend for HipBackend` binds, plus the device-pointer
// causal attention they use. The reference's graph runtime is out of scope;
// these are the Backend surface that LlamaRunner-adjacent callers reach.
#include <hip/hip_runtime.h>
#include <math.h>

#include <algorithm>

#include "aeth_common.hpp"
#include "aeth_internal.hpp"
#include "aeth_ops_internal.hpp"

namespace {

constexpr int CA_WAVES = 4;   // queries per workgroup (one wave each)
constexpr int CA_MAXD = 256;  // head_dim limit: four dims per lane

// Causal attention over [batch][seq][d] rows, head h = columns [h·hd, (h+1)·hd).
// One wave per query i: keys in chunks of 64 (lane ↔ key), the chunk's scores
// (q·k)·scale with online-softmax rescaling of the running (max, sum, out);
// each lane accumulates dims lane + 64t of the output, V rows read coalesced.
// Scores of -inf carry no weight and a row whose scores are all -inf is 0
// (the reference skips such scores).
template <bool VEC4>
__global__ void __launch_bounds__(256) k_causal_attn_bsd(const float* __restrict__ q, const float* __restrict__ k,
                                                         const float* __restrict__ v, int seq, int d, int hd,
                                                         float scale, float* __restrict__ out) {
    __shared__ float qs[CA_WAVES][CA_MAXD];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int i = blockIdx.x * CA_WAVES + w, h = blockIdx.y, b = blockIdx.z;
    const int64_t base = (int64_t)b * seq * d + (int64_t)h * hd;
    const bool live = i < seq;  // a wave past the last query still reaches the barrier
    for (int e = lane; e < hd; e += 64) qs[w][e] = live ? q[base + (int64_t)i * d + e] : 0.0f;
    __syncthreads();
    if (!live) return;
    float m = -INFINITY, l = 0.0f, acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int j0 = 0; j0 <= i; j0 += 64) {
        const int j = j0 + lane;
        float s = -INFINITY;
        if (j <= i) {
            const float* kr = k + base + (int64_t)j * d;
            float dot = 0.0f;
            if (VEC4) {
                for (int e = 0; e < hd; e += 4) {
                    const float4 kv = *(const float4*)(kr + e);
                    dot += qs[w][e] * kv.x + qs[w][e + 1] * kv.y + qs[w][e + 2] * kv.z + qs[w][e + 3] * kv.w;
                }
            } else {
                for (int e = 0; e < hd; e++) dot += qs[w][e] * kr[e];
            }
            s = dot * scale;
        }
        const float m_new = fmaxf(m, aeth_wave_max(s));
        // a -inf score (masked, or q·k overflowing to -inf) gets no weight, as cpu.rs:1705-1721
        // skips it: exp(-inf - m_new) would be NaN while m_new is still -inf
        const float p = j <= i && s != -INFINITY ? expf(s - m_new) : 0.0f;
        const float alpha = m == -INFINITY ? 0.0f : expf(m - m_new);
        l = l * alpha + aeth_wave_sum(p);
        m = m_new;
#pragma unroll
        for (int t = 0; t < 4; t++) acc[t] *= alpha;
        const int cnt = min(64, i - j0 + 1);
        for (int jj = 0; jj < cnt; jj++) {
            const float pj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), jj));
            const float* vr = v + base + (int64_t)(j0 + jj) * d;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int e = lane + 64 * t;
                if (e < hd) acc[t] += pj * vr[e];
            }
        }
    }
    const float inv = 1.0f / l;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int e = lane + 64 * t;
        // every score -inf: the reference sums nothing and leaves the row 0
        if (e < hd) out[base + (int64_t)i * d + e] = l == 0.0f ? 0.0f : acc[t] * inv;
    }
}

__global__ void k_zero_f32(float* __restrict__ p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = 0.0f;
}

int check_attn_shape(int64_t batch, int64_t seq, int64_t d, int64_t num_heads, int64_t* total) {
    int64_t sd = 0;
    if (batch < 0 || seq < 0 || d < 0 || num_heads <= 0 || !aeth_mul_ok(seq, d, &sd) || !aeth_mul_ok(batch, sd, total))
        return aeth_set_error(AETH_EINVAL, "causal_attention: bad shape (batch %lld, seq %lld, d %lld, heads %lld)",
                              (long long)batch, (long long)seq, (long long)d, (long long)num_heads);
    if (d / num_heads > CA_MAXD)
        return aeth_set_error(AETH_EUNSUPPORTED, "causal_attention: head_dim %lld > %d", (long long)(d / num_heads),
                              CA_MAXD);
    if (seq > INT32_MAX || d > INT32_MAX || batch > 65535 || num_heads > 65535 || (seq + CA_WAVES - 1) / CA_WAVES > INT32_MAX)
        return aeth_set_error(AETH_EINVAL, "causal_attention: shape beyond the launch limits");
    return AETH_OK;
}

int causal_attention_launch(const float* q, const float* k, const float* v, int64_t batch, int64_t seq, int64_t d,
                            int64_t num_heads, float scale, float* out, hipStream_t s) {
    int64_t total = 0;
    int rc = check_attn_shape(batch, seq, d, num_heads, &total);
    if (rc) return rc;
    if (total == 0) return AETH_OK;
    const int64_t hd = d / num_heads;
    if (hd * num_heads != d || hd == 0) {  // columns no head owns stay 0 (the reference's zero-initialised output)
        hipLaunchKernelGGL(k_zero_f32, dim3((unsigned)std::min<int64_t>(aeth_cdiv(total, 256), 4096)), dim3(256), 0, s,
                           out, total);
        AETH_LAUNCH_CHECK();
    }
    if (hd == 0) return AETH_OK;
    const dim3 grid((unsigned)aeth_cdiv(seq, CA_WAVES), (unsigned)num_heads, (unsigned)batch);
    const bool vec4 = hd % 4 == 0 && d % 4 == 0 && (((uintptr_t)k) & 15) == 0;
    if (vec4)
        hipLaunchKernelGGL(k_causal_attn_bsd<true>, grid, dim3(64 * CA_WAVES), 0, s, q, k, v, (int)seq, (int)d, (int)hd,
                           scale, out);
    else
        hipLaunchKernelGGL(k_causal_attn_bsd<false>, grid, dim3(64 * CA_WAVES), 0, s, q, k, v, (int)seq, (int)d,
                           (int)hd, scale, out);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}

// Device buffers of one host-slice call, freed on every exit.
struct DevBufs {
    void* p[4] = {nullptr, nullptr, nullptr, nullptr};
    ~DevBufs() {
        for (void* x : p)
            if (x) hipFree(x);
    }
};

int no_device() {
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0)
        return aeth_set_error(AETH_EHIP, "backend op: no HIP device available (no CPU fallback in this library)");
    return AETH_OK;
}

}  // namespace

extern "C" AETH_API int aeth_causal_attention(const float* d_q, const float* d_k, const float* d_v, int64_t batch,
                                              int64_t seq, int64_t d, int64_t num_heads, float scale, float* d_out,
                                              void* stream) {
    int64_t total = 0;
    int rc = check_attn_shape(batch, seq, d, num_heads, &total);
    if (rc) return rc;
    if ((!d_q || !d_k || !d_v || !d_out) && total != 0)
        return aeth_set_error(AETH_EINVAL, "aeth_causal_attention: NULL argument");
    return causal_attention_launch(d_q, d_k, d_v, batch, seq, d, num_heads, scale, d_out, (hipStream_t)stream);
}

extern "C" AETH_API int aeth_backend_causal_attention(const float* q, const float* k, const float* v, int64_t batch,
                                                      int64_t seq, int64_t d, int64_t num_heads, float scale,
                                                      float* out) {
    int64_t total = 0;
    int rc = check_attn_shape(batch, seq, d, num_heads, &total);
    if (rc) return rc;
    if (total == 0) return AETH_OK;
    if (!q || !k || !v || !out) return aeth_set_error(AETH_EINVAL, "aeth_backend_causal_attention: NULL argument");
    if ((rc = no_device())) return rc;
    const size_t bytes = sizeof(float) * (size_t)total;
    DevBufs B;
    for (int i = 0; i < 4; i++) AETH_HIP_CHECK(hipMalloc(&B.p[i], bytes));
    AETH_HIP_CHECK(hipMemcpy(B.p[0], q, bytes, hipMemcpyHostToDevice));
    AETH_HIP_CHECK(hipMemcpy(B.p[1], k, bytes, hipMemcpyHostToDevice));
    AETH_HIP_CHECK(hipMemcpy(B.p[2], v, bytes, hipMemcpyHostToDevice));
    if ((rc = causal_attention_launch((const float*)B.p[0], (const float*)B.p[1], (const float*)B.p[2], batch, seq, d,
                                      num_heads, scale, (float*)B.p[3], nullptr)))
        return rc;
    AETH_HIP_CHECK(hipMemcpy(out, B.p[3], bytes, hipMemcpyDeviceToHost));
    return AETH_OK;
}

extern "C" AETH_API int aeth_backend_rms_norm(const float* x, const float* w, int64_t rows, int64_t last_dim, float eps,
                                              float* out) {
    int64_t total = 0;
    if (rows < 0 || last_dim <= 0 || rows > INT32_MAX || !aeth_mul_ok(rows, last_dim, &total))
        return aeth_set_error(AETH_EINVAL, "aeth_backend_rms_norm: bad shape (rows %lld, last_dim %lld)",
                              (long long)rows, (long long)last_dim);
    if (total == 0) return AETH_OK;
    if (!x || !w || !out) return aeth_set_error(AETH_EINVAL, "aeth_backend_rms_norm: NULL argument");
    int rc = no_device();
    if (rc) return rc;
    DevBufs B;
    AETH_HIP_CHECK(hipMalloc(&B.p[0], sizeof(float) * (size_t)total));
    AETH_HIP_CHECK(hipMalloc(&B.p[1], sizeof(float) * (size_t)last_dim));
    AETH_HIP_CHECK(hipMalloc(&B.p[2], sizeof(float) * (size_t)total));
    AETH_HIP_CHECK(hipMemcpy(B.p[0], x, sizeof(float) * (size_t)total, hipMemcpyHostToDevice));
    AETH_HIP_CHECK(hipMemcpy(B.p[1], w, sizeof(float) * (size_t)last_dim, hipMemcpyHostToDevice));
    if ((rc = aeth_rmsnorm_launch((const float*)B.p[0], (const float*)B.p[1], rows, last_dim, eps, (float*)B.p[2],
                                  nullptr)))
        return rc;
    AETH_HIP_CHECK(hipMemcpy(out, B.p[2], sizeof(float) * (size_t)total, hipMemcpyDeviceToHost));
    return AETH_OK;
}
