// Batched prefill kernels (LlamaRunner::forward_batch, src/inference/runner.rs:833-993):
// the n prompt tokens go through each layer together, token i at position i,
// its K/V written to cache slot i. The projections run on the quantized GEMM
// (aeth_gemm.hip, Q4_K) or the row-batched GEMV (other formats); these kernels
// are the glue around them:
//  * k_embed_rows: token embeddings → rows of x;
//  * k_prefill_rope_kv: RoPE of q and k at each token's position
//    (apply_rope_inplace, runner.rs:1886-1909) and the cache writes (:890-906);
//  * k_attn_prefill: causal attention (attention_batch, runner.rs:1809-1883)
//    as one flash-style pass per (64-query block, head): online softmax over
//    64-key blocks in LDS, 4×4 score and 4×8 output register tiles per thread;
//  * k_silu_pairs: h = g·σ(g)·u on the interleaved gate/up GEMM output
//    (runner.rs:1617-1625 form).
#include <math.h>

#include "aeth_common.hpp"
#include "aeth_internal.hpp"
#include "aeth_ops_internal.hpp"

__global__ void __launch_bounds__(256) k_embed_rows(const float* __restrict__ table, const int* __restrict__ tokens,
                                                    int64_t d, float* __restrict__ x) {
    const int64_t i = blockIdx.x;
    const float* src = table + (int64_t)tokens[i] * d;
    float* dst = x + i * d;
    for (int64_t e = threadIdx.x; e < d; e += 256) dst[e] = src[e];
}

int aeth_embed_rows_launch(const float* table, const int* d_tokens, int64_t n, int64_t d, float* x, hipStream_t s) {
    if (n <= 0) return AETH_OK;
    hipLaunchKernelGGL(k_embed_rows, dim3((unsigned)n), dim3(256), 0, s, table, d_tokens, d, x);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}

// qkv: [n][nh·hd | nkv·hd | nkv·hd]; q and k rotated in place, k and v copied to
// the layer's cache [2][nkv][max_seq][hd] at slot i.
__global__ void __launch_bounds__(256) k_prefill_rope_kv(float* __restrict__ qkv, int64_t stride, int nh, int nkv,
                                                         int hd, const float* __restrict__ sin_t,
                                                         const float* __restrict__ cos_t, int64_t max_seq,
                                                         float* __restrict__ layer_kv) {
    const int64_t i = blockIdx.x;
    const int half = hd / 2;
    const int64_t p = i < max_seq ? i : max_seq - 1;
    float* row = qkv + i * stride;
    const float* sn = sin_t + p * half;
    const float* cs = cos_t + p * half;
    const int64_t hs = max_seq * hd;
    for (int idx = threadIdx.x; idx < (nh + nkv) * half; idx += 256) {
        const int h = idx / half, e = idx - h * half;
        float* v = row + (int64_t)h * hd;  // heads nh.. are the k heads (they follow q in the row)
        const float x0 = v[e], x1 = v[e + half];
        const float r0 = x0 * cs[e] - x1 * sn[e], r1 = x0 * sn[e] + x1 * cs[e];
        v[e] = r0;
        v[e + half] = r1;
        if (h >= nh) {
            float* kd = layer_kv + (int64_t)(h - nh) * hs + i * hd;
            kd[e] = r0;
            kd[e + half] = r1;
        }
    }
    const float* vsrc = row + (int64_t)(nh + nkv) * hd;
    for (int idx = threadIdx.x; idx < nkv * hd; idx += 256) {
        const int h = idx / hd, e = idx - h * hd;
        layer_kv[(int64_t)(nkv + h) * hs + i * hd + e] = vsrc[idx];
    }
}

int aeth_prefill_rope_kv_launch(float* qkv, int64_t n, int64_t nh, int64_t nkv, int64_t hd, const float* sin_t,
                                const float* cos_t, int64_t max_seq, float* layer_kv, hipStream_t s) {
    if (n <= 0) return AETH_OK;
    if (n > max_seq) return aeth_set_error(AETH_EINVAL, "prefill: %lld tokens exceed the cache", (long long)n);
    hipLaunchKernelGGL(k_prefill_rope_kv, dim3((unsigned)n), dim3(256), 0, s, qkv, (nh + 2 * nkv) * hd, (int)nh,
                       (int)nkv, (int)hd, sin_t, cos_t, max_seq, layer_kv);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}

#define PA_BQ 64
#define PA_BK 64

// Causal attention of queries [64·blockIdx.x, +64) of head blockIdx.y over keys
// 0..i of the layer cache (slots written by k_prefill_rope_kv).
template <int HD>
__global__ void __launch_bounds__(256) k_attn_prefill(const float* __restrict__ qkv, int64_t qkv_stride,
                                                      const float* __restrict__ layer_kv, int n, int nh, int nkv,
                                                      int64_t max_seq, float* __restrict__ out) {
    constexpr int LD = HD + 4;  // row stride (floats): 16-byte aligned rows
    extern __shared__ __attribute__((aligned(16))) float sm[];
    float* Qs = sm;
    float* Ks = Qs + PA_BQ * LD;
    float* Vs = Ks + PA_BK * LD;
    float* Ps = Vs + PA_BK * LD;  // [BQ][BK + 1]
    float* mrow = Ps + PA_BQ * (PA_BK + 1);
    float* lrow = mrow + PA_BQ;
    float* arow = lrow + PA_BQ;
    const int tid = threadIdx.x;
    const int h = blockIdx.y, kvh = h / (nh / nkv);
    const int q0 = blockIdx.x * PA_BQ;
    const float* K = layer_kv + (int64_t)kvh * max_seq * HD;
    const float* V = layer_kv + (int64_t)(nkv + kvh) * max_seq * HD;
    const float scale = 1.0f / sqrtf((float)HD);

    for (int idx = tid; idx < PA_BQ * HD / 4; idx += 256) {
        const int r = idx / (HD / 4), c = idx - r * (HD / 4);
        const int qi = min(q0 + r, n - 1);
        *(float4*)(Qs + r * LD + 4 * c) = *(const float4*)(qkv + (int64_t)qi * qkv_stride + (int64_t)h * HD + 4 * c);
    }
    if (tid < PA_BQ) {
        mrow[tid] = -INFINITY;
        lrow[tid] = 0.0f;
    }
    const int qq = tid >> 4, kq = tid & 15;  // score tile: queries 4qq.., keys 4kq..
    const int dq = tid & 15;                 // output tile: queries 4qq.., dims 8dq..
    float o[4][8];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int e = 0; e < 8; e++) o[a][e] = 0.0f;
    const int nkb = (min(q0 + PA_BQ, n) - 1) / PA_BK + 1;
    for (int kb = 0; kb < nkb; kb++) {
        const int k0 = kb * PA_BK;
        __syncthreads();  // the previous block's K/V/P are no longer read
        for (int idx = tid; idx < PA_BK * HD / 4; idx += 256) {
            const int r = idx / (HD / 4), c = idx - r * (HD / 4);
            const int kj = min(k0 + r, n - 1);
            *(float4*)(Ks + r * LD + 4 * c) = *(const float4*)(K + (int64_t)kj * HD + 4 * c);
            *(float4*)(Vs + r * LD + 4 * c) = *(const float4*)(V + (int64_t)kj * HD + 4 * c);
        }
        __syncthreads();
        float sacc[4][4];
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int b = 0; b < 4; b++) sacc[a][b] = 0.0f;
        for (int dd = 0; dd < HD; dd += 4) {
            float4 qv[4], kv[4];
#pragma unroll
            for (int a = 0; a < 4; a++) qv[a] = *(const float4*)(Qs + (4 * qq + a) * LD + dd);
#pragma unroll
            for (int b = 0; b < 4; b++) kv[b] = *(const float4*)(Ks + (4 * kq + b) * LD + dd);
#pragma unroll
            for (int a = 0; a < 4; a++)
#pragma unroll
                for (int b = 0; b < 4; b++)
                    sacc[a][b] += qv[a].x * kv[b].x + qv[a].y * kv[b].y + qv[a].z * kv[b].z + qv[a].w * kv[b].w;
        }
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const int qi = q0 + 4 * qq + a, kj = k0 + 4 * kq + b;
                Ps[(4 * qq + a) * (PA_BK + 1) + 4 * kq + b] = (kj <= qi && kj < n) ? sacc[a][b] * scale : -INFINITY;
            }
        __syncthreads();
        {  // online softmax: 4 threads per query row, 16 keys each
            const int r = tid >> 2, pp = tid & 3;
            float* pr = Ps + r * (PA_BK + 1) + 16 * pp;
            float mx = -INFINITY;
#pragma unroll
            for (int j = 0; j < 16; j++) mx = fmaxf(mx, pr[j]);
            mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
            const float m_old = mrow[r];
            const float m_new = fmaxf(m_old, mx);
            float ps = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const float e = m_new == -INFINITY ? 0.0f : expf(pr[j] - m_new);
                pr[j] = e;
                ps += e;
            }
            ps += __shfl_xor(ps, 1, 64);
            ps += __shfl_xor(ps, 2, 64);
            if (pp == 0) {
                const float alpha = m_new == -INFINITY ? 1.0f : expf(m_old - m_new);
                lrow[r] = lrow[r] * alpha + ps;
                mrow[r] = m_new;
                arow[r] = alpha;
            }
        }
        __syncthreads();
#pragma unroll
        for (int a = 0; a < 4; a++) {
            const float al = arow[4 * qq + a];
#pragma unroll
            for (int e = 0; e < 8; e++) o[a][e] *= al;
        }
        for (int j = 0; j < PA_BK; j++) {
            const float4 v0 = *(const float4*)(Vs + j * LD + 8 * dq);
            const float4 v1 = *(const float4*)(Vs + j * LD + 8 * dq + 4);
#pragma unroll
            for (int a = 0; a < 4; a++) {
                const float p = Ps[(4 * qq + a) * (PA_BK + 1) + j];
                o[a][0] += p * v0.x; o[a][1] += p * v0.y; o[a][2] += p * v0.z; o[a][3] += p * v0.w;
                o[a][4] += p * v1.x; o[a][5] += p * v1.y; o[a][6] += p * v1.z; o[a][7] += p * v1.w;
            }
        }
    }
#pragma unroll
    for (int a = 0; a < 4; a++) {
        const int qi = q0 + 4 * qq + a;
        if (qi < n) {
            const float inv = 1.0f / lrow[4 * qq + a];
            float* dst = out + (int64_t)qi * nh * HD + (int64_t)h * HD + 8 * dq;
            *(float4*)dst = make_float4(o[a][0] * inv, o[a][1] * inv, o[a][2] * inv, o[a][3] * inv);
            *(float4*)(dst + 4) = make_float4(o[a][4] * inv, o[a][5] * inv, o[a][6] * inv, o[a][7] * inv);
        }
    }
}

int aeth_attn_prefill_launch(const float* qkv, const float* layer_kv, int64_t n, int64_t nh, int64_t nkv,
                             int64_t hd, int64_t max_seq, float* out, hipStream_t s) {
    if (n <= 0) return AETH_OK;
    if (hd != 128 || nh % nkv != 0)
        return aeth_set_error(AETH_EUNSUPPORTED, "prefill attention: head_dim %lld (needs 128)", (long long)hd);
    const size_t lds = sizeof(float) * ((size_t)(PA_BQ + 2 * PA_BK) * (128 + 4) + PA_BQ * (PA_BK + 1) + 3 * PA_BQ);
    static bool opted = false;
    if (!opted) {
        AETH_HIP_CHECK(hipFuncSetAttribute((const void*)k_attn_prefill<128>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)lds));
        opted = true;
    }
    hipLaunchKernelGGL(k_attn_prefill<128>, dim3((unsigned)aeth_cdiv(n, PA_BQ), (unsigned)nh), dim3(256), lds, s, qkv,
                       (nh + 2 * nkv) * hd, layer_kv, (int)n, (int)nh, (int)nkv, max_seq, out);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}

// h[i][j] = g·σ(g)·u with (g, u) = gu[i][2j], gu[i][2j+1] (gate/up rows interleaved).
__global__ void k_silu_pairs(const float* __restrict__ gu, int64_t total, float* __restrict__ h) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const float2 p = *(const float2*)(gu + 2 * idx);
    h[idx] = p.x * (1.0f / (1.0f + expf(-p.x))) * p.y;
}

int aeth_silu_pairs_launch(const float* gu, int64_t total, float* h, hipStream_t s) {
    if (total <= 0) return AETH_OK;
    hipLaunchKernelGGL(k_silu_pairs, dim3((unsigned)aeth_cdiv(total, 256)), dim3(256), 0, s, gu, total, h);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}
