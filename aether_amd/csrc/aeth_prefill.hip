// Batched prefill kernels (LlamaRunner::forward_batch, src/inference/runner.rs:833-993):
// the n prompt tokens go through each layer together, token i at position i,
// its K/V written to cache slot i. The projections run on the quantized GEMM
// (aeth_gemm.hip, Q4_K) or the row-batched GEMV (other formats); these kernels
// are the glue around them:
//  * k_embed_rows: token embeddings → rows of x;
//  * k_prefill_rope_kv: RoPE of q and k at each token's position
//    (apply_rope_inplace, runner.rs:1886-1909) and the cache writes (:890-906);
//  * k_attn_prefill_mf: causal attention (attention_batch, runner.rs:1809-1883)
//    on the f32 matrix cores, flash-style (online softmax over 16-key blocks);
//    k_attn_prefill, the f32 VALU form (64-query blocks, 4×4 score and 4×8
//    output register tiles per thread), serves group sizes the MFMA form does
//    not take;
//  * k_silu_pairs: h = g·σ(g)·u on the interleaved gate/up GEMM output
//    (runner.rs:1617-1625 form).
#include <limits.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "aeth_common.hpp"
#include "aeth_internal.hpp"
#include "aeth_ops_internal.hpp"

typedef float f32x4 __attribute__((ext_vector_type(4)));

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

// The same for hd % 8 == 0 on 16-byte aligned rows: float4 pieces (four rotation
// pairs, or four v elements), 4 per thread per batch with every load issued
// before the first store.
__global__ void __launch_bounds__(256) k_prefill_rope_kv4(float* __restrict__ qkv, int64_t stride, int nh, int nkv,
                                                          int hd, const float* __restrict__ sin_t,
                                                          const float* __restrict__ cos_t, int64_t max_seq,
                                                          float* __restrict__ layer_kv) {
    const int64_t i = blockIdx.x;
    const int half = hd / 2, q4 = half / 4;
    const int64_t p = i < max_seq ? i : max_seq - 1;
    float* row = qkv + i * stride;
    const float* sn = sin_t + p * half;
    const float* cs = cos_t + p * half;
    const int64_t hs = max_seq * hd;
    const int units = (nh + nkv) * q4, vunits = nkv * hd / 4;
    for (int u0 = 0; u0 < units; u0 += 1024) {
        float4 a[4], b[4], c[4], t[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int u = min(u0 + (int)threadIdx.x + 256 * k, units - 1), h = u / q4, e = 4 * (u - h * q4);
            a[k] = *(const float4*)(row + (int64_t)h * hd + e);
            b[k] = *(const float4*)(row + (int64_t)h * hd + e + half);
            c[k] = *(const float4*)(cs + e);
            t[k] = *(const float4*)(sn + e);
        }
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int u = u0 + (int)threadIdx.x + 256 * k;
            if (u < units) {
                const int h = u / q4, e = 4 * (u - h * q4);
                const float4 r0 = make_float4(a[k].x * c[k].x - b[k].x * t[k].x, a[k].y * c[k].y - b[k].y * t[k].y,
                                              a[k].z * c[k].z - b[k].z * t[k].z, a[k].w * c[k].w - b[k].w * t[k].w);
                const float4 r1 = make_float4(a[k].x * t[k].x + b[k].x * c[k].x, a[k].y * t[k].y + b[k].y * c[k].y,
                                              a[k].z * t[k].z + b[k].z * c[k].z, a[k].w * t[k].w + b[k].w * c[k].w);
                *(float4*)(row + (int64_t)h * hd + e) = r0;
                *(float4*)(row + (int64_t)h * hd + e + half) = r1;
                if (h >= nh) {
                    float* kd = layer_kv + (int64_t)(h - nh) * hs + i * hd;
                    *(float4*)(kd + e) = r0;
                    *(float4*)(kd + e + half) = r1;
                }
            }
        }
    }
    const float* vsrc = row + (int64_t)(nh + nkv) * hd;
    for (int u = threadIdx.x; u < vunits; u += 256) {
        const int h = (4 * u) / hd, e = 4 * u - h * hd;
        *(float4*)(layer_kv + (int64_t)(nkv + h) * hs + i * hd + e) = *(const float4*)(vsrc + 4 * u);
    }
}

int aeth_prefill_rope_kv_launch(float* qkv, int64_t n, int64_t nh, int64_t nkv, int64_t hd, const float* sin_t,
                                const float* cos_t, int64_t max_seq, float* layer_kv, hipStream_t s) {
    if (n <= 0) return AETH_OK;
    if (n > max_seq) return aeth_set_error(AETH_EINVAL, "prefill: %lld tokens exceed the cache", (long long)n);
    const bool al16 = (((uintptr_t)qkv | (uintptr_t)sin_t | (uintptr_t)cos_t | (uintptr_t)layer_kv) & 15) == 0;
    if (al16 && hd % 8 == 0)
        hipLaunchKernelGGL(k_prefill_rope_kv4, dim3((unsigned)n), dim3(256), 0, s, qkv, (nh + 2 * nkv) * hd, (int)nh,
                           (int)nkv, (int)hd, sin_t, cos_t, max_seq, layer_kv);
    else
        hipLaunchKernelGGL(k_prefill_rope_kv, dim3((unsigned)n), dim3(256), 0, s, qkv, (nh + 2 * nkv) * hd, (int)nh,
                           (int)nkv, (int)hd, sin_t, cos_t, max_seq, layer_kv);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}

#define PA_BQ 64
#define PA_BK 64

// Causal attention of queries [64·blockIdx.x, +64) of head blockIdx.y over keys
// 0..i of the layer cache (slots written by k_prefill_rope_kv); with a sliding
// window w > 0, keys i - w + 1 ..= i (attention_batch, runner.rs:1825-1845).
template <int HD>
__global__ void __launch_bounds__(256) k_attn_prefill(const float* __restrict__ qkv, int64_t qkv_stride,
                                                      const float* __restrict__ layer_kv, int n, int nh, int nkv,
                                                      int64_t max_seq, int window, float* __restrict__ out) {
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
    const int kb0 = window > 0 ? max(0, q0 - window + 1) / PA_BK : 0;  // blocks before every query's window: none
    for (int kb = kb0; kb < nkb; kb++) {
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
                Ps[(4 * qq + a) * (PA_BK + 1) + 4 * kq + b] =
                    (kj <= qi && kj < n && (window <= 0 || kj > qi - window)) ? sacc[a][b] * scale : -INFINITY;
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

// Causal attention on the f32 matrix cores, v_mfma_f32_16x16x4_f32 (lane l
// holds A[l%16][l/16] and B[l/16][l%16]; result register r of lane l is
// D[4(l/16) + r][l%16]). Scores are computed transposed, Sᵀ = K·Qᵀ, so that a
// lane's accumulator holds 4 keys of one score column; those registers are
// then directly the B operand of Oᵀ = Vᵀ·Pᵀ (no transposes). The 16 columns
// are QB = 16/G queries × the G query heads of one KV head (column c: query
// c/G, head c%G), so every K/V element loaded serves all G heads.
// K-index maps: in Sᵀ step i, lane group g (= l/16) contracts d = 32g + i;
// in Oᵀ step j it contracts key t0 + 4g + j (its own score register j), and
// Oᵀ row m of d-tile dt is d = 8m + dt, so a lane (c, g) ends with d = 32g +
// 8r + dt of column c.
// Work: workgroup (KV head, query-block pair {p, nqb−1−p}), which balances the
// causal triangle; its 4 waves take the 16-key blocks of a query block round
// robin, each keeping an online softmax, and merge the partials through LDS.
// Per key block the softmax runs in log2 units (v_exp_f32) and rescales the
// partials only when some column's running max grows by more than 2^8: below
// that the probabilities are taken against the stale max (at most 2^8 each;
// the result o / l does not depend on which max is used). K and V are read as
// buffers of the n filled rows, so the loads of rows ≥ n (the last block's
// tail) return zeros; those keys are masked. Two register sets alternate, the
// next block's loads in flight during the current block. With a sliding window
// w > 0 (attention_batch, runner.rs:1825-1845) query i sees keys i - w + 1 ..= i:
// the waves start at the first key block some query of the block sees, and the
// keys before a query's window are masked like those past it.
// Max / sum of a value over the lane pairs (l, l ^ 16) and (l, l ^ 32): v_permlane16_swap and
// v_permlane32_swap with the same register as both operands leave each lane of a pair the
// lower lane's value in the first result and the upper lane's in the second (register moves,
// no LDS round trip); both lanes then compute lower ∘ upper, the same bits.
__device__ __forceinline__ float pa_max16(float a) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(a), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pa_max32(float a) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(a), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pa_sum16(float a) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(a), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float pa_sum32(float a) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(a), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float4 pa_ld4(__amdgpu_buffer_rsrc_t r, int off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3]));
}

template <int G>
__global__ void __launch_bounds__(256, 2) k_attn_prefill_mf(const float* __restrict__ qkv, int64_t qkv_stride,
                                                         const float* __restrict__ layer_kv, int n, int nh, int nkv,
                                                         int64_t max_seq, int window, float* __restrict__ out) {
    constexpr int QB = 16 / G, HD = 128, PLD = HD + 4;
    constexpr float TH = 8.0f;  // log2 units a running max may grow before the partials are rescaled
    __shared__ __attribute__((aligned(16))) float po[4][16][PLD];  // per wave: column c, d
    __shared__ float pm[4][16], pl[4][16];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int c = lane & 15, grp = lane >> 4;
    const int g = blockIdx.x % nkv, p = blockIdx.x / nkv;
    const int nqb = (n + QB - 1) / QB;
    const int head = g * G + c % G;
    const float* K = layer_kv + (int64_t)g * max_seq * HD;
    const float* V = layer_kv + (int64_t)(nkv + g) * max_seq * HD;
    const __amdgpu_buffer_rsrc_t rK = __builtin_amdgcn_make_buffer_rsrc((void*)K, (short)0, n * HD * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rV = __builtin_amdgcn_make_buffer_rsrc((void*)V, (short)0, n * HD * 4, 0x00020000);
    const float sl2 = 1.4426950408889634f / sqrtf((float)HD);  // scale · log2(e)
    for (int pass = 0; pass < 2; pass++) {
        const int qb = pass == 0 ? p : nqb - 1 - p;
        if (pass == 1 && qb == p) break;  // the middle block of an odd count (uniform)
        const int q0 = qb * QB, query = q0 + c / G;
        float qv[32];
        {
            const float* src = qkv + (int64_t)min(query, n - 1) * qkv_stride + (int64_t)head * HD + 32 * grp;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float4 t = *(const float4*)(src + 4 * i);
                qv[4 * i] = t.x; qv[4 * i + 1] = t.y; qv[4 * i + 2] = t.z; qv[4 * i + 3] = t.w;
            }
        }
        const int kb_end = (min(q0 + QB, n) - 1) / 16;  // last key block, inclusive
        const int kb_beg = window > 0 ? max(0, q0 - window + 1) / 16 : 0;  // first key block any query sees
        // keys t with t > query - window are visible: t ≥ lo_all for every query of the block
        const int lo_all = window > 0 ? q0 + QB - window : INT_MIN;
        // loads of one key block: K rows t0 + c (A of Sᵀ), V rows t0 + 4·grp + j,
        // floats [8c, 8c + 8) (A of Oᵀ)
        auto load = [&](int kb, float4* kk, float4 (*vv)[2]) {
            const int ko = ((16 * kb + c) * HD + 32 * grp) * 4, vo = ((16 * kb + 4 * grp) * HD + 8 * c) * 4;
#pragma unroll
            for (int i = 0; i < 8; i++) kk[i] = pa_ld4(rK, ko + 16 * i);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                vv[j][0] = pa_ld4(rV, vo + j * HD * 4);
                vv[j][1] = pa_ld4(rV, vo + j * HD * 4 + 16);
            }
        };
        float m = -INFINITY, l = 0.0f;
        f32x4 o[8];
#pragma unroll
        for (int dt = 0; dt < 8; dt++) o[dt] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        auto step = [&](int kb, const float4* kr, const float4 (*vr)[2]) {
            const int t0 = 16 * kb;
            // four independent chains of 8 MFMAs (d ≡ i mod 4 of each lane group's 32), summed
            f32x4 s4[4];
#pragma unroll
            for (int u = 0; u < 4; u++) s4[u] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int i = 0; i < 8; i++) {
                s4[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[i].x, qv[4 * i], s4[0], 0, 0, 0);
                s4[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[i].y, qv[4 * i + 1], s4[1], 0, 0, 0);
                s4[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[i].z, qv[4 * i + 2], s4[2], 0, 0, 0);
                s4[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(kr[i].w, qv[4 * i + 3], s4[3], 0, 0, 0);
            }
            f32x4 s = (s4[0] + s4[1]) + (s4[2] + s4[3]);
            if (t0 + 15 <= q0 && t0 + 15 < n && t0 >= lo_all) {  // no key of the block is masked (uniform)
#pragma unroll
                for (int r = 0; r < 4; r++) s[r] *= sl2;
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int t = t0 + 4 * grp + r;
                    s[r] = (t <= query && t < n && (window <= 0 || t > query - window)) ? s[r] * sl2 : -INFINITY;
                }
            }
            float mx = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
            mx = pa_max32(pa_max16(mx));
            if (__any(mx > m + TH)) {  // uniform
                const float m_new = fmaxf(m, mx);
                const float alpha = m_new == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m - m_new);
                l *= alpha;
#pragma unroll
                for (int dt = 0; dt < 8; dt++) o[dt] *= alpha;
                m = m_new;
            }
            float ps = 0.0f;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                s[r] = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s[r] - m);
                ps += s[r];
            }
            l += pa_sum32(pa_sum16(ps));
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float vj[8] = {vr[j][0].x, vr[j][0].y, vr[j][0].z, vr[j][0].w,
                                     vr[j][1].x, vr[j][1].y, vr[j][1].z, vr[j][1].w};
#pragma unroll
                for (int dt = 0; dt < 8; dt++) o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(vj[dt], s[j], o[dt], 0, 0, 0);
            }
        };
        float4 ka[8], va[4][2], kn[8], vn[4][2];
        if (kb_beg + w <= kb_end) load(kb_beg + w, ka, va);
        for (int kb = kb_beg + w; kb <= kb_end; kb += 8) {  // two blocks per trip, the register sets alternating
            load(min(kb + 4, kb_end), kn, vn);
            step(kb, ka, va);
            if (kb + 4 > kb_end) break;
            load(min(kb + 8, kb_end), ka, va);
            step(kb + 4, kn, vn);
        }
        // this wave's partial: column c, d = 32·grp + 8r + dt
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int dt = 0; dt < 8; dt += 4)
                *(float4*)&po[w][c][32 * grp + 8 * r + dt] = make_float4(o[dt][r], o[dt + 1][r], o[dt + 2][r], o[dt + 3][r]);
        if (grp == 0) {
            pm[w][c] = m;
            pl[w][c] = l;
        }
        __syncthreads();
        {  // merge the 4 waves: thread → column tid/16, d [8·(tid%16), +8)
            const int cc = tid >> 4, d0 = 8 * (tid & 15);
            float M = -INFINITY;
#pragma unroll
            for (int v = 0; v < 4; v++) M = fmaxf(M, pm[v][cc]);
            float wgt[4], L = 0.0f;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                wgt[v] = pm[v][cc] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(pm[v][cc] - M);
                L += wgt[v] * pl[v][cc];
            }
            float acc[8] = {};
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const float4 a = *(const float4*)&po[v][cc][d0];
                const float4 b = *(const float4*)&po[v][cc][d0 + 4];
                acc[0] += wgt[v] * a.x; acc[1] += wgt[v] * a.y; acc[2] += wgt[v] * a.z; acc[3] += wgt[v] * a.w;
                acc[4] += wgt[v] * b.x; acc[5] += wgt[v] * b.y; acc[6] += wgt[v] * b.z; acc[7] += wgt[v] * b.w;
            }
            const int qq = q0 + cc / G, hh = g * G + cc % G;
            if (qq < n) {
                const float inv = 1.0f / L;
                float* dst = out + (int64_t)qq * nh * HD + (int64_t)hh * HD + d0;
                *(float4*)dst = make_float4(acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv);
                *(float4*)(dst + 4) = make_float4(acc[4] * inv, acc[5] * inv, acc[6] * inv, acc[7] * inv);
            }
        }
        __syncthreads();  // LDS is reused by the second query block
    }
}

int aeth_attn_prefill_launch(const float* qkv, int64_t stride, const float* layer_kv, int64_t n, int64_t nh,
                             int64_t nkv, int64_t hd, int64_t max_seq, int64_t window, float* out, hipStream_t s) {
    if (n <= 0) return AETH_OK;
    const int win = window > 0 && window < n ? (int)window : 0;  // a window reaching back past key 0 masks nothing
    if (hd != 128 || nh % nkv != 0)
        return aeth_set_error(AETH_EUNSUPPORTED, "prefill attention: head_dim %lld (needs 128)", (long long)hd);
    // AETH_PREFILL_ATTN=valu selects the f32 VALU kernel (comparison, tests)
    static const bool force_valu = getenv("AETH_PREFILL_ATTN") && !strcmp(getenv("AETH_PREFILL_ATTN"), "valu");
    const int64_t G = nh / nkv;
    if (!force_valu && (G == 1 || G == 2 || G == 4 || G == 8)) {
        const int64_t nqb = aeth_cdiv(n, 16 / G);
        const dim3 grid((unsigned)(nkv * aeth_cdiv(nqb, 2)));
        if (G == 1) hipLaunchKernelGGL(k_attn_prefill_mf<1>, grid, dim3(256), 0, s, qkv, stride, layer_kv, (int)n, (int)nh, (int)nkv, max_seq, win, out);
        else if (G == 2) hipLaunchKernelGGL(k_attn_prefill_mf<2>, grid, dim3(256), 0, s, qkv, stride, layer_kv, (int)n, (int)nh, (int)nkv, max_seq, win, out);
        else if (G == 4) hipLaunchKernelGGL(k_attn_prefill_mf<4>, grid, dim3(256), 0, s, qkv, stride, layer_kv, (int)n, (int)nh, (int)nkv, max_seq, win, out);
        else hipLaunchKernelGGL(k_attn_prefill_mf<8>, grid, dim3(256), 0, s, qkv, stride, layer_kv, (int)n, (int)nh, (int)nkv, max_seq, win, out);
        AETH_LAUNCH_CHECK();
        return AETH_OK;
    }
    const size_t lds = sizeof(float) * ((size_t)(PA_BQ + 2 * PA_BK) * (128 + 4) + PA_BQ * (PA_BK + 1) + 3 * PA_BQ);
    static bool opted = false;
    if (!opted) {
        AETH_HIP_CHECK(hipFuncSetAttribute((const void*)k_attn_prefill<128>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)lds));
        opted = true;
    }
    hipLaunchKernelGGL(k_attn_prefill<128>, dim3((unsigned)aeth_cdiv(n, PA_BQ), (unsigned)nh), dim3(256), lds, s, qkv,
                       stride, layer_kv, (int)n, (int)nh, (int)nkv, max_seq, win, out);
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
