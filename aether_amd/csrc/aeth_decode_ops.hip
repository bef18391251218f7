// Decode-step kernels around the quantized GEMVs (src/inference/runner.rs):
// RMSNorm, rotate-half RoPE, KV append, GQA split-sequence attention,
// SiLU·up, residual add, greedy argmax, embedding gather.
//
// Position-dependent kernels take their scalars either as values or from a
// device `int` (the runner keeps token/pos/fill on the device so one decode
// step can be captured once and replayed as a HIP graph).
#include <math.h>

#include "aeth_common.hpp"
#include "aeth_internal.hpp"
#include "aeth_ops_internal.hpp"

__device__ __forceinline__ int64_t scalar_or(const int* p, int64_t v) { return p ? (int64_t)*p : v; }

// ── RMSNorm (runner.rs:1739-1746): rms = sqrt(Σx²/n + eps); out = x / rms * w.
__global__ void __launch_bounds__(256) k_rmsnorm(const float* __restrict__ x, const float* __restrict__ w,
                                                 int64_t n, float eps, float* __restrict__ out) {
    __shared__ float red[4];
    const float* xr = x + (int64_t)blockIdx.x * n;
    float* o = out + (int64_t)blockIdx.x * n;
    float ss = 0.0f;
    for (int64_t i = threadIdx.x; i < n; i += 256) ss += xr[i] * xr[i];
    ss = aeth_wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = (red[0] + red[1]) + (red[2] + red[3]);
    float rms = sqrtf(tot / (float)n + eps);
    for (int64_t i = threadIdx.x; i < n; i += 256) o[i] = xr[i] / rms * w[i];
}

// Rows of n = 1024·V elements with 16-byte aligned x, w and out: one pass, the
// row held in registers (V float4 per thread, all loads issued up front), and
// x / rms as one correctly rounded reciprocal with a residual step per element
// (Markstein's correctly rounded quotient: the same value as the division).
template <int V>
__global__ void __launch_bounds__(256) k_rmsnorm_v(const float* __restrict__ x, const float* __restrict__ w,
                                                   int64_t n, float eps, float* __restrict__ out) {
    __shared__ float red[4];
    const float4* xr = (const float4*)(x + (int64_t)blockIdx.x * n);
    const float4* wr = (const float4*)w;
    float4* o = (float4*)(out + (int64_t)blockIdx.x * n);
    float4 v[V], wv[V];
#pragma unroll
    for (int j = 0; j < V; j++) v[j] = xr[threadIdx.x + 256 * j];
#pragma unroll
    for (int j = 0; j < V; j++) wv[j] = wr[threadIdx.x + 256 * j];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < V; j++) ss += (v[j].x * v[j].x + v[j].y * v[j].y) + (v[j].z * v[j].z + v[j].w * v[j].w);
    ss = aeth_wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float tot = (red[0] + red[1]) + (red[2] + red[3]);
    const float rms = sqrtf(tot / (float)n + eps), inv = 1.0f / rms;
    auto q = [&](float a) { const float q0 = a * inv; return fmaf(fmaf(-q0, rms, a), inv, q0); };
#pragma unroll
    for (int j = 0; j < V; j++)
        o[threadIdx.x + 256 * j] = make_float4(q(v[j].x) * wv[j].x, q(v[j].y) * wv[j].y, q(v[j].z) * wv[j].z,
                                               q(v[j].w) * wv[j].w);
}

int aeth_rmsnorm_launch(const float* x, const float* w, int64_t rows, int64_t n, float eps, float* out,
                        hipStream_t s) {
    if (rows <= 0 || n <= 0) return AETH_OK;
    const bool al16 = (((uintptr_t)x | (uintptr_t)w | (uintptr_t)out) & 15) == 0;
    if (al16 && n % 1024 == 0 && n <= 8192) {
        const dim3 g((unsigned)rows), b(256);
        switch (n / 1024) {
            case 1: hipLaunchKernelGGL(k_rmsnorm_v<1>, g, b, 0, s, x, w, n, eps, out); break;
            case 2: hipLaunchKernelGGL(k_rmsnorm_v<2>, g, b, 0, s, x, w, n, eps, out); break;
            case 3: hipLaunchKernelGGL(k_rmsnorm_v<3>, g, b, 0, s, x, w, n, eps, out); break;
            case 4: hipLaunchKernelGGL(k_rmsnorm_v<4>, g, b, 0, s, x, w, n, eps, out); break;
            case 5: hipLaunchKernelGGL(k_rmsnorm_v<5>, g, b, 0, s, x, w, n, eps, out); break;
            case 6: hipLaunchKernelGGL(k_rmsnorm_v<6>, g, b, 0, s, x, w, n, eps, out); break;
            case 7: hipLaunchKernelGGL(k_rmsnorm_v<7>, g, b, 0, s, x, w, n, eps, out); break;
            default: hipLaunchKernelGGL(k_rmsnorm_v<8>, g, b, 0, s, x, w, n, eps, out); break;
        }
        AETH_LAUNCH_CHECK();
        return AETH_OK;
    }
    hipLaunchKernelGGL(k_rmsnorm, dim3((unsigned)rows), dim3(256), 0, s, x, w, n, eps, out);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}

// ── RoPE (runner.rs:1886-1909): rotate halves (x_i, x_{i+hd/2}) with the
// precompute_rope table row of min(pos, max_seq-1).
__global__ void k_rope(float* __restrict__ x, int n_heads, int head_dim, const int* d_pos, int64_t pos,
                       const float* __restrict__ sin_t, const float* __restrict__ cos_t, int64_t max_seq) {
    int half = head_dim >> 1;
    int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_heads * half) return;
    int h = idx / half, i = idx - h * half;
    int64_t p = scalar_or(d_pos, pos);
    if (p > max_seq - 1) p = max_seq - 1;
    if (p < 0) p = 0;
    float s = sin_t[p * half + i], c = cos_t[p * half + i];
    float* hd = x + (int64_t)h * head_dim;
    float x0 = hd[i], x1 = hd[i + half];
    hd[i] = x0 * c - x1 * s;
    hd[i + half] = x0 * s + x1 * c;
}

int aeth_rope_launch(float* x, int64_t n_heads, int64_t head_dim, const int* d_pos, int64_t pos,
                     const float* sin_t, const float* cos_t, int64_t max_seq, hipStream_t s) {
    int64_t tot = n_heads * (head_dim / 2);
    if (tot <= 0) return AETH_OK;
    hipLaunchKernelGGL(k_rope, dim3((unsigned)aeth_cdiv(tot, 256)), dim3(256), 0, s, x, (int)n_heads,
                       (int)head_dim, d_pos, pos, sin_t, cos_t, max_seq);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}

// ── StaticKVCache::append (kv_cache.rs:40-65); a full cache writes nothing.
__global__ void k_kv_append(float* __restrict__ layer_kv, const float* __restrict__ k, const float* __restrict__ v,
                            int kv_heads, int head_dim, int64_t max_seq, const int* d_slot, int64_t slot) {
    int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= kv_heads * head_dim) return;
    int64_t sl = scalar_or(d_slot, slot);
    if (sl < 0 || sl >= max_seq) return;
    int h = idx / head_dim, e = idx - h * head_dim;
    int64_t hs = max_seq * head_dim;
    layer_kv[h * hs + sl * head_dim + e] = k[idx];
    layer_kv[(int64_t)kv_heads * hs + h * hs + sl * head_dim + e] = v[idx];
}

int aeth_kv_append_launch(float* layer_kv, const float* k, const float* v, int64_t kv_heads, int64_t head_dim,
                          int64_t max_seq, const int* d_slot, int64_t slot, hipStream_t s) {
    int64_t tot = kv_heads * head_dim;
    if (tot <= 0) return AETH_OK;
    hipLaunchKernelGGL(k_kv_append, dim3((unsigned)aeth_cdiv(tot, 256)), dim3(256), 0, s, layer_kv, k, v,
                       (int)kv_heads, (int)head_dim, max_seq, d_slot, slot);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}

// ── GQA decode attention (runner.rs:1579-1603, attn_direct :1757-1801),
// fused with the RoPE of q and k (apply_rope_inplace :1886-1909) and the KV
// append of the new token (StaticKVCache::append, kv_cache.rs:40-65).
//
// Workgroup (chunk c, kv head h) covers positions [Tc, Tc+T) (T = ATTN_T = 128) of
// the sequence [0, seq) for the `groups` query heads sharing h. It writes the
// chunk's softmax partials (max m, Σe^{s-m}, Σe^{s-m}·v); k_attn_merge then
// combines them: out = Σ_c e^{m_c-M} o_c / Σ_c e^{m_c-M} l_c.
//
// With `qkv` set, q/k/v come unrotated from the fused projection output
// [q (n_heads·hd) | k (kv_heads·hd) | v (kv_heads·hd)]: q and the new k are
// rotated here with the table row min(pos, max_seq-1), and the new token is
// position `fill` (the cache fill before this step; seq = fill + 1). The
// chunk holding it reads k/v from registers and stores them in the cache.
// A sliding window w (attn_direct's sliding_window, runner.rs:1768-1777)
// masks the positions before seq - w: chunks wholly before it return at
// once, and the merge leaves them out.
// Chunk shape, compile-time options: ATTN_NT threads (256, 512 or 1024), ATTN_LP lanes per
// position in the scores (2, 4, 8 or 16), ATTN_T = ATTN_NT / ATTN_LP positions per chunk. The 8B
// decode step at 2049-2176 positions measured (tok/s, two runs each): 512 threads × 4 lanes (T =
// 128) 675.6-677.0; 512 × 8 (T = 64) 658.0-660.8; 1024 × 8 (T = 128) 669.5-669.6; 256 × 2 (T = 128)
// 657.3-658.3; 256 × 4 (T = 64) 656.4-656.9; 1024 × 4 and 512 × 2 (T = 256) 640.1-643.6; 32-position
// chunks 617.
#ifndef ATTN_NT
#define ATTN_NT 512
#endif
#ifndef ATTN_LP
#define ATTN_LP 4
#endif
#define ATTN_T (ATTN_NT / ATTN_LP)  // positions per chunk
#define ATTN_MAX_GROUPS 8
#define ATTN_MAX_CHUNKS (8192 / ATTN_T)  // max_seq <= 8192

struct AttnArgs {
    const float* q;      // [n_heads][hd] (already rotated) when qkv == nullptr
    const float* qkv;    // fused projection output, rotated here
    float* layer_kv;     // [2][kv_heads][max_seq][hd]
    const float* sin_t;  // [max_seq][hd/2]
    const float* cos_t;
    const int* st;       // device {token, pos, fill} or nullptr
    int64_t seq_host;    // seq when st == nullptr
    int n_heads, kv_heads, head_dim;
    int64_t max_seq;
    int64_t window;      // sliding window (0: none)
    float* ws;           // [n_heads][max_chunks][hd + 2]
    int max_chunks;
    float* out;          // [n_heads][hd]
};

// Thread layout (shown for the default 512 threads = 8 waves, two per SIMD,
// LP = 4 lanes per position, chunk of T = 128 positions, HD = 128):
//  scores: thread (p = tid/4, e = tid%4) holds K[p][16i + 4e, +4) for i < 8
//          (each load instruction reads 64 contiguous bytes of 16 rows) and
//          dots it with every query head of the group; 4-lane reduction.
//  softmax: wave w takes query heads w, w + 8, ...; lane l the positions l, l + 64.
//  P·V:    thread (dims 4(tid%32), position group pg = tid/32) holds
//          V[8pg + j][4(tid%32), +4) for j < 8; lanes l, l+32 and then the
//          8 waves are summed.
// All loads are unconditional (clamped indices) and issued in one batch in
// the order q/rope inputs → K → V, so each phase waits only for its own data.
template <int HD, int NT>
__global__ void __launch_bounds__(NT) k_attn(AttnArgs A) {
    static_assert(HD == 128 && (NT == 256 || NT == 512 || NT == 1024), "decode attention is laid out for head_dim 128");
    constexpr int HALF = HD / 2, NWV = NT / 64;
    constexpr int LP = ATTN_LP, K4 = HD / LP / 4;  // scores: lanes per position, float4s per lane
    constexpr int T = NT / LP;                                  // positions per chunk (ATTN_T)
    constexpr int PP = T * HD / 4 / NT;                         // P·V: positions per thread
    constexpr int QP = (ATTN_MAX_GROUPS * HALF + NT - 1) / NT;  // rotation pairs of q per thread
    static_assert(T == ATTN_T && PP * (NT / 32) == T, "chunk layout");
    __shared__ __attribute__((aligned(16))) float qs[ATTN_MAX_GROUPS][HD];
    __shared__ __attribute__((aligned(16))) float knew[HD];
    __shared__ __attribute__((aligned(16))) float vnew[HD];
    __shared__ float sc[ATTN_MAX_GROUPS][T];
    __shared__ __attribute__((aligned(16))) float ov[NWV][ATTN_MAX_GROUPS][HD];
    __shared__ float mstat[ATTN_MAX_GROUPS][2];
    // grid (kv head, chunk), kv head fastest: the workgroups of the live chunks are dispatched
    // before those past the sequence (a captured step's grid covers max_seq), which return at
    // once (decode 682.3 tok/s against 679.9 with the chunk index fastest, six runs each)
    const int kvh = blockIdx.x, chunk = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int groups = A.n_heads / A.kv_heads;
    int64_t fill = -1, pos = 0, seq;
    if (A.st) {
        fill = A.st[2];
        pos = A.st[1];
        seq = fill + 1;
    } else {
        seq = A.seq_host;
    }
    if (seq > A.max_seq) seq = A.max_seq;
    const int64_t t0 = (int64_t)chunk * ATTN_T;
    const int64_t wstart = A.window > 0 && seq > A.window ? seq - A.window : 0;  // first visible position
    if (t0 >= seq || t0 + ATTN_T <= wstart) return;
    const int nt = (int)min((int64_t)ATTN_T, seq - t0);
    const int64_t hs = A.max_seq * HD;
    float* K = A.layer_kv + (int64_t)kvh * hs;
    float* V = A.layer_kv + (int64_t)A.kv_heads * hs + (int64_t)kvh * hs;
    const float scale = 1.0f / sqrtf((float)HD);
    const bool fused = A.qkv != nullptr;
    int64_t prow = fused ? pos : 0;
    if (prow > A.max_seq - 1) prow = A.max_seq - 1;
    if (prow < 0) prow = 0;
    const bool has_new = fused && fill >= t0 && fill < t0 + ATTN_T && fill < A.max_seq;

    // 1. q / rope inputs (rotation pairs (e, e + HD/2); one pair per thread covers
    // 8 heads). Without the fused path the table and new-k/v pointers alias q so
    // that the loads stay unconditional; their values are then unused.
    const float* qsrc = (fused ? A.qkv : A.q) + (int64_t)kvh * groups * HD;
    const float* sin_t = fused ? A.sin_t : qsrc;
    const float* cos_t = fused ? A.cos_t : qsrc;
    const float* ksrc = fused ? A.qkv + (int64_t)A.n_heads * HD + (int64_t)kvh * HD : qsrc;
    const float* vsrc = fused ? A.qkv + (int64_t)(A.n_heads + A.kv_heads) * HD + (int64_t)kvh * HD : qsrc;
    float qx0[QP], qx1[QP], qsn[QP], qcs[QP];
#pragma unroll
    for (int u = 0; u < QP; u++) {
        const int i = min(tid + u * NT, groups * HALF - 1), g = i / HALF, e = i - g * HALF;
        qx0[u] = qsrc[g * HD + e];
        qx1[u] = qsrc[g * HD + e + HALF];
        qsn[u] = sin_t[prow * HALF + e];
        qcs[u] = cos_t[prow * HALF + e];
    }
    const float kx0 = ksrc[tid & (HALF - 1)], kx1 = ksrc[(tid & (HALF - 1)) + HALF];
    const float vx = vsrc[tid & (HD - 1)];
    __builtin_amdgcn_sched_barrier(0);  // these small loads go out before the K/V batch
    // 2. K (scores layout) and V (P·V layout) of the chunk, positions past nt clamped
    const int sp = tid / LP, qe = tid % LP;
    float4 kk[K4];
    {
        const float* kr = K + (t0 + min(sp, nt - 1)) * HD + 4 * qe;
#pragma unroll
        for (int i = 0; i < K4; i++) kk[i] = *(const float4*)(kr + 4 * LP * i);
    }
    const int vd4 = tid & 31, pg = tid >> 5;
    float4 vv[PP];
#pragma unroll
    for (int j = 0; j < PP; j++) vv[j] = *(const float4*)(V + (t0 + min(PP * pg + j, nt - 1)) * HD + 4 * vd4);
    // Consume the q / rope inputs here, after the K/V batch is issued: otherwise the
    // compiler sinks their loads into the conditional stores below, behind K and V.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < QP; u++) asm volatile("" : "+v"(qx0[u]), "+v"(qx1[u]), "+v"(qsn[u]), "+v"(qcs[u]));
    float kvx[3] = {kx0, kx1, vx};
    asm volatile("" : "+v"(kvx[0]), "+v"(kvx[1]), "+v"(kvx[2]));

    // 3. rotated q (and the new k / v) to LDS
#pragma unroll
    for (int u = 0; u < QP; u++) {
        const int i = tid + u * NT;
        if (i < groups * HALF) {
            const int g = i / HALF, e = i - g * HALF;
            qs[g][e] = fused ? qx0[u] * qcs[u] - qx1[u] * qsn[u] : qx0[u];
            qs[g][e + HALF] = fused ? qx0[u] * qsn[u] + qx1[u] * qcs[u] : qx1[u];
        }
    }
    if (fused) {
        if (tid < HALF) {  // the pair of thread tid < HALF is (head 0, e = tid): same table entries
            knew[tid] = kvx[0] * qcs[0] - kvx[1] * qsn[0];
            knew[tid + HALF] = kvx[0] * qsn[0] + kvx[1] * qcs[0];
        }
        if (tid < HD) vnew[tid] = kvx[2];
    }
    __syncthreads();
    if (has_new && tid < HD) {  // StaticKVCache::append at slot `fill`
        K[fill * HD + tid] = knew[tid];
        V[fill * HD + tid] = vnew[tid];
    }

    // 4. scores
    const bool knew_here = has_new && t0 + sp == fill;
    if (knew_here) {
#pragma unroll
        for (int i = 0; i < K4; i++) kk[i] = *(const float4*)(&knew[4 * qe + 4 * LP * i]);
    }
#pragma unroll
    for (int g = 0; g < ATTN_MAX_GROUPS; g++) {
        if (g < groups) {
            float a = 0.0f;
#pragma unroll
            for (int i = 0; i < K4; i++) {
                const float4 qv = *(const float4*)(&qs[g][4 * qe + 4 * LP * i]);
                a += qv.x * kk[i].x + qv.y * kk[i].y + qv.z * kk[i].z + qv.w * kk[i].w;
            }
            a += aeth_dpp_xor1f(a);
            if (LP >= 4) a += aeth_dpp_xor2f(a);
            if (LP >= 8) a += aeth_dpp_mirror8f(a);
            if (LP == 16) a += aeth_dpp_mirror16f(a);
            if (qe == 0) sc[g][sp] = sp < nt && t0 + sp >= wstart ? a * scale : -INFINITY;
        }
    }
    __syncthreads();
    // 5. softmax over the chunk: wave w handles heads w, w + NWV, ...; lane l holds positions
    // l, l + 64, ... of the chunk
    constexpr int ST = (T + 63) / 64;
    for (int g = wave; g < groups; g += NWV) {
        float sv[ST], mx = -INFINITY;
#pragma unroll
        for (int u = 0; u < ST; u++) {
            const int p = lane + 64 * u;
            sv[u] = p < T ? sc[g][p] : -INFINITY;
            mx = fmaxf(mx, sv[u]);
        }
        const float m = aeth_wave_max(mx);
        float ps = 0.0f;
#pragma unroll
        for (int u = 0; u < ST; u++) {
            const int p = lane + 64 * u;
            const float pr = p < nt ? expf(sv[u] - m) : 0.0f;
            ps += pr;
            if (p < T) sc[g][p] = pr;
        }
        const float l = aeth_wave_sum(ps);
        if (lane == 0) {
            mstat[g][0] = m;
            mstat[g][1] = l;
        }
    }
    __syncthreads();
    // 6. Σ_t p_t v_t: PP positions per thread, then lanes l / l+32 and the NWV waves
    if (has_new) {
        const float4 nv = *(const float4*)(&vnew[4 * vd4]);
#pragma unroll
        for (int j = 0; j < PP; j++)
            if (t0 + PP * pg + j == fill) vv[j] = nv;
    }
#pragma unroll
    for (int g = 0; g < ATTN_MAX_GROUPS; g++) {
        if (g < groups) {
            float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
            for (int j = 0; j < PP; j++) {
                const float pj = sc[g][PP * pg + j];
                o.x += pj * vv[j].x;
                o.y += pj * vv[j].y;
                o.z += pj * vv[j].z;
                o.w += pj * vv[j].w;
            }
            o.x = aeth_add_halves(o.x);
            o.y = aeth_add_halves(o.y);
            o.z = aeth_add_halves(o.z);
            o.w = aeth_add_halves(o.w);
            if (lane < 32) *(float4*)(&ov[wave][g][4 * vd4]) = o;
        }
    }
    __syncthreads();
    for (int i = tid; i < groups * HD; i += NT) {
        const int g = i / HD, d = i - g * HD;
        float* dst = A.ws + ((int64_t)(kvh * groups + g) * A.max_chunks + chunk) * (HD + 2);
        float t8[NWV];
#pragma unroll
        for (int w = 0; w < NWV; w++) t8[w] = ov[w][g][d];
#pragma unroll
        for (int h = NWV / 2; h >= 1; h >>= 1)  // pairwise, a fixed order
#pragma unroll
            for (int w = 0; w < h; w++) t8[w] += t8[w + h];
        dst[d] = t8[0];
    }
    if (tid < groups) {
        float* dst = A.ws + ((int64_t)(kvh * groups + tid) * A.max_chunks + chunk) * (HD + 2);
        dst[HD] = mstat[tid][0];
        dst[HD + 1] = mstat[tid][1];
    }
}

// Merge of the chunk partials of one query head (grid = n_heads, HD threads):
// out = Σ_c e^{m_c-M} o_c / Σ_c e^{m_c-M} l_c. A separate launch: a kernel
// boundary makes every chunk's partials visible across the XCDs' L2s, which a
// device-scope fence inside one kernel would buy with L2 write-backs.
// Every wave reduces the chunk statistics itself — lane c holds chunks c,
// c + 64, ... — and the weights reach the other lanes by readlane, so the kernel
// has no LDS traffic and no barrier. Thread d loads its column of the chunk
// slots that cover 2560 positions in one batch together with the statistics,
// before the sequence length is known (slots past the live chunks are never
// used); the live chunks of a longer cache follow in batches of 16. (Slots for
// 2560, 3072 and 4096 positions measured 677.6-680.3, 675.8-676.2 and
// 672.8-673.3 tok/s on the 8B decode step at 2049-2176 positions: a slot loaded
// and not used costs more than the later batch at these lengths.)
template <int HD>
__global__ void __launch_bounds__(HD) k_attn_merge(AttnArgs A) {
    constexpr int S = (ATTN_MAX_CHUNKS + 63) / 64;                                  // statistics per lane
    constexpr int CB = 2560 / ATTN_T < ATTN_MAX_CHUNKS ? 2560 / ATTN_T : ATTN_MAX_CHUNKS;  // batched slots
    constexpr int CG = 16;                                                         // later batches
    const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    const float* base = A.ws + (int64_t)h * A.max_chunks * (HD + 2);
    const int cmax = A.max_chunks - 1;
    float m[S], l[S];
#pragma unroll
    for (int u = 0; u < S; u++) {
        const float* st = base + (int64_t)min(lane + 64 * u, cmax) * (HD + 2) + HD;
        m[u] = st[0];
        l[u] = st[1];
    }
    float v[CB];
#pragma unroll
    for (int j = 0; j < CB; j++) v[j] = base[(int64_t)min(j, cmax) * (HD + 2) + tid];
    int64_t seq = A.st ? (int64_t)A.st[2] + 1 : A.seq_host;
    if (seq > A.max_seq) seq = A.max_seq;
    const int nch = (int)((seq + ATTN_T - 1) / ATTN_T);
    const int c_lo = A.window > 0 && seq > A.window ? (int)((seq - A.window) / ATTN_T) : 0;  // chunks before: none
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < S; u++) {
        const int c = lane + 64 * u;
        if (!(c >= c_lo && c < nch)) m[u] = -INFINITY;
        mx = fmaxf(mx, m[u]);
    }
    const float M = aeth_wave_max(mx);
    float w[S], wl = 0.0f;
#pragma unroll
    for (int u = 0; u < S; u++) {  // a slot past the live chunks holds whatever an earlier call left
        const int c = lane + 64 * u;
        const bool live = c >= c_lo && c < nch;
        w[u] = live ? expf(m[u] - M) : 0.0f;
        wl += live ? w[u] * l[u] : 0.0f;
    }
    const float L = aeth_wave_sum(wl);
    // selects, not branches: a branch per chunk let the compiler sink each load into it
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < CB; j++) {
        const bool live = j >= c_lo && j < nch;
        const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w[j / 64]), j % 64));
        acc += (live ? wj : 0.0f) * (live ? v[j] : 0.0f);
    }
    for (int c0 = CB; c0 < nch; c0 += CG) {  // past the first batch: CG slots per batch, loads issued together
        float vr[CG];
#pragma unroll
        for (int j = 0; j < CG; j++) vr[j] = base[(int64_t)min(c0 + j, cmax) * (HD + 2) + tid];
#pragma unroll
        for (int j = 0; j < CG; j++) {
            const int c = c0 + j;
            const bool live = c >= c_lo && c < nch;
            float wc = 0.0f;
#pragma unroll
            for (int u = 0; u < S; u++)
                if (u == c / 64) wc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w[u]), c % 64));
            acc += (live ? wc : 0.0f) * (live ? vr[j] : 0.0f);
        }
    }
    A.out[(int64_t)h * HD + tid] = acc / L;
}

int64_t aeth_attn_ws_floats(int64_t n_heads, int64_t head_dim, int64_t max_seq) {
    return n_heads * aeth_cdiv(max_seq, ATTN_T) * (head_dim + 2);
}

// ws: aeth_attn_ws_floats(...) floats of chunk partials.
int aeth_attn_launch(const float* q, const float* qkv, float* layer_kv, const float* sin_t, const float* cos_t,
                     const int* d_st, int64_t seq, int64_t n_heads, int64_t kv_heads, int64_t head_dim,
                     int64_t max_seq, int64_t window, float* ws, float* out, hipStream_t s) {
    if (kv_heads <= 0 || n_heads % kv_heads != 0 || n_heads / kv_heads > ATTN_MAX_GROUPS || head_dim != 128 ||
        kv_heads > 64 || aeth_cdiv(max_seq, ATTN_T) > ATTN_MAX_CHUNKS)
        return aeth_set_error(AETH_EUNSUPPORTED, "attn: unsupported heads=%lld kv_heads=%lld head_dim=%lld max_seq=%lld",
                              (long long)n_heads, (long long)kv_heads, (long long)head_dim, (long long)max_seq);
    AttnArgs A;
    A.q = q;
    A.qkv = qkv;
    A.layer_kv = layer_kv;
    A.sin_t = sin_t;
    A.cos_t = cos_t;
    A.st = d_st;
    A.seq_host = seq;
    A.n_heads = (int)n_heads;
    A.kv_heads = (int)kv_heads;
    A.head_dim = (int)head_dim;
    A.max_seq = max_seq;
    A.window = window > 0 ? window : 0;
    A.max_chunks = (int)aeth_cdiv(max_seq, ATTN_T);
    A.ws = ws;
    A.out = out;
    const int grid_chunks = d_st ? A.max_chunks : (int)aeth_cdiv(min(seq, max_seq), ATTN_T);
    if (grid_chunks <= 0) return AETH_OK;
    hipLaunchKernelGGL((k_attn<128, ATTN_NT>), dim3((unsigned)kv_heads, (unsigned)grid_chunks), dim3(ATTN_NT), 0, s, A);
    AETH_LAUNCH_CHECK();
    hipLaunchKernelGGL(k_attn_merge<128>, dim3((unsigned)n_heads), dim3(128), 0, s, A);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}

// ── SiLU glue (runner.rs:1617-1625; sigmoid :1749-1751): g = g·σ(g)·up.
__global__ void k_silu_mul(float* __restrict__ g, const float* __restrict__ up, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float v = g[i];
    g[i] = v * (1.0f / (1.0f + expf(-v))) * up[i];
}

int aeth_silu_mul_launch(float* g, const float* up, int64_t n, hipStream_t s) {
    if (n <= 0) return AETH_OK;
    hipLaunchKernelGGL(k_silu_mul, dim3((unsigned)aeth_cdiv(n, 256)), dim3(256), 0, s, g, up, n);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}

__global__ void k_add(float* __restrict__ x, const float* __restrict__ y, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = x[i] + y[i];
}

int aeth_add_launch(float* x, const float* y, int64_t n, hipStream_t s) {
    if (n <= 0) return AETH_OK;
    hipLaunchKernelGGL(k_add, dim3((unsigned)aeth_cdiv(n, 256)), dim3(256), 0, s, x, y, n);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}

// ── Greedy argmax, last maximal index on ties (Iterator::max_by keeps the last
// of equal elements; runner.rs:1964-1973, c_api.rs:384-396). Two passes:
// ARGMAX_WG partial (value, index) pairs, then one workgroup merges them.
#define ARGMAX_WG 256

__device__ __forceinline__ void am_merge(float& bv, int& bi, float v, int i) {
    if (v > bv || (v == bv && i > bi)) { bv = v; bi = i; }
}

__device__ __forceinline__ void am_block(float& bv, int& bi) {
    __shared__ float sv[4];
    __shared__ int si[4];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        float ov = __shfl_xor(bv, off, 64);
        int oi = __shfl_xor(bi, off, 64);
        am_merge(bv, bi, ov, oi);
    }
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = bv; si[threadIdx.x >> 6] = bi; }
    __syncthreads();
    bv = sv[0]; bi = si[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); w++) am_merge(bv, bi, sv[w], si[w]);
}

__global__ void __launch_bounds__(256) k_argmax_partial(const float* __restrict__ x, int64_t n, float* pv, int* pi) {
    float bv = -INFINITY;
    int bi = -1;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        am_merge(bv, bi, x[i], (int)i);
    am_block(bv, bi);
    if (threadIdx.x == 0) { pv[blockIdx.x] = bv; pi[blockIdx.x] = bi; }
}

__global__ void __launch_bounds__(256) k_argmax_final(const float* pv, const int* pi, int np, int* out,
                                                      int* next_token) {
    float bv = -INFINITY;
    int bi = -1;
    for (int i = threadIdx.x; i < np; i += 256) am_merge(bv, bi, pv[i], pi[i]);
    am_block(bv, bi);
    if (threadIdx.x == 0) {
        int r = bi < 0 ? 0 : bi;
        out[0] = r;
        if (next_token) next_token[0] = r;
    }
}

int64_t aeth_argmax_ws_bytes() { return ARGMAX_WG * 8; }

int aeth_argmax_launch(const float* x, int64_t n, int* out, int* next_token, void* ws, hipStream_t s) {
    if (n <= 0) return aeth_set_error(AETH_EINVAL, "argmax: empty input");
    if (n > 0x7FFFFFFF) return aeth_set_error(AETH_EINVAL, "argmax: n too large");
    float* pv = (float*)ws;
    int* pi = (int*)(pv + ARGMAX_WG);
    int grid = (int)min((int64_t)ARGMAX_WG, aeth_cdiv(n, 256));
    hipLaunchKernelGGL(k_argmax_partial, dim3(grid), dim3(256), 0, s, x, n, pv, pi);
    AETH_LAUNCH_CHECK();
    hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(256), 0, s, pv, pi, grid, out, next_token);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}

// ── embedding row gather (runner.rs:1214-1215) with a device token id.
__global__ void k_embed(const float* __restrict__ table, const int* d_token, int64_t token, int64_t d, int64_t vocab,
                        float* __restrict__ x) {
    int64_t t = scalar_or(d_token, token);
    if (t < 0) t = 0;
    if (t >= vocab) t = vocab - 1;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < d; i += (int64_t)gridDim.x * blockDim.x)
        x[i] = table[t * d + i];
}

int aeth_embed_launch(const float* table, const int* d_token, int64_t token, int64_t d, int64_t vocab, float* x,
                      hipStream_t s) {
    hipLaunchKernelGGL(k_embed, dim3((unsigned)min((int64_t)64, aeth_cdiv(d, 256))), dim3(256), 0, s, table, d_token,
                       token, d, vocab, x);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}

// Advances the device decode state {token, pos, fill} after a step:
// StaticKVCache::advance (kv_cache.rs:67-71) and pos += 1; the next token was
// written by the argmax.
__global__ void k_state_advance(int* st, unsigned long long* amax, int* hist, int64_t max_seq) {
    if (threadIdx.x == 0 && blockIdx.x == 0) {
        if (amax) {
            st[0] = (int)(uint32_t)(*amax & 0xFFFFFFFFull);
            st[3] = st[0];
            *amax = 0ull;
            if (hist && st[4] >= 0 && st[4] < max_seq) hist[st[4]++] = st[0];  // the step's token, by step
        }
        st[1] += 1;
        if (st[2] < max_seq) st[2] += 1;
    }
}

int aeth_state_advance_launch(int* st, unsigned long long* amax, int* hist, int64_t max_seq, hipStream_t s) {
    hipLaunchKernelGGL(k_state_advance, dim3(1), dim3(64), 0, s, st, amax, hist, max_seq);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}
