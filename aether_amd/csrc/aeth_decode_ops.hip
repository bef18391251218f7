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

int aeth_rmsnorm_launch(const float* x, const float* w, int64_t rows, int64_t n, float eps, float* out,
                        hipStream_t s) {
    if (rows <= 0 || n <= 0) return AETH_OK;
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
// Workgroup (chunk c, kv head h) covers positions [64c, 64c+64) of the
// sequence [0, seq) for the `groups` query heads sharing h. It writes the
// chunk's softmax partials (max m, Σe^{s-m}, Σe^{s-m}·v); k_attn_merge then
// combines them: out = Σ_c e^{m_c-M} o_c / Σ_c e^{m_c-M} l_c.
//
// With `qkv` set, q/k/v come unrotated from the fused projection output
// [q (n_heads·hd) | k (kv_heads·hd) | v (kv_heads·hd)]: q and the new k are
// rotated here with the table row min(pos, max_seq-1), and the new token is
// position `fill` (the cache fill before this step; seq = fill + 1). The
// chunk holding it reads k/v from registers and stores them in the cache.
#define ATTN_T 64
#define ATTN_MAX_GROUPS 8
#define ATTN_MAX_CHUNKS 128  // max_seq <= 8192

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
    float* ws;           // [n_heads][max_chunks][hd + 2]
    int max_chunks;
    float* out;          // [n_heads][hd]
};

template <int HD>
__global__ void __launch_bounds__(256) k_attn(AttnArgs A) {
    constexpr int HALF = HD / 2;
    constexpr int TPP = HD / 16;   // threads per position in the score pass (16 dims each)
    constexpr int PPW = 256 / TPP;  // positions per score pass
    constexpr int VT = ATTN_T / 2;  // positions per thread in the V pass (two halves of the chunk)
    __shared__ float qs[ATTN_MAX_GROUPS][HD];
    __shared__ float knew[HD], vnew[HD];
    __shared__ float sc[ATTN_MAX_GROUPS][ATTN_T];
    __shared__ float ov[2][ATTN_MAX_GROUPS][HD];
    __shared__ float mstat[ATTN_MAX_GROUPS][2];
    const int kvh = blockIdx.y, chunk = blockIdx.x, tid = threadIdx.x;
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
    if (t0 >= seq) return;
    const int64_t hs = A.max_seq * HD;
    float* K = A.layer_kv + (int64_t)kvh * hs;
    float* V = A.layer_kv + (int64_t)A.kv_heads * hs + (int64_t)kvh * hs;
    const float scale = 1.0f / sqrtf((float)HD);
    int64_t prow = pos;
    if (prow > A.max_seq - 1) prow = A.max_seq - 1;
    if (prow < 0) prow = 0;

    // q (rotated) for this kv head's query heads; the new k/v when fused
    if (A.qkv) {
        const float* qsrc = A.qkv + (int64_t)kvh * groups * HD;
        for (int i = tid; i < groups * HALF; i += 256) {
            const int g = i / HALF, e = i - g * HALF;
            const float x0 = qsrc[g * HD + e], x1 = qsrc[g * HD + e + HALF];
            const float sn = A.sin_t[prow * HALF + e], cs = A.cos_t[prow * HALF + e];
            qs[g][e] = x0 * cs - x1 * sn;
            qs[g][e + HALF] = x0 * sn + x1 * cs;
        }
        const float* ksrc = A.qkv + (int64_t)A.n_heads * HD + (int64_t)kvh * HD;
        const float* vsrc = A.qkv + (int64_t)(A.n_heads + A.kv_heads) * HD + (int64_t)kvh * HD;
        for (int e = tid; e < HALF; e += 256) {
            const float x0 = ksrc[e], x1 = ksrc[e + HALF];
            const float sn = A.sin_t[prow * HALF + e], cs = A.cos_t[prow * HALF + e];
            knew[e] = x0 * cs - x1 * sn;
            knew[e + HALF] = x0 * sn + x1 * cs;
        }
        for (int e = tid; e < HD; e += 256) vnew[e] = vsrc[e];
    } else {
        for (int i = tid; i < groups * HD; i += 256) qs[i / HD][i % HD] = A.q[(int64_t)kvh * groups * HD + i];
    }
    __syncthreads();
    const bool has_new = A.qkv && fill >= t0 && fill < t0 + ATTN_T && fill < A.max_seq;
    if (has_new) {  // StaticKVCache::append at slot `fill`
        for (int e = tid; e < HD; e += 256) {
            K[fill * HD + e] = knew[e];
            V[fill * HD + e] = vnew[e];
        }
    }
    const int nt = (int)min((int64_t)ATTN_T, seq - t0);

    // scores: TPP threads per position, 16 dims each; all passes' K loads first
    constexpr int NP = ATTN_T / PPW;
    float kk[NP][16];
#pragma unroll
    for (int pp = 0; pp < NP; pp++) {
        const int tp = pp * PPW + tid / TPP, part = tid % TPP;
        const int64_t t = t0 + tp;
        if (tp < nt && !(has_new && t == fill)) {
            const float4* kr = (const float4*)(K + t * HD + part * 16);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float4 v4 = kr[e];
                kk[pp][4 * e] = v4.x; kk[pp][4 * e + 1] = v4.y; kk[pp][4 * e + 2] = v4.z; kk[pp][4 * e + 3] = v4.w;
            }
        } else {
#pragma unroll
            for (int e = 0; e < 16; e++) kk[pp][e] = (tp < nt) ? knew[part * 16 + e] : 0.0f;
        }
    }
    // V rows of this thread's half-chunk are loaded right after K, in one batch, and
    // consumed after the softmax
    const int vd = tid % HD, vh = tid / HD;  // HD = 128: vh in {0, 1}
    float vv[VT];
#pragma unroll
    for (int i = 0; i < VT; i++) {
        const int tp = vh * VT + i;
        const int64_t t = t0 + tp;
        vv[i] = (tp < nt) ? ((has_new && t == fill) ? vnew[vd] : V[t * HD + vd]) : 0.0f;
    }

#pragma unroll
    for (int pp = 0; pp < NP; pp++) {
        const int tp = pp * PPW + tid / TPP, part = tid % TPP;
#pragma unroll
        for (int g = 0; g < ATTN_MAX_GROUPS; g++) {
            if (g < groups) {
                float a = 0.0f;
#pragma unroll
                for (int e = 0; e < 16; e++) a += qs[g][part * 16 + e] * kk[pp][e];
#pragma unroll
                for (int off = TPP / 2; off >= 1; off >>= 1) a += __shfl_xor(a, off, 64);
                if (part == 0) sc[g][tp] = tp < nt ? a * scale : -INFINITY;
            }
        }
    }
    __syncthreads();
    // per-head max / exp / sum over the chunk: wave w handles heads w, w+4
    {
        const int lane = tid & 63, wave = tid >> 6;
        for (int g = wave; g < groups; g += 4) {
            float sv = lane < ATTN_T ? sc[g][lane] : -INFINITY;
            float m = aeth_wave_max(sv);
            float pr = lane < nt ? expf(sv - m) : 0.0f;
            float l = aeth_wave_sum(pr);
            if (lane < ATTN_T) sc[g][lane] = pr;
            if (lane == 0) { mstat[g][0] = m; mstat[g][1] = l; }
        }
    }
    __syncthreads();
    // Σ p_t v_t over this thread's half-chunk
    {
        float o[ATTN_MAX_GROUPS];
#pragma unroll
        for (int g = 0; g < ATTN_MAX_GROUPS; g++) o[g] = 0.0f;
#pragma unroll
        for (int i = 0; i < VT; i++) {
#pragma unroll
            for (int g = 0; g < ATTN_MAX_GROUPS; g++)
                if (g < groups) o[g] += sc[g][vh * VT + i] * vv[i];
        }
#pragma unroll
        for (int g = 0; g < ATTN_MAX_GROUPS; g++)
            if (g < groups) ov[vh][g][vd] = o[g];
    }
    __syncthreads();
    for (int i = tid; i < groups * HD; i += 256) {
        const int g = i / HD, d = i - g * HD;
        float* dst = A.ws + ((int64_t)(kvh * groups + g) * A.max_chunks + chunk) * (HD + 2);
        dst[d] = ov[0][g][d] + ov[1][g][d];
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
template <int HD>
__global__ void __launch_bounds__(HD) k_attn_merge(AttnArgs A) {
    __shared__ float cw[ATTN_MAX_CHUNKS];
    __shared__ float cl;
    const int h = blockIdx.x, tid = threadIdx.x;
    int64_t seq = A.st ? (int64_t)A.st[2] + 1 : A.seq_host;
    if (seq > A.max_seq) seq = A.max_seq;
    const int nch = (int)((seq + ATTN_T - 1) / ATTN_T);
    const float* base = A.ws + (int64_t)h * A.max_chunks * (HD + 2);
    if (tid < 64) {
        float M = -INFINITY;
        for (int c = tid; c < nch; c += 64) M = fmaxf(M, base[(int64_t)c * (HD + 2) + HD]);
        M = aeth_wave_max(M);
        float L = 0.0f;
        for (int c = tid; c < nch; c += 64) {
            const float* mc = base + (int64_t)c * (HD + 2);
            const float w = expf(mc[HD] - M);
            cw[c] = w;
            L += w * mc[HD + 1];
        }
        L = aeth_wave_sum(L);
        if (tid == 0) cl = L;
    }
    __syncthreads();
    float acc = 0.0f;
    for (int c0 = 0; c0 < nch; c0 += 8) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = (c0 + j < nch) ? base[(int64_t)(c0 + j) * (HD + 2) + tid] : 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (c0 + j < nch) acc += cw[c0 + j] * v[j];
    }
    A.out[(int64_t)h * HD + tid] = acc / cl;
}

int64_t aeth_attn_ws_floats(int64_t n_heads, int64_t head_dim, int64_t max_seq) {
    return n_heads * aeth_cdiv(max_seq, ATTN_T) * (head_dim + 2);
}

// ws: aeth_attn_ws_floats(...) floats of chunk partials.
int aeth_attn_launch(const float* q, const float* qkv, float* layer_kv, const float* sin_t, const float* cos_t,
                     const int* d_st, int64_t seq, int64_t n_heads, int64_t kv_heads, int64_t head_dim,
                     int64_t max_seq, float* ws, float* out, hipStream_t s) {
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
    A.max_chunks = (int)aeth_cdiv(max_seq, ATTN_T);
    A.ws = ws;
    A.out = out;
    const int grid_chunks = d_st ? A.max_chunks : (int)aeth_cdiv(min(seq, max_seq), ATTN_T);
    if (grid_chunks <= 0) return AETH_OK;
    hipLaunchKernelGGL(k_attn<128>, dim3(grid_chunks, (unsigned)kv_heads), dim3(256), 0, s, A);
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
__global__ void k_state_advance(int* st, unsigned long long* amax, int64_t max_seq) {
    if (threadIdx.x == 0 && blockIdx.x == 0) {
        if (amax) {
            st[0] = (int)(uint32_t)(*amax & 0xFFFFFFFFull);
            st[3] = st[0];
            *amax = 0ull;
        }
        st[1] += 1;
        if (st[2] < max_seq) st[2] += 1;
    }
}

int aeth_state_advance_launch(int* st, unsigned long long* amax, int64_t max_seq, hipStream_t s) {
    hipLaunchKernelGGL(k_state_advance, dim3(1), dim3(64), 0, s, st, amax, max_seq);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}
