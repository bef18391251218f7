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

// ── GQA decode attention (runner.rs:1579-1603, attn_direct :1757-1801).
// Pass 1: workgroup (kv_head, chunk of ATTN_T positions) computes, for each of
// its `groups` query heads, the chunk's max score m, Σexp(s−m) and
// Σexp(s−m)·v. Pass 2 merges the chunks: out = Σ e^{m_c−M} o_c / Σ e^{m_c−M} l_c.
// seq may come from the device (d_seq: cache fill + 1 after append); grids are
// sized for the largest seq and surplus chunks exit.
#define ATTN_T 64
#define ATTN_MAX_GROUPS 8

__global__ void __launch_bounds__(256) k_attn_partial(const float* __restrict__ q, const float* __restrict__ layer_kv,
                                                      int n_heads, int kv_heads, int head_dim, int64_t max_seq,
                                                      const int* d_seq, int64_t seq_v, int seq_add,
                                                      float* __restrict__ ws, int max_chunks) {
    __shared__ float qs[ATTN_MAX_GROUPS][256];
    __shared__ float ps[ATTN_MAX_GROUPS][ATTN_T];
    const int kvh = blockIdx.y;
    const int chunk = blockIdx.x;
    int64_t seq = scalar_or(d_seq, seq_v) + seq_add;
    if (seq > max_seq) seq = max_seq;
    const int64_t t0 = (int64_t)chunk * ATTN_T;
    if (t0 >= seq) return;
    const int groups = n_heads / kv_heads;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float scale = 1.0f / sqrtf((float)head_dim);
    const int64_t hs = max_seq * head_dim;
    const float* K = layer_kv + (int64_t)kvh * hs;
    const float* V = layer_kv + (int64_t)kv_heads * hs + (int64_t)kvh * hs;
    for (int i = tid; i < groups * head_dim; i += 256) qs[i / head_dim][i % head_dim] = q[(int64_t)(kvh * groups) * head_dim + i];
    __syncthreads();
    const int nt = (int)min((int64_t)ATTN_T, seq - t0);
    // scores: wave w handles heads w, w+4, ...; lane = position
    for (int g = wave; g < groups; g += 4) {
        float s = -INFINITY;
        if (lane < nt) {
            const float4* kr = (const float4*)(K + (t0 + lane) * head_dim);
            float dot = 0.0f;
            for (int e = 0; e < head_dim / 4; e++) {
                float4 kv4 = kr[e];
                dot += qs[g][4 * e] * kv4.x;
                dot += qs[g][4 * e + 1] * kv4.y;
                dot += qs[g][4 * e + 2] * kv4.z;
                dot += qs[g][4 * e + 3] * kv4.w;
            }
            s = dot * scale;
        }
        float m = aeth_wave_max(s);
        float p = lane < nt ? expf(s - m) : 0.0f;
        float l = aeth_wave_sum(p);
        ps[g][lane] = p;
        if (lane == 0) {
            float* meta = ws + ((int64_t)(kvh * groups + g) * max_chunks + chunk) * (head_dim + 2);
            meta[head_dim] = m;
            meta[head_dim + 1] = l;
        }
    }
    __syncthreads();
    // weighted V: thread handles dims d = tid, tid+256 for every head
    for (int d = tid; d < head_dim; d += 256) {
        float o[ATTN_MAX_GROUPS];
#pragma unroll
        for (int g = 0; g < ATTN_MAX_GROUPS; g++) o[g] = 0.0f;
        for (int t = 0; t < nt; t++) {
            float vv = V[(t0 + t) * head_dim + d];
#pragma unroll
            for (int g = 0; g < ATTN_MAX_GROUPS; g++)
                if (g < groups) o[g] += ps[g][t] * vv;
        }
#pragma unroll
        for (int g = 0; g < ATTN_MAX_GROUPS; g++)
            if (g < groups) ws[((int64_t)(kvh * groups + g) * max_chunks + chunk) * (head_dim + 2) + d] = o[g];
    }
}

__global__ void __launch_bounds__(256) k_attn_combine(const float* __restrict__ ws, int head_dim, int64_t max_seq,
                                                      const int* d_seq, int64_t seq_v, int seq_add, int max_chunks,
                                                      float* __restrict__ out) {
    const int h = blockIdx.x;
    int64_t seq = scalar_or(d_seq, seq_v) + seq_add;
    if (seq > max_seq) seq = max_seq;
    const int nch = (int)((seq + ATTN_T - 1) / ATTN_T);
    const float* base = ws + (int64_t)h * max_chunks * (head_dim + 2);
    float M = -INFINITY;
    for (int c = 0; c < nch; c++) M = fmaxf(M, base[(int64_t)c * (head_dim + 2) + head_dim]);
    float L = 0.0f;
    for (int c = 0; c < nch; c++) {
        const float* mc = base + (int64_t)c * (head_dim + 2);
        L += expf(mc[head_dim] - M) * mc[head_dim + 1];
    }
    for (int d = threadIdx.x; d < head_dim; d += blockDim.x) {
        float acc = 0.0f;
        for (int c = 0; c < nch; c++) {
            const float* mc = base + (int64_t)c * (head_dim + 2);
            acc += expf(mc[head_dim] - M) * mc[d];
        }
        out[(int64_t)h * head_dim + d] = acc / L;
    }
}

int64_t aeth_attn_ws_floats(int64_t n_heads, int64_t head_dim, int64_t max_seq) {
    return n_heads * aeth_cdiv(max_seq, ATTN_T) * (head_dim + 2);
}

int aeth_attn_decode_launch(const float* q, const float* layer_kv, int64_t n_heads, int64_t kv_heads,
                            int64_t head_dim, int64_t max_seq, const int* d_seq, int64_t seq, int seq_add,
                            float* ws, float* out, hipStream_t s) {
    if (kv_heads <= 0 || n_heads % kv_heads != 0 || n_heads / kv_heads > ATTN_MAX_GROUPS || head_dim % 4 != 0 ||
        head_dim > 256)
        return aeth_set_error(AETH_EUNSUPPORTED, "attn: unsupported heads=%lld kv_heads=%lld head_dim=%lld",
                              (long long)n_heads, (long long)kv_heads, (long long)head_dim);
    int max_chunks = (int)aeth_cdiv(max_seq, ATTN_T);
    int grid_chunks = d_seq ? max_chunks : (int)aeth_cdiv(min(seq + seq_add, max_seq), ATTN_T);
    if (grid_chunks <= 0) return AETH_OK;
    hipLaunchKernelGGL(k_attn_partial, dim3(grid_chunks, (unsigned)kv_heads), dim3(256), 0, s, q, layer_kv,
                       (int)n_heads, (int)kv_heads, (int)head_dim, max_seq, d_seq, seq, seq_add, ws, max_chunks);
    AETH_LAUNCH_CHECK();
    hipLaunchKernelGGL(k_attn_combine, dim3((unsigned)n_heads), dim3(128), 0, s, ws, (int)head_dim, max_seq, d_seq,
                       seq, seq_add, max_chunks, out);
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
__global__ void k_state_advance(int* st, int64_t max_seq) {
    if (threadIdx.x == 0 && blockIdx.x == 0) {
        st[1] += 1;
        if (st[2] < max_seq) st[2] += 1;
    }
}

int aeth_state_advance_launch(int* st, int64_t max_seq, hipStream_t s) {
    hipLaunchKernelGGL(k_state_advance, dim3(1), dim3(64), 0, s, st, max_seq);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}
