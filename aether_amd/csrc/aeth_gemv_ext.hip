// VALU GEMVs for the weight formats without a fused matrix-core kernel:
// F32, F16, Q2_K and Q3_K.
//
//  * GGUF order (AETH_ORDER_GGUF): load_quant keeps these formats as the file
//    holds them, [k][n] (model_loader.rs:344-350), and quantized_matmul_impl
//    multiplies them by dequantize(b, [k, n]) + matmul_f32_gguf
//    (dispatch.rs:126-133, 541-574): c[j] = fma(a_i, b[i·n + j], c[j]) over i,
//    rows with a_i == 0 skipped. Here workgroup (unit u, split s, row group)
//    owns outputs j ∈ [256u, 256u + 256) and inputs i ∈ split s; its four waves
//    take every fourth i, each lane four outputs, one FMA per (row, output) per
//    i with the same zero skip (n % 4 == 0; K-quant blocks may straddle rows). Partials [s][row][j] are then summed in split
//    order by k_col_reduce, which also applies accumulate and the argmax key.
//  * Rows (AETH_ORDER_ROWS): matmul_f16 / matmul_q2_k / matmul_q3_k on [n][k]
//    row blocks (f16.rs, q2_k.rs, q3_k.rs; x86: avx2.rs:210-389). A wave per
//    output row, lanes four elements of each 256-element unit, a wave sum at
//    the end.
//
// Weights are formed exactly as dequant.rs rounds them (contraction off):
// Q2_K d·(sc & 15)·q − dmin·(sc >> 4), Q3_K (d·sc)·q, F16 exact; only the
// summation order differs from the reference.
//
// Lanes own four consecutive elements of the weight's flat element run
// (f, f+1, f+2, f+3 with f % 4 == 0, so they share one K-quant block and
// sub-block): lane l of a 256-wide unit takes its elements 4l .. 4l+3.
#include "aeth_common.hpp"
#include "aeth_internal.hpp"
#include "aeth_ops_internal.hpp"

#pragma clang fp contract(off)

namespace {

template <int F> struct XU;

// Each format splits into load (the raw words a lane needs, issued for a whole
// batch of inputs before any is used) and expand (the four f32 weights).

// dequant_q2_k (dequant.rs:350-398): 84-byte block [d][dmin][scales 16][qs 64];
// element e = 128h + 32t + 16v + i is bits 2t of qs[32h + 16v + i], sub-block
// 8h + 2t + v. Blocks are 4-byte aligned (84 = 4·21) and so are the lane's 4 qs bytes.
template <> struct XU<AETH_DTYPE_Q2_K> {
    struct Raw { uint32_t dd, sc, q; int t; };
    __device__ static Raw load(const uint8_t* W, int64_t f) {
        const uint8_t* b = W + (f >> 8) * Q2K_BLOCK_BYTES;
        const int e = (int)(f & 255), h = e >> 7, t = (e >> 5) & 3, v = (e >> 4) & 1;
        Raw r;
        r.dd = *(const uint32_t*)b;
        r.sc = b[4 + 8 * h + 2 * t + v];
        r.q = *(const uint32_t*)(b + 20 + 32 * h + 16 * v + (e & 15));
        r.t = t;
        return r;
    }
    __device__ static void expand(const Raw& r, float (&w)[4]) {
        const float d = aeth_decode_d(r.dd & 0xFFFFu), dmin = aeth_decode_d(r.dd >> 16);
        const float dl = d * (float)(r.sc & 0xF), ml = dmin * (float)(r.sc >> 4);
#pragma unroll
        for (int c = 0; c < 4; c++) w[c] = dl * (float)((r.q >> (8 * c + 2 * r.t)) & 3) - ml;
    }
};

// dequant_q3_k (dequant.rs:400-451): 110-byte block [hmask 32][qs 64][scales 12][d]
// (2-byte aligned); element e = 128h + 32t + 16v + i: bits 2t of
// qs[32h + 16v + i], bit 4h + t of hmask[16v + i], 6-bit scale of sub-block
// s = 8h + 2t + v (low nibble of scales[s % 8], high pair from scales[8 + s % 4]),
// q = ql − 4·(1 − hbit), w = (d·(scale − 32))·q.
template <> struct XU<AETH_DTYPE_Q3_K> {
    struct Raw { uint32_t q, hm, lob, hib, d; int e; };
    __device__ static Raw load(const uint8_t* W, int64_t f) {
        const uint8_t* b = W + (f >> 8) * Q3K_BLOCK_BYTES;
        const int e = (int)(f & 255), h = e >> 7, t = (e >> 5) & 3, v = (e >> 4) & 1, i = e & 15;
        const uint16_t* qp = (const uint16_t*)(b + 32 + 32 * h + 16 * v + i);
        const uint16_t* hp = (const uint16_t*)(b + 16 * v + i);
        const int s = 8 * h + 2 * t + v;
        Raw r;
        r.q = (uint32_t)qp[0] | ((uint32_t)qp[1] << 16);
        r.hm = (uint32_t)hp[0] | ((uint32_t)hp[1] << 16);
        r.lob = b[96 + (s & 7)];
        r.hib = b[104 + (s & 3)];
        r.d = *(const uint16_t*)(b + 108);
        r.e = e;
        return r;
    }
    __device__ static void expand(const Raw& r, float (&w)[4]) {
        const int h = r.e >> 7, t = (r.e >> 5) & 3, v = (r.e >> 4) & 1, s = 8 * h + 2 * t + v;
        const int sc = (int)((s < 8 ? (r.lob & 0xF) : (r.lob >> 4)) | (((r.hib >> (2 * (s >> 2))) & 3) << 4)) - 32;
        const float dl = aeth_decode_d(r.d) * (float)sc;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int ql = (int)((r.q >> (8 * c + 2 * t)) & 3), hb = (int)((r.hm >> (8 * c + 4 * h + t)) & 1);
            w[c] = dl * (float)(ql - ((hb ^ 1) << 2));
        }
    }
};

template <> struct XU<AETH_DTYPE_F16> {
    typedef uint2 Raw;
    __device__ static Raw load(const uint8_t* W, int64_t f) { return *(const uint2*)(W + 2 * f); }
    __device__ static void expand(const Raw& v, float (&w)[4]) {
        w[0] = aeth_f16_to_f32(v.x & 0xFFFFu);
        w[1] = aeth_f16_to_f32(v.x >> 16);
        w[2] = aeth_f16_to_f32(v.y & 0xFFFFu);
        w[3] = aeth_f16_to_f32(v.y >> 16);
    }
};

template <> struct XU<AETH_DTYPE_F32> {
    typedef float4 Raw;
    __device__ static Raw load(const uint8_t* W, int64_t f) { return *(const float4*)(W + 4 * f); }
    __device__ static void expand(const Raw& v, float (&w)[4]) {
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    }
};

// GGUF order: partials part[s][row][j] of Σ_{i ∈ split s} x[row][i]·W[i][j]
// (element (i, j) is flat element i·n + j; n % 4 == 0). NW waves take every
// NW-th input of the split, NB inputs per batch with all loads issued first.
template <int F, int R, int NW>
__global__ void __launch_bounds__(64 * NW) k_col(const uint8_t* __restrict__ W, int64_t n, int64_t k,
                                                 const float* __restrict__ x, int64_t ldx, int m, int S,
                                                 float* __restrict__ part) {
    constexpr int NB = 8;
    typedef typename XU<F>::Raw Raw;
    __shared__ float4 red[NW][R][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t j0 = (int64_t)blockIdx.x * 256 + 4 * lane;  // this lane's first output
    const int s = blockIdx.y, r0 = blockIdx.z * R;
    const int64_t i0 = k * s / S, i1 = k * (s + 1) / S;
    float acc[R][4];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int t = 0; t < 4; t++) acc[r][t] = 0.0f;
    const float* xr[R];
#pragma unroll
    for (int r = 0; r < R; r++) xr[r] = x + (int64_t)min(r0 + r, m - 1) * ldx;
    const int64_t jl = j0 < n ? j0 : n - 4;  // lanes past n read the last valid group, discarded
    for (int64_t ib = i0 + wave; ib < i1; ib += NW * NB) {
        Raw raw[NB];
        float xv[NB][R];
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const int64_t i = ib + (int64_t)b * NW, ic = i < i1 ? i : i1 - 1;
            raw[b] = XU<F>::load(W, ic * n + jl);
#pragma unroll
            for (int r = 0; r < R; r++) xv[b][r] = i < i1 ? xr[r][ic] : 0.0f;  // past the split: skipped as 0
        }
#pragma unroll
        for (int b = 0; b < NB; b++) {
            float w[4];
            XU<F>::expand(raw[b], w);
#pragma unroll
            for (int r = 0; r < R; r++) {
                const float a = xv[b][r];
                if (a != 0.0f) {  // matmul_f32_gguf skips zero activations (dispatch.rs:548)
#pragma unroll
                    for (int t = 0; t < 4; t++) acc[r][t] = fmaf(a, w[t], acc[r][t]);
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) red[wave][r][lane] = make_float4(acc[r][0], acc[r][1], acc[r][2], acc[r][3]);
    __syncthreads();
    const float* rf = (const float*)red;
    for (int idx = threadIdx.x; idx < R * 256; idx += 64 * NW) {
        const int r = idx >> 8, e = idx & 255;
        const int64_t j = (int64_t)blockIdx.x * 256 + e;
        if (j >= n || r0 + r >= m) continue;
        float v = rf[r * 256 + e];
#pragma unroll
        for (int wv = 1; wv < NW; wv++) v += rf[(wv * R + r) * 256 + e];
        part[((int64_t)s * m + r0 + r) * n + j] = v;
    }
}

// Σ over the S splits, then y = (accumulate ? y : 0) + Σ, and the argmax key.
// G lanes (a power of two ≥ S, at most 64) share one output: lane g loads the
// partials of splits g, g + G, …, and the G lanes combine in a fixed
// butterfly, so the result does not depend on scheduling.
template <int G>
__global__ void __launch_bounds__(256) k_col_reduce(const float* __restrict__ part, int S, int64_t m, int64_t n,
                                                    float* __restrict__ y, int64_t ldy, int accumulate,
                                                    unsigned long long* __restrict__ amax) {
    const int64_t idx = ((int64_t)blockIdx.x * 256 + threadIdx.x) / G;
    const int g = threadIdx.x & (G - 1);
    const bool live = idx < m * n;
    const int64_t row = live ? idx / n : 0, j = live ? idx - row * n : 0;
    float v = 0.0f;
    if (live)
        for (int s = g; s < S; s += G) v += part[((int64_t)s * m + row) * n + j];
#pragma unroll
    for (int off = G / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    unsigned long long best = 0;
    if (live && g == 0) {
        float* dst = y + row * ldy + j;
        if (accumulate) v = *dst + v;
        *dst = v;
        if (amax) best = aeth_amax_key(v, j);
    }
    if (amax) {
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const unsigned long long o = __shfl_xor(best, off, 64);
            best = o > best ? o : best;
        }
        if ((threadIdx.x & 63) == 0 && best) atomicMax(amax, best);
    }
}

// Rows: y[row][j] = Σ_e x[row][e]·W[j][e], a wave per output j, R rows.
// Row j's elements start at flat element j·row_elems (K-quants: k/256 whole
// blocks per row; F16: k values, k % 4 == 0); NB units per batch, loads first.
template <int F, int R>
__global__ void __launch_bounds__(256) k_row(const uint8_t* __restrict__ W, int64_t n, int64_t kr, int64_t row_elems,
                                             const float* __restrict__ x, int64_t ldx, int m, float* __restrict__ y,
                                             int64_t ldy, int accumulate) {
    constexpr int NB = 4;
    typedef typename XU<F>::Raw Raw;
    const int lane = threadIdx.x & 63;
    const int64_t j = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r0 = blockIdx.y * R;
    if (j >= n) return;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    const float* xr[R];
#pragma unroll
    for (int r = 0; r < R; r++) xr[r] = x + (int64_t)min(r0 + r, m - 1) * ldx;
    for (int64_t eb = 4 * lane; eb < kr + 4 * lane; eb += 256 * NB) {  // kr: elements per row (a multiple of 4)
        Raw raw[NB];
        float4 xv[NB][R];
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const int64_t e = eb + 256 * b, ec = e < kr ? e : kr - 4;
            raw[b] = XU<F>::load(W, j * row_elems + ec);
#pragma unroll
            for (int r = 0; r < R; r++) {
                xv[b][r] = *(const float4*)(xr[r] + ec);
                if (e >= kr) xv[b][r] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
        }
#pragma unroll
        for (int b = 0; b < NB; b++) {
            float w[4];
            XU<F>::expand(raw[b], w);
#pragma unroll
            for (int r = 0; r < R; r++) {
                acc[r] = fmaf(xv[b][r].x, w[0], acc[r]);
                acc[r] = fmaf(xv[b][r].y, w[1], acc[r]);
                acc[r] = fmaf(xv[b][r].z, w[2], acc[r]);
                acc[r] = fmaf(xv[b][r].w, w[3], acc[r]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
        const float v = aeth_wave_sum(acc[r]);
        if (lane == 0 && r0 + r < m) {
            float* dst = y + (int64_t)(r0 + r) * ldy + j;
            *dst = accumulate ? *dst + v : v;
        }
    }
}

template <int F>
int launch_col(const aeth_weight* w, const float* x, int64_t m, float* y, int64_t ldy, const GemvEpi& e,
               float* part, int S, hipStream_t s) {
    const int64_t units = aeth_cdiv(w->n, 256);
    if (m == 1) {
        const dim3 grid((unsigned)units, (unsigned)S, 1);
        hipLaunchKernelGGL((k_col<F, 1, 8>), grid, dim3(512), 0, s, w->p0, w->n, w->k, x, w->k, 1, S, part);
    } else {
        const dim3 grid((unsigned)units, (unsigned)S, (unsigned)aeth_cdiv(m, 8));
        hipLaunchKernelGGL((k_col<F, 8, 4>), grid, dim3(256), 0, s, w->p0, w->n, w->k, x, w->k, (int)m, S, part);
    }
    AETH_LAUNCH_CHECK();
    const int64_t tot = m * w->n;
    const int acc = (e.flags & AETH_MM_ACCUMULATE) ? 1 : 0;
#define AETH_COL_REDUCE(G)                                                                                       \
    hipLaunchKernelGGL(k_col_reduce<G>, dim3((unsigned)aeth_cdiv(tot * G, 256)), dim3(256), 0, s, part, S, m,   \
                       w->n, y, ldy, acc, e.amax)
    if (S <= 1) AETH_COL_REDUCE(1);
    else if (S <= 4) AETH_COL_REDUCE(4);
    else if (S <= 16) AETH_COL_REDUCE(16);
    else AETH_COL_REDUCE(64);
#undef AETH_COL_REDUCE
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}

template <int F>
int launch_row(const aeth_weight* w, const float* x, int64_t m, float* y, int64_t ldy, unsigned flags, hipStream_t s) {
    const bool f16 = F == AETH_DTYPE_F16;
    const int64_t kr = f16 ? w->k : w->k / 256 * 256, row_elems = kr;
    const int R = m == 1 ? 1 : 8;
    const dim3 grid((unsigned)aeth_cdiv(w->n, 4), (unsigned)aeth_cdiv(m, R));
    const int acc = (flags & AETH_MM_ACCUMULATE) ? 1 : 0;
    if (R == 1)
        hipLaunchKernelGGL((k_row<F, 1>), grid, dim3(256), 0, s, w->p0, w->n, kr, row_elems, x, w->k, (int)m, y, ldy,
                           acc);
    else
        hipLaunchKernelGGL((k_row<F, 8>), grid, dim3(256), 0, s, w->p0, w->n, kr, row_elems, x, w->k, (int)m, y, ldy,
                           acc);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}

// Splits of k for a GGUF-order launch: enough workgroups to cover the chip
// (≈ 4 per CU), at least one batch of inputs (8 per wave) per wave.
int col_splits(const aeth_weight* w, int64_t m) {
    const int64_t units = aeth_cdiv(w->n, 256), groups = m == 1 ? 1 : aeth_cdiv(m, 8);
    const int64_t per_wave_batch = m == 1 ? 64 : 32;  // NW·NB inputs
    int64_t S = aeth_cdiv(4LL * aeth_num_cus(), units * groups);
    const int64_t smax = w->k / per_wave_batch > 1 ? w->k / per_wave_batch : 1;
    S = S < 1 ? 1 : S > 128 ? 128 : S;
    return (int)(S < smax ? S : smax);
}

}  // namespace

int64_t aeth_xgemv_ws_floats(const aeth_weight* w, int64_t m) {
    if (!w || w->order != AETH_ORDER_GGUF || m <= 0) return 0;
    return (int64_t)col_splits(w, m) * m * w->n + m * w->k;  // partials + a normed copy of x
}

int aeth_xgemv_launch(const aeth_weight* w, const float* d_x, int64_t m, float* d_y, const GemvEpi& e,
                      hipStream_t s) {
    if (m <= 0 || m > 65535) return aeth_set_error(AETH_EINVAL, "gemv: m=%lld out of range", (long long)m);
    if (e.swiglu) return aeth_set_error(AETH_EUNSUPPORTED, "gemv: fused SwiGLU needs a planar weight");
    const int64_t ldy = e.ldc ? e.ldc : w->n;
    if (w->order == AETH_ORDER_ROWS) {
        if (((uintptr_t)d_x & 15) || (m > 1 && (w->k & 3)))  // float4 activation loads
            return aeth_set_error(AETH_EINVAL, "gemv: x rows must be 16-byte aligned");
        if (e.norm_w || e.amax)
            return aeth_set_error(AETH_EUNSUPPORTED, "gemv: row-order weights take no fused norm or argmax");
        switch (w->dtype) {
            case AETH_DTYPE_F16: return launch_row<AETH_DTYPE_F16>(w, d_x, m, d_y, ldy, e.flags, s);
            case AETH_DTYPE_Q2_K: return launch_row<AETH_DTYPE_Q2_K>(w, d_x, m, d_y, ldy, e.flags, s);
            case AETH_DTYPE_Q3_K: return launch_row<AETH_DTYPE_Q3_K>(w, d_x, m, d_y, ldy, e.flags, s);
            default: return aeth_set_error(AETH_EUNSUPPORTED, "gemv: no row kernel for dtype %d", w->dtype);
        }
    }
    if (w->order != AETH_ORDER_GGUF) return aeth_set_error(AETH_EINVAL, "gemv: weight order %d", w->order);
    const int S = col_splits(w, m);
    const int64_t need = aeth_xgemv_ws_floats(w, m);
    float* ws = e.ws;
    if (ws && e.ws_floats < need)
        return aeth_set_error(AETH_EINVAL, "gemv: scratch of %lld floats < %lld needed", (long long)e.ws_floats,
                              (long long)need);
    if (!ws) {  // the library's scratch of this stream
        void* p = nullptr;
        int rc = aeth_stream_scratch(s, AETH_SCRATCH_XGEMV, (size_t)need * sizeof(float), &p);
        if (rc) return rc;
        ws = (float*)p;
    }
    float* part = ws;
    const float* x = d_x;
    if (e.norm_w) {  // rmsnorm_inplace (runner.rs:1739-1746) into the scratch, then the product
        float* xn = ws + (int64_t)S * m * w->n;
        int rc = aeth_rmsnorm_launch(d_x, e.norm_w, m, w->k, e.eps, xn, s);
        if (rc) return rc;
        x = xn;
    }
    switch (w->dtype) {
        case AETH_DTYPE_F32: return launch_col<AETH_DTYPE_F32>(w, x, m, d_y, ldy, e, part, S, s);
        case AETH_DTYPE_F16: return launch_col<AETH_DTYPE_F16>(w, x, m, d_y, ldy, e, part, S, s);
        case AETH_DTYPE_Q2_K: return launch_col<AETH_DTYPE_Q2_K>(w, x, m, d_y, ldy, e, part, S, s);
        case AETH_DTYPE_Q3_K: return launch_col<AETH_DTYPE_Q3_K>(w, x, m, d_y, ldy, e, part, S, s);
        default: return aeth_set_error(AETH_EUNSUPPORTED, "gemv: no GGUF-order kernel for dtype %d", w->dtype);
    }
}
