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

// dequant_q2_k (dequant.rs:350-398): 84-byte block [d][dmin][scales 16][qs 64];
// element e = 128h + 32t + 16v + i is bits 2t of qs[32h + 16v + i], sub-block
// 8h + 2t + v. Blocks are 4-byte aligned (84 = 4·21) and so are the lane's 4 qs bytes.
template <> struct XU<AETH_DTYPE_Q2_K> {
    __device__ static void decode(const uint8_t* W, int64_t f, float (&w)[4]) {
        const uint8_t* b = W + (f >> 8) * Q2K_BLOCK_BYTES;
        const int e = (int)(f & 255), h = e >> 7, t = (e >> 5) & 3, v = (e >> 4) & 1;
        const uint32_t dd = *(const uint32_t*)b;
        const float d = aeth_decode_d(dd & 0xFFFFu), dmin = aeth_decode_d(dd >> 16);
        const uint32_t sc = b[4 + 8 * h + 2 * t + v];
        const uint32_t q = *(const uint32_t*)(b + 20 + 32 * h + 16 * v + (e & 15));
        const float dl = d * (float)(sc & 0xF), ml = dmin * (float)(sc >> 4);
#pragma unroll
        for (int c = 0; c < 4; c++) w[c] = dl * (float)((q >> (8 * c + 2 * t)) & 3) - ml;
    }
};

// dequant_q3_k (dequant.rs:400-451): 110-byte block [hmask 32][qs 64][scales 12][d]
// (2-byte aligned); element e = 128h + 32t + 16v + i: bits 2t of
// qs[32h + 16v + i], bit 4h + t of hmask[16v + i], 6-bit scale of sub-block
// s = 8h + 2t + v (low nibble of scales[s % 8], high pair from scales[8 + s % 4]),
// q = ql − 4·(1 − hbit), w = (d·(scale − 32))·q.
template <> struct XU<AETH_DTYPE_Q3_K> {
    __device__ static void decode(const uint8_t* W, int64_t f, float (&w)[4]) {
        const uint8_t* b = W + (f >> 8) * Q3K_BLOCK_BYTES;
        const int e = (int)(f & 255), h = e >> 7, t = (e >> 5) & 3, v = (e >> 4) & 1, i = e & 15;
        const uint16_t* qp = (const uint16_t*)(b + 32 + 32 * h + 16 * v + i);
        const uint16_t* hp = (const uint16_t*)(b + 16 * v + i);
        const uint32_t q = (uint32_t)qp[0] | ((uint32_t)qp[1] << 16), hm = (uint32_t)hp[0] | ((uint32_t)hp[1] << 16);
        const int s = 8 * h + 2 * t + v;
        const uint32_t lob = b[96 + (s & 7)], hib = b[104 + (s & 3)];
        const int sc = (int)((s < 8 ? (lob & 0xF) : (lob >> 4)) | (((hib >> (2 * (s >> 2))) & 3) << 4)) - 32;
        const float dl = aeth_decode_d(*(const uint16_t*)(b + 108)) * (float)sc;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int ql = (int)((q >> (8 * c + 2 * t)) & 3), hb = (int)((hm >> (8 * c + 4 * h + t)) & 1);
            w[c] = dl * (float)(ql - ((hb ^ 1) << 2));
        }
    }
};

template <> struct XU<AETH_DTYPE_F16> {
    __device__ static void decode(const uint8_t* W, int64_t f, float (&w)[4]) {
        const uint2 v = *(const uint2*)(W + 2 * f);
        w[0] = aeth_f16_to_f32(v.x & 0xFFFFu);
        w[1] = aeth_f16_to_f32(v.x >> 16);
        w[2] = aeth_f16_to_f32(v.y & 0xFFFFu);
        w[3] = aeth_f16_to_f32(v.y >> 16);
    }
};

template <> struct XU<AETH_DTYPE_F32> {
    __device__ static void decode(const uint8_t* W, int64_t f, float (&w)[4]) {
        const float4 v = *(const float4*)(W + 4 * f);
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    }
};

// GGUF order: partials part[s][row][j] of Σ_{i ∈ split s} x[row][i]·W[i][j].
// GGUF order: partials part[s][row][j] of Σ_{i ∈ split s} x[row][i]·W[i][j]
// (element (i, j) is flat element i·n + j; n % 4 == 0).
template <int F, int R>
__global__ void __launch_bounds__(256) k_col(const uint8_t* __restrict__ W, int64_t n, int64_t k,
                                             const float* __restrict__ x, int64_t ldx, int m, int S,
                                             float* __restrict__ part) {
    __shared__ float4 red[4][R][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t j0 = (int64_t)blockIdx.x * 256 + 4 * lane;  // this lane's first output
    const bool live = j0 < n;
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
    const int64_t jl = live ? j0 : n - 4;  // lanes past n read the last valid group, discarded
#pragma unroll 2
    for (int64_t i = i0 + wave; i < i1; i += 4) {
        float w[4];
        XU<F>::decode(W, i * n + jl, w);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float a = xr[r][i];
            if (a != 0.0f) {  // matmul_f32_gguf skips zero activations (dispatch.rs:548)
#pragma unroll
                for (int t = 0; t < 4; t++) acc[r][t] = fmaf(a, w[t], acc[r][t]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) red[wave][r][lane] = make_float4(acc[r][0], acc[r][1], acc[r][2], acc[r][3]);
    __syncthreads();
    const int e = threadIdx.x;  // output 256·blockIdx.x + e
    const int64_t j = (int64_t)blockIdx.x * 256 + e;
    if (j >= n) return;
    const float* rf = (const float*)red;
#pragma unroll
    for (int r = 0; r < R; r++) {
        if (r0 + r >= m) break;
        const float v = ((rf[(0 * R + r) * 256 + e] + rf[(1 * R + r) * 256 + e]) + rf[(2 * R + r) * 256 + e]) +
                        rf[(3 * R + r) * 256 + e];
        part[((int64_t)s * m + r0 + r) * n + j] = v;
    }
}

// Σ over splits in order, then y = (accumulate ? y : 0) + Σ, and the argmax key.
__global__ void __launch_bounds__(256) k_col_reduce(const float* __restrict__ part, int S, int64_t m, int64_t n,
                                                    float* __restrict__ y, int64_t ldy, int accumulate,
                                                    unsigned long long* __restrict__ amax) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    unsigned long long best = 0;
    if (idx < m * n) {
        const int64_t row = idx / n, j = idx - row * n;
        float v = part[row * n + j];
        for (int s = 1; s < S; s++) v += part[((int64_t)s * m + row) * n + j];
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
// blocks per row; F16: k values, k % 4 == 0).
template <int F, int R>
__global__ void __launch_bounds__(256) k_row(const uint8_t* __restrict__ W, int64_t n, int64_t kr, int64_t row_elems,
                                             const float* __restrict__ x, int64_t ldx, int m, float* __restrict__ y,
                                             int64_t ldy, int accumulate) {
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
#pragma unroll 2
    for (int64_t e = 4 * lane; e < kr; e += 256) {  // kr = elements read per row (a multiple of 4)
        float w[4];
        XU<F>::decode(W, j * row_elems + e, w);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float4 xv = *(const float4*)(xr[r] + e);
            acc[r] = fmaf(xv.x, w[0], acc[r]);
            acc[r] = fmaf(xv.y, w[1], acc[r]);
            acc[r] = fmaf(xv.z, w[2], acc[r]);
            acc[r] = fmaf(xv.w, w[3], acc[r]);
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

struct XWs {
    float* ptr = nullptr;
    int64_t floats = 0;
};
XWs g_xws[64];

template <int F>
int launch_col(const aeth_weight* w, const float* x, int64_t m, float* y, int64_t ldy, const GemvEpi& e,
               float* part, int S, hipStream_t s) {
    const int64_t units = aeth_cdiv(w->n, 256);
    const int R = m == 1 ? 1 : 8;
    const dim3 grid((unsigned)units, (unsigned)S, (unsigned)aeth_cdiv(m, R));
    if (R == 1)
        hipLaunchKernelGGL((k_col<F, 1>), grid, dim3(256), 0, s, w->p0, w->n, w->k, x, w->k, (int)m, S, part);
    else
        hipLaunchKernelGGL((k_col<F, 8>), grid, dim3(256), 0, s, w->p0, w->n, w->k, x, w->k, (int)m, S, part);
    AETH_LAUNCH_CHECK();
    const int64_t tot = m * w->n;
    hipLaunchKernelGGL(k_col_reduce, dim3((unsigned)aeth_cdiv(tot, 256)), dim3(256), 0, s, part, S, m, w->n, y, ldy,
                       (e.flags & AETH_MM_ACCUMULATE) ? 1 : 0, e.amax);
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
// (≈ 8 per CU), at least 16 inputs per wave.
int col_splits(const aeth_weight* w, int64_t m) {
    const int64_t units = aeth_cdiv(w->n, 256), groups = aeth_cdiv(m, m == 1 ? 1 : 8);
    int64_t S = aeth_cdiv(8LL * aeth_num_cus(), units * groups);
    S = S < 1 ? 1 : S > 64 ? 64 : S;
    const int64_t smax = w->k / 64 > 1 ? w->k / 64 : 1;
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
    if (!ws) {  // the library's per-device scratch (grow-only)
        int dev = 0;
        AETH_HIP_CHECK(hipGetDevice(&dev));
        if (dev < 0 || dev >= 64) return aeth_set_error(AETH_EINVAL, "gemv: device index");
        XWs& xw = g_xws[dev];
        if (xw.floats < need) {
            if (xw.ptr) AETH_HIP_CHECK(hipFree(xw.ptr));
            xw.ptr = nullptr;
            xw.floats = 0;
            AETH_HIP_CHECK(hipMalloc((void**)&xw.ptr, (size_t)need * sizeof(float)));
            xw.floats = need;
        }
        ws = xw.ptr;
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
