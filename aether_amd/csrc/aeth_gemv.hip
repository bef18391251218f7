// Decode GEMV for Q8_0 / Q4_K / Q6_K weights on gfx950:  y[r] = Σ_k x[k]·W[r][k].
//
// Design (MI355X-first; see DESIGN.md for the derivation):
//  * The weight planes are streamed with 16-byte loads; chunk c of a row is
//    bytes [16c, 16c+16) of that row's quant plane, so lane L of a wave reads
//    bytes [16L, 16L+16) — one wave instruction covers 1 KiB contiguous.
//  * The activation row is converted once per workgroup (in LDS) into an exact
//    integer form: per 16-element group g, x ≈ x_int·2^-S_g with
//    |x_int| ≤ 2^22 (22 bits + sign relative to the group maximum — the f32
//    rounding of x itself is 2^-24), split into three balanced signed byte
//    digits d0 + 256·d1 + 65536·d2. A 4-element weight quad is then dotted
//    with v_dot4_i32_i8 per digit: integer-exact sub-block dots at ~1 VALU op
//    per weight instead of unpack+convert+FMA (~2.4).
//  * Per-sub-block scales are applied in f32 once per 16-element group.
//  * Persistent workgroups: a fixed grid (a small multiple of the CU count)
//    amortises the activation conversion; each wave owns a contiguous run of
//    rows and processes R of them per pass with all loads issued up front.
#include <math.h>
#include <stdlib.h>

#include "aeth_common.hpp"
#include "aeth_internal.hpp"

#define GEMV_THREADS 512
#define GEMV_WAVES (GEMV_THREADS / 64)

// LDS image of one activation row.
struct XDigits {
    int* dig;      // [3][ngroups*4] dwords: 4 signed bytes = digit k of a quad
    int* gexp;     // [ngroups] S_g
    float* gfsum;  // [ngroups] Σx over the group (Q4_K min term)
    int* gisum;    // [3][ngroups] 32·Σ digit_k over the group (Q6_K −32 offset)
    int ngroups;
};

__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

__device__ __forceinline__ int pack4(int a, int b, int c, int d) {
    return (a & 0xFF) | ((b & 0xFF) << 8) | ((c & 0xFF) << 16) | ((int)((unsigned)d << 24));
}

// Builds the digit image of x[0..k) (zero-padded to ngroups*16) in LDS.
// Returns nonzero (uniformly) if x holds a non-finite value.
__device__ int build_digits(const float* __restrict__ x, int k, XDigits X, int* flag_smem) {
    const int tid = threadIdx.x;
    if (tid == 0) *flag_smem = 0;
    __syncthreads();
    const int nhalf = X.ngroups * 2;  // half-groups of 8 elements
    int bad = 0;
    // every thread runs the same number of iterations so the pair shuffles stay converged
    for (int base = 0; base < nhalf; base += GEMV_THREADS) {
        int hg = base + tid;
        bool live = hg < nhalf;
        float v[8];
        int e0 = hg * 8;
#pragma unroll
        for (int t = 0; t < 8; t++) v[t] = (live && e0 + t < k) ? x[e0 + t] : 0.0f;
        float mx = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; t++) mx = fmaxf(mx, fabsf(v[t]));
        mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
        if (!isfinite(mx)) bad = 1;
        int E = 0;
        if (mx > 0.0f) (void)frexpf(mx, &E);
        int S = (mx > 0.0f) ? 22 - E : 0;
        int d0[8], d1[8], d2[8];
        float fs = 0.0f;
        int s0 = 0, s1 = 0, s2 = 0;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            int xi = (mx > 0.0f && isfinite(mx)) ? (int)rintf(ldexpf(v[t], S)) : 0;
            int a = (xi << 24) >> 24;
            int r = (xi - a) >> 8;
            int b = (r << 24) >> 24;
            int c = (r - b) >> 8;
            d0[t] = a; d1[t] = b; d2[t] = c;
            s0 += a; s1 += b; s2 += c;
            fs += v[t];
        }
        fs += __shfl_xor(fs, 1, 64);
        s0 += __shfl_xor(s0, 1, 64);
        s1 += __shfl_xor(s1, 1, 64);
        s2 += __shfl_xor(s2, 1, 64);
        if (live) {
            int q = hg * 2;
            X.dig[q] = pack4(d0[0], d0[1], d0[2], d0[3]);
            X.dig[q + 1] = pack4(d0[4], d0[5], d0[6], d0[7]);
            X.dig[X.ngroups * 4 + q] = pack4(d1[0], d1[1], d1[2], d1[3]);
            X.dig[X.ngroups * 4 + q + 1] = pack4(d1[4], d1[5], d1[6], d1[7]);
            X.dig[X.ngroups * 8 + q] = pack4(d2[0], d2[1], d2[2], d2[3]);
            X.dig[X.ngroups * 8 + q + 1] = pack4(d2[4], d2[5], d2[6], d2[7]);
            if ((hg & 1) == 0) {
                int g = hg >> 1;
                X.gexp[g] = S;
                X.gfsum[g] = fs;
                X.gisum[g] = s0 << 5;
                X.gisum[X.ngroups + g] = s1 << 5;
                X.gisum[2 * X.ngroups + g] = s2 << 5;
            }
        }
    }
    if (bad) *flag_smem = 1;
    __syncthreads();
    return *flag_smem;
}

__device__ __forceinline__ XDigits carve_lds(char* smem, int ngroups) {
    XDigits X;
    X.ngroups = ngroups;
    X.dig = (int*)smem;
    X.gexp = X.dig + 12 * ngroups;
    X.gfsum = (float*)(X.gexp + ngroups);
    X.gisum = (int*)(X.gfsum + ngroups);
    return X;
}

static inline size_t xdigits_lds_bytes(int ngroups) { return (size_t)ngroups * (12 + 1 + 1 + 3) * 4 + 16; }

// Integer dot of 16 weights (4 dwords of signed/unsigned bytes) with the
// digits of group g: returns the three digit accumulators.
struct Dot3 { int a0, a1, a2; };

__device__ __forceinline__ Dot3 dot16(const int4 wq, const XDigits& X, int g) {
    const int4 D0 = *(const int4*)(X.dig + g * 4);
    const int4 D1 = *(const int4*)(X.dig + X.ngroups * 4 + g * 4);
    const int4 D2 = *(const int4*)(X.dig + X.ngroups * 8 + g * 4);
    Dot3 r;
    r.a0 = sdot4(wq.w, D0.w, sdot4(wq.z, D0.z, sdot4(wq.y, D0.y, sdot4(wq.x, D0.x, 0))));
    r.a1 = sdot4(wq.w, D1.w, sdot4(wq.z, D1.z, sdot4(wq.y, D1.y, sdot4(wq.x, D1.x, 0))));
    r.a2 = sdot4(wq.w, D2.w, sdot4(wq.z, D2.z, sdot4(wq.y, D2.y, sdot4(wq.x, D2.x, 0))));
    return r;
}

// Σ q·x over the group as f32 from the digit accumulators.
__device__ __forceinline__ float dot3_value(Dot3 r, int S) {
    float v = (float)r.a2 * 65536.0f + (float)(r.a0 + (r.a1 << 8));
    return ldexpf(v, -S);
}

// get_scale_min_k4 (common.rs:29-38) on the header dwords y = scales[0..3],
// z = scales[4..7], w = scales[8..11], for sub-block s in [0,8).
__device__ __forceinline__ void k4_scale_min(uint32_t y, uint32_t z, uint32_t w, int s, float& sc, float& m) {
    int t = s & 3;
    uint32_t ylo = (y >> (8 * t)) & 0xFFu, zlo = (z >> (8 * t)) & 0xFFu, wb = (w >> (8 * t)) & 0xFFu;
    uint32_t sc_lo = ylo & 63u, m_lo = zlo & 63u;
    uint32_t sc_hi = (wb & 0x0Fu) | ((ylo >> 6) << 4), m_hi = (wb >> 4) | ((zlo >> 6) << 4);
    bool hi = s >= 4;
    sc = (float)(hi ? sc_hi : sc_lo);
    m = (float)(hi ? m_hi : m_lo);
}

struct RowRange { int64_t begin, end; };

// Contiguous rows of this wave: the grid splits [0,n) evenly over workgroups,
// each workgroup evenly over its waves.
__device__ __forceinline__ RowRange wave_rows(int64_t n) {
    int64_t per_wg = (n + gridDim.x - 1) / gridDim.x;
    int64_t wg0 = (int64_t)blockIdx.x * per_wg;
    int64_t wg1 = min(n, wg0 + per_wg);
    int64_t per_wave = (per_wg + GEMV_WAVES - 1) / GEMV_WAVES;
    int wave = threadIdx.x >> 6;
    RowRange r;
    r.begin = min(wg1, wg0 + wave * per_wave);
    r.end = min(wg1, r.begin + per_wave);
    return r;
}

template <int R>
__device__ __forceinline__ void store_rows(float (&acc)[R], int64_t row0, int64_t row_end, float* y,
                                           const float* resid) {
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = aeth_wave_sum(acc[r]);
    if ((threadIdx.x & 63) == 0) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            int64_t row = row0 + r;
            if (row < row_end) y[row] = resid ? resid[row] + acc[r] : acc[r];
        }
    }
}

__device__ __forceinline__ void fill_nan(int64_t n, float* y) {
    RowRange rr = wave_rows(n);
    for (int64_t row = rr.begin + (threadIdx.x & 63); row < rr.end; row += 64) y[row] = __int_as_float(0x7FC00000);
}

// ── Q4_K: planes hdr[row*nb+b][16], qs[row*nb+b][128]. Chunk c (of nb*8):
// block b = c/8, i = c%8 → qs bytes [16i,16i+16): low nibbles are elements
// 64j+16h+t (sub-block 2j), high nibbles 64j+32+16h+t (sub-block 2j+1),
// j = i/2, h = i%2, t = 0..15.
template <int R>
__global__ void __launch_bounds__(GEMV_THREADS) k_gemv_q4k(const uint8_t* __restrict__ hdr,
                                                         const uint8_t* __restrict__ qs, int64_t n, int nb,
                                                         const float* __restrict__ x, int k, int64_t x_stride,
                                                         float* __restrict__ y, int64_t y_stride, int accumulate) {
    extern __shared__ char smem[];
    __shared__ int flag;
    const int ngroups = nb * 16;
    XDigits X = carve_lds(smem, ngroups);
    const float* xr = x + (int64_t)blockIdx.y * x_stride;
    float* yr = y + (int64_t)blockIdx.y * y_stride;
    if (build_digits(xr, k, X, &flag)) { fill_nan(n, yr); return; }
    const float* resid = accumulate ? yr : nullptr;
    const int lane = threadIdx.x & 63;
    const int cpr = nb * 8;
    RowRange rr = wave_rows(n);
    for (int64_t row0 = rr.begin; row0 < rr.end; row0 += R) {
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = 0.0f;
        for (int c = lane; c < cpr; c += 64) {
            const int b = c >> 3, i = c & 7, j = i >> 1, h = i & 1;
            const int glo = b * 16 + j * 4 + h, ghi = glo + 2;
            int4 wv[R];
            uint4 hv[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                int64_t row = min(row0 + r, rr.end - 1);
                wv[r] = *(const int4*)(qs + (row * nb) * 128 + (int64_t)c * 16);
                hv[r] = *(const uint4*)(hdr + (row * nb + b) * 16);
            }
            const int Slo = X.gexp[glo], Shi = X.gexp[ghi];
            const float fslo = X.gfsum[glo], fshi = X.gfsum[ghi];
#pragma unroll
            for (int r = 0; r < R; r++) {
                int4 lo, hi;
                lo.x = wv[r].x & 0x0F0F0F0F; hi.x = (wv[r].x >> 4) & 0x0F0F0F0F;
                lo.y = wv[r].y & 0x0F0F0F0F; hi.y = (wv[r].y >> 4) & 0x0F0F0F0F;
                lo.z = wv[r].z & 0x0F0F0F0F; hi.z = (wv[r].z >> 4) & 0x0F0F0F0F;
                lo.w = wv[r].w & 0x0F0F0F0F; hi.w = (wv[r].w >> 4) & 0x0F0F0F0F;
                Dot3 dl = dot16(lo, X, glo), dh = dot16(hi, X, ghi);
                // |Σ q·x_int| < 16·15·2^22 < 2^31: the digits combine exactly in i32.
                float vlo = ldexpf((float)(dl.a0 + (dl.a1 << 8) + (dl.a2 << 16)), -Slo);
                float vhi = ldexpf((float)(dh.a0 + (dh.a1 << 8) + (dh.a2 << 16)), -Shi);
                float d = aeth_decode_d(hv[r].x), dmin = aeth_decode_d(hv[r].x >> 16);
                float sclo, mlo, schi, mhi;
                k4_scale_min(hv[r].y, hv[r].z, hv[r].w, 2 * j, sclo, mlo);
                k4_scale_min(hv[r].y, hv[r].z, hv[r].w, 2 * j + 1, schi, mhi);
                acc[r] += d * (sclo * vlo + schi * vhi) - dmin * (mlo * fslo + mhi * fshi);
            }
        }
        store_rows<R>(acc, row0, rr.end, yr, resid);
    }
}

// ── Q6_K: planes ql[row*nb+b][128], qh[..][64], sc[..][16], d[..] (f16).
// Chunk c (of nb*4): block b = c/4, half h = (c/2)%2, g = c%2, t = 0..15:
// A = ql[h*64+16g+t], B = ql[h*64+32+16g+t], H = qh[h*32+16g+t] give the
// 6-bit quants of elements h*128 + 16g + 32u + t for u = 0..3, whose scale
// is sc[h*8 + g + 2u] (dequant.rs:301-348).
template <int R>
__global__ void __launch_bounds__(GEMV_THREADS) k_gemv_q6k(const uint8_t* __restrict__ ql,
                                                         const uint8_t* __restrict__ qh,
                                                         const uint8_t* __restrict__ scp,
                                                         const uint16_t* __restrict__ dp, int64_t n, int nb,
                                                         const float* __restrict__ x, int k, int64_t x_stride,
                                                         float* __restrict__ y, int64_t y_stride, int accumulate) {
    extern __shared__ char smem[];
    __shared__ int flag;
    const int ngroups = nb * 16;
    XDigits X = carve_lds(smem, ngroups);
    const float* xr = x + (int64_t)blockIdx.y * x_stride;
    float* yr = y + (int64_t)blockIdx.y * y_stride;
    if (build_digits(xr, k, X, &flag)) { fill_nan(n, yr); return; }
    const float* resid = accumulate ? yr : nullptr;
    const int lane = threadIdx.x & 63;
    const int cpr = nb * 4;
    RowRange rr = wave_rows(n);
    for (int64_t row0 = rr.begin; row0 < rr.end; row0 += R) {
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = 0.0f;
        for (int c = lane; c < cpr; c += 64) {
            const int b = c >> 2, h = (c >> 1) & 1, g = c & 1;
            const int g0 = b * 16 + h * 8 + g;  // group of u = 0; u adds 2
            int4 Av[R], Bv[R], Hv[R];
            uint2 Sv[R];
            uint32_t dv[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                int64_t row = min(row0 + r, rr.end - 1);
                int64_t blk = row * nb + b;
                Av[r] = *(const int4*)(ql + blk * 128 + h * 64 + g * 16);
                Bv[r] = *(const int4*)(ql + blk * 128 + h * 64 + 32 + g * 16);
                Hv[r] = *(const int4*)(qh + blk * 64 + h * 32 + g * 16);
                Sv[r] = *(const uint2*)(scp + blk * 16 + h * 8);
                dv[r] = dp[blk];
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                float part = 0.0f;
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    int4 q;
                    const int* A = (const int*)&Av[r];
                    const int* B = (const int*)&Bv[r];
                    const int* H = (const int*)&Hv[r];
                    int* Q = (int*)&q;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        int v;
                        if (u == 0) v = (A[e] & 0x0F0F0F0F) | ((H[e] << 4) & 0x30303030);
                        else if (u == 1) v = (B[e] & 0x0F0F0F0F) | ((H[e] << 2) & 0x30303030);
                        else if (u == 2) v = ((A[e] >> 4) & 0x0F0F0F0F) | (H[e] & 0x30303030);
                        else v = ((B[e] >> 4) & 0x0F0F0F0F) | ((H[e] >> 2) & 0x30303030);
                        Q[e] = v;
                    }
                    const int grp = g0 + 2 * u;
                    Dot3 dd = dot16(q, X, grp);
                    // quants are stored as q+32 in [0,63]; subtract 32·Σdigit per digit (exact)
                    dd.a0 -= X.gisum[grp];
                    dd.a1 -= X.gisum[X.ngroups + grp];
                    dd.a2 -= X.gisum[2 * X.ngroups + grp];
                    float v = dot3_value(dd, X.gexp[grp]);
                    int sbyte = g + 2 * u;  // byte within sc[h*8 .. h*8+8)
                    uint32_t sw = sbyte < 4 ? Sv[r].x : Sv[r].y;
                    float sc = (float)(int8_t)((sw >> (8 * (sbyte & 3))) & 0xFFu);
                    part += sc * v;
                }
                acc[r] += aeth_decode_d(dv[r]) * part;
            }
        }
        store_rows<R>(acc, row0, rr.end, yr, resid);
    }
}

// ── Q8_0: planes qs[row*nb+b][32] (int8), d[row*nb+b] (f16). Chunk c (of
// nb*2) = elements [16c, 16c+16) = group c, block c/2.
template <int R>
__global__ void __launch_bounds__(GEMV_THREADS) k_gemv_q8_0(const uint8_t* __restrict__ qs,
                                                          const uint16_t* __restrict__ dp, int64_t n, int nb,
                                                          const float* __restrict__ x, int k, int64_t x_stride,
                                                          float* __restrict__ y, int64_t y_stride, int accumulate) {
    extern __shared__ char smem[];
    __shared__ int flag;
    const int ngroups = nb * 2;
    XDigits X = carve_lds(smem, ngroups);
    const float* xr = x + (int64_t)blockIdx.y * x_stride;
    float* yr = y + (int64_t)blockIdx.y * y_stride;
    if (build_digits(xr, k, X, &flag)) { fill_nan(n, yr); return; }
    const float* resid = accumulate ? yr : nullptr;
    const int lane = threadIdx.x & 63;
    const int cpr = nb * 2;
    RowRange rr = wave_rows(n);
    for (int64_t row0 = rr.begin; row0 < rr.end; row0 += R) {
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = 0.0f;
        for (int c = lane; c < cpr; c += 64) {
            int4 wv[R];
            uint32_t dv[R];
#pragma unroll
            for (int r = 0; r < R; r++) {
                int64_t row = min(row0 + r, rr.end - 1);
                wv[r] = *(const int4*)(qs + (row * nb) * 32 + (int64_t)c * 16);
                dv[r] = dp[row * nb + (c >> 1)];
            }
            const int S = X.gexp[c];
#pragma unroll
            for (int r = 0; r < R; r++) {
                Dot3 dd = dot16(wv[r], X, c);
                acc[r] += aeth_f16_to_f32(dv[r]) * dot3_value(dd, S);
            }
        }
        store_rows<R>(acc, row0, rr.end, yr, resid);
    }
}

static int gemv_grid(int64_t n) {
    static int wg_per_cu = -1;
    if (wg_per_cu < 0) {
        const char* e = getenv("AETH_GEMV_WG_PER_CU");
        wg_per_cu = e ? atoi(e) : 2;
        if (wg_per_cu < 1) wg_per_cu = 1;
    }
    int64_t g = (int64_t)aeth_num_cus() * wg_per_cu;
    int64_t need = (n + GEMV_WAVES - 1) / GEMV_WAVES;
    if (need < g) g = need;
    return (int)(g < 1 ? 1 : g);
}

int aeth_gemv_launch(const aeth_weight* w, const float* d_x, int64_t m, float* d_y, unsigned flags,
                     hipStream_t s) {
    if (m > 65535) return aeth_set_error(AETH_EINVAL, "gemv: m=%lld exceeds 65535", (long long)m);
    const int nb = (int)w->nb;
    const int k = (int)w->k;
    const int acc = (flags & AETH_MM_ACCUMULATE) ? 1 : 0;
    dim3 grid(gemv_grid(w->n), (unsigned)m);
    dim3 block(GEMV_THREADS);
    if (w->dtype == AETH_DTYPE_Q4_K) {
        size_t lds = xdigits_lds_bytes(nb * 16);
        if (lds > 150 * 1024) return aeth_set_error(AETH_EUNSUPPORTED, "gemv: k=%d too large for LDS", k);
        hipLaunchKernelGGL(k_gemv_q4k<4>, grid, block, lds, s, w->p0, w->p1, w->n, nb, d_x, k, (int64_t)k, d_y,
                           w->n, acc);
    } else if (w->dtype == AETH_DTYPE_Q6_K) {
        size_t lds = xdigits_lds_bytes(nb * 16);
        if (lds > 150 * 1024) return aeth_set_error(AETH_EUNSUPPORTED, "gemv: k=%d too large for LDS", k);
        hipLaunchKernelGGL(k_gemv_q6k<4>, grid, block, lds, s, w->p0, w->p1, w->p2, (const uint16_t*)w->p3, w->n,
                           nb, d_x, k, (int64_t)k, d_y, w->n, acc);
    } else if (w->dtype == AETH_DTYPE_Q8_0) {
        size_t lds = xdigits_lds_bytes(nb * 2);
        if (lds > 150 * 1024) return aeth_set_error(AETH_EUNSUPPORTED, "gemv: k=%d too large for LDS", k);
        hipLaunchKernelGGL(k_gemv_q8_0<4>, grid, block, lds, s, w->p0, (const uint16_t*)w->p1, w->n, nb, d_x, k,
                           (int64_t)k, d_y, w->n, acc);
    } else {
        return aeth_set_error(AETH_EUNSUPPORTED, "gemv: dtype %d", w->dtype);
    }
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}
