// Decode GEMV for Q8_0 / Q6_K weights on gfx950:  y[r] = Σ_k x[k]·W[r][k]
// (Q4_K runs on the matrix cores, aeth_gemv_q4k.hip).
//
// Design (MI355X-first):
//  * Weights are read from the planar device layout (aeth_weights.hip) in
//    "units" of 32 (Q8_0) or 48 (Q6_K) quant bytes per lane, as
//    16-byte loads; consecutive lanes take consecutive units of a row, so each
//    wave load instruction covers a contiguous span of the row.
//  * The activation row becomes an exact integer form once per workgroup:
//    per 32 elements, x ≈ x_int·2^-S with |x_int| ≤ 2^22 (22 bits + sign
//    relative to the group maximum; f32 itself keeps 24), split into three
//    balanced signed byte digits x_int = d0 + 256·d1 + 65536·d2. A quad of
//    6-bit / 8-bit quants is dotted with v_dot4_i32_i8 per digit:
//    integer-exact sub-block dots for ~1 VALU op per weight instead of
//    unpack + convert + FMA. Scales are applied in f32 per sub-block.
//  * The digits are laid out in LDS per lane unit ("records", strides chosen
//    so that 8 consecutive lanes hit distinct 16-byte bank groups) and, when a
//    lane owns one or two units per row, held in registers for all its rows.
//  * One persistent workgroup of 8 waves per CU; each wave owns a contiguous
//    run of rows, processed R at a time. The first pass's weight loads are
//    issued before the activation conversion, and each pass prefetches the
//    next, so HBM streams while the VALU works.
#include <math.h>
#include <stdlib.h>

#include "aeth_common.hpp"
#include "aeth_internal.hpp"

#define GEMV_THREADS 512
#define GEMV_WAVES (GEMV_THREADS / 64)

enum { FMT_Q80 = 0, FMT_Q6K = 2 };

// Per-format geometry. UE: activation elements per unit; RECB: bytes of one
// LDS digit record; NQ: int4 weight loads per unit.
template <int F> struct Fmt;
template <> struct Fmt<FMT_Q6K> { static constexpr int UE = 64, RECB = 272; };
template <> struct Fmt<FMT_Q80> { static constexpr int UE = 32, RECB = 112; };

__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xFF) | ((uint32_t)(b & 0xFF) << 8) | ((uint32_t)(c & 0xFF) << 16) | ((uint32_t)d << 24);
}

// ── activation → digit records (LDS) ─────────────────────────────────────
// Thread t owns octets o = t + 512·i (i < XO): elements [8o, 8o+8). They are
// loaded first (before any weight traffic is queued), converted after the
// weight loads are in flight. Four consecutive lanes form a 32-element group
// with one exponent S.
// Record contents by format (unit = the weights one lane handles per row):
//  Q6_K unit u = 4b+2h+g: 16 elements h*128+16g+32v+t (t<16) for v = 0..3;
//       slot v digits at v*48 + k*16, meta at 192+16v: {S, 32Σd0, 32Σd1, 32Σd2}.
//  Q8_0 unit u = block u: digits at k*32, meta at 96: {S}.
template <int XO>
__device__ __forceinline__ void load_x(const float* __restrict__ x, int k, int noct, float (&xv)[XO][8]) {
    const bool vec = (k & 7) == 0;
#pragma unroll
    for (int i = 0; i < XO; i++) {
        const int o = threadIdx.x + GEMV_THREADS * i;
        const int e0 = o * 8;
        if (vec && o < noct && e0 + 8 <= k) {
            float4 a = *(const float4*)(x + e0), b = *(const float4*)(x + e0 + 4);
            xv[i][0] = a.x; xv[i][1] = a.y; xv[i][2] = a.z; xv[i][3] = a.w;
            xv[i][4] = b.x; xv[i][5] = b.y; xv[i][6] = b.z; xv[i][7] = b.w;
        } else {
#pragma unroll
            for (int t = 0; t < 8; t++) xv[i][t] = (o < noct && e0 + t < k) ? x[e0 + t] : 0.0f;
        }
    }
}

template <int F, int XO>
__device__ int build_records(const float (&xv)[XO][8], int noct, char* rec, int* flag) {
    const int tid = threadIdx.x;
    if (tid == 0) *flag = 0;
    __syncthreads();
    int bad = 0;
#pragma unroll
    for (int i = 0; i < XO; i++) {
        const int o = tid + GEMV_THREADS * i;
        const bool live = o < noct;
        const int e0 = o * 8;
        const float* v = xv[i];
        float mx = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; t++) mx = fmaxf(mx, fabsf(v[t]));
        mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
        const bool fin = isfinite(mx);
        if (!fin) bad = 1;
        int E = 0;
        if (mx > 0.0f && fin) (void)frexpf(mx, &E);
        const int S = (mx > 0.0f && fin) ? 22 - E : 0;
        int d0[8], d1[8], d2[8];
        int s0 = 0, s1 = 0, s2 = 0;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            int xi = (mx > 0.0f && fin) ? (int)rintf(ldexpf(v[t], S)) : 0;
            int a = (xi << 24) >> 24;
            int r = (xi - a) >> 8;
            int b = (r << 24) >> 24;
            int c = (r - b) >> 8;
            d0[t] = a; d1[t] = b; d2[t] = c;
            s0 += a; s1 += b; s2 += c;
        }
        const int qq = o & 3;  // octet within its 32-group
        char* dst;
        int koff;  // byte stride between the three digits
        if (F == FMT_Q6K) {
            const int b = e0 >> 8, eb = e0 & 255, h = eb >> 7, rr = eb & 127, vv = rr >> 5, w32 = rr & 31;
            const int g = w32 >> 4, half8 = (w32 >> 3) & 1;
            char* r = rec + (size_t)(b * 4 + h * 2 + g) * Fmt<F>::RECB;
            dst = r + vv * 48 + half8 * 8;
            koff = 16;
            s0 += __shfl_xor(s0, 1, 64);
            s1 += __shfl_xor(s1, 1, 64);
            s2 += __shfl_xor(s2, 1, 64);
            if (live && half8 == 0) {
                int4 m;
                m.x = S; m.y = s0 << 5; m.z = s1 << 5; m.w = s2 << 5;
                *(int4*)(r + 192 + 16 * vv) = m;
            }
        } else {
            char* r = rec + (size_t)(e0 >> 5) * Fmt<F>::RECB;
            dst = r + qq * 8;
            koff = 32;
            if (live && qq == 0) *(int*)(r + 96) = S;
        }
        if (live) {
            *(uint2*)(dst) = make_uint2(pack4(d0[0], d0[1], d0[2], d0[3]), pack4(d0[4], d0[5], d0[6], d0[7]));
            *(uint2*)(dst + koff) = make_uint2(pack4(d1[0], d1[1], d1[2], d1[3]), pack4(d1[4], d1[5], d1[6], d1[7]));
            *(uint2*)(dst + 2 * koff) =
                make_uint2(pack4(d2[0], d2[1], d2[2], d2[3]), pack4(d2[4], d2[5], d2[6], d2[7]));
        }
    }
    if (bad) *flag = 1;
    __syncthreads();
    return *flag;
}

// ── per-format unit data, loads and dot products ─────────────────────────

struct UQ6K { int4 a, b, h; uint2 sc; uint32_t d; };
struct UQ80 { int4 q0, q1; uint32_t d; };

template <int F> struct UnitT;
template <> struct UnitT<FMT_Q6K> { typedef UQ6K T; };
template <> struct UnitT<FMT_Q80> { typedef UQ80 T; };

struct Planes {
    const uint8_t* p0;
    const uint8_t* p1;
    const uint8_t* p2;
    const uint8_t* p3;
};

__device__ __forceinline__ void load_unit(UQ6K& d, const Planes& P, int64_t row, int nb, int u) {
    const int b = u >> 2, h = (u >> 1) & 1;
    const int64_t blk = row * nb + b;
    const uint8_t* ql = P.p0 + (row * nb) * 128 + (int64_t)u * 16;
    d.a = *(const int4*)ql;
    d.b = *(const int4*)(ql + nb * 64);
    d.h = *(const int4*)(P.p1 + (row * nb) * 64 + (int64_t)u * 16);
    d.sc = *(const uint2*)(P.p2 + blk * 16 + h * 8);
    d.d = ((const uint16_t*)P.p3)[blk];
}

__device__ __forceinline__ void load_unit(UQ80& d, const Planes& P, int64_t row, int nb, int u) {
    const uint8_t* q = P.p0 + (row * nb) * 32 + (int64_t)u * 16;
    d.q0 = *(const int4*)q;
    d.q1 = *(const int4*)(q + nb * 16);
    d.d = ((const uint16_t*)P.p1)[row * nb + u];
}

// Digit record held in registers (or read from LDS per use).
template <int F> struct Rec { uint4 v[Fmt<F>::RECB / 16]; };

template <int F>
__device__ __forceinline__ void read_rec(Rec<F>& r, const char* p) {
#pragma unroll
    for (int i = 0; i < Fmt<F>::RECB / 16; i++) r.v[i] = *(const uint4*)(p + 16 * i);
}

__device__ __forceinline__ int dot8(const int* q, const uint4* D0) {
    const int* d = (const int*)D0;
    int a = 0;
#pragma unroll
    for (int m = 0; m < 8; m++) a = sdot4(q[m], d[m], a);
    return a;
}

__device__ __forceinline__ int dot4v(const int* q, const uint4& D) {
    return sdot4(q[3], (int)D.w, sdot4(q[2], (int)D.z, sdot4(q[1], (int)D.y, sdot4(q[0], (int)D.x, 0))));
}

// Q6_K unit u = 4b + 2h + g.
__device__ __forceinline__ float unit_dot(const UQ6K& d, const Rec<FMT_Q6K>& R) {
    const int* A = (const int*)&d.a;
    const int* B = (const int*)&d.b;
    const int* H = (const int*)&d.h;
    float part = 0.0f;
#pragma unroll
    for (int v = 0; v < 4; v++) {
        int q[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            if (v == 0) q[e] = (A[e] & 0x0F0F0F0F) | ((H[e] << 4) & 0x30303030);
            else if (v == 1) q[e] = (B[e] & 0x0F0F0F0F) | ((H[e] << 2) & 0x30303030);
            else if (v == 2) q[e] = ((A[e] >> 4) & 0x0F0F0F0F) | (H[e] & 0x30303030);
            else q[e] = ((B[e] >> 4) & 0x0F0F0F0F) | ((H[e] >> 2) & 0x30303030);
        }
        const uint4 meta = R.v[12 + v];
        // quants are stored as q+32 in [0,63]: subtract 32·Σdigit per digit (exact)
        int a0 = dot4v(q, R.v[3 * v]) - (int)meta.y;
        int a1 = dot4v(q, R.v[3 * v + 1]) - (int)meta.z;
        int a2 = dot4v(q, R.v[3 * v + 2]) - (int)meta.w;
        float val = ldexpf((float)a2 * 65536.0f + (float)(a0 + (a1 << 8)), -(int)meta.x);
        uint32_t sw = v < 2 ? d.sc.x : d.sc.y;  // sc[h*8 + g + 2v], pre-shifted by fix_unit
        float sc = (float)(int8_t)((sw >> (16 * (v & 1))) & 0xFFu);
        part += sc * val;
    }
    return aeth_decode_d(d.d) * part;
}

// Q8_0 unit = one block.
__device__ __forceinline__ float unit_dot(const UQ80& d, const Rec<FMT_Q80>& R) {
    int q[8];
#pragma unroll
    for (int m = 0; m < 4; m++) { q[m] = ((const int*)&d.q0)[m]; q[m + 4] = ((const int*)&d.q1)[m]; }
    int a0 = dot8(q, &R.v[0]), a1 = dot8(q, &R.v[2]), a2 = dot8(q, &R.v[4]);
    float val = ldexpf((float)a2 * 65536.0f + (float)(a0 + (a1 << 8)), -(int)R.v[6].x);
    return aeth_f16_to_f32(d.d) * val;
}

// Q6_K scale bytes: the lane's g selects odd/even bytes of sc[h*8 .. h*8+8);
// shifting once per load leaves byte g+2v at bit 16(v&1) of word v/2.
__device__ __forceinline__ void fix_unit(UQ6K& d, int g) {  // g = u & 1
    d.sc.x >>= 8 * g;
    d.sc.y >>= 8 * g;
}
__device__ __forceinline__ void fix_unit(UQ80&, int) {}

// ── reductions: R row sums spread over the wave → one value per row ──────
// Reduce-scatter butterfly: each of the first log2(R) exchange steps halves
// the number of live row sums per lane (lanes on the two sides of the step's
// bit keep different halves), the remaining steps finish the sum. Afterwards
// lane L holds the total of row_of_lane<R>(L), written by the lanes where
// (L & (64/R - 1)) == 0. Six exchange steps move R-1 + 6-log2(R) values
// per lane instead of 6·R.
template <int R>
__device__ __forceinline__ float wave_reduce_rows(const float (&a)[R], int lane) {
    float v[R];
#pragma unroll
    for (int i = 0; i < R; i++) v[i] = a[i];
    int bit = 32;
#pragma unroll
    for (int n = R; n > 1; n >>= 1) {
        const bool hi = lane & bit;
#pragma unroll
        for (int i = 0; i < n / 2; i++) {
            float keep = hi ? v[n / 2 + i] : v[i];
            float send = hi ? v[i] : v[n / 2 + i];
            v[i] = keep + __shfl_xor(send, bit, 64);
        }
        bit >>= 1;
    }
#pragma unroll
    for (int off = 64 / R / 2; off >= 1; off >>= 1) v[0] += __shfl_xor(v[0], off, 64);
    return v[0];
}

template <int R>
__device__ __forceinline__ int row_of_lane(int lane) {
    int row = 0, bit = 32, w = R / 2;
#pragma unroll
    for (int n = R; n > 1; n >>= 1) {
        if (lane & bit) row += w;
        w >>= 1;
        bit >>= 1;
    }
    return row;
}

// ── the kernel ───────────────────────────────────────────────────────────
// WPR waves share a row (wave w of a row handles units [64w, 64w+64)), so
// each lane owns exactly one unit and keeps its digit record in registers;
// the 8 waves form 8/WPR row streams. R rows per pass; XO activation octets
// per thread.
//
// Optional fusions (GemvParams):
//  norm_w   : x ← x / sqrt(Σx²/k + eps) · norm_w before the product
//             (rmsnorm_inplace, runner.rs:1739-1746);
//  swiglu   : rows come in (gate_i, up_i) pairs at 2i, 2i+1 and the output is
//             y[i] = g·σ(g)·u (runner.rs:1617-1625) — WPR == 1 only;
//  amax     : greedy argmax of y folded into a 64-bit atomic max of
//             (orderable(value) << 32 | row): last maximal row wins on ties,
//             as Iterator::max_by (runner.rs:1964-1973);
//  accumulate: y += result (residual adds, runner.rs:1609-1611, 1629-1631).
struct GemvParams {
    Planes P;
    int64_t n;
    int nb, upr;
    const float* x;
    int k;
    int64_t x_stride;
    float* y;
    int64_t y_stride;
    int accumulate;
    int64_t rows_per_wg;
    int npass;
    const float* norm_w;
    float eps;
    int swiglu;
    unsigned long long* amax;
};

__device__ __forceinline__ unsigned long long amax_key(float v, int64_t row) {
    uint32_t f = __float_as_uint(v);
    uint32_t o = (f & 0x80000000u) ? ~f : (f | 0x80000000u);
    return ((unsigned long long)o << 32) | (unsigned long long)(uint32_t)row;
}

__device__ __forceinline__ float silu_mul(float g, float u) { return g * (1.0f / (1.0f + expf(-g))) * u; }

template <int F, int WPR, int R, int XO>
__global__ void __launch_bounds__(GEMV_THREADS) k_gemv(GemvParams G) {
    constexpr int STREAMS = GEMV_WAVES / WPR;
    extern __shared__ __attribute__((aligned(16))) char rec[];
    __shared__ int flag;
    __shared__ float ssum[GEMV_WAVES];
    __shared__ unsigned long long kmax[GEMV_WAVES];
    typedef typename UnitT<F>::T U;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int stream = wave / WPR, wir = wave - stream * WPR;
    const int u = wir * 64 + lane;
    const int upr = G.upr, nb = G.nb;
    const bool valid = u < upr;
    const float* xr = G.x + (int64_t)blockIdx.y * G.x_stride;
    float* yr = G.y + (int64_t)blockIdx.y * G.y_stride;
    const int64_t wg0 = (int64_t)blockIdx.x * G.rows_per_wg;
    const int64_t wg1 = min(G.n, wg0 + G.rows_per_wg);
    const int64_t rps = (G.rows_per_wg + STREAMS - 1) / STREAMS;
    const int64_t sb = min(wg1, wg0 + stream * rps);
    const int64_t se = min(wg1, sb + rps);
    const int noct = upr * Fmt<F>::UE / 8;
    float* red = (float*)(rec + (size_t)upr * Fmt<F>::RECB);  // [2][STREAMS][WPR][R] when WPR > 1

    float xv[XO][8], wv[XO][8];
    load_x<XO>(xr, G.k, noct, xv);
    if (G.norm_w) load_x<XO>(G.norm_w, G.k, noct, wv);

    // Ring of R row buffers: row i of this stream lives in buf[i % R]; each
    // buffer is refilled with the row R ahead as soon as it has been consumed,
    // so every wave keeps R rows of loads in flight and computes on arrival.
    U buf[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        if (valid && sb < se) {
            load_unit(buf[r], G.P, min(sb + r, se - 1), nb, u);
            fix_unit(buf[r], u & 1);
        }
    }

    if (G.norm_w) {  // fused RMSNorm: every workgroup normalises the full row
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < XO; i++)
#pragma unroll
            for (int t = 0; t < 8; t++) ss += xv[i][t] * xv[i][t];
        ss = aeth_wave_sum(ss);
        if (lane == 0) ssum[wave] = ss;
        __syncthreads();
        float tot = 0.0f;
#pragma unroll
        for (int w = 0; w < GEMV_WAVES; w++) tot += ssum[w];
        const float rms = sqrtf(tot / (float)G.k + G.eps);
#pragma unroll
        for (int i = 0; i < XO; i++)
#pragma unroll
            for (int t = 0; t < 8; t++) xv[i][t] = xv[i][t] / rms * wv[i][t];
    }

    if (build_records<F, XO>(xv, noct, rec, &flag)) {
        const int64_t oe = G.swiglu ? se / 2 : se;
        if (wir == 0)
            for (int64_t row = (G.swiglu ? sb / 2 : sb) + lane; row < oe; row += 64) yr[row] = __int_as_float(0x7FC00000);
        return;
    }
    Rec<F> reg;
    if (valid) read_rec<F>(reg, rec + (size_t)u * Fmt<F>::RECB);

    unsigned long long best = 0;
    for (int p = 0; p < G.npass; p++) {
        const int64_t row0 = sb + (int64_t)p * R;
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            acc[r] = (valid && row0 + r < se) ? unit_dot(buf[r], reg) : 0.0f;
            if (valid && p + 1 < G.npass && row0 + R < se) {
                load_unit(buf[r], G.P, min(row0 + R + r, se - 1), nb, u);
                fix_unit(buf[r], u & 1);
            }
        }
        float tot = wave_reduce_rows<R>(acc, lane);
        const int myrow = row_of_lane<R>(lane);
        const bool writer = (lane & (64 / R - 1)) == 0;
        if (WPR == 1) {
            const int64_t row = row0 + myrow;
            if (G.swiglu) {
                const float up = __shfl_xor(tot, 64 / R, 64);  // partner row = row ^ 1
                if (writer && (myrow & 1) == 0 && row < se) yr[row >> 1] = silu_mul(tot, up);
            } else if (writer && row < se) {
                const float v = G.accumulate ? yr[row] + tot : tot;
                yr[row] = v;
                if (G.amax) { unsigned long long kk = amax_key(v, row); best = kk > best ? kk : best; }
            }
        } else {
            float* rb = red + (p & 1) * (STREAMS * WPR * R);
            if (writer) rb[(stream * WPR + wir) * R + myrow] = tot;
            __syncthreads();
            if (threadIdx.x < STREAMS * R) {
                const int s2 = threadIdx.x / R, r2 = threadIdx.x - s2 * R;
                const int64_t sb2 = min(wg1, wg0 + s2 * rps), se2 = min(wg1, sb2 + rps);
                const int64_t row = sb2 + (int64_t)p * R + r2;
                if (row < se2) {
                    float t = 0.0f;
#pragma unroll
                    for (int w = 0; w < WPR; w++) t += rb[(s2 * WPR + w) * R + r2];
                    const float v = G.accumulate ? yr[row] + t : t;
                    yr[row] = v;
                    if (G.amax) { unsigned long long kk = amax_key(v, row); best = kk > best ? kk : best; }
                }
            }
        }
    }
    if (G.amax) {
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            unsigned long long o = __shfl_xor(best, off, 64);
            best = o > best ? o : best;
        }
        if (lane == 0) kmax[wave] = best;
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned long long m = kmax[0];
#pragma unroll
            for (int w = 1; w < GEMV_WAVES; w++) m = kmax[w] > m ? kmax[w] : m;
            atomicMax(G.amax, m);
        }
    }
}

// ── dispatch ─────────────────────────────────────────────────────────────

static int env_int(const char* name, int dflt) {
    const char* e = getenv(name);
    return e ? atoi(e) : dflt;
}

template <int F, int WPR, int R, int XO>
static void launch(dim3 grid, size_t lds, hipStream_t s, GemvParams G) {
    constexpr int STREAMS = GEMV_WAVES / WPR;
    const int64_t rps = (G.rows_per_wg + STREAMS - 1) / STREAMS;
    G.npass = (int)((rps + R - 1) / R);
    hipLaunchKernelGGL((k_gemv<F, WPR, R, XO>), grid, dim3(GEMV_THREADS), lds, s, G);
}

template <int F>
static int dispatch_fmt(GemvParams G, int64_t m, hipStream_t s) {
    static const int wg_per_cu = env_int("AETH_GEMV_WG_PER_CU", 1);
    static const int rsel = env_int("AETH_GEMV_R", 4);
    const int upr = G.upr;
    int wpr = 1;
    while (wpr * 64 < upr) wpr *= 2;
    const int noct = upr * Fmt<F>::UE / 8;
    int xo = 1;
    while (xo * GEMV_THREADS < noct) xo *= 2;
    const size_t lds = (size_t)upr * Fmt<F>::RECB + (wpr > 1 ? 2 * GEMV_WAVES * 4 * sizeof(float) : 0);
    if (wpr > 8 || xo > 4 || lds > 64 * 1024)
        return aeth_set_error(AETH_EUNSUPPORTED, "gemv: k=%d is beyond this kernel's range", G.k);
    if (G.swiglu && (wpr != 1 || (G.n & 1)))
        return aeth_set_error(AETH_EUNSUPPORTED, "gemv: fused SwiGLU needs k <= 4096-wide rows and paired rows");
    const int streams = GEMV_WAVES / wpr;
    int64_t grid = (int64_t)aeth_num_cus() * (wg_per_cu < 1 ? 1 : wg_per_cu);
    const int64_t need = (G.n + streams - 1) / streams;
    if (need < grid) grid = need;
    if (grid < 1) grid = 1;
    int64_t rpg = (G.n + grid - 1) / grid;
    if (G.swiglu) rpg = (rpg + 2 * streams - 1) / (2 * streams) * (2 * streams);  // even rows per stream
    G.rows_per_wg = rpg;
    dim3 g((unsigned)grid, (unsigned)m);
#define L_(W, RR, X) launch<F, W, RR, X>(g, lds, s, G)
    if (wpr == 1 && xo == 1) {
        if (rsel == 2) L_(1, 2, 1);
        else if (rsel == 8) L_(1, 8, 1);
        else L_(1, 4, 1);
    } else if (wpr == 2 && xo == 1) L_(2, 4, 1);
    else if (wpr == 2 && xo == 2) L_(2, 4, 2);
    else if (wpr == 4 && xo == 2) L_(4, 4, 2);
    else if (wpr == 4 && xo == 4) L_(4, 4, 4);
    else if (wpr == 8 && xo == 4) L_(8, 4, 4);
    else if (wpr == 1 && xo == 2) L_(1, 4, 2);
    else if (wpr == 2 && xo == 4) L_(2, 4, 4);
    else return aeth_set_error(AETH_EUNSUPPORTED, "gemv: no kernel for k=%d (wpr %d, xo %d)", G.k, wpr, xo);
#undef L_
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}

int aeth_gemv_launch_ex(const aeth_weight* w, const float* d_x, int64_t m, float* d_y, const GemvEpi& e,
                        hipStream_t s) {
    if (m > 65535) return aeth_set_error(AETH_EINVAL, "gemv: m=%lld exceeds 65535", (long long)m);
    GemvParams G;
    G.P = Planes{w->p0, w->p1, w->p2, w->p3};
    G.n = w->n;
    G.nb = (int)w->nb;
    G.upr = w->dtype == AETH_DTYPE_Q8_0 ? (int)w->nb : (int)w->nb * 4;
    G.x = d_x;
    G.k = (int)w->k;
    G.x_stride = w->k;
    G.y = d_y;
    G.y_stride = e.swiglu ? w->n / 2 : w->n;
    G.accumulate = (e.flags & AETH_MM_ACCUMULATE) ? 1 : 0;
    G.rows_per_wg = 0;
    G.npass = 0;
    G.norm_w = e.norm_w;
    G.eps = e.eps;
    G.swiglu = e.swiglu;
    G.amax = e.amax;
    if (w->dtype == AETH_DTYPE_Q4_K) return aeth_gemv_q4k_launch(w, d_x, m, d_y, e, s);
    if (w->dtype == AETH_DTYPE_Q6_K) return dispatch_fmt<FMT_Q6K>(G, m, s);
    if (w->dtype == AETH_DTYPE_Q8_0) return dispatch_fmt<FMT_Q80>(G, m, s);
    return aeth_set_error(AETH_EUNSUPPORTED, "gemv: dtype %d", w->dtype);
}

int aeth_gemv_launch(const aeth_weight* w, const float* d_x, int64_t m, float* d_y, unsigned flags, hipStream_t s) {
    GemvEpi e;
    e.flags = flags;
    return aeth_gemv_launch_ex(w, d_x, m, d_y, e, s);
}
