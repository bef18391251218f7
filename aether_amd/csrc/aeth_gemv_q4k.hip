// Q4_K decode GEMV on the int8 matrix cores of gfx950:  y[r] = Σ_k x[k]·W[r][k]
// (avx2::matmul_q4_k, src/quant/avx2.rs:23-57, at m = 1; one activation row
// per grid.y for m > 1).
//
// Exact integer core. Once per workgroup the activation row becomes, per
// 32-element sub-block s, x ≈ x_int·2^-S_s with |x_int| ≤ 2^22 (22 bits +
// sign against the sub-block maximum), split into three balanced signed byte
// digits x_int = d0 + 256·d1 + 65536·d2. The digits are the A operand of
// v_mfma_i32_16x16x64_i8 (M = 4 sub-block slots × 4 digit rows, the fourth
// row zero) and 16 weight rows are the B operand (N), so one MFMA returns the
// exact integer dot of every digit with 64 quants of 16 rows. The output lane
// of (slot, row) recombines its three digit sums in i32
// (|Σ q·x_int| ≤ 32·15·2^22 < 2^31) and applies the sub-block scale and min
// in f32:  acc += 2^-S_s·(Σ q·x_int)·d·sc_s − dmin·m_s·Σ_{i∈s} x_i.
//
// Operand mapping for one 128-element half h of super-block b. Lane (n, kg)
// (n = lane % 16 = row in the tile, kg = lane / 16) loads
// qs[64h + 16kg, +16) of row n (one contiguous 1 KiB wave load):
//   kg < 2: bytes of sub-block pair 2h   → low nibbles sub-block 4h,   high 4h+1
//   kg ≥ 2: bytes of sub-block pair 2h+1 → low nibbles sub-block 4h+2, high 4h+3
// MFMA 1 multiplies the low nibbles, MFMA 2 the high nibbles, by the same A:
//   A lane (m, kg), slot s = m / 4, digit d = m % 4, holds the 16 digits d of
//   sub-block 4h+s at elements 16(kg & 1) + [0, 16) when d < 3 and
//   (s ≥ 2) == (kg ≥ 2), and zeros otherwise.
// Rows of even slots are exact in MFMA 1's result and odd slots in MFMA 2's;
// the result lane (n, g = lane / 16) holds slot g's three digit sums of row n,
// i.e. sub-block 4h+g.
//
// Work split: a workgroup (W = 8 or 16 waves) owns a run of 16-row tiles; wave w
// takes super-blocks [nb·w/W, nb·(w+1)/W) of every tile, converts only that slice
// of x, keeps RD tiles of loads in flight, and leaves 16 partial row sums per
// tile in LDS; after the one barrier the partials are summed in a fixed order
// (deterministic) and the epilogue (accumulate, SwiGLU, argmax) runs.
#include <math.h>
#include <stdlib.h>

#include "aeth_common.hpp"
#include "aeth_internal.hpp"

#define MQ_WAVES_MAX 16
#define MQ_TPW_MAX 32   // tiles per workgroup (LDS partials: 64 B per wave each)
#define MQ_NB_MAX 64    // super-blocks per row (k ≤ 16384): LDS digits 2 KiB each

typedef int mq_v4i __attribute__((ext_vector_type(4)));

struct MqParams {
    const uint8_t* hdr;
    const uint8_t* qs;
    int64_t n;
    int nb, ntiles, tpw;
    const float* x;
    int64_t x_stride;
    int k;
    float* y;
    int64_t y_stride;
    int accumulate;
    const float* norm_w;
    float eps;
    int swiglu;
    unsigned long long* amax;
};

__device__ __forceinline__ uint32_t mq_pack4(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xFF) | ((uint32_t)(b & 0xFF) << 8) | ((uint32_t)(c & 0xFF) << 16) | ((uint32_t)d << 24);
}

// Each wave converts only its own K-slice: lane l owns activation octets
// o = o0 + l + 64·i (elements [8o, 8o+8)) below o1.
// Every load in this kernel is issued unconditionally (out-of-range indices
// are clamped to valid addresses and their values discarded): the compiler
// can then count outstanding loads exactly and wait for each one alone,
// instead of draining the whole weight stream at the first use of x.
template <int XO>
__device__ __forceinline__ void mq_load_x(const float* __restrict__ x, int o0, int o1, float (&xv)[XO][8]) {
#pragma unroll
    for (int i = 0; i < XO; i++) {
        const int o = o0 + (threadIdx.x & 63) + 64 * i;
        const int oc = min(o, max(o1 - 1, o0));  // octets past o1 hold copies, masked at their uses
        const float4 a = *(const float4*)(x + 8 * oc), b = *(const float4*)(x + 8 * oc + 4);
        xv[i][0] = a.x; xv[i][1] = a.y; xv[i][2] = a.z; xv[i][3] = a.w;
        xv[i][4] = b.x; xv[i][5] = b.y; xv[i][6] = b.z; xv[i][7] = b.w;
    }
}

// The wave's activation slice → A operands in LDS: V[b][h][lane][16 B]
// (2 KiB per super-block) and meta[b·8 + s] = {−S, Σx} per sub-block, written
// and later read by this wave only (LDS operations of one wave execute in
// order, so no barrier is needed). Each octet writes its three digit pieces,
// the zero piece of digit row 3, and four zero pieces of its slot's lanes in
// the other kg pair, which together cover every byte of V. Returns nonzero
// (wave-uniform) if the slice holds a NaN or an infinity.
template <int XO>
__device__ int mq_build(const float (&xv)[XO][8], int o0, int o1, char* V, int2* meta) {
    const int lane = threadIdx.x & 63;
    int bad = 0;
#pragma unroll
    for (int i = 0; i < XO; i++) {
        const int o = o0 + lane + 64 * i;
        const bool live = o < o1;
        const float* v = xv[i];
        float mx = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; t++) mx = fmaxf(mx, fabsf(v[t]));
        mx = fmaxf(mx, __shfl_xor(mx, 1, 64));  // the 4 octets of a sub-block are adjacent lanes
        mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
        const bool fin = isfinite(mx);
        if (!fin && live) bad = 1;
        const bool use = mx > 0.0f && fin;
        int E = 0;
        if (use) (void)frexpf(mx, &E);
        const int S = use ? 22 - E : 0;
        int d0[8], d1[8], d2[8];
        float fs = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const int xi = use ? (int)rintf(ldexpf(v[t], S)) : 0;
            const int a = (xi << 24) >> 24;
            const int r = (xi - a) >> 8;
            const int b = (r << 24) >> 24;
            d0[t] = a;
            d1[t] = b;
            d2[t] = (r - b) >> 8;
            fs += v[t];
        }
        fs += __shfl_xor(fs, 1, 64);
        fs += __shfl_xor(fs, 2, 64);
        if (live) {
            const int e0 = 8 * o;
            const int b = e0 >> 8, h = (e0 >> 7) & 1, s = (e0 >> 5) & 3, p8 = (e0 >> 3) & 3;
            const int kg = 2 * (s >> 1) + (p8 >> 1), hf = p8 & 1, kgo = 2 - 2 * (s >> 1);
            char* base = V + (size_t)(b * 2 + h) * 1024;
            *(uint2*)(base + (4 * s + 0 + 16 * kg) * 16 + hf * 8) =
                make_uint2(mq_pack4(d0[0], d0[1], d0[2], d0[3]), mq_pack4(d0[4], d0[5], d0[6], d0[7]));
            *(uint2*)(base + (4 * s + 1 + 16 * kg) * 16 + hf * 8) =
                make_uint2(mq_pack4(d1[0], d1[1], d1[2], d1[3]), mq_pack4(d1[4], d1[5], d1[6], d1[7]));
            *(uint2*)(base + (4 * s + 2 + 16 * kg) * 16 + hf * 8) =
                make_uint2(mq_pack4(d2[0], d2[1], d2[2], d2[3]), mq_pack4(d2[4], d2[5], d2[6], d2[7]));
            *(uint2*)(base + (4 * s + 3 + 16 * kg) * 16 + hf * 8) = make_uint2(0u, 0u);
            *(uint4*)(base + (4 * s + p8 + 16 * kgo) * 16) = make_uint4(0u, 0u, 0u, 0u);
            *(uint4*)(base + (4 * s + p8 + 16 * (kgo + 1)) * 16) = make_uint4(0u, 0u, 0u, 0u);
            if (p8 == 0) meta[b * 8 + 4 * h + s] = make_int2(-S, __float_as_int(fs));
        }
    }
    return __any(bad);
}

// Loads of one tile: for each of the wave's super-blocks, the two 1 KiB quant
// halves and the 16-byte header of row (lane % 16). Slots beyond the wave's
// nbw super-blocks reload its last one (bA < nb always), unused.
template <int NBW>
__device__ __forceinline__ void mq_load(int4 (&q)[NBW][2], uint4 (&h)[NBW], const MqParams& G, int64_t t, int bA,
                                        int nbw, int lane) {
#pragma unroll
    for (int i = 0; i < NBW; i++) {
        const int64_t c = t * G.nb + bA + min(i, max(nbw - 1, 0));
        q[i][0] = *(const int4*)(G.qs + (c * 2) * 1024 + lane * 16);
        q[i][1] = *(const int4*)(G.qs + (c * 2 + 1) * 1024 + lane * 16);
        h[i] = *(const uint4*)(G.hdr + (c * 16 + (lane & 15)) * 16);
    }
}

// One tile's partial row sum over the wave's super-blocks (lane (n, g): row n,
// sub-blocks g and 4 + g of each super-block).
template <int NBW>
__device__ __forceinline__ float mq_tile(const int4 (&q)[NBW][2], const uint4 (&h)[NBW], const char* V,
                                         const int2* meta, int bA, int nbw, int lane) {
    const int g = lane >> 4;
    const bool odd = g & 1;
    const mq_v4i zero = {0, 0, 0, 0};
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < NBW; i++) {
        if (i < nbw) {
            const int b = bA + i;
            const uint4 hd = h[i];
            const float d = aeth_decode_d(hd.x), dmin = aeth_decode_d(hd.x >> 16);
            // get_scale_min_k4 (common.rs:29-38) for sub-blocks g and 4+g
            const uint32_t yb = (hd.y >> (8 * g)) & 0xFFu, zb = (hd.z >> (8 * g)) & 0xFFu;
            const uint32_t wb = (hd.w >> (8 * g)) & 0xFFu;
            const float sc[2] = {(float)(yb & 63u), (float)((wb & 15u) | ((yb >> 6) << 4))};
            const float mn[2] = {(float)(zb & 63u), (float)((wb >> 4) | ((zb >> 6) << 4))};
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                const int4 Q = q[i][hh];
                mq_v4i lo, hi;
                lo.x = Q.x & 0x0F0F0F0F; lo.y = Q.y & 0x0F0F0F0F; lo.z = Q.z & 0x0F0F0F0F; lo.w = Q.w & 0x0F0F0F0F;
                hi.x = (Q.x >> 4) & 0x0F0F0F0F; hi.y = (Q.y >> 4) & 0x0F0F0F0F;
                hi.z = (Q.z >> 4) & 0x0F0F0F0F; hi.w = (Q.w >> 4) & 0x0F0F0F0F;
                const mq_v4i A = *(const mq_v4i*)(V + (size_t)(b * 2 + hh) * 1024 + lane * 16);
                const mq_v4i D1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, lo, zero, 0, 0, 0);
                const mq_v4i D2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, hi, zero, 0, 0, 0);
                const int e0 = odd ? D2.x : D1.x, e1 = odd ? D2.y : D1.y, e2 = odd ? D2.z : D1.z;
                const int v = e0 + e1 * 256 + e2 * 65536;
                const int2 mt = meta[b * 8 + 4 * hh + g];
                acc = fmaf(ldexpf((float)v, mt.x), d * sc[hh], acc);
                acc = fmaf(-dmin * mn[hh], __int_as_float(mt.y), acc);
            }
        }
    }
    return acc;
}

__device__ __forceinline__ unsigned long long mq_amax_key(float v, int64_t row) {
    const uint32_t f = __float_as_uint(v);
    const uint32_t o = (f & 0x80000000u) ? ~f : (f | 0x80000000u);
    return ((unsigned long long)o << 32) | (unsigned long long)(uint32_t)row;
}

// Fusions (GemvParams in aeth_gemv.hip has the same meaning):
//  norm_w    : x ← x / sqrt(Σx²/k + eps) · norm_w first (rmsnorm_inplace, runner.rs:1739-1746);
//  swiglu    : rows (2i, 2i+1) = (gate_i, up_i); y[i] = g·σ(g)·u (runner.rs:1617-1625);
//  amax      : 64-bit atomic max of (orderable(y) << 32 | row) — ties → last row
//              (Iterator::max_by, runner.rs:1964-1973);
//  accumulate: y += result (residual adds, runner.rs:1609-1611, 1629-1631).
// RING = false: the workgroup's tiles all fit the RD load slots (issued up
// front); RING = true: the slots are refilled as they are consumed.
template <int NBW, int RD, int XO, bool RING, int W>
__global__ void __launch_bounds__(64 * W) k_gemv_q4k(MqParams G) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    __shared__ float ssum[W];
    __shared__ unsigned long long kmax[W];
    const int nb = G.nb;
    char* V = smem;
    int2* meta = (int2*)(smem + (size_t)nb * 2048);
    float* part = (float*)(smem + (size_t)nb * 2048 + (size_t)nb * 64);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float* xr = G.x + (int64_t)blockIdx.y * G.x_stride;
    float* yr = G.y + (int64_t)blockIdx.y * G.y_stride;
    const int64_t t0 = (int64_t)blockIdx.x * G.tpw;
    const int ntw = (int)min((int64_t)G.tpw, (int64_t)G.ntiles - t0);
    const int bA = nb * wave / W, nbw = nb * (wave + 1) / W - bA;
    const int o0 = 32 * bA, o1 = 32 * (bA + nbw);  // this wave's activation octets

    float xv[XO][8], wv[XO][8];
    mq_load_x<XO>(xr, o0, o1, xv);
    mq_load_x<XO>(G.norm_w ? G.norm_w : xr, o0, o1, wv);
    __builtin_amdgcn_sched_barrier(0);  // keep the activation loads ahead of the weight stream
    int4 q[RD][NBW][2];
    uint4 h[RD][NBW];
#pragma unroll
    for (int r = 0; r < RD; r++) mq_load<NBW>(q[r], h[r], G, t0 + min(r, ntw - 1), bA, nbw, lane);

    if (G.norm_w) {  // fused RMSNorm: the waves' slices tile the row (k = 256·nb); one barrier
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < XO; i++)
#pragma unroll
            for (int t = 0; t < 8; t++) ss += (o0 + lane + 64 * i < o1) ? xv[i][t] * xv[i][t] : 0.0f;
        ss = aeth_wave_sum(ss);
        if (lane == 0) ssum[wave] = ss;
        __syncthreads();
        float tot = 0.0f;
#pragma unroll
        for (int w = 0; w < W; w++) tot += ssum[w];
        const float rms = sqrtf(tot / (float)G.k + G.eps);
#pragma unroll
        for (int i = 0; i < XO; i++)
#pragma unroll
            for (int t = 0; t < 8; t++) xv[i][t] = xv[i][t] / rms * wv[i][t];
    }

    // a NaN or infinity in the slice makes every partial of this wave NaN
    const float poison = mq_build<XO>(xv, o0, o1, V, meta) ? __int_as_float(0x7FC00000) : 0.0f;

    if (!RING) {  // every tile already in flight: no refills
#pragma unroll
        for (int r = 0; r < RD; r++) {
            if (r < ntw) {
                float acc = mq_tile<NBW>(q[r], h[r], V, meta, bA, nbw, lane);
                acc += __shfl_xor(acc, 16, 64);
                acc += __shfl_xor(acc, 32, 64);
                if (lane < 16) part[(r * W + wave) * 16 + lane] = acc + poison;
            }
            __builtin_amdgcn_sched_barrier(0);  // tiles in arrival order: wait for each one alone
        }
    } else {  // ring of RD tiles; each consumed slot is refilled at once (clamped past the end)
        for (int j0 = 0; j0 < ntw; j0 += RD) {
#pragma unroll
            for (int r = 0; r < RD; r++) {
                const int j = j0 + r;
                if (j < ntw) {
                    float acc = mq_tile<NBW>(q[r], h[r], V, meta, bA, nbw, lane);
                    acc += __shfl_xor(acc, 16, 64);
                    acc += __shfl_xor(acc, 32, 64);
                    if (lane < 16) part[(j * W + wave) * 16 + lane] = acc + poison;
                }
                mq_load<NBW>(q[r], h[r], G, t0 + min(j + RD, ntw - 1), bA, nbw, lane);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    __syncthreads();

    unsigned long long best = 0;
    for (int idx = threadIdx.x; idx < ntw * 16; idx += 64 * W) {
        const int jt = idx >> 4, nn = idx & 15;
        const int64_t row = (t0 + jt) * 16 + nn;
        if (row >= G.n) continue;
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < W; w++) sum += part[(jt * W + w) * 16 + nn];
        if (G.swiglu) {
            if ((nn & 1) == 0) {
                float up = 0.0f;
#pragma unroll
                for (int w = 0; w < W; w++) up += part[(jt * W + w) * 16 + nn + 1];
                yr[row >> 1] = sum * (1.0f / (1.0f + expf(-sum))) * up;
            }
        } else {
            const float v = G.accumulate ? yr[row] + sum : sum;
            yr[row] = v;
            if (G.amax) {
                const unsigned long long kk = mq_amax_key(v, row);
                best = kk > best ? kk : best;
            }
        }
    }
    if (G.amax) {
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const unsigned long long o = __shfl_xor(best, off, 64);
            best = o > best ? o : best;
        }
        if (lane == 0) kmax[wave] = best;
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned long long m = kmax[0];
#pragma unroll
            for (int w = 1; w < W; w++) m = kmax[w] > m ? kmax[w] : m;
            atomicMax(G.amax, m);
        }
    }
}

template <int NBW, int RD, int XO, bool RING, int W>
static int mq_launch_k(dim3 grid, size_t lds, hipStream_t s, const MqParams& G) {
    static size_t opted = 64 * 1024;  // dynamic LDS above 64 KiB is opted into per kernel
    if (lds > opted) {
        AETH_HIP_CHECK(hipFuncSetAttribute((const void*)k_gemv_q4k<NBW, RD, XO, RING, W>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        opted = lds;
    }
    hipLaunchKernelGGL((k_gemv_q4k<NBW, RD, XO, RING, W>), grid, dim3(64 * W), lds, s, G);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}

template <int NBW, int RD, int XO, int W>
static int mq_launch(dim3 grid, size_t lds, hipStream_t s, const MqParams& G) {
    return G.tpw <= RD ? mq_launch_k<NBW, RD, XO, false, W>(grid, lds, s, G)
                       : mq_launch_k<NBW, RD, XO, true, W>(grid, lds, s, G);
}

int aeth_gemv_q4k_launch(const aeth_weight* w, const float* d_x, int64_t m, float* d_y, const GemvEpi& e,
                         hipStream_t s) {
    if (m > 65535) return aeth_set_error(AETH_EINVAL, "gemv: m=%lld exceeds 65535", (long long)m);
    const int nb = (int)w->nb;
    if (nb < 1 || nb > MQ_NB_MAX)
        return aeth_set_error(AETH_EUNSUPPORTED, "gemv q4_k: k=%lld outside [256, %d]", (long long)w->k,
                              MQ_NB_MAX * 256);
    if (e.norm_w && w->k != (int64_t)nb * 256)
        return aeth_set_error(AETH_EUNSUPPORTED, "gemv q4_k: fused RMSNorm needs k a multiple of 256");
    if (e.swiglu && (w->n & 1)) return aeth_set_error(AETH_EUNSUPPORTED, "gemv q4_k: SwiGLU needs paired rows");
    if (((uintptr_t)d_x & 15) || (e.norm_w && ((uintptr_t)e.norm_w & 15)))
        return aeth_set_error(AETH_EINVAL, "gemv q4_k: x and norm weight must be 16-byte aligned");
    if (m > 1 && (w->k & 3)) return aeth_set_error(AETH_EINVAL, "gemv q4_k: m > 1 needs k % 4 == 0 (row alignment)");
    MqParams G;
    G.hdr = w->p0;
    G.qs = w->p1;
    G.n = w->n;
    G.nb = nb;
    G.ntiles = (int)aeth_cdiv(w->n, 16);
    // Shape choice: W waves split K; RD tiles per workgroup with all loads issued
    // up front (short memory queues, so each wave's tiles arrive early and
    // their compute overlaps the stream). Taller matrices use the ring with ~2
    // workgroups per CU so the per-workgroup activation conversion stays
    // amortised.
    const int64_t cus = aeth_num_cus();
    // tuning overrides, read once: AETH_GEMV_WAVES (8 | 16), AETH_GEMV_TPW (tiles per workgroup)
    static const int env_w = getenv("AETH_GEMV_WAVES") ? atoi(getenv("AETH_GEMV_WAVES")) : 0;
    static const int env_tpw = getenv("AETH_GEMV_TPW") ? atoi(getenv("AETH_GEMV_TPW")) : 0;
    // (measured: 16 waves pay off only for long rows, k ≥ 8192; one tile per
    // workgroup when there are no more tiles than CUs)
    int W = nb >= 32 ? 16 : 8;
    if (env_w) W = env_w == 16 ? 16 : 8;
    const int nbw = (nb + W - 1) / W;
    const int rd = W == 16 ? (nbw <= 2 ? 2 : 1) : (nbw <= 4 ? 2 : 1);
    int64_t tpw = G.ntiles <= cus ? 1 : G.ntiles <= 8 * cus ? rd : aeth_cdiv(G.ntiles, 2 * cus);
    if (env_tpw > 0) tpw = env_tpw;
    if (tpw > MQ_TPW_MAX) tpw = MQ_TPW_MAX;
    G.tpw = (int)tpw;
    G.x = d_x;
    G.x_stride = w->k;
    G.k = (int)w->k;
    G.y = d_y;
    G.y_stride = e.swiglu ? w->n / 2 : w->n;
    G.accumulate = (e.flags & AETH_MM_ACCUMULATE) ? 1 : 0;
    G.norm_w = e.norm_w;
    G.eps = e.eps;
    G.swiglu = e.swiglu;
    G.amax = e.amax;
    const dim3 grid((unsigned)aeth_cdiv(G.ntiles, tpw), (unsigned)m);
    const size_t lds = (size_t)nb * 2048 + (size_t)nb * 64 + (size_t)tpw * W * 16 * 4;
    if (W == 16) {
        if (nbw <= 1) return mq_launch<1, 2, 1, 16>(grid, lds, s, G);
        if (nbw <= 2) return mq_launch<2, 2, 1, 16>(grid, lds, s, G);
        return mq_launch<4, 1, 2, 16>(grid, lds, s, G);
    }
    if (nbw <= 1) return mq_launch<1, 2, 1, 8>(grid, lds, s, G);
    if (nbw <= 2) return mq_launch<2, 2, 1, 8>(grid, lds, s, G);
    if (nbw <= 4) return mq_launch<4, 2, 2, 8>(grid, lds, s, G);
    return mq_launch<8, 1, 4, 8>(grid, lds, s, G);
}
