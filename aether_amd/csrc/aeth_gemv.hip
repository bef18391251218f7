// Decode GEMV for Q4_K / Q5_K / Q6_K / Q8_0 weights on the int8 matrix cores of gfx950:
//   y[r] = Σ_k x[k]·W[r][k]  (avx2::matmul_q4_k / matmul_q6_k / matmul_q5_k,
//   src/quant/avx2.rs:23-131; scalar matmul_q8_0, src/quant/matmul/q8_0.rs:5-89),
//   one activation row per grid.y.
//
// Exact integer core. Each wave turns its slice of the activation row into an
// exact integer form: per group of 32 (Q4_K, Q5_K, Q8_0) or 16 (Q6_K) elements,
// x = x_int·2^-S with |x_int| < 2^30 against the group maximum — every element
// within 2^7 of the maximum is represented exactly (its 24-bit significand
// fits), smaller ones to 2^-30 of the maximum — split into four balanced
// signed byte digits x_int = d0 + 2^8·d1 + 2^16·d2 + 2^24·d3. The digits are
// the A operand of v_mfma_i32_16x16x64_i8 — M = 4 output slots × 4 digit rows
// — and 16 weight rows are the B operand (N). Lane (n, kg) (n = lane % 16,
// kg = lane / 16) supplies 16 k-slots of row n; A lane (m, kg) holds the
// digits that pair with them, nonzero only where slot m/4 owns those k-slots.
// One MFMA so returns the exact integer dot of every digit with 64 quants of 16
// rows, already split by scale group; the output lane (n, g) holds slot g's
// four digit sums for row n (each exact in i32: |Σ q·d| ≤ 32·63·128), pairs
// them in i32 (d0 + 2^8·d1, d2 + 2^8·d3) and recombines exactly in f64 before
// one rounding to f32 and the group's scales (Q4_K: one f32 fma, exact because
// both pairs fit 24 bits).
//
// Per format ("chunk" = the unit of K a wave steps through):
//  Q4_K, chunk = super-block (256). Per half h, lane (n, kg) loads
//    qs[64h + 16kg, +16) of row n: low nibbles are sub-block 4h + 2(kg ≥ 2),
//    high nibbles the next one. Two chained MFMAs (low, then high nibbles):
//    the even slots' A rows feed the first, the odd slots' the second (each
//    reads the zero slot for the other rows), so slot g ↔ sub-block 4h + g
//    ends complete;  acc += 2^-S·Σq·x_int·d·sc − dmin·m·Σx.
//  Q5_K, as Q4_K (same quant and header planes) plus a plane of fifth bits:
//    lane (n, kg) loads 8 bytes, 16 bits per (half, low / high nibbles) for its
//    16 elements; each bit is spread to 0x10 of its byte before the MFMA.
//  Q8_0, chunk = 4 blocks (128). MFMA j, lane (n, kg): the 16 raw quant bytes
//    [16(kg & 1), +16) of block 2j + (kg ≥ 2) — no unpacking; slot g ↔ block g.
//    acc += 2^-S·(Σ q·x_int)·d.
//  Q6_K, chunk = super-block. Lane (n, kg) loads the 48 bytes of its 2×16
//    elements of half h = kg / 2, g' = kg % 2: ql[64h + 16g', +16),
//    ql[64h + 32 + 16g', +16), qh[32h + 16g', +16), and MFMA v (0..3) takes
//    sub-block (h, v, g') = elements 128h + 32v + 16g' + [0, 16) as the 6-bit
//    q + 32 ∈ [0, 63]; slot g ↔ lane group kg = g. The offset is removed
//    exactly per digit (−32·Σ digit) before   acc += 2^-S·Σ(q)·x_int·sc·d.
//
// A operands are kept compact in LDS: only the digit rows, 16-byte vectors
// indexed (region, kg, slot, digit), 4 bytes per activation element.
// A lane whose (m, kg) holds no digits for an MFMA reads a 16-byte zero slot
// instead (one address select per operand read).
//
// Work split: a workgroup (W = 8 or 16 waves) owns a run of 16-row tiles; wave
// w takes chunks [nc·w/W, nc·(w+1)/W) of every tile, converts only that slice
// of x (no barrier: LDS operations of one wave execute in order), keeps RD
// tiles of loads in flight, and leaves 16 partial row sums per tile in LDS;
// after the one barrier the partials are summed in a fixed order
// (deterministic) and the epilogue (accumulate, SwiGLU, argmax) runs.
//
// Every global load is issued unconditionally (values past a wave's chunks or
// a workgroup's tiles are discarded): the compiler can then count outstanding
// loads exactly and wait for each one alone, instead of draining the whole
// weight stream at the first use of x. Surplus loads repeat a load issued in
// the same batch (still in flight, so they cost no HBM traffic), except the
// ring's refills past the last tile, which read chunk 0 of tile 0.
#include <math.h>
#include <stdlib.h>

#include "aeth_common.hpp"
#include "aeth_internal.hpp"

#define MQ_TPW_MAX 32  // tiles per workgroup (LDS partials: 64 B per wave each)
#define MQ_LDS_MAX (160 * 1024)

typedef int mq_v4i __attribute__((ext_vector_type(4)));

enum { FQ4K = 0, FQ6K = 1, FQ80 = 2, FQ5K = 3 };

struct MqParams {
    const uint8_t* p0;
    const uint8_t* p1;
    const uint8_t* p2;
    int64_t n;
    int nc, ntiles, tpw;  // chunks per row, 16-row tiles, tiles per workgroup
    const float* x;
    int64_t x_stride;
    int k, kx;            // k; activation elements the product reads (kx ≤ k)
    float* y;
    int64_t y_stride;
    int accumulate;
    const float* norm_w;
    float eps;
    int swiglu;
    unsigned long long* amax;
    int plain_d;          // no block scale of the weight has the f16 exponent 31
};

__device__ __forceinline__ uint32_t mq_pack4(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xFF) | ((uint32_t)(b & 0xFF) << 8) | ((uint32_t)(c & 0xFF) << 16) | ((uint32_t)d << 24);
}

__device__ __forceinline__ mq_v4i mq_mfma(const mq_v4i& a, const mq_v4i& b, const mq_v4i& c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// 16 weight bytes, read once per GEMV: a non-temporal (streaming) load, which
// keeps the weight stream from displacing x and the other operands in L2.
__device__ __forceinline__ int4 mq_ld16(const uint8_t* p) {
    const mq_v4i v = __builtin_nontemporal_load((const mq_v4i*)p);
    return make_int4(v.x, v.y, v.z, v.w);
}

// ── per-format traits ────────────────────────────────────────────────────
// CE: activation elements per chunk; AB: LDS bytes of A operands per chunk;
// MB: LDS meta bytes per chunk; GE: elements per exponent group.
template <int F> struct MF;

// Lane constants for reading A: (m, kg) of this lane.
struct MqLane {
    int m, kg, s, d;
};

// Σ q·x_int from its digit pairs lo = Σq·d0 + 2^8·Σq·d1 and hi = Σq·d2 + 2^8·Σq·d3
// (both exact in i32): exact in f64, rounded once to f32.
__device__ __forceinline__ float mq_recombine(int lo, int hi) {
    return (float)fma((double)hi, 65536.0, (double)lo);
}

// Bit i of b (i < 4) → 0x10 in byte i: the fifth quant bit of four elements.
__device__ __forceinline__ int mq_spread4(uint32_t b) { return (int)(((b * 0x00204081u) & 0x01010101u) << 4); }

// Q4_K and Q5_K share the chunk, the A layout and the scale handling; Q5_K adds
// the fifth bits, read per lane as 4 × 16 bits (half h, low / high nibble).
template <bool Q5> struct MFK {
    static constexpr int CE = 256, AB = 1024, MB = 64, GE = 32;
    struct D { int4 q[2]; uint4 h; uint2 qh; };
    // planes: p0 = headers [tile][sb][16 rows][16 B], p1 = quants [tile][sb][h][64][16 B],
    //         Q5: p2 = fifth bits [tile][sb][64][8 B]
    __device__ static void load(D& d, const MqParams& G, int64_t c, int lane) {  // c = tile·nc + chunk
        d.q[0] = mq_ld16(G.p1 + (c * 2) * 1024 + lane * 16);
        d.q[1] = mq_ld16(G.p1 + (c * 2 + 1) * 1024 + lane * 16);
        const int4 h = mq_ld16(G.p0 + (c * 16 + (lane & 15)) * 16);
        d.h = make_uint4(h.x, h.y, h.z, h.w);
        if (Q5) d.qh = *(const uint2*)(G.p2 + (c * 64 + lane) * 8);
    }
    // compact A: per half h, vector ((kg·2 + (s & 1))·4 + d), kg ∈ the pair of slot s.
    // byte offset of an octet's digit-0 piece (digit d: +16·d)
    __device__ static int aoff(int ec) {
        const int h = ec >> 7, s = (ec >> 5) & 3, p = ec & 31, kg = 2 * (s >> 1) + (p >> 4);
        return h * 512 + ((kg * 2 + (s & 1)) * 4) * 16 + (p & 8);
    }
    // PD: the weight holds no d / dmin with the f16 exponent 31 (aeth_weight::special_scales),
    // so decode_d's NaN / infinity rule never applies and a plain f16 conversion is exact
    template <bool Q8A, bool PD>
    __device__ static float dot(const D& dd, const char* A, const char* meta, int lane, const MqLane& L,
                                const char* zs) {
        const int g = lane >> 4;
        // A rows of the even slots pair with the low nibbles, of the odd slots
        // with the high ones: each MFMA reads only its own rows (the others from
        // the zero slot), so the second accumulates onto the first and every
        // output lane ends with its slot's four digit sums
        const bool va = (L.s >> 1) == (L.kg >> 1);
        const bool vlo = va && !(L.s & 1), vhi = va && (L.s & 1);
        const int vo = ((L.kg * 2 + (L.s & 1)) * 4 + L.d) * 16;
        const mq_v4i zero = {0, 0, 0, 0};
        const float d = PD ? aeth_f16_to_f32(dd.h.x) : aeth_decode_d(dd.h.x);
        const float dmin = PD ? aeth_f16_to_f32(dd.h.x >> 16) : aeth_decode_d(dd.h.x >> 16);
        // get_scale_min_k4 (common.rs:29-38) for sub-blocks g and 4 + g
        const uint32_t yb = (dd.h.y >> (8 * g)) & 0xFFu, zb = (dd.h.z >> (8 * g)) & 0xFFu;
        const uint32_t wb = (dd.h.w >> (8 * g)) & 0xFFu;
        const float sc[2] = {(float)(yb & 63u), (float)((wb & 15u) | ((yb >> 6) << 4))};
        const float mn[2] = {(float)(zb & 63u), (float)((wb >> 4) | ((zb >> 6) << 4))};
        float acc = 0.0f;
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            const int4 Q = dd.q[hh];
            mq_v4i lo, hi;
            lo.x = Q.x & 0x0F0F0F0F; lo.y = Q.y & 0x0F0F0F0F; lo.z = Q.z & 0x0F0F0F0F; lo.w = Q.w & 0x0F0F0F0F;
            hi.x = (Q.x >> 4) & 0x0F0F0F0F; hi.y = (Q.y >> 4) & 0x0F0F0F0F;
            hi.z = (Q.z >> 4) & 0x0F0F0F0F; hi.w = (Q.w >> 4) & 0x0F0F0F0F;
            if (Q5) {  // q = nibble | fifth bit << 4 ∈ [0, 31]
                const uint32_t hw = hh ? dd.qh.y : dd.qh.x, hl = hw & 0xFFFFu, hu = hw >> 16;
                lo.x |= mq_spread4(hl & 15u); lo.y |= mq_spread4((hl >> 4) & 15u);
                lo.z |= mq_spread4((hl >> 8) & 15u); lo.w |= mq_spread4(hl >> 12);
                hi.x |= mq_spread4(hu & 15u); hi.y |= mq_spread4((hu >> 4) & 15u);
                hi.z |= mq_spread4((hu >> 8) & 15u); hi.w |= mq_spread4(hu >> 12);
            }
            const mq_v4i alo = *(const mq_v4i*)(vlo ? A + hh * 512 + vo : zs);
            const mq_v4i ahi = *(const mq_v4i*)(vhi ? A + hh * 512 + vo : zs);
            const mq_v4i E = mq_mfma(ahi, hi, mq_mfma(alo, lo, zero));
            const int2 mt = ((const int2*)meta)[4 * hh + g];
            if (Q8A) {  // matmul_q4_k / q5_k_dotprod: d_a·(d1·Σq·q_a − m1·Σq_a) (neon.rs:436-437)
                const float d1 = d * sc[hh], m1 = dmin * mn[hh];
                acc += __int_as_float(mt.y) * (d1 * (float)E.x - m1 * (float)mt.x);
            } else {
                // Q4_K: both pairs fit 24 bits (|Σq·d| ≤ 32·15·128), so one f32
                // fma rounds the exact sum once, as the f64 form does
                const float v = Q5 ? mq_recombine(E.x + E.y * 256, E.z + E.w * 256)
                                   : fmaf((float)(E.z + E.w * 256), 65536.0f, (float)(E.x + E.y * 256));
                acc = fmaf(ldexpf(v, mt.x), d * sc[hh], acc);
                acc = fmaf(-dmin * mn[hh], __int_as_float(mt.y), acc);
            }
        }
        return acc;
    }
};
template <> struct MF<FQ4K> : MFK<false> {};
template <> struct MF<FQ5K> : MFK<true> {};

template <> struct MF<FQ80> {
    static constexpr int CE = 128, AB = 512, MB = 32, GE = 32;
    struct D { int4 q[2]; uint32_t d; };
    // planes: p0 = quants [tile][group][j][64][16 B], p1 = d [tile][group][4 blocks][16 rows] (f16)
    __device__ static void load(D& d, const MqParams& G, int64_t c, int lane) {
        // plain loads: measured faster than streaming ones for this format
        d.q[0] = *(const int4*)(G.p0 + (c * 2) * 1024 + lane * 16);
        d.q[1] = *(const int4*)(G.p0 + (c * 2 + 1) * 1024 + lane * 16);
        d.d = ((const uint16_t*)G.p1)[c * 64 + lane];
    }
    // compact A: per MFMA j, vector (kg·4 + d) (slot s = 2j + (kg ≥ 2))
    __device__ static int aoff(int ec) {
        const int s = ec >> 5, p = ec & 31, kg = 2 * (s & 1) + (p >> 4);
        return (s >> 1) * 256 + (kg * 4) * 16 + (p & 8);
    }
    template <bool Q8A, bool PD>
    __device__ static float dot(const D& dd, const char* A, const char* meta, int lane, const MqLane& L,
                                const char* zs) {
        const int g = lane >> 4;
        const mq_v4i zero = {0, 0, 0, 0};
        const int vo = (L.kg * 4 + L.d) * 16;
        const bool v0 = L.s == (L.kg >> 1), v1 = L.s == 2 + (L.kg >> 1);
        const mq_v4i a0 = *(const mq_v4i*)(v0 ? A + vo : zs), a1 = *(const mq_v4i*)(v1 ? A + 256 + vo : zs);
        const mq_v4i b0 = {dd.q[0].x, dd.q[0].y, dd.q[0].z, dd.q[0].w};
        const mq_v4i b1 = {dd.q[1].x, dd.q[1].y, dd.q[1].z, dd.q[1].w};
        const mq_v4i D = mq_mfma(a1, b1, mq_mfma(a0, b0, zero));
        const int2 mt = ((const int2*)meta)[g];
        if (Q8A)  // matmul_q8_0_dotprod: (Σ q_a·q)·(d_a·d) (tests.rs:44-56)
            return (float)D.x * (__int_as_float(mt.y) * aeth_f16_to_f32(dd.d));
        const float val = mq_recombine(D.x + D.y * 256, D.z + D.w * 256);
        return ldexpf(val, mt.x) * aeth_f16_to_f32(dd.d);  // Q8_0 scales are plain f16 (q8_0.rs)
    }
};

template <> struct MF<FQ6K> {
    static constexpr int CE = 256, AB = 1024, MB = 256, GE = 16;
    struct D { int4 a, b, h; uint2 sc; uint32_t d; };
    // planes: p0 = [tile][sb][part A|B|H][64][16 B], p1 = sc [tile][sb][16 rows][16 B],
    //         p2 = d [tile][sb][16 rows] (f16)
    __device__ static void load(D& d, const MqParams& G, int64_t c, int lane) {
        d.a = mq_ld16(G.p0 + (c * 3) * 1024 + lane * 16);
        d.b = mq_ld16(G.p0 + (c * 3 + 1) * 1024 + lane * 16);
        d.h = mq_ld16(G.p0 + (c * 3 + 2) * 1024 + lane * 16);
        d.sc = *(const uint2*)(G.p1 + (c * 16 + (lane & 15)) * 16 + ((lane >> 5) & 1) * 8);
        d.d = ((const uint16_t*)G.p2)[c * 16 + (lane & 15)];
    }
    // compact A: per MFMA v, vector (kg·4 + d) (slot = kg)
    __device__ static int aoff(int ec) {
        const int h = ec >> 7, r = ec & 127, v = r >> 5, kg = 2 * h + ((r >> 4) & 1);
        return v * 256 + (kg * 4) * 16 + (r & 8);
    }
    template <bool Q8A, bool PD>
    __device__ static float dot(const D& dd, const char* A, const char* meta, int lane, const MqLane& L,
                                const char* zs) {
        const int g = lane >> 4;
        const bool va = L.s == L.kg;
        const int vo = (L.kg * 4 + L.d) * 16;
        const mq_v4i zero = {0, 0, 0, 0};
        const int* Aw = (const int*)&dd.a;
        const int* Bw = (const int*)&dd.b;
        const int* Hw = (const int*)&dd.h;
        // scale bytes sc[8h + 2v + g'] (the half h = g / 2 was picked at load; g' = g % 2)
        const uint32_t s01 = dd.sc.x >> (8 * (g & 1)), s23 = dd.sc.y >> (8 * (g & 1));
        float part = 0.0f;
#pragma unroll
        for (int v = 0; v < 4; v++) {
            mq_v4i q;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                int w;
                if (v == 0) w = (Aw[e] & 0x0F0F0F0F) | ((Hw[e] << 4) & 0x30303030);
                else if (v == 1) w = (Bw[e] & 0x0F0F0F0F) | ((Hw[e] << 2) & 0x30303030);
                else if (v == 2) w = ((Aw[e] >> 4) & 0x0F0F0F0F) | (Hw[e] & 0x30303030);
                else w = ((Bw[e] >> 4) & 0x0F0F0F0F) | ((Hw[e] >> 2) & 0x30303030);
                q[e] = w;
            }
            const mq_v4i a = *(const mq_v4i*)(va ? A + v * 256 + vo : zs);
            const mq_v4i Dv = mq_mfma(a, q, zero);
            const int4 mt = ((const int4*)meta)[8 * (g >> 1) + 2 * v + (g & 1)];
            const uint32_t sw = v < 2 ? s01 : s23;
            const float scv = (float)(int8_t)((sw >> (16 * (v & 1))) & 0xFFu);
            if (Q8A) {  // matmul_q6_k_dotprod: (d·s·d_a)·Σ q_a·(q − 32) (neon.rs / tests.rs:227-237)
                part += (aeth_decode_d(dd.d) * scv * __int_as_float(mt.y)) * (float)(Dv.x - 32 * mt.x);
                continue;
            }
            // stored q + 32 ∈ [0, 63]: subtract 32·Σ x_int per digit pair (exact in i32)
            const float val = ldexpf(mq_recombine(Dv.x + Dv.y * 256 - mt.y, Dv.z + Dv.w * 256 - mt.z), mt.x);
            part += scv * val;
        }
        return Q8A ? part : aeth_decode_d(dd.d) * part;
    }
};

// Lane l of the wave owns activation octets o = o0 + l + 64·i (elements
// [8o, 8o+8)) below o1; elements at or past kx read as zero.
template <int XO, bool RAG>
__device__ __forceinline__ void mq_load_x(const float* __restrict__ x, int o0, int o1, int kx,
                                          float (&xv)[XO][8]) {
#pragma unroll
    for (int i = 0; i < XO; i++) {
        const int o = o0 + (threadIdx.x & 63) + 64 * i;
        if (!RAG) {  // kx % 8 == 0: copies past o1 / kx are masked at their uses
            const int oc = min(o, max(min(o1, kx / 8) - 1, 0));
            const float4 a = *(const float4*)(x + 8 * oc), b = *(const float4*)(x + 8 * oc + 4);
            xv[i][0] = a.x; xv[i][1] = a.y; xv[i][2] = a.z; xv[i][3] = a.w;
            xv[i][4] = b.x; xv[i][5] = b.y; xv[i][6] = b.z; xv[i][7] = b.w;
        } else {  // k not a multiple of 8 (Q8_0 only): element-wise
#pragma unroll
            for (int t = 0; t < 8; t++) xv[i][t] = x[min(8 * o + t, kx - 1)];
        }
    }
}

// The wave's activation slice → compact A operands (every byte of the slice's
// regions is written) and per-group meta: Q4_K / Q5_K {−S, Σx}, Q8_0 {−S, 0},
// Q6_K {−S, 32·(Σd0 + 2^8·Σd1), 32·(Σd2 + 2^8·Σd3), 0}. Written and later
// read by this wave only.
// Q8A (the int8 dot-product path): the slice becomes Q8_0 activation blocks
// instead, byte for byte as quantize_q8_0_block (neon.rs:45-104) makes them:
// per 32 elements d = max|x|/127 (a NaN anywhere gives NaN), stored as f16,
// q = sat_i8(RNE(x·(1/d))) with the f32 d, zeros when d is not > 0; digit 0
// holds q, the others zero; meta Q4_K / Q5_K {Σq, d_a}, Q8_0 {0, d_a}, Q6_K
// per 16 elements {Σq, d_a} (d_a = the stored f16 scale as f32).
// Converts the octet sets xv[ib .. ie) (set i: this lane's octet o0 + lane + 64i), each set
// independently; returns nonzero (wave-uniform) if they hold a NaN or an infinity.
template <int F, int XO, bool Q8A>
__device__ __forceinline__ int mq_build(float (&xv)[XO][8], int c0, int nbw, int kx, char* Abase, char* Mbase,
                                        int ib = 0, int ie = XO) {
    typedef MF<F> T;
    const int lane = threadIdx.x & 63;
    const int o0 = c0 * (T::CE / 8), o1 = (c0 + nbw) * (T::CE / 8);
    int bad = 0;
#pragma unroll
    for (int i = ib; i < ie; i++) {
        const int o = o0 + lane + 64 * i;
        const bool live = o < o1;
        float* v = xv[i];
        if (8 * o1 > kx) {  // the slice runs past k (Q8_0 padding blocks, ragged k): zeros there
#pragma unroll
            for (int t = 0; t < 8; t++)
                if (8 * o + t >= kx) v[t] = 0.0f;
        }
        float mx = 0.0f;
        bool nan = false;  // fmaxf drops NaN operands: test for them explicitly
#pragma unroll
        for (int t = 0; t < 8; t++) {
            mx = fmaxf(mx, fabsf(v[t]));
            nan |= v[t] != v[t];
        }
        mx = fmaxf(mx, aeth_dpp_xor1f(mx));  // the octets of a group are adjacent lanes
        if (T::GE == 32 || Q8A) mx = fmaxf(mx, aeth_dpp_xor2f(mx));  // Q8_0 activation blocks are 32 wide
        const bool fin = isfinite(mx);
        if ((!fin || nan) && live) bad = 1;
        if (Q8A) {
            int nb4 = nan ? 1 : 0;
            nb4 |= aeth_dpp_xor1(nb4);
            nb4 |= aeth_dpp_xor2(nb4);
            const float dq = nb4 ? __int_as_float(0x7FC00000) : mx / 127.0f;
            const float da = aeth_f16_to_f32(aeth_f32_to_f16_bits(dq));
            const float inv = 1.0f / dq;
            int q[8], sq = 0;
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const float pr = v[t] * inv;
                q[t] = dq > 0.0f && pr == pr ? max(-128, min(127, (int)rintf(fminf(fmaxf(pr, -256.0f), 256.0f)))) : 0;
                sq += q[t];
            }
            sq += aeth_dpp_xor1(sq);
            if (T::GE == 32) sq += aeth_dpp_xor2(sq);
            if (live) {
                const int c = o / (T::CE / 8), ec = 8 * o - c * T::CE;
                char* dst = Abase + (size_t)c * T::AB + T::aoff(ec);
                *(uint2*)(dst) = make_uint2(mq_pack4(q[0], q[1], q[2], q[3]), mq_pack4(q[4], q[5], q[6], q[7]));
                *(uint2*)(dst + 16) = make_uint2(0u, 0u);
                *(uint2*)(dst + 32) = make_uint2(0u, 0u);
                *(uint2*)(dst + 48) = make_uint2(0u, 0u);
                char* mb = Mbase + (size_t)c * T::MB;
                if (F != FQ6K && (ec & 31) == 0) ((int2*)mb)[ec >> 5] = make_int2(F == FQ80 ? 0 : sq, __float_as_int(da));
                if (F == FQ6K && (ec & 15) == 0) ((int4*)mb)[ec >> 4] = make_int4(sq, __float_as_int(da), 0, 0);
            }
            continue;
        }
        const bool use = mx > 0.0f && fin;
        int E = 0;
        if (use) (void)frexpf(mx, &E);
        const int S = use ? 30 - E : 0;  // max|x| < 2^E, so |x_int| < 2^30
        // Balanced digits by one biased add: y = x_int + 0x808080 has bytes
        // (d0 + 128, d1 + 128, d2 + 128, d3) — each (d + 128) ∈ [0, 255] absorbs
        // the borrow the balanced split would propagate, and d3 = y >> 24 ∈ [−64, 64].
        // The bytes are then transposed (element-major → digit-major) and the
        // bias flipped off with one xor per word (−128 ≡ ^0x80 on a byte).
        uint32_t y[8];
        uint32_t sx = 0, sh = 0;  // Q6_K: Σ x_int and Σ (y >> 16), both mod 2^32
        float fs = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const int xi = use ? (int)rintf(ldexpf(v[t], S)) : 0;
            y[t] = (uint32_t)xi + 0x00808080u;
            sx += (uint32_t)xi;
            sh += (uint32_t)((int)y[t] >> 16);  // (d2 + 128) + 2^8·d3
            fs += v[t];
        }
        uint32_t dg[4][2];  // digit d of elements 4j .. 4j + 3
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const uint32_t *z = y + 4 * j;
            const uint32_t l01 = __builtin_amdgcn_perm(z[1], z[0], 0x05010400u);  // z0.b0 z1.b0 z0.b1 z1.b1
            const uint32_t h01 = __builtin_amdgcn_perm(z[1], z[0], 0x07030602u);  // z0.b2 z1.b2 z0.b3 z1.b3
            const uint32_t l23 = __builtin_amdgcn_perm(z[3], z[2], 0x05010400u);
            const uint32_t h23 = __builtin_amdgcn_perm(z[3], z[2], 0x07030602u);
            dg[0][j] = __builtin_amdgcn_perm(l23, l01, 0x05040100u) ^ 0x80808080u;
            dg[1][j] = __builtin_amdgcn_perm(l23, l01, 0x07060302u) ^ 0x80808080u;
            dg[2][j] = __builtin_amdgcn_perm(h23, h01, 0x05040100u) ^ 0x80808080u;
            dg[3][j] = __builtin_amdgcn_perm(h23, h01, 0x07060302u);
        }
        if (F == FQ4K || F == FQ5K) {
            fs += aeth_dpp_xor1f(fs);
            fs += aeth_dpp_xor2f(fs);
        }
        int slo = 0, shi = 0;
        if (F == FQ6K) {  // per 16 elements: Σ(d0 + 2^8·d1) and Σ(d2 + 2^8·d3), exact in i32
            sx += (uint32_t)aeth_dpp_xor1((int)sx);
            sh += (uint32_t)aeth_dpp_xor1((int)sh);
            shi = (int)(sh - 128u * 16u);
            slo = (int)(sx - ((uint32_t)shi << 16));
        }
        if (live) {
            const int c = o / (T::CE / 8), ec = 8 * o - c * T::CE;
            char* dst = Abase + (size_t)c * T::AB + T::aoff(ec);
            *(uint2*)(dst) = make_uint2(dg[0][0], dg[0][1]);
            *(uint2*)(dst + 16) = make_uint2(dg[1][0], dg[1][1]);
            *(uint2*)(dst + 32) = make_uint2(dg[2][0], dg[2][1]);
            *(uint2*)(dst + 48) = make_uint2(dg[3][0], dg[3][1]);
            char* mb = Mbase + (size_t)c * T::MB;
            if ((F == FQ4K || F == FQ5K) && (ec & 31) == 0) ((int2*)mb)[ec >> 5] = make_int2(-S, __float_as_int(fs));
            if (F == FQ80 && (ec & 31) == 0) ((int2*)mb)[ec >> 5] = make_int2(-S, 0);
            if (F == FQ6K && (ec & 15) == 0) ((int4*)mb)[ec >> 4] = make_int4(-S, 32 * slo, 32 * shi, 0);
        }
    }
    return __any(bad);
}

// Fusions:
//  norm_w    : x ← x / sqrt(Σx²/k + eps) · norm_w first (rmsnorm_inplace, runner.rs:1739-1746);
//              exact path: (W·(x·norm_w)) / rms, the epilogue divides; Q8A: x / rms · norm_w, then quantized;
//  swiglu    : rows (2i, 2i+1) = (gate_i, up_i); y[i] = g·σ(g)·u (runner.rs:1617-1625);
//  amax      : 64-bit atomic max of (orderable(y) << 32 | row) — ties → last row
//              (Iterator::max_by, runner.rs:1964-1973);
//  accumulate: y += result (residual adds, runner.rs:1609-1611, 1629-1631).
// RING = false: the workgroup's tiles all fit the RD load slots (issued up
// front); RING = true: the slots are refilled as they are consumed.
// NORM: the exact path's fused RMSNorm, with the division moved to the epilogue (G.norm_w set,
// !Q8A); other instances apply a G.norm_w to the row first.
template <int F, int NBW, int RD, int XO, bool RING, int W, bool RAG, bool Q8A, bool NORM, bool PD>
__global__ void __launch_bounds__(64 * W) k_gemv_mf(MqParams G) {
    typedef MF<F> T;
    typedef typename T::D Dt;
    extern __shared__ __attribute__((aligned(16))) char smem[];
    __shared__ float ssum[W];
    __shared__ unsigned long long kmax[W];
    const int nc = G.nc;
    char* Abase = smem;
    char* Mbase = smem + (size_t)nc * T::AB;
    float* part = (float*)(smem + (size_t)nc * (T::AB + T::MB));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    char* zs = (char*)(part + (size_t)G.tpw * W * 16) + 16 * wave;  // this wave's zero slot
    MqLane L;
    L.m = lane & 15;
    L.kg = lane >> 4;
    L.s = L.m >> 2;
    L.d = L.m & 3;
    const float* xr = G.x + (int64_t)blockIdx.y * G.x_stride;
    float* yr = G.y + (int64_t)blockIdx.y * G.y_stride;
    const int64_t t0 = (int64_t)blockIdx.x * G.tpw;
    const int ntw = (int)min((int64_t)G.tpw, (int64_t)G.ntiles - t0);
    const int c0 = nc * wave / W, nbw = nc * (wave + 1) / W - c0;
    const int o0 = c0 * (T::CE / 8), o1 = (c0 + nbw) * (T::CE / 8);

    float xv[XO][8], wv[XO][8];
    mq_load_x<XO, RAG>(xr, o0, o1, G.kx, xv);
    if (NORM || G.norm_w) mq_load_x<XO, RAG>(G.norm_w, o0, o1, G.kx, wv);  // (a uniform branch)
    // the residual this thread adds in the epilogue (row t0·16 + thread, the epilogue's first
    // pass), loaded now so that its latency hides behind the weight stream; unconditional, from
    // x when there is none to add (a load under a branch would be waited for at its end)
    const float* yp = G.accumulate && !G.swiglu ? yr + min(t0 * 16 + (int64_t)threadIdx.x, G.n - 1) : xr;
    const float yprev = *yp;
    __builtin_amdgcn_sched_barrier(0);  // keep the activation loads ahead of the weight stream
    Dt buf[RD][NBW];
#pragma unroll
    for (int r = 0; r < RD; r++)
#pragma unroll
        for (int i = 0; i < NBW; i++)
            T::load(buf[r][i], G, (t0 + min(r, ntw - 1)) * nc + c0 + min(i, max(nbw - 1, 0)), lane);

    if (NORM) {
        // fused RMSNorm, exact dots: 1/rms is one factor of every output, so the slice
        // becomes x·w at once and each output row is divided by rms in the epilogue, after
        // the barrier that is there anyway — no wave waits for the others before its first
        // dot; each wave leaves its slice's Σx² (the slices tile the row)
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < XO; i++) {
            const int o = o0 + lane + 64 * i;
#pragma unroll
            for (int t = 0; t < 8; t++) ss += (o < o1 && 8 * o + t < G.kx) ? xv[i][t] * xv[i][t] : 0.0f;
        }
        ss = aeth_wave_sum(ss);
        if (lane == 0) ssum[wave] = ss;
#pragma unroll
        for (int i = 0; i < XO; i++)
#pragma unroll
            for (int t = 0; t < 8; t++) xv[i][t] *= wv[i][t];
    } else if (G.norm_w) {
        // fused RMSNorm applied to the row first — for the dot-product mode, whose Q8_0
        // activation blocks must be made from the normalised row itself (byte for byte as
        // the reference quantizes it): one barrier for Σx², then x / rms · w. No caller
        // combines that mode with a fused norm today (the runner decodes on the exact
        // path). The plain instances carry the block as well: without it the compiler
        // lays them out differently and the C2 GEMV measured 8.12 µs instead of 8.02.
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < XO; i++) {
            const int o = o0 + lane + 64 * i;
#pragma unroll
            for (int t = 0; t < 8; t++) ss += (o < o1 && 8 * o + t < G.kx) ? xv[i][t] * xv[i][t] : 0.0f;
        }
        ss = aeth_wave_sum(ss);
        if (lane == 0) ssum[wave] = ss;
        __syncthreads();
        float tot = 0.0f;
#pragma unroll
        for (int w = 0; w < W; w++) tot += ssum[w];
        const float rms = sqrtf(tot / (float)G.k + G.eps);
        // x / rms by one correctly rounded reciprocal and a residual step per
        // element (Markstein: q0 = x·r, q = q0 + (x − q0·rms)·r rounds x / rms
        // correctly away from overflow and underflow), then · w
        const float inv = 1.0f / rms;
#pragma unroll
        for (int i = 0; i < XO; i++)
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const float q0 = xv[i][t] * inv;
                xv[i][t] = fmaf(fmaf(-q0, rms, xv[i][t]), inv, q0) * wv[i][t];
            }
    }

    // a NaN or infinity in the slice makes every partial of this wave NaN
    if (lane == 0) *(uint4*)zs = make_uint4(0u, 0u, 0u, 0u);
    // With several octet sets per lane (long rows), only the first is converted before the
    // first tile's dots; set x is converted within them, just before chunk CPX·x, the first it
    // feeds, so that the conversion of a long slice does not hold back every dot
    constexpr int CPX = 512 / T::CE;  // chunks per octet set
    constexpr bool LAZY = XO > 1 && !Q8A;
    int bad = mq_build<F, XO, Q8A>(xv, c0, nbw, G.kx, Abase, Mbase, 0, LAZY ? 1 : XO);

    auto tile = [&](const Dt (&b)[NBW], bool first) {
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < NBW; i++) {
            if (LAZY && first && i > 0 && i % CPX == 0 && i / CPX < XO)
                bad |= mq_build<F, XO, Q8A>(xv, c0, nbw, G.kx, Abase, Mbase, i / CPX, i / CPX + 1);
            if (i < nbw)
                acc += T::template dot<Q8A, PD>(b[i], Abase + (size_t)(c0 + i) * T::AB, Mbase + (size_t)(c0 + i) * T::MB,
                                            lane, L, zs);
        }
        return aeth_sum_rows(acc) + (bad ? __int_as_float(0x7FC00000) : 0.0f);
    };
    if (!RING) {  // every tile already in flight: no refills
#pragma unroll
        for (int r = 0; r < RD; r++) {
            if (r < ntw) {
                const float acc = tile(buf[r], r == 0);
                if (lane < 16) part[(r * W + wave) * 16 + lane] = acc;
            }
            __builtin_amdgcn_sched_barrier(0);  // tiles in arrival order: wait for each one alone
        }
    } else {  // ring of RD tiles; each consumed slot is refilled at once (clamped past the end)
        for (int j0 = 0; j0 < ntw; j0 += RD) {
#pragma unroll
            for (int r = 0; r < RD; r++) {
                const int j = j0 + r;
                if (j < ntw) {
                    const float acc = tile(buf[r], j == 0);
                    if (lane < 16) part[(j * W + wave) * 16 + lane] = acc;
                }
                // refill with tile j + RD; past the run, the same loads of chunk 0 of tile 0,
                // which every wave's surplus refills share (so they hit in cache), instead of
                // re-streaming the last tile (branching around the loads would leave the
                // compiler's per-tile waits inexact)
#pragma unroll
                for (int i = 0; i < NBW; i++)
                    T::load(buf[r][i], G, j + RD < ntw ? (t0 + j + RD) * nc + c0 + min(i, max(nbw - 1, 0)) : 0, lane);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    __syncthreads();

    float rms = 1.0f;  // the exact path's fused RMSNorm: rms = sqrt(Σx²/k + eps), the waves' slices in order
    constexpr bool div_rms = NORM;
    if (div_rms) {
        float tot = 0.0f;
#pragma unroll
        for (int w = 0; w < W; w++) tot += ssum[w];
        rms = sqrtf(tot / (float)G.k + G.eps);
    }
    unsigned long long best = 0;
    for (int idx = threadIdx.x; idx < ntw * 16; idx += 64 * W) {
        const int jt = idx >> 4, nn = idx & 15;
        const int64_t row = (t0 + jt) * 16 + nn;
        if (row >= G.n) continue;
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < W; w++) sum += part[(jt * W + w) * 16 + nn];
        if (div_rms) sum = sum / rms;
        if (G.swiglu) {
            if ((nn & 1) == 0) {
                float up = 0.0f;
#pragma unroll
                for (int w = 0; w < W; w++) up += part[(jt * W + w) * 16 + nn + 1];
                if (div_rms) up = up / rms;
                yr[row >> 1] = sum * (1.0f / (1.0f + expf(-sum))) * up;
            }
        } else {
            const float v = G.accumulate ? (idx == (int)threadIdx.x ? yprev : yr[row]) + sum : sum;
            yr[row] = v;
            if (G.amax) {
                const unsigned long long kk = aeth_amax_key(v, row);
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

// ── dispatch ─────────────────────────────────────────────────────────────

template <int F, int NBW, int RD, int XO, bool RING, int W, bool RAG, bool Q8A, bool NORM, bool PD>
static int mq_launch_k2(dim3 grid, size_t lds, hipStream_t s, const MqParams& G) {
    static size_t opted = 64 * 1024;  // dynamic LDS above 64 KiB is opted into per kernel
    if (lds > opted) {
        AETH_HIP_CHECK(hipFuncSetAttribute((const void*)k_gemv_mf<F, NBW, RD, XO, RING, W, RAG, Q8A, NORM, PD>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        opted = lds;
    }
    hipLaunchKernelGGL((k_gemv_mf<F, NBW, RD, XO, RING, W, RAG, Q8A, NORM, PD>), grid, dim3(64 * W), lds, s, G);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}

// Q4_K / Q5_K on the exact path: the instance without decode_d's NaN / infinity rule when the
// weight has no such scale (measured 1.7-1.8 % faster on the Q4_K decode shapes; Q6_K and Q8_0
// gain nothing and keep one instance)
template <int F, int NBW, int RD, int XO, bool RING, int W, bool RAG, bool Q8A, bool NORM>
static int mq_launch_k(dim3 grid, size_t lds, hipStream_t s, const MqParams& G) {
    if constexpr ((F == FQ4K || F == FQ5K) && !Q8A) {
        if (G.plain_d) return mq_launch_k2<F, NBW, RD, XO, RING, W, RAG, Q8A, NORM, true>(grid, lds, s, G);
    }
    return mq_launch_k2<F, NBW, RD, XO, RING, W, RAG, Q8A, NORM, false>(grid, lds, s, G);
}

template <int F, int NBW, int RD, int W, bool RAG, bool Q8A>
static int mq_launch(dim3 grid, size_t lds, hipStream_t s, const MqParams& G) {
    constexpr int XO = (NBW * MF<F>::CE / 8 + 63) / 64;
    if (!RAG && !Q8A && G.norm_w)  // (a fused RMSNorm needs whole 256-element rows: never ragged)
        return G.tpw <= RD ? mq_launch_k<F, NBW, RD, XO, false, W, RAG, Q8A, !RAG && !Q8A>(grid, lds, s, G)
                           : mq_launch_k<F, NBW, RD, XO, true, W, RAG, Q8A, !RAG && !Q8A>(grid, lds, s, G);
    return G.tpw <= RD ? mq_launch_k<F, NBW, RD, XO, false, W, RAG, Q8A, false>(grid, lds, s, G)
                       : mq_launch_k<F, NBW, RD, XO, true, W, RAG, Q8A, false>(grid, lds, s, G);
}

template <int F, bool RAG, bool Q8A>
static int mq_dispatch(MqParams G, int64_t m, hipStream_t s) {
    typedef MF<F> T;
    const int nc = G.nc;
    // Shape choice (measured on the decode and benchmark shapes): W waves split
    // K, 16 only for long rows; RD tiles per workgroup with all loads issued up
    // front (short memory queues, so each wave's tiles arrive early and their
    // compute overlaps the stream); one tile per workgroup when there are no
    // more tiles than CUs; taller matrices use the ring with ~2 workgroups per
    // CU (Q6_K: ~4) so the per-workgroup activation conversion stays amortised.
    // Tuning overrides, read once: AETH_GEMV_WAVES (8 | 16), AETH_GEMV_TPW.
    static const int env_w = getenv("AETH_GEMV_WAVES") ? atoi(getenv("AETH_GEMV_WAVES")) : 0;
    static const int env_tpw = getenv("AETH_GEMV_TPW") ? atoi(getenv("AETH_GEMV_TPW")) : 0;
    const int64_t cus = aeth_num_cus();
    int W = (int64_t)nc * T::CE >= 8192 ? 16 : 8;
    if (env_w) W = env_w == 16 ? 16 : 8;
    const int nbw = (nc + W - 1) / W;
    const int NBW = nbw <= 1 ? 1 : nbw <= 2 ? 2 : nbw <= 4 ? 4 : 8;
    if (nbw > 8) return aeth_set_error(AETH_EUNSUPPORTED, "gemv: k=%d is beyond this kernel's range", G.k);
    int RD = NBW <= 2 || (W == 8 && NBW == 4 && F != FQ6K) ? 2 : 1;
    // (Q6_K on the ring: ~4 workgroups per CU, measured 1.5 % faster on the 128256-row LM head)
    // (4 to 8 tiles per CU, other formats: one workgroup per CU on the ring — the 28672-row gate|up GEMV
    // of the 8B decode step, 3.6 % faster decode than 2 tiles per workgroup)
    const int64_t wpc = F == FQ6K ? 4 : 2;
    int64_t tpw;
    if (G.ntiles <= cus) tpw = 1;
    else if (G.ntiles <= 4 * cus || (F == FQ6K && G.ntiles <= 8 * cus)) tpw = RD;
    else if (G.ntiles <= 8 * cus) tpw = aeth_cdiv(G.ntiles, cus);
    else tpw = aeth_cdiv(G.ntiles, wpc * cus);
    if (env_tpw > 0) tpw = env_tpw;
    if (tpw > MQ_TPW_MAX) tpw = MQ_TPW_MAX;
    G.tpw = (int)tpw;
    // one tile per workgroup: a single load slot (with two, the second repeats the first tile's loads;
    // the o GEMV of the 8B decode step measured 4.17 -> 3.92 us)
    if (tpw == 1 && W == 8 && (NBW == 2 || NBW == 4)) RD = 1;
    const size_t lds = (size_t)nc * (T::AB + T::MB) + (size_t)tpw * W * 16 * 4 + (size_t)W * 16;
    if (lds > MQ_LDS_MAX)
        return aeth_set_error(AETH_EUNSUPPORTED, "gemv: k=%d needs %zu B of LDS (max %d)", G.k, lds, MQ_LDS_MAX);
    const dim3 grid((unsigned)aeth_cdiv(G.ntiles, tpw), (unsigned)m);
    if (W == 16) {
        if (NBW == 1) return mq_launch<F, 1, 2, 16, RAG, Q8A>(grid, lds, s, G);
        if (NBW == 2) return mq_launch<F, 2, 2, 16, RAG, Q8A>(grid, lds, s, G);
        if (NBW == 4) return mq_launch<F, 4, 1, 16, RAG, Q8A>(grid, lds, s, G);
        return mq_launch<F, 8, 1, 16, RAG, Q8A>(grid, lds, s, G);
    }
    if (NBW == 1) return mq_launch<F, 1, 2, 8, RAG, Q8A>(grid, lds, s, G);
    if (NBW == 2) {
        if (RD == 1) return mq_launch<F, 2, 1, 8, RAG, Q8A>(grid, lds, s, G);
        return mq_launch<F, 2, 2, 8, RAG, Q8A>(grid, lds, s, G);
    }
    if (NBW == 4) {
        if (RD == 2) return mq_launch<F, 4, 2, 8, RAG, Q8A>(grid, lds, s, G);
        return mq_launch<F, 4, 1, 8, RAG, Q8A>(grid, lds, s, G);
    }
    return mq_launch<F, 8, 1, 8, RAG, Q8A>(grid, lds, s, G);
}

int aeth_gemv_launch_ex(const aeth_weight* w, const float* d_x, int64_t m, float* d_y, const GemvEpi& e,
                        hipStream_t s) {
    if (w->order != AETH_ORDER_PLANAR) return aeth_xgemv_launch(w, d_x, m, d_y, e, s);
    if (m > 65535) return aeth_set_error(AETH_EINVAL, "gemv: m=%lld exceeds 65535", (long long)m);
    MqParams G;
    G.p0 = w->p0;
    G.p1 = w->p1;
    G.p2 = w->p2;
    G.n = w->n;
    G.ntiles = (int)aeth_cdiv(w->n, 16);
    G.tpw = 1;
    G.x = d_x;
    G.x_stride = w->k;
    G.k = (int)w->k;
    G.y = d_y;
    G.y_stride = e.ldc ? e.ldc : e.swiglu ? w->n / 2 : w->n;
    G.accumulate = (e.flags & AETH_MM_ACCUMULATE) ? 1 : 0;
    G.norm_w = e.norm_w;
    G.eps = e.eps;
    G.swiglu = e.swiglu;
    G.amax = e.amax;
    G.plain_d = !w->special_scales;
    const bool q8 = w->dtype == AETH_DTYPE_Q8_0;
    G.nc = q8 ? (int)aeth_cdiv(w->nb, 4) : (int)w->nb;
    G.kx = q8 ? (int)w->k : (int)w->nb * 256;  // K-quants read k/256 whole blocks (avx2.rs:26)
    if (G.nc < 1) return aeth_set_error(AETH_EINVAL, "gemv: empty rows (k=%d)", G.k);
    if (e.swiglu && (w->n & 1)) return aeth_set_error(AETH_EUNSUPPORTED, "gemv: fused SwiGLU needs paired rows");
    if (e.norm_w && G.kx != G.k)
        return aeth_set_error(AETH_EUNSUPPORTED, "gemv: fused RMSNorm needs k a multiple of 256");
    const bool rag = (G.kx & 7) != 0;
    if (!rag && (((uintptr_t)d_x & 15) || (e.norm_w && ((uintptr_t)e.norm_w & 15)) || (m > 1 && (G.k & 3))))
        return aeth_set_error(AETH_EINVAL, "gemv: x rows and the norm weight must be 16-byte aligned");
    if (e.flags & AETH_MM_Q8_ACTIVATIONS) {  // the int8 dot-product path (a14 activations)
        if (w->dtype == AETH_DTYPE_Q4_K) return mq_dispatch<FQ4K, false, true>(G, m, s);
        if (w->dtype == AETH_DTYPE_Q5_K) return mq_dispatch<FQ5K, false, true>(G, m, s);
        if (w->dtype == AETH_DTYPE_Q6_K) return mq_dispatch<FQ6K, false, true>(G, m, s);
        if (q8) return rag ? mq_dispatch<FQ80, true, true>(G, m, s) : mq_dispatch<FQ80, false, true>(G, m, s);
    }
    if (w->dtype == AETH_DTYPE_Q4_K) return mq_dispatch<FQ4K, false, false>(G, m, s);
    if (w->dtype == AETH_DTYPE_Q5_K) return mq_dispatch<FQ5K, false, false>(G, m, s);
    if (w->dtype == AETH_DTYPE_Q6_K) return mq_dispatch<FQ6K, false, false>(G, m, s);
    if (q8) return rag ? mq_dispatch<FQ80, true, false>(G, m, s) : mq_dispatch<FQ80, false, false>(G, m, s);
    return aeth_set_error(AETH_EUNSUPPORTED, "gemv: dtype %d", w->dtype);
}

int aeth_gemv_launch(const aeth_weight* w, const float* d_x, int64_t m, float* d_y, unsigned flags, hipStream_t s) {
    GemvEpi e;
    e.flags = flags;
    return aeth_gemv_launch_ex(w, d_x, m, d_y, e, s);
}
