// Prefill GEMM for Q4_K weights (m > 1):  C[m][n] = Σ_k A[m][k]·W[n][k]
// (avx2::matmul_q4_k with m rows, src/quant/avx2.rs:23-57; quantized_matmul_impl).
//
// "Exact" mode on fp16 MFMA (v_mfma_f32_32x32x16_f16, fp32 accumulate):
//  * A is split into two fp16 parts, A·2^-e = Ah + Al (Ah = fp16(A·2^-e),
//    Al = fp16(A·2^-e − Ah)): 22 significant bits, f32-level. The power of two
//    2^e is chosen per row so that the parts stay in fp16 range (e = 0 unless
//    the row holds a value of magnitude ≥ 2^14); a shared exponent for several
//    rows would push the lo parts of a small row next to a large one into fp16
//    subnormals.
//  * Q4_K weights become exact fp16 integers w = q·sc (q ≤ 15, sc ≤ 63), so
//    every MFMA product is exact and the K-sum is an f32 accumulation.
//  * Per 256-element super-block b:  C += 2^e·(d_b·Σ A·(q·sc) − dmin_b·Σ_s m_s·S_s)
//    with S_s = Σ_{i∈s} A_i·2^-e the 32-element sub-block sums, themselves split
//    hi/lo and contracted by one extra MFMA (k = 8 sub-blocks × {hi, lo}).
//    Scales are therefore applied once per super-block, not per element.
// Each product A_hi·w and A_lo·w costs one MFMA pass, so the useful rate is
// half the fp16 MFMA rate.
//
// Weight dequantisation in packed fp16: the half with bits 0x6400 | q is
// 1024 + q (q < 1024), and one v_pk_fma_f16 with (sc, −1024·sc) gives q·sc
// exactly (the fused product is exact, the result an integer below 2048).
// Masking a dword with 0x000F000F yields the pair (elements 0, 2) of its four
// bytes and (w >> 8) the pair (1, 3), so each group of 4 k-positions is taken
// in the order [0, 2, 1, 3]; the activation prep writes A in the same order,
// and every dot product is unchanged.
//
// Data movement (gfx950): workgroup tile 64 × 128 of C. K advances 64 positions
// (a quarter super-block) per stage through a 3-stage LDS ring filled with
// direct-to-LDS loads (global_load_lds_dwordx4 / buffer_load_dwordx4 … lds:
// lane i of a wave writes LDS bytes [16i, 16i+16) of the destination, from any
// address): A as MFMA fragments written by the prep kernel in operand order (so
// every operand read is one contiguous ds_read_b128), the raw Q4_K quants of the
// 16-row tile layout, and the tiles' headers. The waves dequantise their own B
// operands from the raw bytes in LDS straight into registers. One barrier per
// stage; the loads of stage s+2 are issued right after it, while stage s computes.
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

#include <algorithm>

#include "aeth_common.hpp"
#include "aeth_internal.hpp"

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

#define G2_BM 64
#define G2_BN 128
#define G2_A 16384  // one stage's A: 2 m-tiles × 4 k-slices × {hi, lo} fragments of 1 KiB
#define G2_B 4096   // one stage's quants: 8 tiles × 512 B
#define G2_H 4096   // 2 KiB of headers per stage, each half loaded by two waves
#define G2_STAGE (G2_A + G2_B + G2_H)
#define G2_NST 3
#define G2_LOADS 6

// positions 1 and 2 of each group of 4 exchanged (an involution)
__device__ __forceinline__ int perm4(int i) { return (i & ~3) | ((0x3120 >> (4 * (i & 3))) & 3); }

// ── activation prep, two passes over A (f32 [m][k]; rows m..mp-1 read as zero).
// Row scales: escale[r] = 2^e, e ≥ 0 the least with |A[r]·2^-e| < 2^14. One
// wave per row, 16 loads per lane in flight.
template <bool AL16>
__global__ void __launch_bounds__(256) k_gemm_rowscale(const float* __restrict__ A, int m, int mp, int k,
                                                       float* __restrict__ escale) {
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (r >= mp) return;
    if (r >= m) {
        if (lane == 0) escale[r] = 1.0f;
        return;
    }
    const float* a = A + (int64_t)r * k;
    float mx = 0.0f;
    if (AL16) {
        for (int base = 0; base < k / 4; base += 1024) {
            float4 t[16];
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const int i = min(base + lane + 64 * j, k / 4 - 1);  // repeats are harmless for a max
                t[j] = *(const float4*)(a + 4 * i);
            }
#pragma unroll
            for (int j = 0; j < 16; j++)
                mx = fmaxf(mx, fmaxf(fmaxf(fabsf(t[j].x), fabsf(t[j].y)), fmaxf(fabsf(t[j].z), fabsf(t[j].w))));
        }
    } else {
        for (int i = lane; i < k; i += 64) mx = fmaxf(mx, fabsf(a[i]));
    }
    mx = aeth_wave_max(mx);
    if (lane == 0) {
        int E = 0;
        if (mx > 0.0f && isfinite(mx)) (void)frexpf(mx, &E);
        escale[r] = ldexpf(1.0f, E > 14 ? E - 14 : 0);
    }
}

// Fragments. Workgroup (m-tile mt, super-block sb) = 32 rows × 256 columns,
// staged through LDS with whole-row loads. Writes
//  * fragment (mt, ks, part) = 1 KiB at ((mt·nks + ks)·2 + part)·1024 bytes
//    (nks = k/16): lane l holds row 32·mt + l%32 at k-positions
//    16·ks + 8·(l/32) + perm4(i), i < 8, of A·2^-e, part 0 = hi, 1 = lo;
//  * Sh/Sl [row][k/32] = Σ of each 32-element sub-block of A·2^-(e+5), hi/lo.
// Thread (row lr = tid/8, sub-block q = tid%8) converts 32 elements.
//
// Q8 = true (AETH_MM_Q8_ACTIVATIONS, the dot-product mode): each 32-element
// sub-block is first replaced by its Q8_0 activation block, dequantized —
// quantize_q8_0_block (neon.rs:45-104): d = max|x|/127 (NaN-propagating max),
// q = sat_i8(RNE(x·(1/d))) with the f32 d, and the value q·f16(d) the integer
// dot of the reference scales with (d_a = the stored f16 d). q·f16(d) has at
// most 18 significant bits, so it is exact in f32 and in the hi/lo split: the
// GEMM then computes Σ (q_a·d_a)·(q·sc·d) exactly per product, i.e. the
// reference's per-term d_a·(d1·Σ q·q_a − m1·Σ q_a) up to f32 summation order.
#define GF_LD 260  // LDS row stride in floats
template <bool AL16, bool Q8>
__global__ void __launch_bounds__(256) k_gemm_frag(const float* __restrict__ A, int m, int k,
                                                   const float* __restrict__ escale, _Float16* __restrict__ frag,
                                                   _Float16* __restrict__ Sh, _Float16* __restrict__ Sl) {
    __shared__ __attribute__((aligned(16))) float blk[32 * GF_LD];
    const int mt = blockIdx.x, sb = blockIdx.y, tid = threadIdx.x;
    const int lane = tid & 63, wv = tid >> 6;
#pragma unroll
    for (int i = 0; i < 8; i++) {  // wave wv loads rows 8wv..8wv+7, one row per instruction
        const int row = 8 * wv + i, r = 32 * mt + row;
        const float* src = A + (int64_t)min(r, m - 1) * k + 256 * sb;
        float4 t;
        if (AL16) {
            t = *(const float4*)(src + 4 * lane);
        } else {
            t.x = src[4 * lane];
            t.y = src[4 * lane + 1];
            t.z = src[4 * lane + 2];
            t.w = src[4 * lane + 3];
        }
        if (r >= m) t = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        *(float4*)(blk + row * GF_LD + 4 * lane) = t;
    }
    __syncthreads();
    const int lr = tid >> 3, q = tid & 7, r = 32 * mt + lr;
    const float inv = 1.0f / escale[r];  // a power of two: the products below are exact scalings
    float v[32];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float4 t = *(const float4*)(blk + lr * GF_LD + 32 * q + 4 * i);
        v[4 * i] = t.x;
        v[4 * i + 1] = t.y;
        v[4 * i + 2] = t.z;
        v[4 * i + 3] = t.w;
    }
    if (Q8) {
        bool nan = false;
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            nan |= v[i] != v[i];
            mx = fmaxf(mx, fabsf(v[i]));
        }
        const float d = nan ? __uint_as_float(0x7FC00000u) : mx / 127.0f;
        const float da = aeth_f16_to_f32(aeth_f32_to_f16_bits(d));  // d_a as the block stores it
        const float id = d > 0.0f ? 1.0f / d : 0.0f;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const float p = v[i] * id;  // RNE with saturation, NaN → 0 (vcvtnq_s32_f32, sqxtn)
            const float q = p != p ? 0.0f : fminf(fmaxf(rintf(p), -128.0f), 127.0f);
            v[i] = d > 0.0f ? q * da : (d == 0.0f ? 0.0f : da);  // a NaN block dequantizes to NaN
        }
    }
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) sum += v[i];
    const int nks = k / 16;
#pragma unroll
    for (int x = 0; x < 2; x++) {       // k-slice 16·sb + 2q + x
#pragma unroll
        for (int h = 0; h < 2; h++) {   // lane lr + 32h: elements 16x + 8h + perm4(i)
            half8_t hi, lo;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float t = v[16 * x + 8 * h + perm4(i)] * inv;
                const _Float16 th = (_Float16)t;
                hi[i] = th;
                lo[i] = (_Float16)(t - (float)th);
            }
            _Float16* dst = frag + ((int64_t)(mt * nks + 16 * sb + 2 * q + x) * 2) * 512 + (lr + 32 * h) * 8;
            *(half8_t*)dst = hi;
            *(half8_t*)(dst + 512) = lo;
        }
    }
    const float sv = sum * inv * 0.03125f;
    const _Float16 sh = (_Float16)sv;
    Sh[(int64_t)r * (k / 32) + 8 * sb + q] = sh;
    Sl[(int64_t)r * (k / 32) + 8 * sb + q] = (_Float16)(sv - (float)sh);
}

struct GemmArgs {
    const uint8_t* frag;
    const _Float16 *Sh, *Sl;
    const float* escale;  // [row]: 2^e
    const uint8_t* hdr;   // Q4_K tile layout (aeth_q4k_hdr_off)
    const uint8_t* qs;    // Q4_K tile layout (aeth_q4k_qs_off)
    int m, n, k, nb, ntiles;
    int gm, gn;                     // 64-row and 128-column tiles of C
    int a_bytes, q_bytes, h_bytes;  // buffer extents for the buffer-resource loads
    float* C;
    int64_t ldc;  // row stride of C
    int accumulate;
};

// ── Single-K-group variant (used when the super-block count is odd or a buffer
// exceeds 2 GiB): 4 waves of 32 × 64 (2 m-tiles × 2 column halves); one stage =
// 16 A fragments, 8 tiles × 512 B of quants, the super-block's headers. Each wave
// issues the same 6 loads per stage, so a fixed vmcnt marks a stage's arrival.
__device__ __forceinline__ void g_dma(const void* g, char* l) {
    __builtin_amdgcn_global_load_lds(g, (lds_void*)l, 16, 0, 0);
}

// bytes (b0, b1, b2, b3) of w as fp16 pairs (b0, b1) and (b2, b3): (0x64 | b) is 1024 + b
__device__ __forceinline__ void bytes_to_h2(uint32_t w, half2_t& p01, half2_t& p23) {
    const half2_t k1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f};
    p01 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, w, 0x07010700u)) + k1024;
    p23 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, w, 0x07030702u)) + k1024;
}

__device__ __forceinline__ uint32_t pkfma(uint32_t q, half2_t s, half2_t z) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(half2_t, q), s, z));
}

// Eight quants of (x, y) → the B operand (k-order [0, 2, 1, 3] per 4). The
// nibble pairs come from one v_and_or_b32 each: MASK 0x000F000F keeps the low
// nibbles of bytes (0, 2) as halves 1024 + q (scales s = sc, z = −1024·sc),
// MASK 0x00F000F0 the high nibbles as 1024 + 16q (s = sc/16, z = −64·sc); bytes
// (1, 3) after a shift by 8. c64 holds 0x64006400 in a VGPR, so that the OR's
// constant does not need a second scalar operand (VOP3 takes one).
template <uint32_t MASK>
__device__ __forceinline__ half8_t dq8(uint32_t x, uint32_t y, uint32_t c64, half2_t s, half2_t z) {
    const uint32_t x8 = x >> 8, y8 = y >> 8;
    const uint32_t q0 = pkfma((x & MASK) | c64, s, z);
    const uint32_t q1 = pkfma((x8 & MASK) | c64, s, z);
    const uint32_t q2 = pkfma((y & MASK) | c64, s, z);
    const uint32_t q3 = pkfma((y8 & MASK) | c64, s, z);
    return __builtin_bit_cast(half8_t, make_uint4(q0, q1, q2, q3));
}

// LDS reads issued as inline asm: the compiler would otherwise order every LDS
// read after all outstanding direct-to-LDS loads (vmcnt(0)), since it cannot tell
// the ring's slots apart. The kernel waits with lgkmcnt itself, then passes each
// value through pin() so no use is scheduled above its wait.
typedef __attribute__((address_space(3))) char lds_char;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(const lds_char*)p; }
template <int OFF>
__device__ __forceinline__ u32x4 lds_b128(uint32_t a) {
    u32x4 v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(a), "i"(OFF));
    return v;
}
template <int OFF>
__device__ __forceinline__ half8_t lds_b128h(uint32_t a) {
    half8_t v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(a), "i"(OFF));
    return v;
}
// two 8-byte reads, at a and a + 256
__device__ __forceinline__ u32x4 lds_2b64_256(uint32_t a) {
    u32x4 v;
    asm volatile("ds_read2_b64 %0, %1 offset1:32" : "=v"(v) : "v"(a));
    return v;
}
template <int N>
__device__ __forceinline__ void lgkm_wait() {
    static_assert(N >= 0 && N < 16, "lgkmcnt range");
    __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (N << 8) | (3 << 14));  // vmcnt, expcnt at their maximum
}
template <class T>
__device__ __forceinline__ void pin(T& v) {
    asm volatile("" : "+v"(v));
}

// Workgroup → tile: the 8 XCDs take workgroup ids round-robin; each XCD gets a
// contiguous run of tiles, ordered in groups of 4 row-tiles so that the
// workgroups resident on one XCD share A rows and weight tiles in its L2.
__device__ __forceinline__ void g2_tile(int id, int gm, int gn, int& tm, int& tn) {
    const int T = gm * gn;
    if ((T & 7) == 0) id = (id & 7) * (T >> 3) + (id >> 3);
    const int GM = 4, per = GM * gn, grp = id / per, first = grp * GM, rows = min(GM, gm - first);
    const int in = id - grp * per;
    tm = first + in % rows;
    tn = in / rows;
}

__global__ void __launch_bounds__(256) k_gemm_q4k_ring(GemmArgs G) {
    __shared__ __attribute__((aligned(1024))) char ring[G2_NST * G2_STAGE];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    int tm, tn;
    g2_tile(blockIdx.x, G.gm, G.gn, tm, tn);
    const int n0 = tn * G2_BN, m0 = tm * G2_BM;
    const int nb = G.nb, nst = 4 * nb, nks = G.k / 16;

    // direct-load sources: a uniform base per stage (s·8 KiB of A fragments, s·512 B
    // of quants, (s/4)·256 B of headers) plus a fixed 32-bit offset per lane. Tiles
    // past the last are clamped (never written back).
    uint32_t a_lo[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int f = wave + 4 * j;  // local fragment: m-tile f/8, k-slice (f/2)%4, part f%2
        a_lo[j] = (uint32_t)((((2 * tm + (f >> 3)) * nks + ((f >> 1) & 3)) * 2 + (f & 1)) * 1024 + lane * 16);
    }
    const int bt = min(n0 / 16 + 2 * wave + (lane >> 5), G.ntiles - 1);
    const uint32_t b_lo = (uint32_t)(bt * nb * 2048 + (lane & 31) * 16);
    const int ht = min(n0 / 16 + 4 * (wave & 1) + (lane >> 4), G.ntiles - 1);
    const uint32_t h_lo = (uint32_t)((ht * nb * 16 + (lane & 15)) * 16);
    auto issue = [&](int s, char* st) {
        s = min(s, nst - 1);  // the ring's tail reloads the last stage into a free buffer
        const uint8_t* ab = G.frag + (size_t)s * 8192;
#pragma unroll
        for (int j = 0; j < 4; j++) g_dma(ab + a_lo[j], st + (wave + 4 * j) * 1024);
        g_dma(G.qs + (size_t)s * 512 + b_lo, st + G2_A + wave * 1024);
        g_dma(G.hdr + (size_t)(s >> 2) * 256 + h_lo, st + G2_A + G2_B + wave * 1024);
    };

    // LDS offsets: A fragment (wm, ks, part) at a_off + (2ks + part)·1024; quants of
    // column c's tile, lane (n, kg) at b_off[c] + 256·kg; its header at h_off[c]
    const int a_off = wm * 8192 + lane * 16;
    int b_off[2], h_off[2];
#pragma unroll
    for (int c = 0; c < 2; c++) {
        const int nc = 64 * wn + 32 * c + (lane & 31), t = nc >> 4, n = nc & 15;
        b_off[c] = G2_A + t * 512 + n * 16 + 8 * (lane >> 5);
        h_off[c] = G2_A + G2_B + (t >> 2) * 1024 + ((t & 3) * 16 + n) * 16;
    }
    const int srow = min(m0 + 32 * wm + (lane & 31), G.m - 1);
    const _Float16* s_src = ((lane >> 5) ? G.Sl : G.Sh) + (int64_t)srow * (G.k / 32);

    f32x16 acc[2], part[2];
#pragma unroll
    for (int c = 0; c < 2; c++) {
        acc[c] = (f32x16){};
        part[c] = (f32x16){};
    }
    u32x4 hd[2] = {};
    half8_t sv = {};

    uint32_t c64;  // 0x64006400 in a VGPR (see dq8)
    asm("v_mov_b32 %0, 0x64006400" : "=v"(c64));
    issue(0, ring);
    issue(1, ring + G2_STAGE);
    const uint32_t ring_lds = lds_addr(ring);
    int cur = 0;  // ring slot of stage s
    for (int b = 0; b < nb; b++) {
#pragma unroll
        for (int J = 0; J < 4; J++) {
            const int s = 4 * b + J;
            const uint32_t st = ring_lds + cur * G2_STAGE;
            const int nx = cur == 0 ? 2 : cur - 1;  // slot of stage s + 2 (= slot of s - 1)
            // this wave's loads of stage s have landed (those of s + 1 may be in flight)
            __builtin_amdgcn_s_waitcnt((G2_LOADS & 15) | (7 << 4) | (15 << 8) | ((G2_LOADS >> 4) << 14));
            __builtin_amdgcn_s_barrier();  // every wave's part of stage s is in; slot nx is free
            issue(s + 2, ring + nx * G2_STAGE);
            cur = cur == 2 ? 0 : cur + 1;
            if (J == 0) sv = *(const half8_t*)(s_src + b * 8);
            // LDS reads in one batch, consumed in order under lgkmcnt
            if (J == 0) {
                hd[0] = lds_b128<0>(st + h_off[0]);
                hd[1] = lds_b128<0>(st + h_off[1]);
            }
            u32x4 raw[2];  // .xy: k-group 0, .zw: k-group 1 (256 B further)
            raw[0] = lds_2b64_256(st + b_off[0]);
            raw[1] = lds_2b64_256(st + b_off[1]);
            const uint32_t pa = st + a_off;
            half8_t a[4][2];
            a[0][0] = lds_b128h<0>(pa);
            a[0][1] = lds_b128h<1024>(pa);
            a[1][0] = lds_b128h<2048>(pa);
            a[1][1] = lds_b128h<3072>(pa);
            a[2][0] = lds_b128h<4096>(pa);
            a[2][1] = lds_b128h<5120>(pa);
            a[3][0] = lds_b128h<6144>(pa);
            a[3][1] = lds_b128h<7168>(pa);
            lgkm_wait<6>();
            pin(hd[0]);
            pin(hd[1]);
            pin(raw[0]);
            pin(raw[1]);
            pin(a[0][0]);
            pin(a[0][1]);
            // scales of sub-blocks 2J (low nibbles) and 2J + 1 (high nibbles), get_scale_min_k4:
            // sp = (sc, sc'/16), zp = (−1024·sc, −64·sc'), used as broadcast halves
            half2_t sp[2], zp[2];
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const uint32_t y = hd[c][1], w = hd[c][3];
                const uint32_t sc4 = J < 2 ? (y & 0x3F3F3F3Fu) : ((w & 0x0F0F0F0Fu) | ((y >> 2) & 0x30303030u));
                half2_t p01, p23;
                bytes_to_h2(sc4, p01, p23);
                const half2_t pr = (J & 1) ? p23 : p01;
                const half2_t k_s = {(_Float16)1.0f, (_Float16)0.0625f}, k_z = {(_Float16)-1024.0f, (_Float16)-64.0f};
                sp[c] = pr * k_s;
                zp[c] = pr * k_z;
            }
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                const int nib = ks >> 1, kg = ks & 1;
                if (ks == 1) lgkm_wait<4>();
                if (ks == 2) lgkm_wait<2>();
                if (ks == 3) lgkm_wait<0>();
                if (ks > 0) {
                    pin(a[ks][0]);
                    pin(a[ks][1]);
                }
                half8_t bv[2];
#pragma unroll
                for (int c = 0; c < 2; c++) {
                    const uint32_t x = raw[c][2 * kg], y = raw[c][2 * kg + 1];
                    if (nib == 0)
                        bv[c] = dq8<0x000F000Fu>(x, y, c64, __builtin_shufflevector(sp[c], sp[c], 0, 0),
                                                 __builtin_shufflevector(zp[c], zp[c], 0, 0));
                    else
                        bv[c] = dq8<0x00F000F0u>(x, y, c64, __builtin_shufflevector(sp[c], sp[c], 1, 1),
                                                 __builtin_shufflevector(zp[c], zp[c], 1, 1));
                }
#pragma unroll
                for (int p = 0; p < 2; p++)
#pragma unroll
                    for (int c = 0; c < 2; c++)
                        part[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[ks][p], bv[c], part[c], 0, 0, 0);
            }
            if (J == 3) {
                // super-block done: C·2^-e += d·P − 32·dmin·Σ_s m_s·S_s (S carries 2^-(e+5))
#pragma unroll
                for (int c = 0; c < 2; c++) {
                    const float d = aeth_decode_d(hd[c][0]), ndm = -32.0f * aeth_decode_d(hd[c][0] >> 16);
                    const uint32_t z = hd[c][2], w = hd[c][3];
                    half2_t m01, m23, m45, m67;
                    bytes_to_h2(z & 0x3F3F3F3Fu, m01, m23);
                    bytes_to_h2(((w >> 4) & 0x0F0F0F0Fu) | ((z >> 2) & 0x30303030u), m45, m67);
                    const half8_t mv = {m01[0], m01[1], m23[0], m23[1], m45[0], m45[1], m67[0], m67[1]};
                    const f32x16 q = __builtin_amdgcn_mfma_f32_32x32x16_f16(sv, mv, (f32x16){}, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; r++) acc[c][r] = fmaf(ndm, q[r], fmaf(d, part[c][r], acc[c][r]));
                    part[c] = (f32x16){};
                }
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0);  // the tail's loads land before the workgroup's LDS is released

    const int lr = lane & 31;
#pragma unroll
    for (int c = 0; c < 2; c++) {
        const int col = n0 + 64 * wn + 32 * c + lr;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int row = m0 + 32 * wm + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
            if (row < G.m && col < G.n) {
                const float v = acc[c][r] * G.escale[row];
                float* dst = G.C + (int64_t)row * G.ldc + col;
                *dst = G.accumulate ? *dst + v : v;
            }
        }
    }
}

// ── Split-K variant: the same 64 × 128 workgroup tile, computed by 4 waves as
// 2 column halves × 2 K halves, each wave a 64 × 64 tile over half of K. Every
// dequantised weight fragment then feeds 4 MFMAs (2 m-tiles × {hi, lo}) instead
// of 2, halving the VALU work per MFMA; the two K halves meet in LDS at the end.
// A stage holds 64 K-positions of both halves (2 × 22 KiB), the ring 3 stages
// (132 KiB: one workgroup per CU). Per stage and wave: 11 loads through buffer
// resources (the stage offset is a scalar), 32 MFMAs. The default launches the
// 8-wave form (k_gemm_q4k_sk8: the two m-tiles on separate waves, two waves per
// SIMD, 6 loads and 16 MFMAs per stage and wave), measured 2-5 % faster; splitting
// the columns instead (dequantisation not repeated, A read twice from LDS) gained
// nothing.
#define G3_HALF (G2_A + G2_B + 2048)  // one K half: A fragments, quants, headers
#define G3_STAGE (2 * G3_HALF)
#define G3_LOADS 11

template <int MS>
__device__ __forceinline__ void gemm_sk_body(const GemmArgs& G) {
    // MS = 1: 4 waves, each both m-tiles of its (column half, K half).
    // MS = 2: 8 waves, waves w and w + 4 take m-tile 0 and 1 of the same (column
    // half, K half), two waves per SIMD, so one wave's dequantisation and LDS
    // waits overlap the other's MFMAs; the LDS ring is the same.
    constexpr int NM = 2 / MS;                // m-tiles per wave
    constexpr int LOADS = MS == 1 ? G3_LOADS : 6;
    __shared__ __attribute__((aligned(1024))) char ring[G2_NST * G3_STAGE];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wq = wave & 3, wn = wave & 1, kh = (wave >> 1) & 1;  // loader slot, column half, K half
    const int mb = MS == 2 ? wave >> 2 : 0;                      // first m-tile of this wave
    int tm, tn;
    g2_tile(blockIdx.x, G.gm, G.gn, tm, tn);
    const int n0 = tn * G2_BN, m0 = tm * G2_BM;
    const int nb = G.nb, hsb = nb / 2, nst = 4 * hsb, nks = G.k / 16;

    // Direct loads: 44 pieces of 1 KiB per stage. MS = 1: piece w + 4i to wave w
    // (i < 11): i < 8: A fragment (K half i/4, local fragment w + 4(i%4)); i = 8, 9:
    // quants of tiles 2w, 2w+1 for K half i-8; i = 10: headers of tiles
    // 4(w%2)..+3 for K half w/2. MS = 2: wave w takes the A fragments of m-tile
    // mb (local fragments w%4 + 8mb, w%4 + 8mb + 4, both K halves), the quants of
    // K half mb and the same header piece as wave w%4 (a duplicate of identical
    // bytes, so every wave issues 6 loads). Lane offsets are fixed; stage s of K
    // half h adds (h·nst + s)·8 KiB (A), ·512 B (quants), ((h·nst + s)/4)·256 B
    // (headers).
    constexpr int NJ = 4 / MS;
    uint32_t a_lo[NJ];
    int a_f[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int f = wq + 4 * (MS == 2 ? 2 * mb + j : j);  // m-tile f/8, k-slice (f/2)%4, part f%2
        a_f[j] = f;
        a_lo[j] = (uint32_t)((((2 * tm + (f >> 3)) * nks + ((f >> 1) & 3)) * 2 + (f & 1)) * 1024 + lane * 16);
    }
    const int bt = min(n0 / 16 + 2 * wq + (lane >> 5), G.ntiles - 1);
    const uint32_t b_lo = (uint32_t)(bt * nb * 2048 + (lane & 31) * 16);
    const int ht = min(n0 / 16 + 4 * (wq & 1) + (lane >> 4), G.ntiles - 1);
    const uint32_t h_lo = (uint32_t)((ht * nb * 16 + (lane & 15)) * 16);
    // buffer resources (loads past an extent read zeros); the per-stage offset goes in
    // the scalar offset, so a load needs no vector address arithmetic
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void*)G.frag, (short)0, G.a_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc((void*)G.qs, (short)0, G.q_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc((void*)G.hdr, (short)0, G.h_bytes, 0x00020000);
    auto issue = [&](int s, char* st) {
        s = min(s, nst - 1);  // the ring's tail reloads the last stage into a free slot
#pragma unroll
        for (int h = 0; h < 2; h++) {
#pragma unroll
            for (int j = 0; j < NJ; j++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void*)(st + h * G3_HALF + a_f[j] * 1024), 16,
                                                         a_lo[j], (h * nst + s) * 8192, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 2 / MS; i++) {
            const int h = MS == 1 ? i : mb;  // (no branch around a load: the wait counts stay exact)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, (lds_void*)(st + h * G3_HALF + G2_A + wq * 1024), 16, b_lo,
                                                     (h * nst + s) * 512, 0, 0);
        }
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rh, (lds_void*)(st + kh * G3_HALF + G2_A + G2_B + (wq & 1) * 1024),
                                                 16, h_lo, ((kh * nst + s) >> 2) * 256, 0, 0);
    };

    // LDS offsets within the wave's K half: A fragment (mt, ks, part) at
    // a_off + (8mt + 2ks + part)·1024; column c's quants (lane (n, kg)) at
    // b_off[c] + 256·kg; its header at h_off[c]
    const int a_off = kh * G3_HALF + lane * 16 + mb * 8192;
    int b_off[2], h_off[2];
#pragma unroll
    for (int c = 0; c < 2; c++) {
        const int nc = 64 * wn + 32 * c + (lane & 31), t = nc >> 4, n = nc & 15;
        b_off[c] = kh * G3_HALF + G2_A + t * 512 + n * 16 + 8 * (lane >> 5);
        h_off[c] = kh * G3_HALF + G2_A + G2_B + t * 256 + n * 16;
    }
    const _Float16* s_src[NM];
#pragma unroll
    for (int mt = 0; mt < NM; mt++) {
        const int srow = min(m0 + 32 * (mb + mt) + (lane & 31), G.m - 1);
        s_src[mt] = ((lane >> 5) ? G.Sl : G.Sh) + (int64_t)srow * (G.k / 32) + kh * hsb * 8;
    }

    f32x16 acc[NM][2], part[NM][2];
#pragma unroll
    for (int mt = 0; mt < NM; mt++)
#pragma unroll
        for (int c = 0; c < 2; c++) {
            acc[mt][c] = (f32x16){};
            part[mt][c] = (f32x16){};
        }
    u32x4 hd[2] = {};
    half8_t sv[NM] = {};
    uint32_t c64;  // 0x64006400 in a VGPR (see dq8)
    asm("v_mov_b32 %0, 0x64006400" : "=v"(c64));

    issue(0, ring);
    issue(1, ring + G3_STAGE);
    const uint32_t ring_lds = lds_addr(ring);
    int cur = 0;  // ring slot of stage s
    for (int b = 0; b < hsb; b++) {
#pragma unroll
        for (int J = 0; J < 4; J++) {
            const int s = 4 * b + J;
            const uint32_t st = ring_lds + cur * G3_STAGE;
            const int nx = cur == 0 ? 2 : cur - 1;  // slot of stage s + 2 (= slot of s - 1)
            // this wave's loads of stage s have landed (those of s + 1 may be in flight)
            __builtin_amdgcn_s_waitcnt((LOADS & 15) | (7 << 4) | (15 << 8) | ((LOADS >> 4) << 14));
            __builtin_amdgcn_s_barrier();  // every wave's part of stage s is in; slot nx is free
            if (J == 0) {
#pragma unroll
                for (int mt = 0; mt < NM; mt++) sv[mt] = *(const half8_t*)(s_src[mt] + b * 8);
            }
            issue(s + 2, ring + nx * G3_STAGE);
            cur = cur == 2 ? 0 : cur + 1;
            // LDS reads, one k-slice ahead of the MFMAs, consumed under lgkmcnt
            // (2·NM A reads per k-slice)
            if (J == 0) {
                hd[0] = lds_b128<0>(st + h_off[0]);
                hd[1] = lds_b128<0>(st + h_off[1]);
            }
            u32x4 raw[2];  // [0..1]: k-group 0, [2..3]: k-group 1 (256 B further)
            raw[0] = lds_2b64_256(st + b_off[0]);
            raw[1] = lds_2b64_256(st + b_off[1]);
            const uint32_t pa = st + a_off;
            half8_t a[4][NM][2];  // [ks][mt][part]
            a[0][0][0] = lds_b128h<0>(pa);
            a[0][0][1] = lds_b128h<1024>(pa);
            if constexpr (NM == 2) {
                a[0][NM - 1][0] = lds_b128h<8192>(pa);
                a[0][NM - 1][1] = lds_b128h<9216>(pa);
            }
            a[1][0][0] = lds_b128h<2048>(pa);
            a[1][0][1] = lds_b128h<3072>(pa);
            if constexpr (NM == 2) {
                a[1][NM - 1][0] = lds_b128h<10240>(pa);
                a[1][NM - 1][1] = lds_b128h<11264>(pa);
            }
            lgkm_wait<2 * NM>();
            pin(hd[0]);
            pin(hd[1]);
            pin(raw[0]);
            pin(raw[1]);
            a[2][0][0] = lds_b128h<4096>(pa);
            a[2][0][1] = lds_b128h<5120>(pa);
            if constexpr (NM == 2) {
                a[2][NM - 1][0] = lds_b128h<12288>(pa);
                a[2][NM - 1][1] = lds_b128h<13312>(pa);
            }
            // scales of sub-blocks 2J (low nibbles) and 2J + 1 (high nibbles), get_scale_min_k4:
            // sp = (sc, sc'/16), zp = (−1024·sc, −64·sc'), used as broadcast halves
            half2_t sp[2], zp[2];
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const uint32_t y = hd[c][1], w = hd[c][3];
                const uint32_t sc4 = J < 2 ? (y & 0x3F3F3F3Fu) : ((w & 0x0F0F0F0Fu) | ((y >> 2) & 0x30303030u));
                half2_t p01, p23;
                bytes_to_h2(sc4, p01, p23);
                const half2_t pr = (J & 1) ? p23 : p01;
                const half2_t k_s = {(_Float16)1.0f, (_Float16)0.0625f}, k_z = {(_Float16)-1024.0f, (_Float16)-64.0f};
                sp[c] = pr * k_s;
                zp[c] = pr * k_z;
            }
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                const int nib = ks >> 1, kg = ks & 1;
                if (ks == 1) {
                    lgkm_wait<2 * NM>();
                    a[3][0][0] = lds_b128h<6144>(pa);
                    a[3][0][1] = lds_b128h<7168>(pa);
                    if constexpr (NM == 2) {
                        a[3][NM - 1][0] = lds_b128h<14336>(pa);
                        a[3][NM - 1][1] = lds_b128h<15360>(pa);
                    }
                }
                if (ks == 2) lgkm_wait<2 * NM>();
                if (ks == 3) lgkm_wait<0>();
#pragma unroll
                for (int mt = 0; mt < NM; mt++) {
                    pin(a[ks][mt][0]);
                    pin(a[ks][mt][1]);
                }
                half8_t bv[2];
#pragma unroll
                for (int c = 0; c < 2; c++) {
                    const uint32_t x = raw[c][2 * kg], y = raw[c][2 * kg + 1];
                    if (nib == 0)
                        bv[c] = dq8<0x000F000Fu>(x, y, c64, __builtin_shufflevector(sp[c], sp[c], 0, 0),
                                                 __builtin_shufflevector(zp[c], zp[c], 0, 0));
                    else
                        bv[c] = dq8<0x00F000F0u>(x, y, c64, __builtin_shufflevector(sp[c], sp[c], 1, 1),
                                                 __builtin_shufflevector(zp[c], zp[c], 1, 1));
                }
#pragma unroll
                for (int p = 0; p < 2; p++)
#pragma unroll
                    for (int mt = 0; mt < NM; mt++)
#pragma unroll
                        for (int c = 0; c < 2; c++)
                            part[mt][c] =
                                __builtin_amdgcn_mfma_f32_32x32x16_f16(a[ks][mt][p], bv[c], part[mt][c], 0, 0, 0);
            }
#if AETH_GEMM_IGLP
            // interleave: each MFMA followed by a few VALU ops (next k-slice's dequantisation)
#pragma unroll
            for (int i = 0; i < 16 * NM; i++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, AETH_GEMM_IGLP, 0);
            }
#endif
            if (J == 3) {
                // super-block done: C·2^-e += d·P − 32·dmin·Σ_s m_s·S_s (S carries 2^-(e+5))
#pragma unroll
                for (int c = 0; c < 2; c++) {
                    const float d = aeth_decode_d(hd[c][0]), ndm = -32.0f * aeth_decode_d(hd[c][0] >> 16);
                    const uint32_t z = hd[c][2], w = hd[c][3];
                    half2_t m01, m23, m45, m67;
                    bytes_to_h2(z & 0x3F3F3F3Fu, m01, m23);
                    bytes_to_h2(((w >> 4) & 0x0F0F0F0Fu) | ((z >> 2) & 0x30303030u), m45, m67);
                    const half8_t mv = {m01[0], m01[1], m23[0], m23[1], m45[0], m45[1], m67[0], m67[1]};
#pragma unroll
                    for (int mt = 0; mt < NM; mt++) {
                        const f32x16 q = __builtin_amdgcn_mfma_f32_32x32x16_f16(sv[mt], mv, (f32x16){}, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 16; r++)
                            acc[mt][c][r] = fmaf(ndm, q[r], fmaf(d, part[mt][c][r], acc[mt][c][r]));
                        part[mt][c] = (f32x16){};
                    }
                }
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0);  // the tail's loads have landed
    __syncthreads();                // and every wave is done reading the ring

    // K half 1 hands its partial sums to K half 0 through LDS ([wn][mt][c][r][lane] floats)
    float* red = (float*)ring + wn * 4096;
    if (kh == 1) {
#pragma unroll
        for (int mt = 0; mt < NM; mt++)
#pragma unroll
            for (int c = 0; c < 2; c++)
#pragma unroll
                for (int r = 0; r < 16; r++) red[(((mb + mt) * 2 + c) * 16 + r) * 64 + lane] = acc[mt][c][r];
    }
    __syncthreads();
    if (kh == 1) return;
    const int lr = lane & 31;
#pragma unroll
    for (int mt = 0; mt < NM; mt++)
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const int col = n0 + 64 * wn + 32 * c + lr;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = m0 + 32 * (mb + mt) + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
                const float sum = acc[mt][c][r] + red[(((mb + mt) * 2 + c) * 16 + r) * 64 + lane];
                if (row < G.m && col < G.n) {
                    const float v = sum * G.escale[row];
                    float* dst = G.C + (int64_t)row * G.ldc + col;
                    *dst = G.accumulate ? *dst + v : v;
                }
            }
        }
}

__global__ void __launch_bounds__(256) k_gemm_q4k_sk(GemmArgs G) { gemm_sk_body<1>(G); }
__global__ void __launch_bounds__(512) k_gemm_q4k_sk8(GemmArgs G) { gemm_sk_body<2>(G); }

int64_t aeth_gemm_ws_bytes(int64_t m, int64_t k) {
    // fragments [mp][k] × {hi, lo}, Sh, Sl [mp][k/32] (fp16), escale [mp] (f32)
    const int64_t mp = aeth_cdiv(m, G2_BM) * G2_BM;
    return mp * k * 2 * 2 + mp * (k / 32) * 2 * 2 + mp * 4 + 256;
}

int aeth_gemm_q4k_launch(const aeth_weight* w, const float* d_a, int64_t m, float* d_c, unsigned flags,
                         hipStream_t s, int64_t ldc, void* ws, size_t ws_bytes) {
    const int k = (int)w->k, nb = (int)w->nb;
    if (ldc <= 0) ldc = w->n;
    if (k != nb * 256) {  // ragged K: row-batched GEMV
        GemvEpi e;
        e.flags = flags;
        e.ldc = ldc;
        return aeth_gemv_launch_ex(w, d_a, m, d_c, e, s);
    }
    const int64_t mp = aeth_cdiv(m, G2_BM) * G2_BM;  // fragment rows: whole 64-row tiles
    if (mp > (1LL << 20) || mp * k > (1LL << 29)) return aeth_set_error(AETH_EINVAL, "gemm: m=%lld too large", (long long)m);
    const size_t need = (size_t)aeth_gemm_ws_bytes(m, k);
    if (ws && ws_bytes < need)
        return aeth_set_error(AETH_EINVAL, "gemm: workspace of %zu bytes < %zu needed", ws_bytes, need);
    if (!ws) {
        int rc = aeth_stream_scratch(s, AETH_SCRATCH_GEMM, need, &ws);
        if (rc) return rc;
    }
    _Float16* frag = (_Float16*)ws;
    _Float16* Sh = frag + (size_t)mp * k * 2;
    _Float16* Sl = Sh + (size_t)mp * (k / 32);
    float* esc = (float*)(Sl + (size_t)mp * (k / 32));
    const bool al16 = ((uintptr_t)d_a & 15) == 0;
    const dim3 rg((unsigned)aeth_cdiv(mp, 4)), fg((unsigned)(mp / 32), (unsigned)nb);
    if (al16) hipLaunchKernelGGL(k_gemm_rowscale<true>, rg, dim3(256), 0, s, d_a, (int)m, (int)mp, k, esc);
    else hipLaunchKernelGGL(k_gemm_rowscale<false>, rg, dim3(256), 0, s, d_a, (int)m, (int)mp, k, esc);
    AETH_LAUNCH_CHECK();
    const bool q8 = (flags & AETH_MM_Q8_ACTIVATIONS) != 0;
    if (al16 && q8) hipLaunchKernelGGL((k_gemm_frag<true, true>), fg, dim3(256), 0, s, d_a, (int)m, k, esc, frag, Sh, Sl);
    else if (q8) hipLaunchKernelGGL((k_gemm_frag<false, true>), fg, dim3(256), 0, s, d_a, (int)m, k, esc, frag, Sh, Sl);
    else if (al16) hipLaunchKernelGGL((k_gemm_frag<true, false>), fg, dim3(256), 0, s, d_a, (int)m, k, esc, frag, Sh, Sl);
    else hipLaunchKernelGGL((k_gemm_frag<false, false>), fg, dim3(256), 0, s, d_a, (int)m, k, esc, frag, Sh, Sl);
    AETH_LAUNCH_CHECK();
    const int gm = (int)(mp / G2_BM), gn = (int)aeth_cdiv(w->n, G2_BN);
    const int64_t ntiles = aeth_cdiv(w->n, 16);
    const int64_t qb = ntiles * nb * 2048, hb = ntiles * nb * 256, ab = mp * k * 4;
    GemmArgs G{(const uint8_t*)frag, Sh, Sl, esc, w->p0, w->p1, (int)m, (int)w->n, k, nb, (int)ntiles, gm, gn,
               (int)std::min(ab, (int64_t)INT32_MAX), (int)std::min(qb, (int64_t)INT32_MAX),
               (int)std::min(hb, (int64_t)INT32_MAX), d_c, ldc, (flags & AETH_MM_ACCUMULATE) ? 1 : 0};
    const bool fits32 = qb < INT32_MAX && ab < INT32_MAX;  // buffer offsets are 32-bit
    // AETH_GEMM_KERNEL=2 forces the single-K-group kernel, =3 the 4-wave split-K kernel (tuning and tests)
    static const int env_kernel = getenv("AETH_GEMM_KERNEL") ? atoi(getenv("AETH_GEMM_KERNEL")) : 0;
    if ((nb & 1) == 0 && fits32 && env_kernel == 3)
        hipLaunchKernelGGL(k_gemm_q4k_sk, dim3((unsigned)(gm * gn)), dim3(256), 0, s, G);
    else if ((nb & 1) == 0 && fits32 && env_kernel != 2)
        hipLaunchKernelGGL(k_gemm_q4k_sk8, dim3((unsigned)(gm * gn)), dim3(512), 0, s, G);
    else
        hipLaunchKernelGGL(k_gemm_q4k_ring, dim3((unsigned)(gm * gn)), dim3(256), 0, s, G);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}
