// Prefill GEMM for Q4_K weights (m > 1):  C[m][n] = Σ_k A[m][k]·W[n][k].
//
// "Exact" mode on fp16 MFMA (v_mfma_f32_32x32x16_f16, fp32 accumulate):
//  * A is split into two fp16 parts, A = Ah + Al (Ah = fp16(A·2^-e),
//    Al = fp16(A·2^-e − Ah)): 22 significant bits, f32-level, with a per-row
//    power-of-two e keeping the parts in fp16 range.
//  * Q4_K weights become exact fp16 integers w = q·sc (q ≤ 15, sc ≤ 63), so
//    every MFMA product is exact and the K-sum is an f32 accumulation.
//  * Per 256-element super-block b:  C += d_b·Σ A·(q·sc) − dmin_b·Σ_s m_s·S_s
//    with S_s = Σ_{i∈s} A_i the 32-element sub-block sums, themselves split
//    hi/lo and contracted by one extra MFMA (k = 8 sub-blocks × {hi, lo}).
//    Scales are therefore applied once per super-block, not per element.
// Each product A_hi·w and A_lo·w costs one MFMA pass, so the useful rate is
// half the fp16 MFMA rate.
//
// Weight dequantisation in packed fp16: the half with bits 0x6400 | q is
// 1024 + q (q < 1024), and one v_pk_fma_f16 with (sc, −1024·sc) gives q·sc
// exactly (the fused product is exact, the result an integer below 2048).
// Masking a dword with 0x000F000F yields the pair (elements 0, 2) of its four
// bytes and (w >> 8) the pair (1, 3), so each group of 4 k-positions is stored
// in the order [0, 2, 1, 3]; the activation prep writes A in the same order,
// and every dot product is unchanged.
#include <math.h>
#include <stdlib.h>

#include "aeth_common.hpp"
#include "aeth_internal.hpp"

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// ── activation prep: A (f32) → Ah, Al (fp16), Sh, Sl (fp16 sub-block sums),
// escale[m] = 2^e (A was scaled by 2^-e; S by 2^-(e+5)).
__global__ void __launch_bounds__(256) k_gemm_prep(const float* __restrict__ A, int k, _Float16* __restrict__ Ah,
                                                   _Float16* __restrict__ Al, _Float16* __restrict__ Sh,
                                                   _Float16* __restrict__ Sl, float* __restrict__ escale) {
    __shared__ float red[4];
    const int m = blockIdx.x, tid = threadIdx.x;
    const float* a = A + (int64_t)m * k;
    float mx = 0.0f;
    for (int i = tid; i < k; i += 256) mx = fmaxf(mx, fabsf(a[i]));
    mx = aeth_wave_max(mx);
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int E = 0;
    if (mx > 0.0f && isfinite(mx)) (void)frexpf(mx, &E);
    const int e = E > 14 ? E - 14 : 0;  // |A·2^-e| < 2^14
    if (tid == 0) escale[m] = ldexpf(1.0f, e);
    for (int i = tid; i < k; i += 256) {
        const float v = ldexpf(a[i], -e);
        const _Float16 h = (_Float16)v;
        const int pi = (i & ~3) | ((0x3120 >> (4 * (i & 3))) & 3);  // positions 1 and 2 of each 4 swapped
        Ah[(int64_t)m * k + pi] = h;
        Al[(int64_t)m * k + pi] = (_Float16)(v - (float)h);
    }
    for (int s = tid; s < k / 32; s += 256) {
        float sum = 0.0f;
        for (int i = 0; i < 32; i++) sum += a[s * 32 + i];
        const float v = ldexpf(sum, -(e + 5));
        const _Float16 h = (_Float16)v;
        Sh[(int64_t)m * (k / 32) + s] = h;
        Sl[(int64_t)m * (k / 32) + s] = (_Float16)(v - (float)h);
    }
}

#define GEMM_BN 128
#define GEMM_BK 64
#define GEMM_LDR 72  // LDS row stride in halves (64 + 8 pad: 144 B, conflict-free b128 reads)

struct GemmArgs {
    const _Float16 *Ah, *Al, *Sh, *Sl;
    const float* escale;
    const uint8_t* hdr;  // Q4_K tile layout (aeth_q4k_hdr_off)
    const uint8_t* qs;   // Q4_K tile layout (aeth_q4k_qs_off)
    int m, n, k, nb;
    float* C;
    int accumulate;
};

// get_scale_min_k4 (common.rs:29-38) for sub-block s on header dwords.
__device__ __forceinline__ void k4_sm(const uint4& h, int s, int& sc, int& m) {
    const uint32_t y = h.y, z = h.z, w = h.w;
    const int t = s & 3;
    const uint32_t yb = (y >> (8 * t)) & 0xFFu, zb = (z >> (8 * t)) & 0xFFu, wb = (w >> (8 * t)) & 0xFFu;
    if (s < 4) {
        sc = (int)(yb & 63u);
        m = (int)(zb & 63u);
    } else {
        sc = (int)((wb & 0x0Fu) | ((yb >> 6) << 4));
        m = (int)((wb >> 4) | ((zb >> 6) << 4));
    }
}

// Workgroup: BM × 128 tile of C, 4 waves in 2 × 2, wave tile (BM/2) × 64 =
// TM × 2 MFMA tiles of 32 × 32. K advances by 64 (a quarter super-block).
// Global loads run D steps ahead of the LDS stores (register staging slots
// j % D of the 4 unrolled steps of a super-block), so each step's loads have D
// steps of MFMA work to arrive in.
template <int BM, int D>
__global__ void __launch_bounds__(256) k_gemm_q4k(GemmArgs G) {
    static_assert(D == 1 || D == 2 || D == 4, "prefetch distance divides the 4 steps of a super-block");
    constexpr int TM = BM / 64;  // 32-row MFMA tiles per wave
    __shared__ __attribute__((aligned(16))) _Float16 sA[2][2][BM * GEMM_LDR];  // [buf][hi/lo]
    __shared__ __attribute__((aligned(16))) _Float16 sB[2][GEMM_BN * GEMM_LDR];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int n0 = blockIdx.x * GEMM_BN, m0 = blockIdx.y * BM;
    const int nb = G.nb;
    const int nsteps = nb * 4;

    // global → register staging for one K-step. Every load is unconditional
    // (rows past m / n are clamped to valid rows and never written back).
    // A: BM rows × 64 halves × {hi, lo}: 16-byte pieces, 8 per row per part
    constexpr int A_PIECES = BM * 8 * 2;
    constexpr int A_PER_T = A_PIECES / 256;
    // piece i = tid + 256·i: part (hi/lo) = 256·i / (8·BM) is known at compile time
    uint4 ra[D][A_PER_T];
    const int a_rr = (tid / 8) % BM, a_c = tid % 8;
    // B: 128 rows × one Q4_K unit (32 qs bytes): 2 threads per row, 16 bytes each
    uint4 rq[D];
    uint4 rh[D];
    const int brow = tid >> 1, bhalf = tid & 1;
    const int64_t nrow = min(n0 + brow, G.n - 1);
    const uint8_t* q_src = G.qs + aeth_q4k_qs_off(nrow, 0, 16 * bhalf, nb);
    const uint8_t* h_src = G.hdr + aeth_q4k_hdr_off(nrow, 0, nb);

    auto load_step = [&](int step, int slot) {
        const int b = step >> 2, j = step & 3;
#pragma unroll
        for (int i = 0; i < A_PER_T; i++) {
            const int part = (256 * i) / (BM * 8), rshift = ((256 * i) % (BM * 8)) / 8;
            const int row_i = min(m0 + (a_rr + rshift) % BM, G.m - 1);
            ra[slot][i] = *(const uint4*)((part ? G.Al : G.Ah) + (int64_t)row_i * G.k + a_c * 8 + step * 64);
        }
        rq[slot] = *(const uint4*)(q_src + b * 2048 + (j >> 1) * 1024 + (j & 1) * 512);
        rh[slot] = *(const uint4*)(h_src + b * 256);
    };
    auto store_step = [&](int step, int buf, int slot) {
        const int j = step & 3;
#pragma unroll
        for (int i = 0; i < A_PER_T; i++) {
            const int part = (256 * i) / (BM * 8), rshift = ((256 * i) % (BM * 8)) / 8;
            *(uint4*)(&sA[buf][part][((a_rr + rshift) % BM) * GEMM_LDR + a_c * 8]) = ra[slot][i];
        }
        // unit bytes [16·bhalf, 16·bhalf+16) of qs[32j .. 32j+32): byte l → low nibble
        // is element l (sub-block 2j), high nibble element 32 + l (sub-block 2j+1)
        int sc0, m_, sc1;
        k4_sm(rh[slot], 2 * j, sc0, m_);
        k4_sm(rh[slot], 2 * j + 1, sc1, m_);
        const half2_t s0 = {(_Float16)sc0, (_Float16)sc0}, z0 = {(_Float16)(-1024 * sc0), (_Float16)(-1024 * sc0)};
        const half2_t s1 = {(_Float16)sc1, (_Float16)sc1}, z1 = {(_Float16)(-1024 * sc1), (_Float16)(-1024 * sc1)};
        const uint32_t* qw = (const uint32_t*)&rq[slot];
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const uint32_t w = qw[e];
            const uint32_t q[4] = {(w & 0x000F000Fu) | 0x64006400u, ((w >> 8) & 0x000F000Fu) | 0x64006400u,
                                   ((w >> 4) & 0x000F000Fu) | 0x64006400u, ((w >> 12) & 0x000F000Fu) | 0x64006400u};
            lo[2 * e] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(half2_t, q[0]), s0, z0));
            lo[2 * e + 1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(half2_t, q[1]), s0, z0));
            hi[2 * e] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(half2_t, q[2]), s1, z1));
            hi[2 * e + 1] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(half2_t, q[3]), s1, z1));
        }
        _Float16* dst = &sB[buf][brow * GEMM_LDR];
        *(uint4*)(dst + bhalf * 16) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        *(uint4*)(dst + bhalf * 16 + 8) = make_uint4(lo[4], lo[5], lo[6], lo[7]);
        *(uint4*)(dst + 32 + bhalf * 16) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
        *(uint4*)(dst + 32 + bhalf * 16 + 8) = make_uint4(hi[4], hi[5], hi[6], hi[7]);
    };

    f32x16 acc[TM][2], part[TM][2];
#pragma unroll
    for (int a = 0; a < TM; a++)
#pragma unroll
        for (int c = 0; c < 2; c++) {
            acc[a][c] = (f32x16){};
            part[a][c] = (f32x16){};
        }

#pragma unroll
    for (int d = 0; d < D; d++) load_step(min(d, nsteps - 1), d);
    const int lr = lane & 31, lk = (lane >> 5) * 8;
    int hcol[2], srow[TM];
#pragma unroll
    for (int c = 0; c < 2; c++) hcol[c] = min(n0 + wn * 64 + c * 32 + lr, G.n - 1);
#pragma unroll
    for (int a = 0; a < TM; a++) srow[a] = min(m0 + wm * (BM / 2) + a * 32 + lr, G.m - 1);
    for (int b = 0; b < nb; b++) {
        // this super-block's scales and sub-block sums, issued ahead of the steps' loads
        uint4 h[2];
        half8_t sv[TM];
#pragma unroll
        for (int c = 0; c < 2; c++) h[c] = *(const uint4*)(G.hdr + aeth_q4k_hdr_off(hcol[c], b, nb));
#pragma unroll
        for (int a = 0; a < TM; a++)
            sv[a] = *(const half8_t*)((lk ? G.Sl : G.Sh) + (int64_t)srow[a] * (G.k / 32) + b * 8);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int step = 4 * b + j, buf = j & 1;
            // LDS buffer buf was last read by step - 2, which every wave finished before
            // the barrier of step - 1
            store_step(step, buf, j % D);
            __syncthreads();
            load_step(min(step + D, nsteps - 1), j % D);
            // MFMAs of this K-step: 4 k-slices of 16, hi and lo parts
#pragma unroll
            for (int ks = 0; ks < GEMM_BK / 16; ks++) {
                half8_t bv[2];
#pragma unroll
                for (int c = 0; c < 2; c++)
                    bv[c] = *(const half8_t*)(&sB[buf][(wn * 64 + c * 32 + lr) * GEMM_LDR + ks * 16 + lk]);
#pragma unroll
                for (int a = 0; a < TM; a++) {
                    const int row = wm * (BM / 2) + a * 32 + lr;
                    const half8_t ah = *(const half8_t*)(&sA[buf][0][row * GEMM_LDR + ks * 16 + lk]);
                    const half8_t al = *(const half8_t*)(&sA[buf][1][row * GEMM_LDR + ks * 16 + lk]);
#pragma unroll
                    for (int c = 0; c < 2; c++) {
                        part[a][c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bv[c], part[a][c], 0, 0, 0);
                        part[a][c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, bv[c], part[a][c], 0, 0, 0);
                    }
                }
            }
            if (j == 3) {
                // super-block done: C += d·P − dmin·Q, Q = Σ_s m_s·S_s (hi/lo) by one MFMA per tile
#pragma unroll
                for (int c = 0; c < 2; c++) {
                    const float d = aeth_decode_d(h[c].x), dmin = aeth_decode_d(h[c].x >> 16);
                    half8_t mv;
#pragma unroll
                    for (int s = 0; s < 8; s++) {
                        int scv, mm;
                        k4_sm(h[c], s, scv, mm);
                        mv[s] = (_Float16)(float)mm;
                    }
#pragma unroll
                    for (int a = 0; a < TM; a++) {
                        f32x16 q = __builtin_amdgcn_mfma_f32_32x32x16_f16(sv[a], mv, (f32x16){}, 0, 0, 0);
                        // S was scaled by 2^-(e+5) against A's 2^-e: fold the 2^5 into dmin
                        const float dm = dmin * 32.0f;
#pragma unroll
                        for (int r = 0; r < 16; r++) acc[a][c][r] += d * part[a][c][r] - dm * q[r];
                        part[a][c] = (f32x16){};
                    }
                }
            }
        }
    }
    // epilogue: undo the row scale 2^-e, write (or accumulate) C
#pragma unroll
    for (int a = 0; a < TM; a++)
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const int col = n0 + wn * 64 + c * 32 + lr;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = m0 + wm * (BM / 2) + a * 32 + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
                if (row < G.m && col < G.n) {
                    const float v = acc[a][c][r] * G.escale[row];
                    float* dst = G.C + (int64_t)row * G.n + col;
                    *dst = G.accumulate ? *dst + v : v;
                }
            }
        }
}

// ── Ring-buffered variant (the default): A arrives as MFMA fragments, weights as
// raw quants, both through a 3-stage LDS ring filled by global_load_lds_dwordx4
// (lane i of a wave writes LDS bytes [16i, 16i+16) of the destination, from any
// global address), so no VGPR staging and no LDS stores by the waves.
// Workgroup tile 64 × 128, 4 waves of 32 × 64; one stage = 64 K-positions (a
// quarter super-block): 16 A fragments (2 m-tiles × 4 k-slices × {hi, lo}),
// 8 tiles × 512 B of quants, the super-block's headers. Each wave issues the
// same 6 loads per stage, so a fixed vmcnt marks the arrival of a stage.
#define G2_BM 64
#define G2_BN 128
#define G2_A 16384
#define G2_B 4096
#define G2_H 4096  // 2 KiB of headers per stage, each half loaded by two waves
#define G2_STAGE (G2_A + G2_B + G2_H)
#define G2_NST 3
#define G2_LOADS 6

typedef __attribute__((address_space(3))) void lds_void;

// positions 1 and 2 of each group of 4 exchanged (an involution)
__device__ __forceinline__ int perm4(int i) { return (i & ~3) | ((0x3120 >> (4 * (i & 3))) & 3); }

// A (f32 [m][k]) → fragments: fragment (mt, ks, part) = 1 KiB at ((mt·nks + ks)·2 + part)·1024
// bytes (nks = k/16); lane l holds row 32·mt + l%32 at k-positions 16·ks + 8·(l/32) + perm4(i),
// i < 8, part 0 = hi, 1 = lo. Rows m..mp-1 are zero. Sh/Sl and escale as k_gemm_prep.
__global__ void __launch_bounds__(256) k_gemm_prep_frag(const float* __restrict__ A, int m, int k,
                                                        _Float16* __restrict__ frag, _Float16* __restrict__ Sh,
                                                        _Float16* __restrict__ Sl, float* __restrict__ escale) {
    __shared__ float red[4];
    const int r = blockIdx.x, tid = threadIdx.x;
    const bool live = r < m;
    const float* a = A + (int64_t)min(r, m - 1) * k;
    float mx = 0.0f;
    for (int i = tid; i < k; i += 256) mx = fmaxf(mx, fabsf(a[i]));
    mx = aeth_wave_max(mx);
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int E = 0;
    if (mx > 0.0f && isfinite(mx)) (void)frexpf(mx, &E);
    const int e = E > 14 ? E - 14 : 0;  // |A·2^-e| < 2^14
    if (tid == 0) escale[r] = ldexpf(1.0f, e);
    const int nks = k / 16, mt = r / 32, lr = r % 32;
    // 8-element groups g; groups 4q..4q+3 form sub-block q (k is a multiple of 256,
    // so every lane of a wave that enters an iteration has its whole aligned 4-group)
    for (int g = tid; g < k / 8; g += 256) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = live ? a[8 * g + i] : 0.0f;
        float fs = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) fs += v[i];
        half8_t hi, lo;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float x = ldexpf(v[perm4(i)], -e);
            const _Float16 h = (_Float16)x;
            hi[i] = h;
            lo[i] = (_Float16)(x - (float)h);
        }
        _Float16* dst = frag + ((int64_t)(mt * nks + (g >> 1)) * 2) * 512 + (lr + 32 * (g & 1)) * 8;
        *(half8_t*)dst = hi;
        *(half8_t*)(dst + 512) = lo;
        fs += __shfl_xor(fs, 1, 64);
        fs += __shfl_xor(fs, 2, 64);
        if ((g & 3) == 0) {
            const float sv = ldexpf(fs, -(e + 5));
            const _Float16 h = (_Float16)sv;
            Sh[(int64_t)r * (k / 32) + g / 4] = h;
            Sl[(int64_t)r * (k / 32) + g / 4] = (_Float16)(sv - (float)h);
        }
    }
}

struct Gemm2Args {
    const uint8_t* frag;
    const _Float16 *Sh, *Sl;
    const float* escale;
    const uint8_t* hdr;
    const uint8_t* qs;
    int m, n, k, nb, ntiles;
    int gm, gn;  // 64-row and 128-column tiles of C
    float* C;
    int accumulate;
};

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

// 8 quants (one nibble of 8 bytes) → the B operand, k-order [0, 2, 1, 3] per 4
__device__ __forceinline__ half8_t dq8(uint2 raw, int nib, half2_t s, half2_t z) {
    const uint32_t x = raw.x >> (4 * nib), y = raw.y >> (4 * nib);
    const uint32_t q0 = pkfma((x & 0x000F000Fu) | 0x64006400u, s, z);
    const uint32_t q1 = pkfma(((x >> 8) & 0x000F000Fu) | 0x64006400u, s, z);
    const uint32_t q2 = pkfma((y & 0x000F000Fu) | 0x64006400u, s, z);
    const uint32_t q3 = pkfma(((y >> 8) & 0x000F000Fu) | 0x64006400u, s, z);
    return __builtin_bit_cast(half8_t, make_uint4(q0, q1, q2, q3));
}

// LDS reads issued as inline asm: the compiler would otherwise order every LDS
// read after all outstanding direct-to-LDS loads (vmcnt(0)), since it cannot tell
// the ring's slots apart. The kernel waits with lgkmcnt itself, then passes each
// value through pin() so no use is scheduled above its wait.
typedef __attribute__((address_space(3))) char lds_char;
__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(const lds_char*)p; }
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
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

__global__ void __launch_bounds__(256) k_gemm_q4k_ring(Gemm2Args G) {
    __shared__ __attribute__((aligned(1024))) char ring[G2_NST * G2_STAGE];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    int tm, tn;
    g2_tile(blockIdx.x, G.gm, G.gn, tm, tn);
    const int n0 = tn * G2_BN, m0 = tm * G2_BM;
    const int nb = G.nb, nst = 4 * nb, nks = G.k / 16;

    // direct-load sources for stage 0; stage s adds s·8 KiB (A), s·512 B (quants),
    // (s/4)·256 B (headers). Tiles past the last are clamped (never written back).
    const uint8_t* a_src[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int f = wave + 4 * j;  // local fragment: m-tile f/8, k-slice (f/2)%4, part f%2
        a_src[j] = G.frag + ((int64_t)((2 * tm + (f >> 3)) * nks + ((f >> 1) & 3)) * 2 + (f & 1)) * 1024 + lane * 16;
    }
    const int bt = min(n0 / 16 + 2 * wave + (lane >> 5), G.ntiles - 1);
    const uint8_t* b_src = G.qs + (int64_t)bt * nb * 2048 + (lane & 31) * 16;
    const int ht = min(n0 / 16 + 4 * (wave & 1) + (lane >> 4), G.ntiles - 1);
    const uint8_t* h_src = G.hdr + ((int64_t)ht * nb * 16 + (lane & 15)) * 16;
    auto issue = [&](int s, char* st) {
        s = min(s, nst - 1);  // the ring's tail reloads the last stage into a free buffer
#pragma unroll
        for (int j = 0; j < 4; j++) g_dma(a_src[j] + (int64_t)s * 8192, st + (wave + 4 * j) * 1024);
        g_dma(b_src + (int64_t)s * 512, st + G2_A + wave * 1024);
        g_dma(h_src + (int64_t)(s >> 2) * 256, st + G2_A + G2_B + wave * 1024);
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
            // scales of sub-blocks 2J (low nibbles) and 2J + 1 (high nibbles), get_scale_min_k4
            half2_t sn[2][2], zn[2][2];
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const uint32_t y = hd[c].y, w = hd[c].w;
                const uint32_t sc4 = J < 2 ? (y & 0x3F3F3F3Fu) : ((w & 0x0F0F0F0Fu) | ((y >> 2) & 0x30303030u));
                half2_t p01, p23;
                bytes_to_h2(sc4, p01, p23);
                const half2_t pr = (J & 1) ? p23 : p01;
                const half2_t m1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f};
                sn[c][0] = __builtin_shufflevector(pr, pr, 0, 0);
                sn[c][1] = __builtin_shufflevector(pr, pr, 1, 1);
                zn[c][0] = sn[c][0] * m1024;
                zn[c][1] = sn[c][1] * m1024;
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
                    const uint2 r2 = kg ? make_uint2(raw[c].z, raw[c].w) : make_uint2(raw[c].x, raw[c].y);
                    bv[c] = dq8(r2, nib, sn[c][nib], zn[c][nib]);
                }
#pragma unroll
                for (int p = 0; p < 2; p++)
#pragma unroll
                    for (int c = 0; c < 2; c++)
                        part[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[ks][p], bv[c], part[c], 0, 0, 0);
            }
            if (J == 3) {
                // super-block done: C += d·P − 32·dmin·Σ_s m_s·S_s (S scaled by 2^-(e+5))
#pragma unroll
                for (int c = 0; c < 2; c++) {
                    const float d = aeth_decode_d(hd[c].x), dmin = aeth_decode_d(hd[c].x >> 16);
                    const uint32_t z = hd[c].z, w = hd[c].w;
                    half2_t m01, m23, m45, m67;
                    bytes_to_h2(z & 0x3F3F3F3Fu, m01, m23);
                    bytes_to_h2(((w >> 4) & 0x0F0F0F0Fu) | ((z >> 2) & 0x30303030u), m45, m67);
                    const half8_t mv = {m01[0], m01[1], m23[0], m23[1], m45[0], m45[1], m67[0], m67[1]};
                    const f32x16 q = __builtin_amdgcn_mfma_f32_32x32x16_f16(sv, mv, (f32x16){}, 0, 0, 0);
                    const float dm = dmin * 32.0f;
#pragma unroll
                    for (int r = 0; r < 16; r++) acc[c][r] += d * part[c][r] - dm * q[r];
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
                float* dst = G.C + (int64_t)row * G.n + col;
                *dst = G.accumulate ? *dst + v : v;
            }
        }
    }
}

namespace {
struct GemmWs {
    void* ptr = nullptr;
    size_t bytes = 0;
};
GemmWs g_gemm_ws[64];
}  // namespace

int aeth_gemm_q4k_launch(const aeth_weight* w, const float* d_a, int64_t m, float* d_c, unsigned flags,
                         hipStream_t s) {
    const int k = (int)w->k, nb = (int)w->nb;
    if (k != nb * 256) return aeth_gemv_launch(w, d_a, m, d_c, flags, s);  // ragged K: row-batched GEMV
    // AETH_GEMM_KERNEL=1 selects the register-staged kernel (k_gemm_q4k) instead of the ring
    static const int env_kernel = getenv("AETH_GEMM_KERNEL") ? atoi(getenv("AETH_GEMM_KERNEL")) : 0;
    const bool ring = env_kernel != 1;
    const int64_t mp = ring ? aeth_cdiv(m, G2_BM) * G2_BM : m;  // fragment rows: whole 64-row tiles
    if (mp > (1LL << 20) || mp * k > (1LL << 30)) return aeth_set_error(AETH_EINVAL, "gemm: m=%lld too large", (long long)m);
    // workspace: A parts [mp][k] × {hi, lo}, Sh, Sl [mp][k/32] (fp16), escale [mp] (f32)
    const size_t need = (size_t)mp * k * 2 * 2 + (size_t)mp * (k / 32) * 2 * 2 + (size_t)mp * 4 + 256;
    int dev = 0;
    AETH_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return aeth_set_error(AETH_EINVAL, "gemm: device index");
    GemmWs& ws = g_gemm_ws[dev];
    if (ws.bytes < need) {
        if (ws.ptr) AETH_HIP_CHECK(hipFree(ws.ptr));
        ws.ptr = nullptr;
        ws.bytes = 0;
        AETH_HIP_CHECK(hipMalloc(&ws.ptr, need));
        ws.bytes = need;
    }
    _Float16* Ah = (_Float16*)ws.ptr;
    _Float16* Al = Ah + (size_t)mp * k;
    _Float16* Sh = Al + (size_t)mp * k;
    _Float16* Sl = Sh + (size_t)mp * (k / 32);
    float* esc = (float*)(Sl + (size_t)mp * (k / 32));
    if (ring) {
        hipLaunchKernelGGL(k_gemm_prep_frag, dim3((unsigned)mp), dim3(256), 0, s, d_a, (int)m, k, Ah, Sh, Sl, esc);
        AETH_LAUNCH_CHECK();
        const int gm = (int)(mp / G2_BM), gn = (int)aeth_cdiv(w->n, G2_BN);
        Gemm2Args G{(const uint8_t*)Ah, Sh, Sl, esc, w->p0, w->p1, (int)m, (int)w->n, k, nb,
                    (int)aeth_cdiv(w->n, 16), gm, gn, d_c, (flags & AETH_MM_ACCUMULATE) ? 1 : 0};
        hipLaunchKernelGGL(k_gemm_q4k_ring, dim3((unsigned)(gm * gn)), dim3(256), 0, s, G);
        AETH_LAUNCH_CHECK();
        return AETH_OK;
    }
    hipLaunchKernelGGL(k_gemm_prep, dim3((unsigned)m), dim3(256), 0, s, d_a, k, Ah, Al, Sh, Sl, esc);
    AETH_LAUNCH_CHECK();
    GemmArgs G{Ah, Al, Sh, Sl, esc, w->p0, w->p1, (int)m, (int)w->n, k, nb, d_c,
               (flags & AETH_MM_ACCUMULATE) ? 1 : 0};
    // tuning override, read once: AETH_GEMM_D (prefetch distance 1, 2 or 4)
    static const int env_d = getenv("AETH_GEMM_D") ? atoi(getenv("AETH_GEMM_D")) : 0;
    // measured at m = 512, n = 4096 / 14336: BM = 64 with a one-step prefetch is
    // best of this kernel (two workgroups per CU where the grid allows)
    dim3 grid((unsigned)aeth_cdiv(w->n, GEMM_BN), (unsigned)aeth_cdiv(m, 64));
    if (env_d == 2) hipLaunchKernelGGL((k_gemm_q4k<64, 2>), grid, dim3(256), 0, s, G);
    else if (env_d == 4) hipLaunchKernelGGL((k_gemm_q4k<64, 4>), grid, dim3(256), 0, s, G);
    else hipLaunchKernelGGL((k_gemm_q4k<64, 1>), grid, dim3(256), 0, s, G);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}
