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
// This file holds the activation prep (k_gemm_prep), the launcher and the
// single-K-group kernel for buffers past 32-bit offsets; the default main
// kernel is the K-split one in aeth_gemm_kq.hip. Both use a workgroup tile of
// 64 × 128 of C and stage their operands through LDS rings filled with
// direct-to-LDS loads (global_load_lds_dwordx4 / buffer_load_dwordx4 … lds: lane
// i of a wave writes LDS bytes [16i, 16i+16) of the destination, from any
// address): A as MFMA fragments written by the prep kernel in operand order (so
// every operand read is one contiguous ds_read_b128), the raw Q4_K quants of the
// 16-row tile layout, and the tiles' headers. The waves dequantise their own B
// operands from the raw bytes in LDS straight into registers. Their epilogue
// (aeth_gemm_common.hpp) stores C, adds it to C (accumulate), or for a gate|up
// weight of interleaved (g, u) rows stores h = g·σ(g)·u (GemmIn::swiglu_out).
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

#include <algorithm>

#include "aeth_common.hpp"
#include "aeth_gemm_common.hpp"
#include "aeth_internal.hpp"

#define G2_BM 64
#define G2_BN 128
#define G2_A 16384  // one stage's A: 2 m-tiles × 4 k-slices × {hi, lo} fragments of 1 KiB
#define G2_B 4096   // one stage's quants: 8 tiles × 512 B
#define G2_H 4096   // 2 KiB of headers per stage, each half loaded by two waves
#define G2_STAGE (G2_A + G2_B + G2_H)
#define G2_NST 3
#define G2_LOADS 6

// ── activation prep (f32 A [m][k]; rows m..mp-1 read as zero). Writes
//  * escale[r] = 2^e, e ≥ 0 the least with |A[r]·2^-e| < 2^14;
//  * fragment (mt, ks, part) = 1 KiB at ((mt·nks + ks)·2 + part)·1024 bytes
//    (nks = k/16): lane l holds row 32·mt + l%32 at k-positions
//    16·ks + 8·(l/32) + perm4(i), i < 8, of A·2^-e, part 0 = hi, 1 = lo;
//  * Sh/Sl [row][k/32] = Σ of each 32-element sub-block of A·2^-(e+5), hi/lo.
// A may be produced here from the previous op's output (GemmIn): the RMSNorm
// of the row (runner.rs:1739-1746, the element formula of k_rmsnorm_v), or
// h = g·σ(g)·u over the interleaved gate/up pairs (the formula of k_silu_pairs),
// so the GEMM reads the producer's input and the normalised / gated rows never
// go through memory.
//
// Workgroup = 4 rows (2 for the RMSNorm / SwiGLU producers holding 8 steps of
// inputs) × 4 K-parts, one wave per (row, part): wave (ri, j) takes
// the steps [S·j/4, S·(j+1)/4) of its row (a step = 64 groups of 8 elements,
// S = ⌈k/512⌉), all of its loads in flight at once (SPW steps in registers,
// sized to the share; longer rows of the plain input are read in chunks and
// re-read for the conversion). The row's sum of squares and maximum meet in LDS.
// Lane l of a step converts group gi = 64·step + l, group gi being (k-slice
// gi/2, k-group gi%2) of the row's fragment lane; a step's pieces go through LDS
// so that each store writes the 4 rows' pieces of a fragment as 64 contiguous
// bytes (measured at k = 4096: 2 rows 6.8 µs, 4 rows 5.7 µs, 8 rows 7.5 µs — 64
// workgroups for m = 512). A 32-element sub-block is the groups of four
// adjacent lanes; its sums (and its Q8_0 block) meet by DPP.
//
// Q8 = true (AETH_MM_Q8_ACTIVATIONS, the dot-product mode; plain input only): each 32-element
// sub-block is first replaced by its Q8_0 activation block, dequantized —
// quantize_q8_0_block (neon.rs:45-104): d = max|x|/127 (NaN-propagating max),
// q = sat_i8(RNE(x·(1/d))) with the f32 d, and the value q·f16(d) the integer
// dot of the reference scales with (d_a = the stored f16 d). q·f16(d) has at
// most 18 significant bits, so it is exact in f32 and in the hi/lo split: the
// GEMM then computes Σ (q_a·d_a)·(q·sc·d) exactly per product, i.e. the
// reference's per-term d_a·(d1·Σ q·q_a − m1·Σ q_a) up to f32 summation order.
#define PREP_WK 4    // K-parts per row (one wave each)
#define PREP_LD 5    // LDS stride in 16-byte pieces between groups (odd: lanes spread over the banks)

struct PrepArgs {
    const float* A;       // [m][k], or [m][2k] (g, u) pairs for PREP_SWIGLU
    const float* norm_w;  // [k] for PREP_RMSNORM
    float eps;
    int m, k;
    float* escale;
    _Float16 *frag, *Sh, *Sl;
};

// 8 consecutive floats at p (16-byte aligned when AL16)
template <bool AL16>
__device__ __forceinline__ void prep_ld8(const float* __restrict__ p, float* v) {
    if (AL16) {
        const float4 x0 = *(const float4*)p, x1 = *(const float4*)(p + 4);
        v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w;
        v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = p[i];
    }
}

// SPW: steps a wave holds in registers, at least its share ⌈S/4⌉ (1, 2, 4 or 8: k ≤ 16384 in one chunk).
// PREP_ROWS: rows per workgroup, 4 (2 where the producer's 8 steps of inputs need more than the
// 128 registers of a 16-wave workgroup; 1 for at most 128 rows, which then take more CUs).
template <bool AL16, bool Q8, int MODE, int SPW, int PREP_ROWS>
__global__ void __launch_bounds__(64 * PREP_ROWS * PREP_WK) k_gemm_prep(PrepArgs P) {
    static_assert(!Q8 || MODE == PREP_PLAIN, "the producers feed the exact mode");
    constexpr int WK = PREP_WK;
    __shared__ __attribute__((aligned(16))) uint4 stage[WK][2][64][PREP_LD];  // [part j][hi/lo][group][row]
    __shared__ float red[2][PREP_ROWS * WK];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, ri = wv % PREP_ROWS, j = wv / PREP_ROWS;
    const int r0 = blockIdx.x * PREP_ROWS, r = r0 + ri;
    const bool live = r < P.m;
    const int k = P.k, ng = k / 8, nks = k / 16, mt = r0 >> 5, rr0 = r0 & 31;
    const int S = (ng + 63) / 64, s0 = S * j / WK, ns = S * (j + 1) / WK - s0, nsmax = (S + WK - 1) / WK;
    const float* a = P.A + (int64_t)min(r, P.m - 1) * (MODE == PREP_SWIGLU ? 2 * k : k);
    float v[SPW][8], v2[SPW][8];
    // loads of the SPW steps from step t0 of this part. Every load is issued, from a clamped
    // address, and values outside the row, the part or the live rows are zeroed afterwards: a
    // load under a branch would make the compiler wait for it at the branch's end, one round
    // trip per load.
    auto load = [&](int t0) {
        bool ok[SPW];
#pragma unroll
        for (int t = 0; t < SPW; t++) {
            const int gi = 64 * (s0 + t0 + t) + lane, gc = min(gi, ng - 1);
            ok[t] = live && t0 + t < ns && gi < ng;
            if (MODE == PREP_SWIGLU) {
                prep_ld8<AL16>(a + 16 * gc, v[t]);
                prep_ld8<AL16>(a + 16 * gc + 8, v2[t]);
            } else {
                prep_ld8<AL16>(a + 8 * gc, v[t]);
                if (MODE == PREP_RMSNORM) prep_ld8<AL16>(P.norm_w + 8 * gc, v2[t]);
            }
        }
#pragma unroll
        for (int t = 0; t < SPW; t++)
#pragma unroll
            for (int i = 0; i < 8; i++) {
                v[t][i] = ok[t] ? v[t][i] : 0.0f;
                v2[t][i] = ok[t] ? v2[t][i] : 0.0f;
            }
        if (MODE == PREP_SWIGLU) {  // (g, u) pairs → g·σ(g)·u, in k order
#pragma unroll
            for (int t = 0; t < SPW; t++) {
                float h[8];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float g0 = v[t][2 * i], u0 = v[t][2 * i + 1], g1 = v2[t][2 * i], u1 = v2[t][2 * i + 1];
                    h[i] = g0 * (1.0f / (1.0f + expf(-g0))) * u0;
                    h[4 + i] = g1 * (1.0f / (1.0f + expf(-g1))) * u1;
                }
#pragma unroll
                for (int i = 0; i < 8; i++) v[t][i] = h[i];
            }
        }
    };
    const int nck = (nsmax + SPW - 1) / SPW;  // chunks (1 unless a plain row is longer than 16384)
    float mx = 0.0f;
    for (int c = 0; c < nck; c++) {
        load(c * SPW);
        if (MODE == PREP_RMSNORM) {  // rms = sqrt(Σx²/k + eps); x ← (x / rms)·w (one chunk: k ≤ 16384)
            float ss = 0.0f;
#pragma unroll
            for (int t = 0; t < SPW; t++)
#pragma unroll
                for (int i = 0; i < 8; i++) ss += v[t][i] * v[t][i];
            ss = aeth_wave_sum(ss);
            if (lane == 0) red[0][wv] = ss;
            __syncthreads();
            float tot = 0.0f;
#pragma unroll
            for (int q = 0; q < WK; q++) tot += red[0][PREP_ROWS * q + ri];
            const float rms = sqrtf(tot / (float)k + P.eps), inv = 1.0f / rms;
#pragma unroll
            for (int t = 0; t < SPW; t++)
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const float x = v[t][i], q0 = x * inv;  // the correctly rounded x / rms
                    v[t][i] = fmaf(fmaf(-q0, rms, x), inv, q0) * v2[t][i];
                }
        }
#pragma unroll
        for (int t = 0; t < SPW; t++)
#pragma unroll
            for (int i = 0; i < 8; i++) mx = fmaxf(mx, fabsf(v[t][i]));
    }
    mx = aeth_wave_max(mx);
    if (lane == 0) red[1][wv] = mx;
    __syncthreads();
    mx = 0.0f;
#pragma unroll
    for (int q = 0; q < WK; q++) mx = fmaxf(mx, red[1][PREP_ROWS * q + ri]);
    int E = 0;
    if (mx > 0.0f && isfinite(mx)) (void)frexpf(mx, &E);
    const float esc = ldexpf(1.0f, E > 14 ? E - 14 : 0);
    if (j == 0 && lane == 0) P.escale[r] = esc;
    const float inv = 1.0f / esc;  // a power of two: the products below are exact scalings
    const int tp = tid % (64 * PREP_ROWS);  // thread of the part's PREP_ROWS waves
    for (int c = 0; c < nck; c++) {
        if (nck > 1) load(c * SPW);  // (one chunk: still in registers)
#pragma unroll
        for (int t = 0; t < SPW; t++) {
            if (c * SPW + t >= nsmax) break;  // uniform
            const int gb = 64 * (s0 + c * SPW + t), gi = gb + lane;
            const bool sl = c * SPW + t < ns;  // this part has the step (uniform per wave)
            float* x = v[t];
            if (Q8) {  // quantize_q8_0_block (neon.rs:45-104), then the value q·f16(d)
                int nan = 0;
                float bm = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    nan |= x[i] != x[i];
                    bm = fmaxf(bm, fabsf(x[i]));
                }
                nan |= aeth_dpp_xor1(nan);
                nan |= aeth_dpp_xor2(nan);
                bm = fmaxf(bm, aeth_dpp_xor1f(bm));
                bm = fmaxf(bm, aeth_dpp_xor2f(bm));
                const float d = nan ? __uint_as_float(0x7FC00000u) : bm / 127.0f;
                const float da = aeth_f16_to_f32(aeth_f32_to_f16_bits(d));
                const float id = d > 0.0f ? 1.0f / d : 0.0f;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const float p = x[i] * id;  // RNE with saturation, NaN → 0 (vcvtnq_s32_f32, sqxtn)
                    const float q = p != p ? 0.0f : fminf(fmaxf(rintf(p), -128.0f), 127.0f);
                    x[i] = d > 0.0f ? q * da : (d == 0.0f ? 0.0f : da);  // a NaN block dequantizes to NaN
                }
            }
            float sum = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) sum += x[i];
            sum += aeth_dpp_xor1f(sum);
            sum += aeth_dpp_xor2f(sum);
            half8_t hi, lo;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float tv = x[perm4(i)] * inv;
                const _Float16 th = (_Float16)tv;
                hi[i] = th;
                lo[i] = (_Float16)(tv - (float)th);
            }
            if (sl && gi < ng && (lane & 3) == 0) {  // gi < ng is uniform per four lanes (ng % 32 == 0)
                const float sv = sum * inv * 0.03125f;
                const _Float16 sh = (_Float16)sv;
                P.Sh[(int64_t)r * (k / 32) + (gi >> 2)] = sh;
                P.Sl[(int64_t)r * (k / 32) + (gi >> 2)] = (_Float16)(sv - (float)sh);
            }
            __syncthreads();  // the previous step's pieces have been stored
            stage[j][0][lane][ri] = __builtin_bit_cast(uint4, hi);
            stage[j][1][lane][ri] = __builtin_bit_cast(uint4, lo);
            __syncthreads();
            // piece (part, group, row) = (Q / 64R, (Q / R) % 64, Q % R), R = PREP_ROWS: R consecutive
            // threads store one group's R rows, 16·R contiguous bytes of fragment (mt, group/2, part)
            // at lane rows rr0 .. rr0 + R − 1, k-group group%2
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int Q = tp + 64 * PREP_ROWS * h, i = Q % PREP_ROWS, g = (Q / PREP_ROWS) & 63;
                const int part = Q / (64 * PREP_ROWS);
                if (sl && gb + g < ng) {
                    const int gg = gb + g;
                    uint4* dst = (uint4*)(P.frag + ((int64_t)(mt * nks + (gg >> 1)) * 2 + part) * 512) +
                                 rr0 + i + 32 * (gg & 1);
                    *dst = stage[j][part][g][i];
                }
            }
        }
    }
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
    int swiglu;   // C[row][col/2] = g·σ(g)·u over the (g, u) column pairs
};

// ── Single-K-group kernel (buffers past 2 GiB; the default is the K-split kernel
// of aeth_gemm_kq.hip): 4 waves of 32 × 64 (2 m-tiles × 2 column halves); one stage =
// 16 A fragments, 8 tiles × 512 B of quants, the super-block's headers. Each wave
// issues the same 6 loads per stage, so a fixed vmcnt marks a stage's arrival.
__device__ __forceinline__ void g_dma(const void* g, char* l) {
    __builtin_amdgcn_global_load_lds(g, (lds_void*)l, 16, 0, 0);
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
    int rows[16];
#pragma unroll
    for (int r = 0; r < 16; r++) rows[r] = m0 + 32 * wm + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
    G2Epi E[2];
#pragma unroll
    for (int c = 0; c < 2; c++)
        g2_epi_load(E[c], G.escale, G.C, G.ldc, G.m, G.n, rows, n0 + 64 * wn + 32 * c + lr, G.accumulate);
    if (G.swiglu) {
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int r = 0; r < 16; r += 2)
                g2_store_swiglu(E[c], r, G.C, G.ldc, G.m, G.n, rows[r], n0 + 64 * wn + 32 * c + lr, acc[c][r],
                                acc[c][r + 1]);
    } else {
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int r = 0; r < 16; r++)
                g2_store(E[c], r, G.C, G.ldc, G.m, G.n, rows[r], n0 + 64 * wn + 32 * c + lr, acc[c][r], G.accumulate);
    }
}

int64_t aeth_gemm_ws_bytes(int64_t m, int64_t k) {
    // fragments [mp][k] × {hi, lo}, Sh, Sl [mp][k/32] (fp16), escale [mp] (f32)
    const int64_t mp = aeth_cdiv(m, G2_BM) * G2_BM;
    return mp * k * 2 * 2 + mp * (k / 32) * 2 * 2 + mp * 4 + 256;
}

template <bool AL16, bool Q8, int MODE, int SPW>
static void prep_launch_r(unsigned mp, hipStream_t s, const PrepArgs& P) {
    constexpr int R = SPW == 8 && MODE != PREP_PLAIN ? 2 : 4;
    if (mp <= 128)  // few rows: one row per workgroup, so that they spread over more CUs
        hipLaunchKernelGGL((k_gemm_prep<AL16, Q8, MODE, SPW, 1>), dim3(mp), dim3(64 * PREP_WK), 0, s, P);
    else
        hipLaunchKernelGGL((k_gemm_prep<AL16, Q8, MODE, SPW, R>), dim3(mp / R), dim3(64 * R * PREP_WK), 0, s, P);
}
template <bool AL16, bool Q8, int MODE>
static void prep_launch(int spw, unsigned mp, hipStream_t s, const PrepArgs& P) {
    if (spw == 1) prep_launch_r<AL16, Q8, MODE, 1>(mp, s, P);
    else if (spw == 2) prep_launch_r<AL16, Q8, MODE, 2>(mp, s, P);
    else if (spw == 4) prep_launch_r<AL16, Q8, MODE, 4>(mp, s, P);
    else prep_launch_r<AL16, Q8, MODE, 8>(mp, s, P);
}

// The activation prep of the Q4_K and Q6_K GEMMs: A (or, with `in`, its producer's input) into
// hi/lo fp16 MFMA fragments, sub-block sums and row scales in ws (the stream's scratch when null).
static int gemm_prep(const float* d_a, int64_t m, int k, unsigned flags, const GemmIn* in, hipStream_t s, void* ws,
                     size_t ws_bytes, _Float16*& frag, _Float16*& Sh, float*& esc) {
    const int mode = in ? in->mode : PREP_PLAIN;
    const int64_t mp = aeth_cdiv(m, G2_BM) * G2_BM;  // fragment rows: whole 64-row tiles
    if (mp > (1LL << 20) || mp * k > (1LL << 29)) return aeth_set_error(AETH_EINVAL, "gemm: m=%lld too large", (long long)m);
    const size_t need = (size_t)aeth_gemm_ws_bytes(m, k);
    if (ws && ws_bytes < need)
        return aeth_set_error(AETH_EINVAL, "gemm: workspace of %zu bytes < %zu needed", ws_bytes, need);
    if (!ws) {
        int rc = aeth_stream_scratch(s, AETH_SCRATCH_GEMM, need, &ws);
        if (rc) return rc;
    }
    frag = (_Float16*)ws;
    Sh = frag + (size_t)mp * k * 2;
    _Float16* Sl = Sh + (size_t)mp * (k / 32);
    esc = (float*)(Sl + (size_t)mp * (k / 32));
    if (in && in->prepared) return AETH_OK;
    const bool al16 = ((uintptr_t)d_a & 15) == 0;
    const bool q8 = (flags & AETH_MM_Q8_ACTIVATIONS) != 0;
    // registers per wave: its share of the row's steps, rounded up to 1, 2, 4 or 8 (past 8: chunks)
    const int share = (int)aeth_cdiv(aeth_cdiv(k, 512), PREP_WK);
    const int spw = share <= 1 ? 1 : share <= 2 ? 2 : share <= 4 ? 4 : 8;
    const PrepArgs P{d_a, in ? in->norm_w : nullptr, in ? in->eps : 0.0f, (int)m, k, esc, frag, Sh, Sl};
    const unsigned pg = (unsigned)mp;  // fragment rows (whole 64-row tiles)
    if (mode == PREP_RMSNORM) prep_launch<true, false, PREP_RMSNORM>(spw, pg, s, P);
    else if (mode == PREP_SWIGLU) prep_launch<true, false, PREP_SWIGLU>(spw, pg, s, P);
    else if (al16 && q8) prep_launch<true, true, PREP_PLAIN>(spw, pg, s, P);
    else if (q8) prep_launch<false, true, PREP_PLAIN>(spw, pg, s, P);
    else if (al16) prep_launch<true, false, PREP_PLAIN>(spw, pg, s, P);
    else prep_launch<false, false, PREP_PLAIN>(spw, pg, s, P);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}

bool aeth_q4k_gemm_rows(const aeth_weight* w, int64_t m) {
    // AETH_Q4K_GEMM_ROWS=r takes the GEMM from r rows (tests and measurements; read once)
    static const int64_t env_rows = getenv("AETH_Q4K_GEMM_ROWS") ? atoll(getenv("AETH_Q4K_GEMM_ROWS")) : 0;
    if (env_rows > 0) return m >= env_rows;
    // The row-batched GEMV streams the weight once per row; the GEMM (its K split over workgroups
    // while its tiles are at most half the CUs) costs a near-constant 24 µs (k = 4096) to 42 µs
    // (28672 × 4096) up to 64 rows. Measured crossovers (prep + GEMM against the GEMV, rotated
    // weight copies): 4096 × 4096 ≈ 13 rows, 6144 × 4096 ≈ 12, 4096 × 14336, 14336 × 4096 and
    // 28672 × 4096 ≈ 5, i.e. where m · (weight bytes) reaches ≈ 150 MB; from 16 rows the GEMM
    // takes any weight (a 1024 × 4096 one would gain from the GEMV up to ≈ 50 rows).
    return m >= 16 || (m >= 5 && m * w->nb * w->n * 144 >= 150000000LL);
}

bool aeth_q5k_gemm_rows(const aeth_weight* w, int64_t m) {
    if (!w || w->dtype != AETH_DTYPE_Q5_K || w->order != AETH_ORDER_PLANAR || w->k != w->nb * 256 || m <= 1)
        return false;
    const int64_t mp = aeth_cdiv(m, G2_BM) * G2_BM, ntiles = aeth_cdiv(w->n, 16);
    // buffer offsets are 32-bit (larger products take the dequantized product)
    if (ntiles * w->nb * 2048 >= INT32_MAX || mp * w->k * 4 >= INT32_MAX || mp > (1LL << 20)) return false;
    // AETH_Q5K_GEMM_ROWS=r takes the GEMM from r rows (tests and measurements; read once)
    static const int64_t env_rows = getenv("AETH_Q5K_GEMM_ROWS") ? atoll(getenv("AETH_Q5K_GEMM_ROWS")) : 0;
    if (env_rows > 0) return m >= env_rows;
    return m >= 16 || (m >= 5 && m * w->nb * w->n * 176 >= 150000000LL);
}

// planar Q4_K or Q5_K weights at m rows that the K-split GEMM takes
static bool kq_gemm_rows(const aeth_weight* w, int64_t m) {
    if (!w || w->order != AETH_ORDER_PLANAR) return false;
    if (w->dtype == AETH_DTYPE_Q4_K) return aeth_q4k_gemm_rows(w, m);
    return aeth_q5k_gemm_rows(w, m);
}

bool aeth_gemm_fuses(const aeth_weight* w, int64_t m, int mode, const float* d_a, const float* norm_w) {
    if (!w || (w->dtype != AETH_DTYPE_Q4_K && w->dtype != AETH_DTYPE_Q5_K) || w->order != AETH_ORDER_PLANAR || m <= 1)
        return false;
    if (!kq_gemm_rows(w, m)) return false;  // the runner takes the GEMV path and its own producers
    if (mode == PREP_PLAIN) return true;
    if (w->k != w->nb * 256) return false;  // ragged K goes to the row-batched GEMV
    if (w->k > 16384 || ((uintptr_t)d_a & 15)) return false;  // one chunk of registers per wave, float4 loads
    if (mode == PREP_RMSNORM) return norm_w && ((uintptr_t)norm_w & 15) == 0;
    return mode == PREP_SWIGLU;
}

bool aeth_gemm_swiglu_out(const aeth_weight* w, int64_t m) {
    return w && (w->dtype == AETH_DTYPE_Q4_K || w->dtype == AETH_DTYPE_Q5_K) && w->order == AETH_ORDER_PLANAR &&
           m > 1 && w->k == w->nb * 256 && (w->n & 1) == 0 && kq_gemm_rows(w, m);
}

// AETH_GEMM_TAIL_SPLIT=0 turns the last-round K split off (A/B timing; the results agree to rounding)
static bool tail_split_off() {
    static const bool off = getenv("AETH_GEMM_TAIL_SPLIT") && atoi(getenv("AETH_GEMM_TAIL_SPLIT")) == 0;
    return off;
}

// K splits of a K-split GEMM launch over gm × gn tiles (at most maxsplit ways, so that every wave
// keeps whole units of K): with at most half as many tiles as CUs, ksplit ways for
// every tile, as many as fit one round of workgroups; with more tiles than CUs and a last round at
// most half full, tsplit ways for that round's tiles (g2_tail_ways). The partial tiles go to the
// stream's scratch (g2_part's layouts: all of C per split, or the tail tiles only); with `whole`
// (a caller's workspace) nothing is split.
struct SplitPlan {
    int ksplit = 1, tsplit = 1, t_full = 0;
    float* part = nullptr;
};
static int split_plan(hipStream_t s, int64_t gm, int64_t gn, int64_t maxsplit, bool whole, SplitPlan& P) {
    P = SplitPlan{};
    if (whole) return AETH_OK;
    const int64_t cus = aeth_num_cus(), T = gm * gn;
    P.ksplit = (int)std::max<int64_t>(1, std::min<int64_t>(cus / T, maxsplit));
    if (P.ksplit == 1 && !tail_split_off()) {
        P.tsplit = g2_tail_ways(T, cus, maxsplit);
        if (P.tsplit > 1) P.t_full = (int)(T - T % cus);
    }
    if (P.ksplit == 1 && P.tsplit == 1) return AETH_OK;
    const size_t floats = P.tsplit > 1 ? (size_t)P.tsplit * (size_t)(T - P.t_full) * G2_BM * G2_BN
                                       : (size_t)P.ksplit * gm * G2_BM * gn * G2_BN;
    void* p = nullptr;
    const int rc = aeth_stream_scratch(s, AETH_SCRATCH_SPLIT, floats * sizeof(float), &p);
    P.part = (float*)p;
    return rc;
}

int aeth_gemm_q4k_launch(const aeth_weight* w, const float* d_a, int64_t m, float* d_c, unsigned flags,
                         hipStream_t s, int64_t ldc, void* ws, size_t ws_bytes, const GemmIn* in) {
    const int k = (int)w->k, nb = (int)w->nb;
    const int mode = in ? in->mode : PREP_PLAIN;
    const bool swo = in && in->swiglu_out;
    if (ldc <= 0) ldc = swo ? w->n / 2 : w->n;
    if (mode != PREP_PLAIN && !aeth_gemm_fuses(w, m, mode, d_a, in->norm_w))
        return aeth_set_error(AETH_EINVAL, "gemm: fused producer %d not available for k=%d", mode, k);
    if (mode != PREP_PLAIN && (flags & AETH_MM_Q8_ACTIVATIONS))  // the producers feed the exact (f32) mode only
        return aeth_set_error(AETH_EINVAL, "gemm: fused producer %d with Q8 activations", mode);
    if (swo && (!aeth_gemm_swiglu_out(w, m) || (flags & AETH_MM_ACCUMULATE)))
        return aeth_set_error(AETH_EINVAL, "gemm: SwiGLU output needs whole super-blocks, even n, no accumulate");
    const bool q5 = w->dtype == AETH_DTYPE_Q5_K;
    if (q5 && !aeth_q5k_gemm_rows(w, m))
        return aeth_set_error(AETH_EINVAL, "gemm q5_k: shape not taken (m=%lld)", (long long)m);
    if (k != nb * 256) {  // ragged K: row-batched GEMV
        GemvEpi e;
        e.flags = flags;
        e.ldc = ldc;
        return aeth_gemv_launch_ex(w, d_a, m, d_c, e, s);
    }
    const int64_t mp = aeth_cdiv(m, G2_BM) * G2_BM;  // fragment rows: whole 64-row tiles
    _Float16 *frag, *Sh;
    float* esc;
    int rc = gemm_prep(d_a, m, k, flags, in, s, ws, ws_bytes, frag, Sh, esc);
    if (rc) return rc;
    const _Float16* Sl = Sh + (size_t)mp * (k / 32);
    const int gm = (int)(mp / G2_BM), gn = (int)aeth_cdiv(w->n, G2_BN);
    const int64_t ntiles = aeth_cdiv(w->n, 16);
    const int64_t qb = ntiles * nb * 2048, hb = ntiles * nb * 256, ab = mp * k * 4;
    GemmArgs G{(const uint8_t*)frag, Sh, Sl, esc, w->p0, w->p1, (int)m, (int)w->n, k, nb, (int)ntiles, gm, gn,
               (int)std::min(ab, (int64_t)INT32_MAX), (int)std::min(qb, (int64_t)INT32_MAX),
               (int)std::min(hb, (int64_t)INT32_MAX), d_c, ldc, (flags & AETH_MM_ACCUMULATE) ? 1 : 0, swo ? 1 : 0};
    const bool fits32 = qb < INT32_MAX && ab < INT32_MAX;  // buffer offsets are 32-bit
    // The K-split kernel (aeth_gemm_kq.hip); the single-K-group kernel serves buffers past the 32-bit
    // offsets of the buffer loads, and AETH_GEMM_KERNEL=2 forces it (tests)
    static const int env_kernel = getenv("AETH_GEMM_KERNEL") ? atoi(getenv("AETH_GEMM_KERNEL")) : 0;
    if (fits32 && (env_kernel != 2 || q5)) {
        // at most half as many tiles as CUs: K split over workgroups too, as many splits as fit in one
        // round of workgroups (each wave keeps at least one super-block), the partial tiles in the
        // stream's scratch (not with a caller's workspace)
        SplitPlan P;
        if ((rc = split_plan(s, gm, gn, nb / 8, ws != nullptr, P))) return rc;
        KqArgs Q{(const uint8_t*)frag, (const uint8_t*)Sh, esc, w->p0, w->p1, (int)m, (int)w->n, k, nb, (int)ntiles,
                 (int)mp, gm, gn, (int)ab, (int)(mp * (k / 32) * 4), (int)qb, (int)std::min(hb, (int64_t)INT32_MAX),
                 d_c, ldc, (flags & AETH_MM_ACCUMULATE) ? 1 : 0, swo ? 1 : 0, P.ksplit, P.part, gn * G2_BN,
                 q5 ? w->p3 : nullptr, q5 ? (int)(ntiles * nb * 512) : 0, P.t_full, P.tsplit};
        return aeth_gemm_kq_launch(Q, s);
    }
    hipLaunchKernelGGL(k_gemm_q4k_ring, dim3((unsigned)(gm * gn)), dim3(256), 0, s, G);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}

bool aeth_q6k_gemm_rows(const aeth_weight* w, int64_t m) {
    if (!w || w->dtype != AETH_DTYPE_Q6_K || w->order != AETH_ORDER_PLANAR || w->k != w->nb * 256) return false;
    const int64_t mp = aeth_cdiv(m, G2_BM) * G2_BM, ntiles = aeth_cdiv(w->n, 16);
    // buffer offsets are 32-bit (the larger products take the dequantized DGEMM)
    if (ntiles * w->nb * 3072 >= INT32_MAX || mp * w->k * 4 >= INT32_MAX || mp > (1LL << 20)) return false;
    // AETH_Q6K_GEMM_ROWS=r takes the GEMM from r rows whatever the weight's size (tests; read once)
    static const int64_t env_rows = getenv("AETH_Q6K_GEMM_ROWS") ? atoll(getenv("AETH_Q6K_GEMM_ROWS")) : 0;
    if (env_rows > 0) return m >= env_rows;
    // The row-batched GEMV streams the weight once per row; the GEMM costs a near-constant
    // ≈ 31 µs (k = 4096) to 45 µs (k = 14336) up to 64 rows. Measured crossovers (HIP events,
    // rotated weight copies): 1024 × 4096 ≈ 53 rows, 4096 × 4096 ≈ 13, 4096 × 14336 and
    // 14336 × 4096 ≈ 5, i.e. where m · (weight bytes) reaches ≈ 200 MB.
    return m * w->nb * w->n * 210 >= 200000000LL;
}

bool aeth_q6k_gemm_fuses(const aeth_weight* w, int64_t m, int mode, const float* d_a, const float* norm_w) {
    if (m <= 1 || !aeth_q6k_gemm_rows(w, m)) return false;
    if (mode == PREP_PLAIN) return true;
    if (w->k > 16384 || ((uintptr_t)d_a & 15)) return false;  // one chunk of registers per wave, float4 loads
    if (mode == PREP_RMSNORM) return norm_w && ((uintptr_t)norm_w & 15) == 0;
    return mode == PREP_SWIGLU;
}

int aeth_gemm_q6k_launch(const aeth_weight* w, const float* d_a, int64_t m, float* d_c, unsigned flags,
                         hipStream_t s, int64_t ldc, const GemmIn* in) {
    if (!aeth_q6k_gemm_rows(w, m)) return aeth_set_error(AETH_EINVAL, "gemm q6_k: shape not taken (m=%lld)", (long long)m);
    const int mode = in ? in->mode : PREP_PLAIN;
    if (in && in->swiglu_out) return aeth_set_error(AETH_EINVAL, "gemm q6_k: no SwiGLU output");
    if (mode != PREP_PLAIN && !aeth_q6k_gemm_fuses(w, m, mode, d_a, in->norm_w))
        return aeth_set_error(AETH_EINVAL, "gemm q6_k: fused producer %d not available", mode);
    if (mode != PREP_PLAIN && (flags & AETH_MM_Q8_ACTIVATIONS))  // the producers feed the exact (f32) mode only
        return aeth_set_error(AETH_EINVAL, "gemm q6_k: fused producer %d with Q8 activations", mode);
    const int k = (int)w->k, nb = (int)w->nb;
    if (ldc <= 0) ldc = w->n;
    const int64_t mp = aeth_cdiv(m, G2_BM) * G2_BM;
    _Float16 *frag, *Sh;
    float* esc;
    int rc = gemm_prep(d_a, m, k, flags, in, s, nullptr, 0, frag, Sh, esc);
    if (rc) return rc;
    const int64_t ntiles = aeth_cdiv(w->n, 16), gm = mp / G2_BM, gn = aeth_cdiv(w->n, G2_BN);
    // K split over workgroups (split_plan; each wave keeps at least one super-block)
    SplitPlan P;
    if ((rc = split_plan(s, gm, gn, nb / 8, false, P))) return rc;
    Q6Args Q{(const uint8_t*)frag, esc, w->p0, w->p1, w->p2, (int)m, (int)w->n, k, nb, (int)ntiles, (int)mp,
             (int)gm, (int)gn, (int)(mp * k * 4), (int)(ntiles * nb * 3072), (int)(ntiles * nb * 256),
             (int)(ntiles * nb * 32), d_c, ldc, (flags & AETH_MM_ACCUMULATE) ? 1 : 0, 0,
             P.ksplit, P.part, (int)(gn * G2_BN), P.t_full, P.tsplit};
    return aeth_gemm_q6k_kq_launch(Q, s);
}

bool aeth_q80_gemm_rows(const aeth_weight* w, int64_t m) {
    if (!w || w->dtype != AETH_DTYPE_Q8_0 || w->order != AETH_ORDER_PLANAR || w->k != w->nb * 32 || m <= 1) return false;
    // a NaN or infinite block scale: the rescaled accumulator (U ← U·d_old/d_new) cannot carry
    // it (entering an infinite d zeroes U, the next one makes Inf·0 = NaN); q8_0.rs adds d·Σ per
    // block, as the GEMV does, so such weights stay on the GEMV
    if (w->special_scales) return false;
    const int64_t mp = aeth_cdiv(m, G2_BM) * G2_BM, ntiles = aeth_cdiv(w->n, 16), ngr = aeth_cdiv(w->nb, 4);
    if (ntiles * ngr * 2048 >= INT32_MAX || mp * w->k * 4 >= INT32_MAX || mp > (1LL << 20)) return false;
    // AETH_Q80_GEMM_ROWS=r takes the GEMM from r rows (tests and measurements; read once)
    static const int64_t env_rows = getenv("AETH_Q80_GEMM_ROWS") ? atoll(getenv("AETH_Q80_GEMM_ROWS")) : 0;
    if (env_rows > 0) return m >= env_rows;
    // The GEMM's cost is nearly flat in m (26.9 / 34.4 / 30.0 / 26.1 us for 4096 x 4096, 4096 x 14336,
    // 14336 x 4096, 1024 x 4096 at m = 2 ... 48); the row-batched GEMV adds one weight stream per row,
    // ~1.2 us for a weight the memory-side cache holds (17.8 MB) and ~8-12 us for 62 MB. Measured
    // crossovers: 4096 x 4096 at ~21 rows, 4096 x 14336 ~2.6, 14336 x 4096 ~3.5, 1024 x 4096 past 48.
    const int64_t bytes = w->nb * w->n * 34;
    return m >= 4096 || (m >= 3 && m * bytes >= (bytes <= (32LL << 20) ? 380000000LL : 180000000LL));
}

bool aeth_q80_gemm_fuses(const aeth_weight* w, int64_t m, int mode, const float* d_a, const float* norm_w) {
    if (!aeth_q80_gemm_rows(w, m)) return false;
    if (mode == PREP_PLAIN) return true;
    if (w->k > 16384 || ((uintptr_t)d_a & 15)) return false;  // one chunk of registers per wave, float4 loads
    if (mode == PREP_RMSNORM) return norm_w && ((uintptr_t)norm_w & 15) == 0;
    return mode == PREP_SWIGLU;
}

int aeth_gemm_q80_launch(const aeth_weight* w, const float* d_a, int64_t m, float* d_c, unsigned flags,
                         hipStream_t s, int64_t ldc, const GemmIn* in) {
    if (!aeth_q80_gemm_rows(w, m)) return aeth_set_error(AETH_EINVAL, "gemm q8_0: shape not taken (m=%lld)", (long long)m);
    const int mode = in ? in->mode : PREP_PLAIN;
    const bool swo = in && in->swiglu_out;
    if (mode != PREP_PLAIN && !aeth_q80_gemm_fuses(w, m, mode, d_a, in->norm_w))
        return aeth_set_error(AETH_EINVAL, "gemm q8_0: fused producer %d not available", mode);
    if (mode != PREP_PLAIN && (flags & AETH_MM_Q8_ACTIVATIONS))  // the producers feed the exact (f32) mode only
        return aeth_set_error(AETH_EINVAL, "gemm q8_0: fused producer %d with Q8 activations", mode);
    if (swo && ((w->n & 1) || (flags & AETH_MM_ACCUMULATE)))
        return aeth_set_error(AETH_EINVAL, "gemm q8_0: SwiGLU output needs even n, no accumulate");
    const int k = (int)w->k, nb = (int)w->nb;
    if (ldc <= 0) ldc = swo ? w->n / 2 : w->n;
    const int64_t mp = aeth_cdiv(m, G2_BM) * G2_BM;
    _Float16 *frag, *Sh;
    float* esc;
    int rc = gemm_prep(d_a, m, k, flags, in, s, nullptr, 0, frag, Sh, esc);
    if (rc) return rc;
    const int64_t ntiles = aeth_cdiv(w->n, 16), ngr = aeth_cdiv(nb, 4), gm = mp / G2_BM, gn = aeth_cdiv(w->n, G2_BN);
    // K split over workgroups (split_plan; each wave keeps 8 blocks at least, the 256 elements of a
    // K-quant super-block)
    SplitPlan P;
    if ((rc = split_plan(s, gm, gn, nb / 64, false, P))) return rc;
    Q80Args Q{(const uint8_t*)frag, esc, w->p0, w->p1, (int)m, (int)w->n, k, nb, (int)ngr, (int)ntiles, (int)mp,
              (int)gm, (int)gn, (int)(mp * k * 4), (int)(ntiles * ngr * 2048), (int)(ntiles * ngr * 128), d_c, ldc,
              (flags & AETH_MM_ACCUMULATE) ? 1 : 0, swo ? 1 : 0, P.ksplit, P.part, (int)(gn * G2_BN), P.t_full,
              P.tsplit};
    return aeth_gemm_q80_kq_launch(Q, s);
}

bool aeth_gemm_fused_ok(const aeth_weight* w, int64_t m, int mode, const float* d_a, const float* norm_w) {
    if (!w) return false;
    if (w->dtype == AETH_DTYPE_Q4_K || w->dtype == AETH_DTYPE_Q5_K) return aeth_gemm_fuses(w, m, mode, d_a, norm_w);
    if (w->dtype == AETH_DTYPE_Q6_K) return aeth_q6k_gemm_fuses(w, m, mode, d_a, norm_w);
    if (w->dtype == AETH_DTYPE_Q8_0) return aeth_q80_gemm_fuses(w, m, mode, d_a, norm_w);
    return false;
}

bool aeth_gemm_swo_ok(const aeth_weight* w, int64_t m) {
    if (!w) return false;
    if (w->dtype == AETH_DTYPE_Q4_K || w->dtype == AETH_DTYPE_Q5_K) return aeth_gemm_swiglu_out(w, m);
    return w->dtype == AETH_DTYPE_Q8_0 && (w->n & 1) == 0 && aeth_q80_gemm_rows(w, m);
}

int aeth_gemm_fused_launch(const aeth_weight* w, const float* d_a, int64_t m, float* d_c, unsigned flags,
                           hipStream_t s, int64_t ldc, const GemmIn* in) {
    if (w->dtype == AETH_DTYPE_Q4_K || w->dtype == AETH_DTYPE_Q5_K)
        return aeth_gemm_q4k_launch(w, d_a, m, d_c, flags, s, ldc, nullptr, 0, in);
    if (w->dtype == AETH_DTYPE_Q6_K) return aeth_gemm_q6k_launch(w, d_a, m, d_c, flags, s, ldc, in);
    if (w->dtype == AETH_DTYPE_Q8_0) return aeth_gemm_q80_launch(w, d_a, m, d_c, flags, s, ldc, in);
    return aeth_set_error(AETH_EINVAL, "gemm: no fused GEMM for dtype %d", w->dtype);
}
