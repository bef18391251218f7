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
    if (m > 65535 * 128) return aeth_set_error(AETH_EINVAL, "gemm: m too large");
    // workspace: Ah, Al [m][k], Sh, Sl [m][k/32] (fp16), escale [m] (f32)
    const size_t need = (size_t)m * k * 2 * 2 + (size_t)m * (k / 32) * 2 * 2 + (size_t)m * 4 + 256;
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
    _Float16* Al = Ah + (size_t)m * k;
    _Float16* Sh = Al + (size_t)m * k;
    _Float16* Sl = Sh + (size_t)m * (k / 32);
    float* esc = (float*)(Sl + (size_t)m * (k / 32));
    hipLaunchKernelGGL(k_gemm_prep, dim3((unsigned)m), dim3(256), 0, s, d_a, k, Ah, Al, Sh, Sl, esc);
    AETH_LAUNCH_CHECK();
    GemmArgs G{Ah, Al, Sh, Sl, esc, w->p0, w->p1, (int)m, (int)w->n, k, nb, d_c,
               (flags & AETH_MM_ACCUMULATE) ? 1 : 0};
    // tuning overrides, read once: AETH_GEMM_D (prefetch distance 1, 2 or 4), AETH_GEMM_BM (64 | 128)
    static const int env_d = getenv("AETH_GEMM_D") ? atoi(getenv("AETH_GEMM_D")) : 0;
    static const int env_bm = getenv("AETH_GEMM_BM") ? atoi(getenv("AETH_GEMM_BM")) : 0;
    // measured at m = 512, n = 4096 / 14336: BM = 64 with a one-step prefetch is
    // best (two workgroups per CU where the grid allows); AETH_GEMM_BM=128 forces
    // the 128-row tile
    if (env_bm == 128) {
        dim3 grid((unsigned)aeth_cdiv(w->n, GEMM_BN), (unsigned)aeth_cdiv(m, 128));
        if (env_d == 2) hipLaunchKernelGGL((k_gemm_q4k<128, 2>), grid, dim3(256), 0, s, G);
        else hipLaunchKernelGGL((k_gemm_q4k<128, 1>), grid, dim3(256), 0, s, G);
    } else {
        dim3 grid((unsigned)aeth_cdiv(w->n, GEMM_BN), (unsigned)aeth_cdiv(m, 64));
        if (env_d == 2) hipLaunchKernelGGL((k_gemm_q4k<64, 2>), grid, dim3(256), 0, s, G);
        else if (env_d == 4) hipLaunchKernelGGL((k_gemm_q4k<64, 4>), grid, dim3(256), 0, s, G);
        else hipLaunchKernelGGL((k_gemm_q4k<64, 1>), grid, dim3(256), 0, s, G);
    }
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}
