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
#include <math.h>
#include <stdlib.h>

#include "aeth_common.hpp"
#include "aeth_internal.hpp"

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
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
        Ah[(int64_t)m * k + i] = h;
        Al[(int64_t)m * k + i] = (_Float16)(v - (float)h);
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
template <int BM>
__global__ void __launch_bounds__(256) k_gemm_q4k(GemmArgs G) {
    constexpr int TM = BM / 64;  // 32-row MFMA tiles per wave
    __shared__ __attribute__((aligned(16))) _Float16 sA[2][2][BM * GEMM_LDR];  // [buf][hi/lo]
    __shared__ __attribute__((aligned(16))) _Float16 sB[2][GEMM_BN * GEMM_LDR];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int n0 = blockIdx.x * GEMM_BN, m0 = blockIdx.y * BM;
    const int nb = G.nb;
    const int nsteps = nb * 4;

    // global → register staging for one K-step
    // A: BM rows × 64 halves × {hi, lo}: 16-byte pieces, 8 per row per part
    constexpr int A_PIECES = BM * 8 * 2;
    constexpr int A_PER_T = A_PIECES / 256;
    uint4 ra[A_PER_T];
    // B: 128 rows × one Q4_K unit (32 qs bytes): 2 threads per row, 16 bytes each
    uint4 rq;
    uint4 rh;
    const int brow = tid >> 1, bhalf = tid & 1;

    auto load_step = [&](int step) {
        const int b = step >> 2, j = step & 3;
#pragma unroll
        for (int i = 0; i < A_PER_T; i++) {
            const int p = tid + 256 * i;
            const int part = p / (BM * 8), rr = (p / 8) % BM, c = p % 8;
            const int row = m0 + rr;
            const _Float16* src = part ? G.Al : G.Ah;
            ra[i] = row < G.m ? *(const uint4*)(src + (int64_t)row * G.k + b * 256 + j * 64 + c * 8) : make_uint4(0, 0, 0, 0);
        }
        const int nrow = n0 + brow;
        if (nrow < G.n) {
            rq = *(const uint4*)(G.qs + aeth_q4k_qs_off(nrow, b, 32 * j + 16 * bhalf, nb));
            rh = *(const uint4*)(G.hdr + aeth_q4k_hdr_off(nrow, b, nb));
        } else {
            rq = make_uint4(0, 0, 0, 0);
            rh = make_uint4(0, 0, 0, 0);
        }
    };
    auto store_step = [&](int step, int buf) {
        const int j = step & 3;
#pragma unroll
        for (int i = 0; i < A_PER_T; i++) {
            const int p = tid + 256 * i;
            const int part = p / (BM * 8), rr = (p / 8) % BM, c = p % 8;
            *(uint4*)(&sA[buf][part][rr * GEMM_LDR + c * 8]) = ra[i];
        }
        // unit bytes [16·bhalf, 16·bhalf+16) of qs[32j .. 32j+32): byte l → low nibble
        // is element l (sub-block 2j), high nibble element 32 + l (sub-block 2j+1)
        int sc0, m_, sc1;
        k4_sm(rh, 2 * j, sc0, m_);
        k4_sm(rh, 2 * j + 1, sc1, m_);
        const uint32_t* qw = (const uint32_t*)&rq;
        _Float16 lo[16], hi[16];
#pragma unroll
        for (int t = 0; t < 16; t++) {
            const uint32_t byte = (qw[t >> 2] >> (8 * (t & 3))) & 0xFFu;
            lo[t] = (_Float16)(float)((int)(byte & 15u) * sc0);
            hi[t] = (_Float16)(float)((int)(byte >> 4) * sc1);
        }
        _Float16* dst = &sB[buf][brow * GEMM_LDR];
        *(half8_t*)(dst + bhalf * 16) = *(half8_t*)&lo[0];
        *(half8_t*)(dst + bhalf * 16 + 8) = *(half8_t*)&lo[8];
        *(half8_t*)(dst + 32 + bhalf * 16) = *(half8_t*)&hi[0];
        *(half8_t*)(dst + 32 + bhalf * 16 + 8) = *(half8_t*)&hi[8];
    };

    f32x16 acc[TM][2], part[TM][2];
#pragma unroll
    for (int a = 0; a < TM; a++)
#pragma unroll
        for (int c = 0; c < 2; c++) {
            acc[a][c] = (f32x16){};
            part[a][c] = (f32x16){};
        }

    load_step(0);
    store_step(0, 0);
    __syncthreads();
    const int lr = lane & 31, lk = (lane >> 5) * 8;
    for (int step = 0; step < nsteps; step++) {
        const int buf = step & 1;
        if (step + 1 < nsteps) load_step(step + 1);
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
        if ((step & 3) == 3) {
            // super-block done: C += d·P − dmin·Q, Q = Σ_s m_s·S_s (hi/lo) by one MFMA per tile
            const int b = step >> 2;
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const int col = n0 + wn * 64 + c * 32 + lr;
                uint4 h = make_uint4(0, 0, 0, 0);
                if (col < G.n) h = *(const uint4*)(G.hdr + aeth_q4k_hdr_off(col, b, nb));
                const float d = aeth_decode_d(h.x), dmin = aeth_decode_d(h.x >> 16);
                half8_t mv;
#pragma unroll
                for (int s = 0; s < 8; s++) {
                    int scv, mm;
                    k4_sm(h, s, scv, mm);
                    mv[s] = (_Float16)(float)mm;
                }
#pragma unroll
                for (int a = 0; a < TM; a++) {
                    const int row = m0 + wm * (BM / 2) + a * 32 + lr;
                    half8_t sv = (half8_t){};
                    if (row < G.m) sv = *(const half8_t*)((lk ? G.Sl : G.Sh) + (int64_t)row * (G.k / 32) + b * 8);
                    f32x16 q = __builtin_amdgcn_mfma_f32_32x32x16_f16(sv, mv, (f32x16){}, 0, 0, 0);
                    // S was scaled by 2^-(e+5) against A's 2^-e: fold the 2^5 into dmin
                    const float dm = dmin * 32.0f;
#pragma unroll
                    for (int r = 0; r < 16; r++) acc[a][c][r] += d * part[a][c][r] - dm * q[r];
                    part[a][c] = (f32x16){};
                }
            }
        }
        if (step + 1 < nsteps) {
            store_step(step + 1, buf ^ 1);
            __syncthreads();
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
    const int64_t tiles128 = aeth_cdiv(w->n, GEMM_BN) * aeth_cdiv(m, 128);
    if (tiles128 >= aeth_num_cus()) {
        dim3 grid((unsigned)aeth_cdiv(w->n, GEMM_BN), (unsigned)aeth_cdiv(m, 128));
        hipLaunchKernelGGL(k_gemm_q4k<128>, grid, dim3(256), 0, s, G);
    } else {
        dim3 grid((unsigned)aeth_cdiv(w->n, GEMM_BN), (unsigned)aeth_cdiv(m, 64));
        hipLaunchKernelGGL(k_gemm_q4k<64>, grid, dim3(256), 0, s, G);
    }
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}
