// Q8_0 prefill GEMM (m rows from aeth_q80_gemm_rows on):  C[m][n] = Σ_k A[m][k]·W[n][k]
// (matmul_q8_0 with m rows, src/quant/matmul/q8_0.rs:5-89; quantized_matmul_impl).
//
// The exact mode of the Q4_K GEMM: A·2^-e split into fp16 hi/lo MFMA fragments (k_gemm_prep in
// aeth_gemm.hip), f32 accumulation on v_mfma_f32_32x32x16_f16, two passes per product. A Q8_0
// weight is w = d·q: d (f16) per 32-element block, q ∈ [−128, 127] an exact fp16 operand. d enters
// through the rescaled accumulator, here once per block: entering block b, U ← U·D_{b−1}/D_b, the
// block's two slices add Σ A·q, and the result is D_last·U (a zero d keeps the scale and zeroes
// the block's operands).
//
// Work split as aeth_gemm_q6k.hip: 64 × 128 workgroup tiles, 8 waves over eighths of the blocks
// (and K over several workgroups when the tiles are few), each wave filling a private LDS ring with
// direct-to-LDS buffer loads and waiting with its own vmcnt. A 16-position slice is half a block.
// In the weight planes (aeth_weights.hip) the 16 quants of (row n, block b, half hf) are the 16
// bytes of lane n + 16·(2·(b & 1) + hf) in the 1 KiB piece (tile, group b/4, pair (b/2) & 1): a
// slice of the workgroup's 8 tiles is 8 contiguous 256-byte runs (2 KiB), loaded two slices
// ahead; the 16 rows' d of a block are 32 contiguous bytes per tile (one 4-byte load per lane), a
// block ahead. Every load of the main loop is a direct-to-LDS buffer load, so program order is the
// order the vmcnt waits count; loads past the wave's last block re-read the last block.
#include <math.h>
#include <stdint.h>

#include "aeth_common.hpp"
#include "aeth_gemm_common.hpp"
#include "aeth_internal.hpp"

#define K0_A 4096                            // A fragments of a slice
#define K0_B 2048                            // quants of a slice: [tile 8][row 16][16 B]
#define K0_D 256                             // d of a block: [tile 8][row 16] (f16)
#define K0_NS 3                              // A and quant slots
#define K0_BOFF (K0_NS * K0_A)               // quant slots
#define K0_DOFF (K0_BOFF + K0_NS * K0_B)     // d slots (2)
#define K0_WAVE (K0_DOFF + 2 * K0_D)         // LDS per wave: 18.5 KiB
#define K0_W 8

__global__ void __launch_bounds__(64 * K0_W) k_gemm_q80_kq(Q80Args G) {
    __shared__ __attribute__((aligned(1024))) char smem[K0_W * K0_WAVE];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int tile, ks, nsplit, tm, tn;
    g2_work((int)blockIdx.x, G.gm, G.gn, G.ksplit, G.t_full, G.tsplit, tile, ks, nsplit);
    g2_tile(tile, G.gm, G.gn, tm, tn);
    const int n0 = tn * 128, m0 = tm * 64, t0 = n0 >> 4;
    const int nb = G.nb, nks = G.k >> 4;
    const int lo = nb * ks / nsplit, len = nb * (ks + 1) / nsplit - lo;  // this split's blocks
    const int b0 = lo + len * wave / K0_W, nbw = lo + len * (wave + 1) / K0_W - b0;
    char* wl = smem + wave * K0_WAVE;
    const uint32_t wl_lds = lds_addr(wl);

    const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc((void*)G.frag, (short)0, G.a_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rQ = __builtin_amdgcn_make_buffer_rsrc((void*)G.q, (short)0, G.q_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rD = __builtin_amdgcn_make_buffer_rsrc((void*)G.dd, (short)0, G.d_bytes, 0x00020000);
    // DMA lanes (16 B): lane → tile 4i + lane/16 of the workgroup's 8, row lane%16; the d DMA (4 B):
    // lane → tile lane/8, rows 2·(lane%8), +1. Tiles past the last are clamped (never stored).
    uint32_t q_v[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int t = min(t0 + 4 * i + (lane >> 4), G.ntiles - 1);
        q_v[i] = (uint32_t)(t * G.ngr * 2048 + (lane & 15) * 16);
    }
    const uint32_t dv_v = (uint32_t)((min(t0 + (lane >> 3), G.ntiles - 1) * G.ngr * 64 + 2 * (lane & 7)) * 2);
    const uint32_t a_v = (uint32_t)(lane * 16);
    const int aB0 = 2 * tm * nks * 2048, aB1 = (2 * tm + 1) * nks * 2048;  // A fragments of the two m-tiles
    // this lane's columns 32c + lane%32: tile 2c + (lane%32)/16, row lane%16; k half lane/32 of a slice
    int q_off[4], d_off[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const int tl = 2 * c + ((lane & 31) >> 4), r = lane & 15;
        q_off[c] = tl * 256 + r * 16 + 8 * (lane >> 5);
        d_off[c] = (tl * 16 + r) * 2;
    }

    // slice s = 2b + hf of the weight (b clamped to the last block): A fragments, quants
    auto issueS = [&](int b, int hf, int slot) {
        const int kso = (2 * b + hf) * 2048;
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int p = 0; p < 2; p++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, (lds_void*)(wl + slot * K0_A + (mt * 2 + p) * 1024), 16, a_v,
                                                         (mt ? aB1 : aB0) + kso + p * 1024, 0, 0);
        const int qso = ((b >> 2) * 2 + ((b >> 1) & 1)) * 1024 + (2 * (b & 1) + hf) * 256;
#pragma unroll
        for (int i = 0; i < 2; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rQ, (lds_void*)(wl + K0_BOFF + slot * K0_B + i * 1024), 16, q_v[i],
                                                     qso, 0, 0);
    };
    auto issueD = [&](int b, int slot) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rD, (lds_void*)(wl + K0_DOFF + slot * K0_D), 4, dv_v,
                                                 ((b >> 2) * 4 + (b & 3)) * 32, 0, 0);
    };

    f32x16 U[2][4];
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
        for (int c = 0; c < 4; c++) U[mt][c] = (f32x16){};
    float D[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    uint32_t zm[4] = {0u, 0u, 0u, 0u};  // all ones where this block's d is zero (its operands are zeroed)
    uint32_t c64;  // 0x64646464 in a VGPR (the perm's constant byte source)
    asm("v_mov_b32 %0, 0x64646464" : "=v"(c64));
    const half2_t k1152 = {(_Float16)-1152.0f, (_Float16)-1152.0f};

    if (nbw > 0) {  // prologue: d of the first block, then slices 0 and 1
        issueD(b0, 0);
        issueS(b0, 0, 0);
        issueS(b0, 1, 1);
    }
    int s3 = 0;  // (2·bi) mod 3: slice 2·bi + hf uses slot (s3 + hf) mod 3
    for (int bi = 0; bi < nbw; bi++) {
        const int b = b0 + bi;
#pragma unroll
        for (int hf = 0; hf < 2; hf++) {
            // slice hf = 0 needs this block's d (issued last two slices ago: one slice's 6 loads since),
            // hf = 1 its A and quants (then the d of the next block and the 6 loads of slice hf = 0 since)
            if (hf == 0) vm_wait<6>();
            else vm_wait<7>();
            {  // slice + 2: the next block's slice hf, and at hf = 0 the next block's d
                int sl = s3 + (hf + 2) % 3;
                sl = sl >= 3 ? sl - 3 : sl;
                const int bn = min(b + 1, nb - 1);
                issueS(bn, hf, sl);
                if (hf == 0) issueD(bn, (bi + 1) & 1);
            }
            int sc3 = s3 + hf;
            sc3 = sc3 >= 3 ? sc3 - 3 : sc3;
            const uint32_t sa = wl_lds + sc3 * K0_A, sq = wl_lds + K0_BOFF + sc3 * K0_B;
            uint32_t dq[4];
            if (hf == 0) {
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    asm volatile("ds_read_u16 %0, %1" : "=v"(dq[c]) : "v"(wl_lds + K0_DOFF + (bi & 1) * K0_D + d_off[c]));
                }
            }
            u32x2 qw[4];
#pragma unroll
            for (int c = 0; c < 4; c++) qw[c] = lds_b64<0>(sq + q_off[c]);
            half8_t a[2][2];  // [mt][part]
            a[0][0] = lds_b128h<0>(sa + a_v);
            a[0][1] = lds_b128h<1024>(sa + a_v);
            a[1][0] = lds_b128h<2048>(sa + a_v);
            a[1][1] = lds_b128h<3072>(sa + a_v);
            lgkm_wait<4>();  // all but the A fragments
#pragma unroll
            for (int c = 0; c < 4; c++) pin(qw[c]);
            if (hf == 0) {
                // entering the block: rescale U to this block's d (a zero d keeps the scale; its
                // operands are zeroed for both slices)
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    pin(dq[c]);
                    const float d = aeth_f16_to_f32(dq[c] & 0xFFFFu);
                    const bool z = (dq[c] & 0x7FFFu) == 0u;
                    zm[c] = z ? 0xFFFFFFFFu : 0u;
                    const float Dn = z ? D[c] : d;
                    if (bi > 0) {
                        const float r = D[c] * __builtin_amdgcn_rcpf(Dn);
#pragma unroll
                        for (int mt = 0; mt < 2; mt++)
#pragma unroll
                            for (int q = 0; q < 16; q++) U[mt][c][q] *= r;
                    }
                    D[c] = Dn;
                }
            }
            // operands q as exact halves, k-order [0, 2, 1, 3] per 4 (bytes (0, 2) and (1, 3) of each
            // dword, as the prep orders A): q + 128 as 0x64 | byte is the half 1152 + q; a zero-d block's
            // quants are masked to 0 first (byte 0x80 after the flip, the half 0)
            auto build = [&](int c, half8_t& bq) {
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    const uint32_t w = (qw[c][e] & ~zm[c]) ^ 0x80808080u;
                    const half2_t x0 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(c64, w, 0x04020400u)) + k1152;
                    const half2_t x1 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(c64, w, 0x04030401u)) + k1152;
                    bq[4 * e] = x0[0];
                    bq[4 * e + 1] = x0[1];
                    bq[4 * e + 2] = x1[0];
                    bq[4 * e + 3] = x1[1];
                }
            };
            half8_t bq[4];
            build(0, bq[0]);
            lgkm_wait<0>();
#pragma unroll
            for (int mt = 0; mt < 2; mt++) {
                pin(a[mt][0]);
                pin(a[mt][1]);
            }
#pragma unroll
            for (int c = 0; c < 4; c++) {
                __builtin_amdgcn_sched_barrier(0);
                if (c < 3) build(c + 1, bq[c + 1]);
#pragma unroll
                for (int pa = 0; pa < 2; pa++)
#pragma unroll
                    for (int mt = 0; mt < 2; mt++)
                        U[mt][c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[mt][pa], bq[c], U[mt][c], 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                    __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // three VALU
                }
            }
        }
        s3 = s3 == 0 ? 2 : s3 - 1;  // (s3 + 2) mod 3
    }
    __builtin_amdgcn_s_waitcnt(0);  // the tail's loads have landed
    __syncthreads();                // and every wave is done with its ring

    // the eight K-eighth tiles meet in LDS as in aeth_gemm_kq.hip
    float* red = (float*)smem;  // [4][2][4][16][64] floats = 128 KiB
    const int mt = wave >> 2, c = wave & 3, lr = lane & 31;
    const int col = n0 + 32 * c + lr;
    int rows[16];
#pragma unroll
    for (int r = 0; r < 16; r++) rows[r] = m0 + 32 * mt + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
    G2Epi E;
    if (nsplit == 1) g2_epi_load(E, G.escale, G.C, G.ldc, G.m, G.n, rows, col, G.accumulate);
#pragma unroll
    for (int q = 0; q < 2; q++)
#pragma unroll
        for (int cc = 0; cc < 4; cc++)
#pragma unroll
            for (int r = 0; r < 16; r++) U[q][cc][r] *= D[cc];
    if (wave >= 4) {
#pragma unroll
        for (int q = 0; q < 2; q++)
#pragma unroll
            for (int cc = 0; cc < 4; cc++)
#pragma unroll
                for (int r = 0; r < 16; r++) red[((((wave - 4) * 2 + q) * 4 + cc) * 16 + r) * 64 + lane] = U[q][cc][r];
    }
    __syncthreads();
    if (wave < 4) {
#pragma unroll
        for (int q = 0; q < 2; q++)
#pragma unroll
            for (int cc = 0; cc < 4; cc++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int i = (((wave * 2 + q) * 4 + cc) * 16 + r) * 64 + lane;
                    red[i] = U[q][cc][r] + red[i];
                }
    }
    __syncthreads();
    float sum[16];
#pragma unroll
    for (int r = 0; r < 16; r++) {
        sum[r] = red[(((0 * 2 + mt) * 4 + c) * 16 + r) * 64 + lane];
#pragma unroll
        for (int w = 1; w < 4; w++) sum[r] += red[(((w * 2 + mt) * 4 + c) * 16 + r) * 64 + lane];
    }
    if (nsplit > 1) {  // the split's partial tile (rows < mp, columns < pld: no bounds to check)
        int ld;
        float* P = g2_part(G.part, ks, tile, G.t_full, G.tsplit, G.gm * G.gn, G.mp, G.pld, m0, n0, ld) + (col - n0);
#pragma unroll
        for (int r = 0; r < 16; r++) P[(int64_t)(rows[r] - m0) * ld] = sum[r];
    } else if (G.swiglu) {
#pragma unroll
        for (int r = 0; r < 16; r += 2) g2_store_swiglu(E, r, G.C, G.ldc, G.m, G.n, rows[r], col, sum[r], sum[r + 1]);
    } else {
#pragma unroll
        for (int r = 0; r < 16; r++) g2_store(E, r, G.C, G.ldc, G.m, G.n, rows[r], col, sum[r], G.accumulate);
    }
}

int aeth_gemm_q80_kq_launch(const Q80Args& G, hipStream_t s) {
    hipLaunchKernelGGL(k_gemm_q80_kq, dim3(g2_grid(G)), dim3(64 * K0_W), 0, s, G);
    AETH_LAUNCH_CHECK();
    return g2_split_sum(G, s);
}
