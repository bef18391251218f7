// Q6_K prefill GEMM (m rows from aeth_q6k_gemm_rows on):  C[m][n] = Σ_k A[m][k]·W[n][k]
// (avx2::matmul_q6_k with m rows, src/quant/avx2.rs:60-94; quantized_matmul_impl).
//
// The exact mode of the Q4_K GEMM: A·2^-e split into fp16 hi/lo MFMA fragments (k_gemm_prep
// in aeth_gemm.hip), f32 accumulation on v_mfma_f32_32x32x16_f16. A Q6_K weight is
// w = d·sc_s·(q − 32): d (f16) per 256-element super-block, sc_s (int8) per 16-element
// sub-block s, q ∈ [0, 63]. sc·(q − 32) needs 13 bits, more than an fp16 integer holds, so
// against A_hi it enters as two exact fp16 operands B1 = lo·(q − 32) and B2 = 16·hi·(q − 32),
// sc = 16·hi + lo (lo ∈ [0, 15], hi ∈ [−8, 7]; |B1| ≤ 480, B2 a multiple of 16 of at most
// 4096), and against A_lo (≤ 2^-11·|A|) as one operand Bs = fp16(sc·(q − 32)) (relative
// rounding ≤ 2^-11): three MFMA passes per product, each product within 2^-22·|A·w| of exact
// beyond the hi/lo split's own 2^-22.
// d enters per super-block through the rescaled accumulator of aeth_gemm_kq.hip: entering
// super-block b, U ← U·D_{b−1}/D_b (a zero d keeps the scale and zeroes the block's
// operands); the result is D_last·U. There is no min term.
//
// Work split as aeth_gemm_kq.hip: 64 × 128 workgroup tiles, 8 waves over eighths of the
// super-blocks, each filling a private 20 KiB LDS ring with direct-to-LDS buffer loads and
// waiting with its own vmcnt; no barrier until the 8 partial tiles meet in LDS.
//
// A 16-position slice is one sub-block. In the weight planes (aeth_weights.hip), lane
// (n, kg = 2h + g') of a 16-row tile holds for its row ql[64h + 16g', +16) (part 0),
// ql[64h + 32 + 16g', +16) (part 1) and qh[32h + 16g', +16) (part 2): byte i of them carries
// element i of the four sub-blocks s = 8h + g' + 2v (get_q6k, dequant.rs: v = 0 part 0's low
// nibble and qh bits 0-1, v = 1 part 1's low nibble and bits 2-3, v = 2 part 0's high nibble
// and bits 4-5, v = 3 part 1's high nibble and bits 6-7). A super-block's slices are taken in
// groups kg = 0..3 of four, v in the order 0, 2, 1, 3, so that a group reads part 0 and qh at
// its first slice and part 1 at its third: the 4 KiB group slot takes part 0 and qh for 128
// columns, is read into registers, then takes part 1, is read, then the next group's part 0
// and qh, each 2 slices ahead. The super-block's 16 scale bytes per column (2 KiB) and its d
// (256 B) pass through slots of their own, loaded a super-block ahead. Every load of the main
// loop is a direct-to-LDS buffer load (their order is the program order the vmcnt waits count).
#include <math.h>
#include <stdint.h>

#include "aeth_common.hpp"
#include "aeth_gemm_common.hpp"
#include "aeth_internal.hpp"

#define K6_A 4096                 // A fragments of a slice
#define K6_NA 3                   // A slots
#define K6_G 4096                 // group slot: [part 0 or 1 | qh][tile 8][row 16][16 B]
#define K6_S 2048                 // a super-block's scales: [tile 8][row 16][16 B]
#define K6_D 256                  // a super-block's d: [tile 8][row 16] (f16)
#define K6_GOFF (K6_NA * K6_A)    // group slot
#define K6_SOFF (K6_GOFF + K6_G)  // scale slot
#define K6_DOFF (K6_SOFF + K6_S)  // d slot
#define K6_WAVE (K6_DOFF + K6_D)  // LDS per wave: 18.25 KiB
#define K6_W 8

// slice position j of a super-block (group j / 4, p = j % 4): v = 0, 2, 1, 3 for p = 0..3
__host__ __device__ constexpr int k6_v(int j) { return (j & 3) == 1 ? 2 : (j & 3) == 2 ? 1 : (j & 3); }
__host__ __device__ constexpr int k6_sub(int j) { return 8 * (j >> 3) + ((j >> 2) & 1) + 2 * k6_v(j); }
// loads issued at position j after its A fragments: part 1 of the group at p = 0 (2), the next
// group's part 0 and qh at p = 2 (4), the next super-block's scales (2) and d (1) at j = 0
__host__ __device__ constexpr int k6_extra(int j) {
    return ((j & 3) == 0 ? 2 : 0) + ((j & 3) == 2 ? 4 : 0) + (j == 0 ? 3 : 0);
}
// loads allowed outstanding when position j starts: its A fragments must have landed, and at
// p = 0 / 2 also the group part issued after them at position j − 2 (its extras)
__host__ __device__ constexpr int k6_wait(int j) {
    return ((j & 3) == 0 || (j & 3) == 2) ? 4 + k6_extra((j + 15) & 15)
                                          : k6_extra((j + 14) & 15) + 4 + k6_extra((j + 15) & 15);
}

// two 8-byte reads, at a and a + 2048
__device__ __forceinline__ u32x4 lds_2b64_2k(uint32_t a) {
    u32x4 v;
    asm volatile("ds_read2st64_b64 %0, %1 offset1:4" : "=v"(v) : "v"(a));
    return v;
}

__global__ void __launch_bounds__(64 * K6_W) k_gemm_q6k_kq(Q6Args G) {
    __shared__ __attribute__((aligned(1024))) char smem[K6_W * K6_WAVE];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int tile, ks, nsplit, tm, tn;
    g2_work((int)blockIdx.x, G.gm, G.gn, G.ksplit, G.t_full, G.tsplit, tile, ks, nsplit);
    g2_tile(tile, G.gm, G.gn, tm, tn);
    const int n0 = tn * 128, m0 = tm * 64, t0 = n0 >> 4;
    const int nb = G.nb, nks = G.k >> 4;
    const int lo = nb * ks / nsplit, len = nb * (ks + 1) / nsplit - lo;  // this split's super-blocks
    const int sb0 = lo + len * wave / K6_W, nsb = lo + len * (wave + 1) / K6_W - sb0;
    char* wl = smem + wave * K6_WAVE;
    const uint32_t wl_lds = lds_addr(wl);

    // buffer resources; per-lane offsets fixed, per-load offsets in the scalar offset
    const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc((void*)G.frag, (short)0, G.a_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rQ = __builtin_amdgcn_make_buffer_rsrc((void*)G.q, (short)0, G.q_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rS = __builtin_amdgcn_make_buffer_rsrc((void*)G.sc, (short)0, G.s_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rD = __builtin_amdgcn_make_buffer_rsrc((void*)G.dd, (short)0, G.d_bytes, 0x00020000);
    // DMA lanes (16 B): lane → tile 4i + lane/16 of the workgroup's 8, row lane%16; the d DMA (4 B):
    // lane → tile lane/8, rows 2·(lane%8), +1. Tiles past the last are clamped (never stored).
    uint32_t gq_v[2], sv_v[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int t = min(t0 + 4 * i + (lane >> 4), G.ntiles - 1);
        gq_v[i] = (uint32_t)(t * nb * 3072 + (lane & 15) * 16);
        sv_v[i] = (uint32_t)((t * nb * 16 + (lane & 15)) * 16);
    }
    const uint32_t dv_v = (uint32_t)((min(t0 + (lane >> 3), G.ntiles - 1) * nb * 16 + 2 * (lane & 7)) * 2);
    const uint32_t a_v = (uint32_t)(lane * 16);
    const int aB0 = 2 * tm * nks * 2048, aB1 = (2 * tm + 1) * nks * 2048;  // A fragments of the two m-tiles
    // this lane's columns 32c + lane%32: tile 2c + (lane%32)/16, row lane%16; k half lane/32 of a slice
    int g_off[4], s_off[4], d_off[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const int tl = 2 * c + ((lane & 31) >> 4), r = lane & 15;
        g_off[c] = tl * 256 + r * 16 + 8 * (lane >> 5);
        s_off[c] = tl * 256 + r * 16;
        d_off[c] = (tl * 16 + r) * 2;
    }

    // A fragments of slice position j of super-block b, into A slot sa
    auto issueA = [&](int b, int j, int sa) {
        const int kso = b * 32768 + k6_sub(j) * 2048;
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int p = 0; p < 2; p++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, (lds_void*)(wl + sa + (mt * 2 + p) * 1024), 16, a_v,
                                                         (mt ? aB1 : aB0) + kso + p * 1024, 0, 0);
    };
    // part 0 and qh of group kg of super-block b (slot halves 0 / 1), or its part 1 (half 0)
    auto issueG0 = [&](int b, int kg) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rQ, (lds_void*)(wl + K6_GOFF + i * 1024), 16, gq_v[i & 1],
                                                     (3 * b + (i < 2 ? 0 : 2)) * 1024 + kg * 256, 0, 0);
    };
    auto issueG1 = [&](int b, int kg) {
#pragma unroll
        for (int i = 0; i < 2; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rQ, (lds_void*)(wl + K6_GOFF + i * 1024), 16, gq_v[i],
                                                     (3 * b + 1) * 1024 + kg * 256, 0, 0);
    };
    auto issueSD = [&](int b) {
#pragma unroll
        for (int i = 0; i < 2; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rS, (lds_void*)(wl + K6_SOFF + i * 1024), 16, sv_v[i], b * 256, 0,
                                                     0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rD, (lds_void*)(wl + K6_DOFF), 4, dv_v, b * 32, 0, 0);
    };

    f32x16 U[2][4];
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
        for (int c = 0; c < 4; c++) U[mt][c] = (f32x16){};
    float D[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    u32x4 scr[4] = {};  // this super-block's 16 scale bytes of each column
    uint32_t dq[4] = {};
    u32x2 rp0[4] = {}, rp1[4] = {}, rph[4] = {};  // this group's part 0 / part 1 / qh bytes of each column
    uint32_t c64;  // 0x64006400 in a VGPR (the OR's constant beside a VGPR operand)
    asm("v_mov_b32 %0, 0x64006400" : "=v"(c64));

    if (nsb > 0) {
        issueG0(sb0, 0);
        issueSD(sb0);
        issueA(sb0, 0, 0);
        issueA(sb0, 1, K6_A);
    }
    int s3 = 0;  // (16·bi) mod 3: slice position 16·bi + j uses A slot (s3 + j) mod 3
    for (int bi = 0; bi < nsb; bi++) {
        const int b = sb0 + bi;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const int p = j & 3, kg = j >> 2, v = k6_v(j), s = k6_sub(j);
            const int nw = k6_wait(j);  // 4, 6, 8 or 9 (folded: j is unrolled)
            if (nw == 9) vm_wait<9>();
            else if (nw == 8) vm_wait<8>();
            else if (nw == 6) vm_wait<6>();
            else vm_wait<4>();
            {
                int sl = s3 + (j + 2) % 3;
                sl = sl >= 3 ? sl - 3 : sl;
                // slices past the last super-block (the ring's tail, never read) load the last one's
                // again: every load stays inside its buffer, whatever part of the offset is range-checked
                issueA(j < 14 ? b : min(b + 1, nb - 1), (j + 2) & 15, sl * K6_A);
            }
            int sc3 = s3 + j % 3;
            sc3 = sc3 >= 3 ? sc3 - 3 : sc3;
            const uint32_t sa = wl_lds + sc3 * K6_A;
            if (j == 0) {  // the super-block's scales and d (read alone: their own wait)
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    scr[c] = lds_b128<0>(wl_lds + K6_SOFF + s_off[c]);
                    dq[c] = lds_u16<0>(wl_lds + K6_DOFF + d_off[c]);
                }
                lgkm_wait<0>();
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    pin(scr[c]);
                    pin(dq[c]);
                }
            }
            if (p == 0) {
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const u32x4 t = lds_2b64_2k(wl_lds + K6_GOFF + g_off[c]);
                    rp0[c] = (u32x2){t[0], t[1]};
                    rph[c] = (u32x2){t[2], t[3]};
                }
            } else if (p == 2) {
#pragma unroll
                for (int c = 0; c < 4; c++) rp1[c] = lds_b64<0>(wl_lds + K6_GOFF + g_off[c]);
            }
            half8_t a[2][2];  // [mt][part]
            a[0][0] = lds_b128h<0>(sa + a_v);
            a[0][1] = lds_b128h<1024>(sa + a_v);
            a[1][0] = lds_b128h<2048>(sa + a_v);
            a[1][1] = lds_b128h<3072>(sa + a_v);
            lgkm_wait<4>();  // all but the A fragments
            if (p == 0) {
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    pin(rp0[c]);
                    pin(rph[c]);
                }
                issueG1(b, kg);  // the slot is read: this group's part 1
            } else if (p == 2) {
#pragma unroll
                for (int c = 0; c < 4; c++) pin(rp1[c]);
                // the next group's part 0 and qh (past the last super-block: the last one's again, unread —
                // these weight loads stay inside the planes whatever the range check covers)
                if (kg < 3) issueG0(b, kg + 1);
                else issueG0(min(b + 1, nb - 1), 0);
            }
            if (j == 0) {
                // entering the super-block: rescale U to this block's d (a zero d keeps the scale;
                // its operands are zeroed through the scales)
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const float d = aeth_decode_d(dq[c]);
                    const float Dn = d != 0.0f ? d : D[c];
                    if ((dq[c] & 0x7FFFu) == 0u) scr[c] = (u32x4){0u, 0u, 0u, 0u};  // d = ±0
                    if (bi > 0) {
                        const float r = D[c] * __builtin_amdgcn_rcpf(Dn);
#pragma unroll
                        for (int mt = 0; mt < 2; mt++)
#pragma unroll
                            for (int q = 0; q < 16; q++) U[mt][c][q] *= r;
                    }
                    D[c] = Dn;
                }
                issueSD(min(b + 1, nb - 1));  // the slots are read: the next super-block's scales and d
            }
            // this slice's operands: B1 = lo·(q − 32), B2 = 16·hi·(q − 32), Bs = fp16(sc·(q − 32))
            // for sub-block s, k-order [0, 2, 1, 3] per 4 (the pairs of bytes (0, 2) and (1, 3) of
            // each dword, as the prep orders A); 0x64 | q is the half 1024 + q
            const half2_t k1056 = {(_Float16)-1056.0f, (_Float16)-1056.0f};
            auto build = [&](int c, half8_t& b1, half8_t& b2, half8_t& bs) {
                const int sc = (int)(int8_t)((scr[c][s >> 2] >> (8 * (s & 3))) & 0xFFu);
                const int lo = sc & 15;
                const _Float16 flo = (_Float16)(float)lo, fhi = (_Float16)(float)(sc - lo), fsc = (_Float16)(float)sc;
                const half2_t slo = {flo, flo}, shi = {fhi, fhi}, ssc = {fsc, fsc};
                const u32x2 P = (v & 1) ? rp1[c] : rp0[c];
                uint32_t w[2];
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    const uint32_t nib = v >= 2 ? (P[e] >> 4) & 0x0F0F0F0Fu : P[e] & 0x0F0F0F0Fu;
                    const uint32_t hb = 2 * v <= 4 ? (rph[c][e] << (4 - 2 * v)) & 0x30303030u
                                                   : (rph[c][e] >> (2 * v - 4)) & 0x30303030u;
                    w[e] = nib | hb;
                }
                half2_t x[4];
                x[0] = __builtin_bit_cast(half2_t, (w[0] & 0x00FF00FFu) | c64) + k1056;
                x[1] = __builtin_bit_cast(half2_t, ((w[0] >> 8) & 0x00FF00FFu) | c64) + k1056;
                x[2] = __builtin_bit_cast(half2_t, (w[1] & 0x00FF00FFu) | c64) + k1056;
                x[3] = __builtin_bit_cast(half2_t, ((w[1] >> 8) & 0x00FF00FFu) | c64) + k1056;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const half2_t y1 = x[i] * slo, y2 = x[i] * shi, y3 = x[i] * ssc;
                    b1[2 * i] = y1[0];
                    b1[2 * i + 1] = y1[1];
                    b2[2 * i] = y2[0];
                    b2[2 * i + 1] = y2[1];
                    bs[2 * i] = y3[0];
                    bs[2 * i + 1] = y3[1];
                }
            };
            // Column groups in turn: group c's eight MFMAs are issued between the VALU
            // instructions that build group c + 1's operands, so the dequantisation runs in the
            // shadow of the matrix core (the scheduling groups fix that interleave)
            half8_t b1[4], b2[4], bs[4];
            build(0, b1[0], b2[0], bs[0]);
            lgkm_wait<0>();
#pragma unroll
            for (int mt = 0; mt < 2; mt++) {
                pin(a[mt][0]);
                pin(a[mt][1]);
            }
#pragma unroll
            for (int c = 0; c < 4; c++) {
                __builtin_amdgcn_sched_barrier(0);
                if (c < 3) build(c + 1, b1[c + 1], b2[c + 1], bs[c + 1]);
#pragma unroll
                for (int h = 0; h < 3; h++)
#pragma unroll
                    for (int mt = 0; mt < 2; mt++)
                        U[mt][c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[mt][h == 2], h == 0 ? b1[c] : h == 1 ? b2[c] : bs[c],
                                                                          U[mt][c], 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 6; i++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                    __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // six VALU
                }
            }
        }
        s3 = s3 == 2 ? 0 : s3 + 1;
    }
    __builtin_amdgcn_s_waitcnt(0);  // the tail's loads have landed
    __syncthreads();                // and every wave is done with its ring

    // The eight K-eighth tiles meet in LDS as in aeth_gemm_kq.hip: waves 4..7 hand theirs to
    // waves 0..3, which write the pair sums; wave w sums (mt, c) = (w / 4, w % 4) in order.
    float* red = (float*)smem;  // [4][2][4][16][64] floats = 128 KiB
    const int mt = wave >> 2, c = wave & 3, lr = lane & 31;
    const int col = n0 + 32 * c + lr;
    int rows[16];
#pragma unroll
    for (int r = 0; r < 16; r++) rows[r] = m0 + 32 * mt + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
    G2Epi E;  // in flight during the reduction
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
        float* P = g2_part(G.part, ks, tile, G.t_full, G.tsplit, G.gm * G.gn, G.mp, G.pld, m0, n0, ld) +
                   32 * mt * ld + (col - n0);
#pragma unroll
        for (int r = 0; r < 16; r++) P[(int64_t)(rows[r] - m0 - 32 * mt) * ld] = sum[r];
    } else if (G.swiglu) {
#pragma unroll
        for (int r = 0; r < 16; r += 2) g2_store_swiglu(E, r, G.C, G.ldc, G.m, G.n, rows[r], col, sum[r], sum[r + 1]);
    } else {
#pragma unroll
        for (int r = 0; r < 16; r++) g2_store(E, r, G.C, G.ldc, G.m, G.n, rows[r], col, sum[r], G.accumulate);
    }
}

// Sum of the K splits, in split order, and the epilogue (SplitSum), for 4 columns of a row: the
// splits' partials at P, P + split, ... (float4 units).
__device__ __forceinline__ void split_sum_out(const SplitSum& G, const float4* P, int64_t split, int row, int col) {
    float4 v = P[0];
    for (int s = 1; s < G.ksplit; s++) {
        const float4 t = P[s * split];
        v.x += t.x;
        v.y += t.y;
        v.z += t.z;
        v.w += t.w;
    }
    const float e = G.escale[row];
    const float o[4] = {v.x * e, v.y * e, v.z * e, v.w * e};
    float* C = G.C + (int64_t)row * G.ldc;
    if (G.swiglu) {
#pragma unroll
        for (int j = 0; j < 4; j += 2)
            if (col + j + 1 < G.n) C[(col + j) >> 1] = o[j] * __builtin_amdgcn_rcpf(1.0f + expf(-o[j])) * o[j + 1];
    } else {
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (col + j < G.n) C[col + j] = G.accumulate ? C[col + j] + o[j] : o[j];
    }
}

// Every row of C: one thread per 4 columns of a row.
__global__ void __launch_bounds__(256) k_gemm_split_sum(SplitSum G) {
    const int q4 = G.pld >> 2;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)G.m * q4) return;
    const int row = (int)(i / q4), col = (int)(i - (int64_t)row * q4) * 4;
    if (col >= G.n) return;
    split_sum_out(G, (const float4*)(G.part + (int64_t)row * G.pld + col), (int64_t)G.mp * G.pld / 4, row, col);
}

// The tiles of a tail split only: 8 workgroups per 64 × 128 tile, one thread per 4 columns of a
// row, the tile found by the GEMM's own order (g2_tile).
__global__ void __launch_bounds__(256) k_gemm_tail_sum(SplitSum G) {
    const int tile = G.t_full + (int)blockIdx.x / 8, idx = ((int)blockIdx.x % 8) * 256 + (int)threadIdx.x;
    int tm, tn;
    g2_tile(tile, G.gm, G.gn, tm, tn);
    const int row = tm * 64 + (idx >> 5), col = tn * 128 + (idx & 31) * 4;
    if (row >= G.m || col >= G.n) return;
    const int ntail = G.gm * G.gn - G.t_full;
    const float* P = G.part + (int64_t)(tile - G.t_full) * (64 * 128) + (idx >> 5) * 128 + (idx & 31) * 4;
    split_sum_out(G, (const float4*)P, (int64_t)ntail * (64 * 128 / 4), row, col);
}

int aeth_gemm_split_sum_launch(const SplitSum& S, hipStream_t s) {
    if (S.gm > 0) {
        const int ntail = S.gm * S.gn - S.t_full;
        if (ntail <= 0) return AETH_OK;
        hipLaunchKernelGGL(k_gemm_tail_sum, dim3((unsigned)ntail * 8), dim3(256), 0, s, S);
        AETH_LAUNCH_CHECK();
        return AETH_OK;
    }
    const int64_t threads = (int64_t)S.m * (S.pld / 4);
    hipLaunchKernelGGL(k_gemm_split_sum, dim3((unsigned)aeth_cdiv(threads, 256)), dim3(256), 0, s, S);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}

int aeth_gemm_q6k_kq_launch(const Q6Args& G, hipStream_t s) {
    hipLaunchKernelGGL(k_gemm_q6k_kq, dim3(g2_grid(G)), dim3(64 * K6_W), 0, s, G);
    AETH_LAUNCH_CHECK();
    return g2_split_sum(G, s);
}
