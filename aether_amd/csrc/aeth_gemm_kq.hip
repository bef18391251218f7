// Q4_K and Q5_K prefill GEMM, K-split form (m > 1):  C[m][n] = Σ_k A[m][k]·W[n][k]
// (avx2::matmul_q4_k with m rows, src/quant/avx2.rs:23-57; quantized_matmul_impl).
//
// Operands as in the exact mode of aeth_gemm.hip: A·2^-e split into fp16 hi/lo
// MFMA fragments (k_gemm_prep), weights as exact fp16 integers q·sc, f32
// accumulation on v_mfma_f32_32x32x16_f16; the mins enter per super-block through
// the sub-block sums S (one more MFMA, k = 8 sub-blocks × {hi, lo}).
//
// Work split. A workgroup owns a 64 × 128 tile of C and has 8 waves, two per
// SIMD; wave w computes the whole tile over the w-th eighth of the super-blocks.
// A wave so holds 2 m-tiles × 4 column tiles of accumulators: every A fragment it
// reads feeds 4 MFMAs and every dequantised weight fragment 4 (2 m-tiles × {hi,
// lo}). The waves share no data: each streams its own A fragments, quants,
// headers and sub-block sums into a private LDS ring with direct-to-LDS buffer
// loads and waits for them with its own vmcnt, so the main loop has no barrier;
// the two waves of a SIMD cover each other's waits. The eight partial tiles meet
// in LDS at the end and are summed in a fixed order (deterministic).
//
// One accumulator per output. A column's contribution of super-block b is
// d_b·P_b − 32·dmin_b·Q_b (P_b = Σ A·(q·sc) from the MFMAs, Q_b = Σ_s m_s·S_s).
// Instead of a separate P_b per super-block the accumulator U holds the running
// sum in units of the current scale D_b (= d_b; a zero d_b keeps the previous
// scale and zeroes the super-block's weight operands): entering b, U ← U·D_{b-1}/D_b
// (one multiply per output), the MFMAs then add P_b in place, and leaving b,
// U ← U + (−32·dmin_b/D_b)·Q_b; the result is D_last·U. The rescaling rounds once
// per super-block, at the level of the running sum, like the f32 sum it replaces.
//
// Ring. A slice is 16 K positions: 4 A fragments of 1 KiB (2 m-tiles × {hi, lo}).
// Two consecutive slices read the low and the high nibbles of the same quant
// bytes qs[32J + 16kg, +16) (128 rows × 16 B = 2 KiB, loaded with the first).
// A super-block's first slice also loads its headers (128 × 16 B) and the 64
// rows' sub-block sums (2 KiB), which the wave copies to registers when it starts
// the super-block. Per wave: 3 A slots, 2 quant slots, 1 header slot (20 KiB);
// slice s + 2 is issued before slice s is computed.
//
// Q5_K (avx2::matmul_q5_k with m rows, src/quant/avx2.rs:97-131) runs the same kernel with a
// fifth bit per quant: w = d·sc·(q + 16·h) − dmin·m, h bit 32·s + l of the block's qh for
// element l of sub-block s (q5_k.rs:49-56). q5·sc ≤ 1953 is still an exact fp16 integer, so
// the two MFMA passes and the min term are Q4_K's. The GEMM's fifth-bit plane (p3,
// aeth_weights.hip) holds per 16-row tile and super-block [J 4][kg 2][row 16][half 2] 16-bit
// words: the bits of the 8 elements a lane takes in the slice pair (J, kg), arranged for
// dq8s5; a slice pair's words for the workgroup's 128 columns (512 B) ride in its quant slot.
// The LDS they need comes from the header slot: the sub-block sums go to registers instead
// (loaded a super-block ahead, after the last slice used them). Per wave: 3 A slots, 2 quant
// slots of 2.5 KiB, 1 header slot of 2 KiB (19 KiB).
#include <math.h>
#include <stdint.h>

#include "aeth_common.hpp"
#include "aeth_gemm_common.hpp"
#include "aeth_internal.hpp"

#define K8_A 4096   // A fragments of a slice
#define K8_NA 3     // A slots
#define K8_W 8      // waves

// LDS of a wave: A slots, the quant slots of a slice pair (Q5_K: + its fifth bits), the
// header slot of a super-block (Q4_K: + its sub-block sums)
template <bool Q5>
struct K8L {
    static constexpr int B = Q5 ? 2560 : 2048;
    static constexpr int HS = Q5 ? 2048 : 4096;
    static constexpr int BOFF = K8_NA * K8_A;
    static constexpr int HOFF = BOFF + 2 * B;
    static constexpr int WAVE = HOFF + HS;  // 20 KiB (Q4_K), 19 KiB (Q5_K)
};

// buffer loads issued for slice s (s = position in the wave's run): A fragments, a pair's quants
// (Q5_K: and fifth bits), a super-block's headers (Q4_K: and sums)
template <bool Q5>
__host__ __device__ constexpr int k8_loads(int s) {
    return 4 + ((s & 1) == 0 ? (Q5 ? 4 : 2) : 0) + ((s & 15) == 0 ? (Q5 ? 2 : 4) : 0);
}
// loads allowed outstanding when slice position j starts: slice j + 1's, and at j = 0 (Q5_K) the
// two sub-block-sum loads issued after it, at the end of the previous super-block
template <bool Q5>
__host__ __device__ constexpr int k8_wait(int j) {
    return k8_loads<Q5>(j + 1) + (Q5 && j == 0 ? 2 : 0);
}

template <bool Q5>
__global__ void __launch_bounds__(64 * K8_W) k_gemm_kq(KqArgs G) {
    using L = K8L<Q5>;
    __shared__ __attribute__((aligned(1024))) char smem[K8_W * L::WAVE];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int tile, ks, nsplit, tm, tn;
    g2_work((int)blockIdx.x, G.gm, G.gn, G.ksplit, G.t_full, G.tsplit, tile, ks, nsplit);
    g2_tile(tile, G.gm, G.gn, tm, tn);
    const int n0 = tn * 128, m0 = tm * 64, t0 = n0 >> 4;
    const int nb = G.nb, nks = G.k >> 4, ksb = G.k >> 5;
    const int lo = nb * ks / nsplit, len = nb * (ks + 1) / nsplit - lo;  // this split's super-blocks
    const int sb0 = lo + len * wave / K8_W, nsb = lo + len * (wave + 1) / K8_W - sb0, ns = 16 * nsb;
    char* wl = smem + wave * L::WAVE;
    const uint32_t wl_lds = lds_addr(wl);

    // buffer resources; per-lane offsets are fixed, per-slice offsets go in the scalar offset
    const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc((void*)G.frag, (short)0, G.a_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rS = __builtin_amdgcn_make_buffer_rsrc((void*)G.sums, (short)0, G.s_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rQ = __builtin_amdgcn_make_buffer_rsrc((void*)G.qs, (short)0, G.q_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rH = __builtin_amdgcn_make_buffer_rsrc((void*)G.hdr, (short)0, G.h_bytes, 0x00020000);
    // DMA piece i (i = 0, 1) of quants / headers: lane → row tile 4i + lane/16 of the workgroup's 8, row lane%16
    uint32_t q_v[2], h_v[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int t = min(t0 + 4 * i + (lane >> 4), G.ntiles - 1);  // tiles past the last: clamped, never stored
        q_v[i] = (uint32_t)(t * nb * 2048 + (lane & 15) * 16);
        h_v[i] = (uint32_t)(t * nb * 256 + (lane & 15) * 16);
    }
    // sub-block sums of m-tile mt: lane → row m0 + 32mt + lane%32, hi (lane < 32) or lo
    uint32_t s_v[2];
#pragma unroll
    for (int mt = 0; mt < 2; mt++) {
        const int row = min(m0 + 32 * mt + (lane & 31), G.mp - 1);
        s_v[mt] = (uint32_t)(((lane >> 5) * G.mp * ksb + row * ksb) * 2);
    }
    const uint32_t a_v = (uint32_t)(lane * 16);
    // Q5_K fifth bits, DMA piece i (4 B): lane → tile 4i + lane/16 of the workgroup's 8, row
    // lane%16 (both halves' words), at q_v[i] / 4
    __amdgpu_buffer_rsrc_t rF = rQ;
    if constexpr (Q5) rF = __builtin_amdgcn_make_buffer_rsrc((void*)G.fifth, (short)0, G.f_bytes, 0x00020000);

    // Loads of slice s = 16·(b − sb0) + jl of this wave, into A slot sa (a byte
    // offset in the wave's LDS). Offsets are a per-super-block scalar base plus
    // constants (jl is known at compile time). Slices past the run (the ring's
    // tail) read whatever lies beyond it: the next K range's data, or zeros past
    // a buffer's extent (buffer loads check it); their slots are never read.
    const int aB0 = 2 * tm * nks * 2048, aB1 = (2 * tm + 1) * nks * 2048;  // A fragments of the two m-tiles
    auto issue = [&](int b, int jl, int sa) {
        const int J = jl >> 2, kg = (jl >> 1) & 1, nib = jl & 1;
        const int kso = b * 32768 + (4 * J + 2 * nib + kg) * 2048;
        char* st = wl + sa;
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int p = 0; p < 2; p++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rA, (lds_void*)(st + (mt * 2 + p) * 1024), 16, a_v,
                                                         (mt ? aB1 : aB0) + kso + p * 1024, 0, 0);
        if ((jl & 1) == 0) {
            char* sq = wl + L::BOFF + ((jl >> 1) & 1) * L::B;
            const int qoff = b * 2048 + (J >> 1) * 1024 + (2 * (J & 1) + kg) * 256;
#pragma unroll
            for (int i = 0; i < 2; i++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rQ, (lds_void*)(sq + i * 1024), 16, q_v[i], qoff, 0, 0);
            if constexpr (Q5) {
                const int foff = b * 512 + (2 * J + kg) * 64;
#pragma unroll
                for (int i = 0; i < 2; i++)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rF, (lds_void*)(sq + 2048 + i * 256), 4, q_v[i] >> 2, foff, 0,
                                                             0);
            }
        }
        if (jl == 0) {
            char* hs = wl + L::HOFF;
#pragma unroll
            for (int i = 0; i < 2; i++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rH, (lds_void*)(hs + i * 1024), 16, h_v[i], b * 256, 0, 0);
            if constexpr (!Q5) {
#pragma unroll
                for (int mt = 0; mt < 2; mt++)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rS, (lds_void*)(hs + 2048 + mt * 1024), 16, s_v[mt],
                                                             b * 16, 0, 0);
            }
        }
    };
    // Q5_K: the sub-block sums of super-block b straight into registers
    auto load_sums = [&](int b, half8_t* sv) {
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
            sv[mt] = __builtin_bit_cast(half8_t, __builtin_amdgcn_raw_buffer_load_b128(rS, s_v[mt], b * 16, 0));
    };

    // LDS offsets of column tile 0: quants of lane (col, k-group lane/32), header of col (column
    // tile c: + 512c)
    const int h_off = ((lane & 31) >> 4) * 256 + (lane & 15) * 16, b_off = h_off + 8 * (lane >> 5);
    // Q5_K: this lane's fifth-bit word of column tile c in a quant slot: + 2048 + 128c
    const int f_off = (lane & 31) * 4 + 2 * (lane >> 5);

    f32x16 U[2][4];
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
        for (int c = 0; c < 4; c++) U[mt][c] = (f32x16){};
    float D[4] = {1.0f, 1.0f, 1.0f, 1.0f};  // current scale of column tile c (this lane's column)
    u32x4 hd[4] = {};
    half8_t sv[2] = {};
    half2_t sp[4] = {}, zp[4] = {};
    u32x2 raw[4] = {};
    uint32_t x8[4] = {}, y8[4] = {};
    uint32_t P5[4] = {};  // Q5_K: this slice pair's fifth bits of each column (dq8s5)
    uint32_t c64;  // 0x64006400 in a VGPR (see dq8s)
    asm("v_mov_b32 %0, 0x64006400" : "=v"(c64));

    if (ns > 0) {
        issue(sb0, 0, 0);
        issue(sb0, 1, K8_A);
        if constexpr (Q5) load_sums(sb0, sv);
    }
    int s3 = 0;  // (16·bi) mod 3: slice 16·bi + j uses A slot (s3 + j) mod 3
    for (int bi = 0; bi < nsb; bi++) {
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const int nib = j & 1;
            // slice s has landed when only slice s + 1's loads (and at j = 0 the sums, Q5_K) are
            // outstanding
            const int nw = k8_wait<Q5>(j);  // 4, 6, 8 or 10 (folded: j is unrolled)
            if (nw == 10) vm_wait<10>();
            else if (nw == 8) vm_wait<8>();
            else if (nw == 6) vm_wait<6>();
            else vm_wait<4>();
            {
                int sl = s3 + (j + 2) % 3;
                sl = sl >= 3 ? sl - 3 : sl;
                issue(sb0 + bi + (j + 2) / 16, (j + 2) & 15, sl * K8_A);
            }
            int sc3 = s3 + j % 3;
            sc3 = sc3 >= 3 ? sc3 - 3 : sc3;
            const uint32_t sa = wl_lds + sc3 * K8_A;
            const uint32_t sq = wl_lds + L::BOFF + ((j >> 1) & 1) * L::B;
            if (j == 0) {
                const uint32_t hs = wl_lds + L::HOFF;
                hd[0] = lds_b128<0>(hs + h_off);
                hd[1] = lds_b128<512>(hs + h_off);
                hd[2] = lds_b128<1024>(hs + h_off);
                hd[3] = lds_b128<1536>(hs + h_off);
                if constexpr (!Q5) {
                    sv[0] = lds_b128h<2048>(hs + a_v);
                    sv[1] = lds_b128h<3072>(hs + a_v);
                }
            }
            if (nib == 0) {
                raw[0] = lds_b64<0>(sq + b_off);
                raw[1] = lds_b64<512>(sq + b_off);
                raw[2] = lds_b64<1024>(sq + b_off);
                raw[3] = lds_b64<1536>(sq + b_off);
                if constexpr (Q5) {
                    P5[0] = lds_u16<2048>(sq + f_off);
                    P5[1] = lds_u16<2048 + 128>(sq + f_off);
                    P5[2] = lds_u16<2048 + 256>(sq + f_off);
                    P5[3] = lds_u16<2048 + 384>(sq + f_off);
                }
            }
            if constexpr (Q5) {
                if (j == 0) lgkm_wait<11>();  // at most 15 LDS reads outstanding: the first header read is back
            }
            half8_t a[2][2];  // [mt][part]
            a[0][0] = lds_b128h<0>(sa + a_v);
            a[0][1] = lds_b128h<1024>(sa + a_v);
            a[1][0] = lds_b128h<2048>(sa + a_v);
            a[1][1] = lds_b128h<3072>(sa + a_v);
            lgkm_wait<4>();  // all but the A fragments
            if (j == 0) {
#pragma unroll
                for (int c = 0; c < 4; c++) pin(hd[c]);
                if constexpr (!Q5) {
                    pin(sv[0]);
                    pin(sv[1]);
                }
                // entering the super-block: rescale U to this block's d (a zero d keeps the scale;
                // its weights are zeroed through the scales below)
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const float d = aeth_decode_d(hd[c][0]);
                    const float Dn = d != 0.0f ? d : D[c];
                    if (bi > 0) {
                        const float r = D[c] * __builtin_amdgcn_rcpf(Dn);  // one rounding per block
#pragma unroll
                        for (int mt = 0; mt < 2; mt++)
#pragma unroll
                            for (int q = 0; q < 16; q++) U[mt][c][q] *= r;
                    }
                    D[c] = Dn;
                }
            }
            if ((j & 3) == 0) {
                // scales of sub-blocks 2J (low nibbles) and 2J + 1 (high nibbles), get_scale_min_k4
                // (common.rs:29-38): sp = (sc, sc'/16), zp = (−1024·sc, −64·sc'), used as broadcast
                // halves; all zero when the block's d is zero
                const int J = j >> 2;
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const uint32_t y = hd[c][1], w = hd[c][3];
                    uint32_t sc4 = J < 2 ? (y & 0x3F3F3F3Fu) : ((w & 0x0F0F0F0Fu) | ((y >> 2) & 0x30303030u));
                    if ((hd[c][0] & 0x7FFFu) == 0u) sc4 = 0u;  // d = ±0
                    half2_t p01, p23;
                    bytes_to_h2(sc4, p01, p23);
                    const half2_t pr = (J & 1) ? p23 : p01;
                    const half2_t k_s = {(_Float16)1.0f, (_Float16)0.0625f};
                    const half2_t k_z = {(_Float16)-1024.0f, (_Float16)-64.0f};
                    sp[c] = pr * k_s;
                    zp[c] = pr * k_z;
                }
            }
            if (nib == 0) {
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    pin(raw[c]);
                    if constexpr (Q5) {
                        pin(P5[c]);
                        P5[c] = __builtin_amdgcn_perm(0u, P5[c], 0x0C010C00u);  // word bytes → bits 0-7, 16-23
                    } else {
                        x8[c] = raw[c][0] >> 8;
                        y8[c] = raw[c][1] >> 8;
                    }
                }
            }
            if constexpr (Q5) {
                // the shifted quant words are formed in each slice (registers: Q5_K holds the fifth
                // bits instead); a fresh name per slice keeps the two slices' shifts apart
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    if (nib == 1) pin(raw[c]);
                    x8[c] = raw[c][0] >> 8;
                    y8[c] = raw[c][1] >> 8;
                }
            }
            half8_t bv[4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                if constexpr (Q5) {
                    if (nib == 0)
                        bv[c] = dq8s5<0x000F000Fu, 0x00100010u>(raw[c][0], raw[c][1], x8[c], y8[c], P5[c], c64,
                                                                __builtin_shufflevector(sp[c], sp[c], 0, 0),
                                                                __builtin_shufflevector(zp[c], zp[c], 0, 0));
                    else
                        bv[c] = dq8s5<0x00F000F0u, 0x01000100u>(raw[c][0], raw[c][1], x8[c], y8[c], P5[c], c64,
                                                                __builtin_shufflevector(sp[c], sp[c], 1, 1),
                                                                __builtin_shufflevector(zp[c], zp[c], 1, 1));
                    continue;
                }
                if (nib == 0)
                    bv[c] = dq8s<0x000F000Fu>(raw[c][0], raw[c][1], x8[c], y8[c], c64,
                                              __builtin_shufflevector(sp[c], sp[c], 0, 0),
                                              __builtin_shufflevector(zp[c], zp[c], 0, 0));
                else
                    bv[c] = dq8s<0x00F000F0u>(raw[c][0], raw[c][1], x8[c], y8[c], c64,
                                              __builtin_shufflevector(sp[c], sp[c], 1, 1),
                                              __builtin_shufflevector(zp[c], zp[c], 1, 1));
            }
            lgkm_wait<0>();
#pragma unroll
            for (int mt = 0; mt < 2; mt++) {
                pin(a[mt][0]);
                pin(a[mt][1]);
            }
#pragma unroll
            for (int p = 0; p < 2; p++)
#pragma unroll
                for (int mt = 0; mt < 2; mt++)
#pragma unroll
                    for (int c = 0; c < 4; c++)
                        U[mt][c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[mt][p], bv[c], U[mt][c], 0, 0, 0);
            if (j == 15) {
                // leaving the super-block: U += (−32·dmin/D)·Σ_s m_s·S_s (S carries 2^-(e+5))
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const float ndm = -32.0f * aeth_decode_d(hd[c][0] >> 16) * __builtin_amdgcn_rcpf(D[c]);
                    const uint32_t z = hd[c][2], w = hd[c][3];
                    half2_t m01, m23, m45, m67;
                    bytes_to_h2(z & 0x3F3F3F3Fu, m01, m23);
                    bytes_to_h2(((w >> 4) & 0x0F0F0F0Fu) | ((z >> 2) & 0x30303030u), m45, m67);
                    const half8_t mv = {m01[0], m01[1], m23[0], m23[1], m45[0], m45[1], m67[0], m67[1]};
#pragma unroll
                    for (int mt = 0; mt < 2; mt++) {
                        const f32x16 q = __builtin_amdgcn_mfma_f32_32x32x16_f16(sv[mt], mv, (f32x16){}, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 16; r++) U[mt][c][r] = fmaf(ndm, q[r], U[mt][c][r]);
                    }
                }
                if constexpr (Q5) load_sums(sb0 + bi + 1, sv);  // the next super-block's (past the run: unread)
            }
        }
        s3 = s3 == 2 ? 0 : s3 + 1;
    }
    __builtin_amdgcn_s_waitcnt(0);  // the tail's loads have landed
    __syncthreads();                // and every wave is done with its ring

    // The eight K-eighth tiles meet in LDS. Round 1: waves 4..7 hand theirs to
    // waves 0..3 (slot [w - 4]); round 2: waves 0..3 write the pair sums and wave w
    // (0..7) sums (mt, c) = (w / 4, w % 4) over them in order and stores it.
    float* red = (float*)smem;  // [4][2][4][16][64] floats = 128 KiB
    const int mt = wave >> 2, c = wave & 3, lr = lane & 31;
    const int col = n0 + 32 * c + lr;
    int rows[16];
#pragma unroll
    for (int r = 0; r < 16; r++) rows[r] = m0 + 32 * mt + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
    G2Epi E;  // in flight during the reduction
    if (nsplit == 1) g2_epi_load(E, G.escale, G.C, G.ldc, G.m, G.n, rows, col, G.accumulate);
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int r = 0; r < 16; r++) U[mt][c][r] *= D[c];
    if (wave >= 4) {
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int c = 0; c < 4; c++)
#pragma unroll
                for (int r = 0; r < 16; r++) red[((((wave - 4) * 2 + mt) * 4 + c) * 16 + r) * 64 + lane] = U[mt][c][r];
    }
    __syncthreads();
    if (wave < 4) {
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int c = 0; c < 4; c++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int i = (((wave * 2 + mt) * 4 + c) * 16 + r) * 64 + lane;
                    red[i] = U[mt][c][r] + red[i];
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

int aeth_gemm_kq_launch(const KqArgs& G, hipStream_t s) {
    if (G.fifth)
        hipLaunchKernelGGL(k_gemm_kq<true>, dim3(g2_grid(G)), dim3(64 * K8_W), 0, s, G);
    else
        hipLaunchKernelGGL(k_gemm_kq<false>, dim3(g2_grid(G)), dim3(64 * K8_W), 0, s, G);
    AETH_LAUNCH_CHECK();
    return g2_split_sum(G, s);
}
