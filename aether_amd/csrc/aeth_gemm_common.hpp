// Shared pieces of the Q4_K prefill GEMM kernels (aeth_gemm.hip, aeth_gemm_kq.hip):
// operand types, the packed-fp16 weight dequantisation, LDS reads under manual
// lgkmcnt and the XCD-aware tile order.
#pragma once
#include <stdint.h>

#include "aeth_common.hpp"

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) char lds_char;

// positions 1 and 2 of each group of 4 exchanged (an involution)
__device__ __forceinline__ int perm4(int i) { return (i & ~3) | ((0x3120 >> (4 * (i & 3))) & 3); }

// bytes (b0, b1, b2, b3) of w as fp16 pairs (b0, b1) and (b2, b3): (0x64 | b) is 1024 + b
__device__ __forceinline__ void bytes_to_h2(uint32_t w, half2_t& p01, half2_t& p23) {
    const half2_t k1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f};
    p01 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, w, 0x07010700u)) + k1024;
    p23 = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, w, 0x07030702u)) + k1024;
}

__device__ __forceinline__ uint32_t pkfma(uint32_t q, half2_t s, half2_t z) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(half2_t, q), s, z));
}

// Eight quants of (x, y) → an fp16 MFMA operand (k-order [0, 2, 1, 3] per 4).
// The nibble pairs come from one v_and_or_b32 each: MASK 0x000F000F keeps the
// low nibbles of bytes (0, 2) as halves 1024 + q (scales s = sc, z = −1024·sc),
// MASK 0x00F000F0 the high nibbles as 1024 + 16q (s = sc/16, z = −64·sc); bytes
// (1, 3) after a shift by 8 (x8, y8). c64 holds 0x64006400 in a VGPR, so that
// the OR's constant does not need a second scalar operand (VOP3 takes one).
// Every result q·sc ≤ 945 is an exact fp16 integer (the fused product is exact).
template <uint32_t MASK>
__device__ __forceinline__ half8_t dq8s(uint32_t x, uint32_t y, uint32_t x8, uint32_t y8, uint32_t c64, half2_t s,
                                        half2_t z) {
    const uint32_t q0 = pkfma((x & MASK) | c64, s, z);
    const uint32_t q1 = pkfma((x8 & MASK) | c64, s, z);
    const uint32_t q2 = pkfma((y & MASK) | c64, s, z);
    const uint32_t q3 = pkfma((y8 & MASK) | c64, s, z);
    return __builtin_bit_cast(half8_t, make_uint4(q0, q1, q2, q3));
}
// dq8s for Q5_K: q gains its fifth bit, 16 (low nibbles, MASK 0x000F000F: bit 4 of each half,
// M5 = 0x00100010) or 256 in the in-place high nibble's units (MASK 0x00F000F0: bit 8, M5 =
// 0x01000100), so the halves are 1024 + q5 or 1024 + 16·q5 and every result q5·sc ≤ 1953 is
// exact. P holds the eight fifth bits of this slice's pair of sub-blocks (bits 0-3: the four
// dwords' first halves of the low-nibble sub-block, 4-7 the high-nibble one's; bits 16-23 the
// second halves): dword i takes its bits shifted left by 4 − i.
template <uint32_t MASK, uint32_t M5>
__device__ __forceinline__ half8_t dq8s5(uint32_t x, uint32_t y, uint32_t x8, uint32_t y8, uint32_t P, uint32_t c64,
                                         half2_t s, half2_t z) {
    const uint32_t q0 = pkfma((x & MASK) | (((P << 4) & M5) | c64), s, z);
    const uint32_t q1 = pkfma((x8 & MASK) | (((P << 3) & M5) | c64), s, z);
    const uint32_t q2 = pkfma((y & MASK) | (((P << 2) & M5) | c64), s, z);
    const uint32_t q3 = pkfma((y8 & MASK) | (((P << 1) & M5) | c64), s, z);
    return __builtin_bit_cast(half8_t, make_uint4(q0, q1, q2, q3));
}
template <uint32_t MASK>
__device__ __forceinline__ half8_t dq8(uint32_t x, uint32_t y, uint32_t c64, half2_t s, half2_t z) {
    return dq8s<MASK>(x, y, x >> 8, y >> 8, c64, s, z);
}

// LDS reads issued as inline asm: the compiler would otherwise order every LDS
// read after all outstanding direct-to-LDS loads (vmcnt(0)), since it cannot
// tell the ring's slots apart. Kernels wait with lgkmcnt themselves, then pass
// each value through pin() so no use is scheduled above its wait.
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
template <int OFF>
__device__ __forceinline__ u32x2 lds_b64(uint32_t a) {
    u32x2 v;
    asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(v) : "v"(a), "i"(OFF));
    return v;
}
template <int OFF>
__device__ __forceinline__ uint32_t lds_u16(uint32_t a) {
    uint32_t v;
    asm volatile("ds_read_u16 %0, %1 offset:%2" : "=v"(v) : "v"(a), "i"(OFF));
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
template <int N>
__device__ __forceinline__ void vm_wait() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));  // lgkmcnt at its maximum
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

// Workgroup bid → (tile, K part ks of nsplit). Without a tail split the ksplit parts of a tile
// are T = gm·gn workgroups apart (each keeps the tile's XCD when T is a multiple of 8). With one
// (ksplit == 1, tsplit > 1) the workgroups below t_full take the whole tiles [0, t_full) and the
// rest the tsplit parts of the tail tiles [t_full, T), the parts of one tile T − t_full apart.
__device__ __forceinline__ void g2_work(int bid, int gm, int gn, int ksplit, int t_full, int tsplit, int& tile,
                                        int& ks, int& nsplit) {
    const int T = gm * gn;
    if (tsplit > 1 && bid >= t_full) {
        const int ntail = T - t_full, jt = bid - t_full;
        nsplit = tsplit;
        ks = jt / ntail;
        tile = t_full + (jt - ks * ntail);
    } else {
        nsplit = ksplit;
        ks = bid / T;
        tile = bid - ks * T;
    }
}

// Partial tile of split ks of `tile` (its 64 × 128 block at rows m0, columns n0 of C): the address of
// its element (0, 0) and the row stride ld. A K split over every tile keeps C's layout, part[ks][mp][pld];
// a tail split stores only the tail tiles, part[ks][tile − t_full][64][128].
__device__ __forceinline__ float* g2_part(float* part, int ks, int tile, int t_full, int tsplit, int T, int mp, int pld,
                                          int m0, int n0, int& ld) {
    if (tsplit > 1) {
        ld = 128;
        return part + ((int64_t)ks * (T - t_full) + (tile - t_full)) * (64 * 128);
    }
    ld = pld;
    return part + ((int64_t)ks * mp + m0) * pld + n0;
}

// Ways to split the K range of every tile of a short last round (the launch has no K split):
// more tiles than CUs and a last round at most half full → as many ways as fill the idle CUs,
// at most maxsplit; otherwise 1.
inline int g2_tail_ways(int64_t T, int64_t cus, int64_t maxsplit) {
    const int64_t tail = T % cus;
    if (T < cus || tail == 0 || 2 * tail > cus) return 1;
    const int64_t w = cus / tail < maxsplit ? cus / tail : maxsplit;
    return w > 1 ? (int)w : 1;
}

// Epilogue of one lane: 16 outputs at rows row(r) (r < 16, each < mp) of column col.
// g2_epi_load fetches the rows' scales 2^e and, with accumulate, C's previous values
// (from clamped addresses, so every load is issued) before the first store: a store to C
// may alias them, so a load after one waits for it, one round trip per output.
struct G2Epi {
    float es[16], pv[16];
};
__device__ __forceinline__ void g2_epi_load(G2Epi& E, const float* escale, const float* C, int64_t ldc, int m, int n,
                                            const int* row, int col, int accumulate) {
#pragma unroll
    for (int r = 0; r < 16; r++) E.es[r] = escale[row[r]];
    if (accumulate) {
        const int cc = min(col, n - 1);
#pragma unroll
        for (int r = 0; r < 16; r++) E.pv[r] = C[(int64_t)min(row[r], m - 1) * ldc + cc];
    }
}
// Store of output r: C[row][col] = sum·2^e (+ the previous value with accumulate).
__device__ __forceinline__ void g2_store(const G2Epi& E, int r, float* C, int64_t ldc, int m, int n, int row, int col,
                                         float sum, int accumulate) {
    const float v = sum * E.es[r];
    if (row < m && col < n) C[(int64_t)row * ldc + col] = accumulate ? E.pv[r] + v : v;
}
// SwiGLU store of outputs r and r + 1 (r even: rows row0 and row0 + 1; columns = (g, u)
// pairs, lane l holding column col and lane l ^ 1 its neighbour; every lane calls it): after
// one lane swap the even lane of a pair holds (g, u) of row row0 and the odd lane those of
// row0 + 1, and each stores h = g·σ(g)·u at C[row][col/2] (σ(g) = 1/(1 + e^-g) with the
// reciprocal instruction).
__device__ __forceinline__ void g2_store_swiglu(const G2Epi& E, int r, float* C, int64_t ldc, int m, int n, int row0,
                                                int col, float sum0, float sum1) {
    const float v0 = sum0 * E.es[r], v1 = sum1 * E.es[r + 1];
    const int odd = col & 1;
    const float y = __shfl_xor(odd ? v0 : v1, 1);
    const float g = odd ? y : v0, u = odd ? v1 : y;
    const int row = row0 + odd;
    if (row < m && col < n) C[(int64_t)row * ldc + (col >> 1)] = g * __builtin_amdgcn_rcpf(1.0f + expf(-g)) * u;
}

// Arguments of the K-split GEMM kernel (aeth_gemm_kq.hip).
struct KqArgs {
    const uint8_t* frag;   // A·2^-e as fp16 MFMA fragments: ((mt·(k/16) + ks)·2 + part)·1 KiB (k_gemm_prep)
    const uint8_t* sums;   // sub-block sums of A·2^-(e+5): hi [mp][k/32] then lo [mp][k/32] (fp16)
    const float* escale;   // [mp]: 2^e
    const uint8_t* hdr;    // Q4_K tile layout (aeth_q4k_hdr_off)
    const uint8_t* qs;     // Q4_K tile layout (aeth_q4k_qs_off)
    int m, n, k, nb, ntiles, mp;
    int gm, gn;            // 64-row and 128-column tiles of C
    int a_bytes, s_bytes, q_bytes, h_bytes;  // buffer extents (each < 2^31)
    float* C;
    int64_t ldc;
    int accumulate;
    int swiglu;            // C[row][col/2] = g·σ(g)·u over the (g, u) column pairs
    // K split over workgroups (ksplit > 1): as Q6Args
    int ksplit;
    float* part;
    int pld;
    // Q5_K: the fifth-bit plane of the GEMM (aeth_weights.hip, p3), null for Q4_K
    const uint8_t* fifth;
    int f_bytes;
    // Tail split (ksplit == 1, tsplit > 1): tiles [t_full, gm·gn) — the last, partial round of
    // workgroups — have K split over tsplit workgroups each (partials in part as g2_part lays them
    // out) and are summed by the tail-sum kernel; tiles below t_full run whole
    int t_full = 0, tsplit = 1;
};
int aeth_gemm_kq_launch(const KqArgs& G, hipStream_t s);

// The second kernel of a GEMM split over K across workgroups (aeth_gemm_q6k.hip): the splits'
// tile sums part[split][row][col] (rows mp, pld columns) added in split order, then the
// epilogue: C[row][col] = Σ·2^e (+ C with accumulate), or with swiglu h = g·σ(g)·u of the
// (g, u) column pairs at C[row][col/2].
struct SplitSum {
    const float* part;
    int ksplit, mp, pld;
    const float* escale;
    float* C;
    int64_t ldc;
    int m, n, accumulate, swiglu;
    // gm > 0: only the 64 × 128 tiles [t_full, gm·gn) in g2_tile's order (a tail split; partials
    // part[split][tile − t_full][64][128])
    int t_full = 0, gm = 0, gn = 0;
};
int aeth_gemm_split_sum_launch(const SplitSum& S, hipStream_t s);

// Arguments of the Q6_K GEMM kernel (aeth_gemm_q6k.hip): A as for KqArgs, the Q6_K weight
// planes (aeth_weights.hip).
struct Q6Args {
    const uint8_t* frag;   // A·2^-e as fp16 MFMA fragments (k_gemm_prep)
    const float* escale;   // [mp]: 2^e
    const uint8_t* q;      // [tile][b][part 3][lane][16 B]
    const uint8_t* sc;     // [tile][b][16 rows][16 B]
    const uint8_t* dd;     // [tile][b][16 rows] (f16)
    int m, n, k, nb, ntiles, mp;
    int gm, gn;            // 64-row and 128-column tiles of C
    int a_bytes, q_bytes, s_bytes, d_bytes;  // buffer extents (each < 2^31)
    float* C;
    int64_t ldc;
    int accumulate;
    int swiglu;
    // K split over workgroups: ksplit > 1 runs ksplit workgroups per tile, each over its share
    // of the super-blocks, writing its tile's sum to part[split][row][col] (rows mp, pld = 128·gn
    // columns); a second kernel adds the splits in order and applies the epilogue
    int ksplit;
    float* part;
    int pld;
    int t_full = 0, tsplit = 1;  // tail split: as KqArgs
};
int aeth_gemm_q6k_kq_launch(const Q6Args& G, hipStream_t s);

// Arguments of the Q8_0 GEMM kernel (aeth_gemm_q80.hip): A as for KqArgs, the Q8_0 weight planes
// (aeth_weights.hip: blocks in groups of 4 per row).
struct Q80Args {
    const uint8_t* frag;   // A·2^-e as fp16 MFMA fragments (k_gemm_prep)
    const float* escale;   // [mp]: 2^e
    const uint8_t* q;      // [tile][group][pair 2][lane][16 B]
    const uint8_t* dd;     // [tile][group][4 blocks][16 rows] (f16)
    int m, n, k, nb, ngr, ntiles, mp;
    int gm, gn;            // 64-row and 128-column tiles of C
    int a_bytes, q_bytes, d_bytes;  // buffer extents (each < 2^31)
    float* C;
    int64_t ldc;
    int accumulate;
    int swiglu;
    int ksplit;            // K split over workgroups: as Q6Args
    float* part;
    int pld;
    int t_full = 0, tsplit = 1;  // tail split: as KqArgs
};
int aeth_gemm_q80_kq_launch(const Q80Args& G, hipStream_t s);

// Grid of a K-split GEMM launch (see g2_work) and its second kernel (none without a split).
template <class Args>
unsigned g2_grid(const Args& G) {
    const int T = G.gm * G.gn;
    return (unsigned)(G.tsplit > 1 ? G.t_full + (T - G.t_full) * G.tsplit : T * G.ksplit);
}
template <class Args>
int g2_split_sum(const Args& G, hipStream_t s) {
    const bool tail = G.tsplit > 1;
    if (G.ksplit == 1 && !tail) return 0;
    SplitSum S{G.part, tail ? G.tsplit : G.ksplit, G.mp, G.pld, G.escale, G.C, G.ldc, G.m, G.n, G.accumulate, G.swiglu};
    if (tail) {
        S.t_full = G.t_full;
        S.gm = G.gm;
        S.gn = G.gn;
    }
    return aeth_gemm_split_sum_launch(S, s);
}
