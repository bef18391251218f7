// GGUF block → f32 dequantization, bit-exact with src/loader/dequant.rs.
//
// The reference rounds every multiply and subtract separately (Rust never
// fuses). With a NaN/Inf-pattern scale (bits/65536: 16 significant bits) the
// product d1*q is not exact in f32, so fusing it with the subtraction would
// change results: contraction is switched off for this file (the library is
// built with -ffp-contract=fast-honor-pragmas, which honours the pragma).
#include "aeth_common.hpp"
#include "aeth_internal.hpp"

#pragma clang fp contract(off)

// dequant_q8_0, dequant.rs:103-127: out = (f32)(i8)q * d, d plain f16.
__global__ void k_dequant_q8_0(const uint8_t* __restrict__ raw, int64_t n, float* __restrict__ out) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int64_t blk = i >> 5;
    int l = (int)(i & 31);
    const uint8_t* b = raw + blk * Q8_BLOCK_BYTES;
    float d = aeth_f16_to_f32((uint32_t)b[0] | ((uint32_t)b[1] << 8));
    out[i] = (float)(int8_t)b[2 + l] * d;
}

// get_scale_min_k4, common.rs:29-38.
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t* s, int& sc, int& m) {
    if (j < 4) {
        sc = s[j] & 63;
        m = s[j + 4] & 63;
    } else {
        sc = (s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4);
        m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

// dequant_q4_k, dequant.rs:195-227. Thread (block, t<128) owns qs byte t:
// group j = t/32, l = t%32 → out[64j+l] (low nibble), out[64j+32+l] (high).
__global__ void k_dequant_q4_k(const uint8_t* __restrict__ raw, int64_t nblk, float* __restrict__ out) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblk * 128) return;
    int64_t blk = i >> 7;
    int t = (int)(i & 127);
    int j = t >> 5, l = t & 31;
    const uint8_t* b = raw + blk * Q4K_BLOCK_BYTES;
    float d = aeth_decode_d((uint32_t)b[0] | ((uint32_t)b[1] << 8));
    float dmin = aeth_decode_d((uint32_t)b[2] | ((uint32_t)b[3] << 8));
    int sc0, m0, sc1, m1;
    scale_min_k4(2 * j, b + 4, sc0, m0);
    scale_min_k4(2 * j + 1, b + 4, sc1, m1);
    float d1 = d * (float)sc0, mm1 = dmin * (float)m0;
    float d2 = d * (float)sc1, mm2 = dmin * (float)m1;
    uint32_t q = b[16 + t];
    float* o = out + blk * 256 + 64 * j + l;
    o[0] = d1 * (float)(q & 0x0F) - mm1;
    o[32] = d2 * (float)((q >> 4) & 0x0F) - mm2;
}

// dequant_q6_k, dequant.rs:301-348. Thread (block, t<64): half h = t/32,
// l = t%32 → 4 outputs at h*128 + l + {0,32,64,96}.
__global__ void k_dequant_q6_k(const uint8_t* __restrict__ raw, int64_t nblk, float* __restrict__ out) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblk * 64) return;
    int64_t blk = i >> 6;
    int t = (int)(i & 63);
    int h = t >> 5, l = t & 31, is = l >> 4;
    const uint8_t* b = raw + blk * Q6K_BLOCK_BYTES;
    float d = aeth_decode_d((uint32_t)b[208] | ((uint32_t)b[209] << 8));
    uint32_t a = b[h * 64 + l], a32 = b[h * 64 + l + 32], hb = b[128 + h * 32 + l];
    int q1 = (int)((a & 0x0F) | ((hb & 0x03) << 4)) - 32;
    int q2 = (int)((a32 & 0x0F) | ((hb & 0x0C) << 2)) - 32;
    int q3 = (int)((a >> 4) | (hb & 0x30)) - 32;
    int q4 = (int)((a32 >> 4) | ((hb & 0xC0) >> 2)) - 32;
    const int8_t* sc = (const int8_t*)(b + 192 + h * 8);
    float* o = out + blk * 256 + h * 128 + l;
    o[0] = d * (float)sc[is] * (float)q1;
    o[32] = d * (float)sc[is + 2] * (float)q2;
    o[64] = d * (float)sc[is + 4] * (float)q3;
    o[96] = d * (float)sc[is + 6] * (float)q4;
}

// dequant_q5_k, dequant.rs:229-285 (block form :542-584): Q4_K's fields plus a
// fifth bit per element e at bit e % 8 of qh[e / 8]. Thread (block, t < 128)
// owns qs byte t as in k_dequant_q4_k.
__global__ void k_dequant_q5_k(const uint8_t* __restrict__ raw, int64_t nblk, float* __restrict__ out) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblk * 128) return;
    int64_t blk = i >> 7;
    int t = (int)(i & 127);
    int j = t >> 5, l = t & 31;
    const uint8_t* b = raw + blk * Q5K_BLOCK_BYTES;
    float d = aeth_decode_d((uint32_t)b[0] | ((uint32_t)b[1] << 8));
    float dmin = aeth_decode_d((uint32_t)b[2] | ((uint32_t)b[3] << 8));
    int sc0, m0, sc1, m1;
    scale_min_k4(2 * j, b + 4, sc0, m0);
    scale_min_k4(2 * j + 1, b + 4, sc1, m1);
    float d1 = d * (float)sc0, mm1 = dmin * (float)m0;
    float d2 = d * (float)sc1, mm2 = dmin * (float)m1;
    const int elo = 64 * j + l, ehi = elo + 32;
    uint32_t q = b[48 + t];
    uint32_t qlo = (q & 0x0F) | (((uint32_t)(b[16 + (elo >> 3)] >> (elo & 7)) & 1u) << 4);
    uint32_t qhi = ((q >> 4) & 0x0F) | (((uint32_t)(b[16 + (ehi >> 3)] >> (ehi & 7)) & 1u) << 4);
    float* o = out + blk * 256;
    o[elo] = d1 * (float)qlo - mm1;
    o[ehi] = d2 * (float)qhi - mm2;
}

// dequant_q2_k, dequant.rs:350-398. Thread (block, t < 64) owns qs byte t:
// half h = t/32, r = t%32 → elements 128h + 32s + r (s = 0..3, bits 2s), of
// sub-block 8h + 2s + r/16; out = d·(sc & 15)·q − dmin·(sc >> 4).
__global__ void k_dequant_q2_k(const uint8_t* __restrict__ raw, int64_t nblk, float* __restrict__ out) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblk * 64) return;
    int64_t blk = i >> 6;
    int t = (int)(i & 63), h = t >> 5, r = t & 31;
    const uint8_t* b = raw + blk * Q2K_BLOCK_BYTES;
    float d = aeth_decode_d((uint32_t)b[0] | ((uint32_t)b[1] << 8));
    float dmin = aeth_decode_d((uint32_t)b[2] | ((uint32_t)b[3] << 8));
    uint32_t q = b[20 + t];
    float* o = out + blk * 256 + 128 * h + r;
#pragma unroll
    for (int s = 0; s < 4; s++) {
        uint32_t sc = b[4 + 8 * h + 2 * s + (r >> 4)];
        float dl = d * (float)(sc & 0xF), ml = dmin * (float)(sc >> 4);
        o[32 * s] = dl * (float)((q >> (2 * s)) & 3) - ml;
    }
}

// Q3_K's 16 six-bit scales (dequant.rs:412-425), centred by −32.
__device__ __forceinline__ int q3k_scale(const uint8_t* sr, int s) {
    const int lo = s < 8 ? (sr[s] & 0x0F) : (sr[s - 8] >> 4);
    const int hi = (sr[8 + (s & 3)] >> (2 * (s >> 2))) & 3;
    return (lo | (hi << 4)) - 32;
}

// dequant_q3_k, dequant.rs:400-451. Thread (block, t < 64) owns qs byte t:
// half h = t/32, r = t%32, elements 128h + 32s + r of sub-block
// 8h + 2s + r/16 (bits 2s of the byte), high-mask bit 4h + s of hmask[r];
// q = ql − 4·(1 − hbit), out = (d·sc)·q.
__global__ void k_dequant_q3_k(const uint8_t* __restrict__ raw, int64_t nblk, float* __restrict__ out) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblk * 64) return;
    int64_t blk = i >> 6;
    int t = (int)(i & 63), h = t >> 5, r = t & 31;
    const uint8_t* b = raw + blk * Q3K_BLOCK_BYTES;
    float d = aeth_decode_d((uint32_t)b[108] | ((uint32_t)b[109] << 8));
    uint32_t q = b[32 + t], hm = b[r];
    float* o = out + blk * 256 + 128 * h + r;
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const int sub = 8 * h + 2 * s + (r >> 4);
        const int ql = (int)((q >> (2 * s)) & 3), hb = (int)((hm >> (4 * h + s)) & 1);
        float dl = d * (float)q3k_scale(b + 96, sub);
        o[32 * s] = dl * (float)(ql - ((hb ^ 1) << 2));
    }
}

// dequant_f16 / dequant_f32, dequant.rs:57-95.
__global__ void k_dequant_f16(const uint16_t* __restrict__ raw, int64_t n, float* __restrict__ out) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = aeth_f16_to_f32(raw[i]);
}

extern "C" AETH_API int aeth_dequant(int dtype, const void* d_raw, int64_t n_elems, float* d_out, void* stream) {
    if (!d_raw || !d_out || n_elems < 0) return aeth_set_error(AETH_EINVAL, "aeth_dequant: bad argument");
    hipStream_t s = (hipStream_t)stream;
    const uint8_t* raw = (const uint8_t*)d_raw;
    if (dtype == AETH_DTYPE_Q8_0) {
        if (n_elems == 0) return AETH_OK;
        hipLaunchKernelGGL(k_dequant_q8_0, dim3((unsigned)aeth_cdiv(n_elems, 256)), dim3(256), 0, s, raw, n_elems,
                           d_out);
    } else if (dtype == AETH_DTYPE_Q4_K) {
        int64_t nblk = n_elems / 256;
        if (nblk == 0) return AETH_OK;
        hipLaunchKernelGGL(k_dequant_q4_k, dim3((unsigned)aeth_cdiv(nblk * 128, 256)), dim3(256), 0, s, raw, nblk,
                           d_out);
    } else if (dtype == AETH_DTYPE_Q6_K || dtype == AETH_DTYPE_Q2_K || dtype == AETH_DTYPE_Q3_K) {
        int64_t nblk = n_elems / 256;
        if (nblk == 0) return AETH_OK;
        auto kern = dtype == AETH_DTYPE_Q6_K ? k_dequant_q6_k : dtype == AETH_DTYPE_Q2_K ? k_dequant_q2_k : k_dequant_q3_k;
        hipLaunchKernelGGL(kern, dim3((unsigned)aeth_cdiv(nblk * 64, 256)), dim3(256), 0, s, raw, nblk, d_out);
    } else if (dtype == AETH_DTYPE_Q5_K) {
        int64_t nblk = n_elems / 256;
        if (nblk == 0) return AETH_OK;
        hipLaunchKernelGGL(k_dequant_q5_k, dim3((unsigned)aeth_cdiv(nblk * 128, 256)), dim3(256), 0, s, raw, nblk,
                           d_out);
    } else if (dtype == AETH_DTYPE_F16) {
        if (n_elems == 0) return AETH_OK;
        hipLaunchKernelGGL(k_dequant_f16, dim3((unsigned)aeth_cdiv(n_elems, 256)), dim3(256), 0, s,
                           (const uint16_t*)raw, n_elems, d_out);
    } else if (dtype == AETH_DTYPE_F32) {
        if (n_elems == 0) return AETH_OK;
        AETH_HIP_CHECK(hipMemcpyAsync(d_out, raw, (size_t)n_elems * 4, hipMemcpyDeviceToDevice, s));
        return AETH_OK;
    } else {
        return aeth_set_error(AETH_EUNSUPPORTED, "aeth_dequant: unsupported dtype %d", dtype);
    }
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}
