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
    } else if (dtype == AETH_DTYPE_Q6_K) {
        int64_t nblk = n_elems / 256;
        if (nblk == 0) return AETH_OK;
        hipLaunchKernelGGL(k_dequant_q6_k, dim3((unsigned)aeth_cdiv(nblk * 64, 256)), dim3(256), 0, s, raw, nblk,
                           d_out);
    } else {
        return aeth_set_error(AETH_EUNSUPPORTED, "aeth_dequant: unsupported dtype %d", dtype);
    }
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}
