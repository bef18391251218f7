// Shared device/host helpers for the gfx950 quantized-matmul library.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/aether_hip.h"

// GGUF block geometry (src/quant/matmul/common.rs:1-8; gguf.rs:137-173).
#define Q8_BLOCK_ELEMS 32
#define Q8_BLOCK_BYTES 34
#define QK_BLOCK_ELEMS 256
#define Q2K_BLOCK_BYTES 84
#define Q3K_BLOCK_BYTES 110
#define Q4K_BLOCK_BYTES 144
#define Q5K_BLOCK_BYTES 176
#define Q6K_BLOCK_BYTES 210

// Records a message for aeth_last_error() and returns `code`.
int aeth_set_error(int code, const char* fmt, ...);

#define AETH_HIP_CHECK(expr)                                                          \
    do {                                                                              \
        hipError_t _e = (expr);                                                       \
        if (_e != hipSuccess)                                                         \
            return aeth_set_error(AETH_EHIP, "%s failed: %s (%s:%d)", #expr,          \
                                  hipGetErrorString(_e), __FILE__, __LINE__);         \
    } while (0)

#define AETH_LAUNCH_CHECK()                                                           \
    do {                                                                              \
        hipError_t _e = hipGetLastError();                                            \
        if (_e != hipSuccess)                                                         \
            return aeth_set_error(AETH_EHIP, "kernel launch failed: %s (%s:%d)",     \
                                  hipGetErrorString(_e), __FILE__, __LINE__);         \
    } while (0)

// binary32 → binary16 bits, round to nearest even (the hardware conversion),
// NaN as sign | 0x7E00 | payload >> 13 (half::f16::from_f32).
__device__ __forceinline__ uint32_t aeth_f32_to_f16_bits(float f) {
    const uint32_t x = __float_as_uint(f);
    if ((x & 0x7F800000u) == 0x7F800000u && (x & 0x7FFFFFu))
        return ((x >> 16) & 0x8000u) | 0x7E00u | ((x & 0x7FFFFFu) >> 13);
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

// Exact binary16 -> binary32.
__device__ __forceinline__ float aeth_f16_to_f32(uint32_t bits16) {
    return __half2float(__ushort_as_half((unsigned short)bits16));
}

// decode_f16_scale / decode_d (common.rs:19-27, dequant.rs:161-168): K-quant
// scales whose f16 pattern is NaN or Inf decode to bits/65536 instead.
__device__ __forceinline__ float aeth_decode_d(uint32_t bits16) {
    bits16 &= 0xFFFFu;
    const float alt = (float)bits16 * (1.0f / 65536.0f);  // exact: 16-bit integer × 2^-16
    const float f = aeth_f16_to_f32(bits16);
    return ((bits16 & 0x7C00u) == 0x7C00u) ? alt : f;  // select, not a branch
}

// Lane exchanges without the LDS crossbar: DPP quad_perm moves (lane ^ 1,
// lane ^ 2) and row mirrors (lane i of 8 ↔ 7 − i, of 16 ↔ 15 − i), and
// gfx950's permlane16/32 swaps, which exchange whole 16- and 32-lane rows.
// Callers keep all 64 lanes of the wave active.
__device__ __forceinline__ int aeth_dpp_xor1(int v) { return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false); }
__device__ __forceinline__ int aeth_dpp_xor2(int v) { return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false); }
__device__ __forceinline__ float aeth_dpp_xor1f(float v) { return __int_as_float(aeth_dpp_xor1(__float_as_int(v))); }
__device__ __forceinline__ float aeth_dpp_xor2f(float v) { return __int_as_float(aeth_dpp_xor2(__float_as_int(v))); }
__device__ __forceinline__ float aeth_dpp_mirror8f(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false));
}
__device__ __forceinline__ float aeth_dpp_mirror16f(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, false));
}

// v[l] + v[l ^ 16], then the same across l ^ 32: after a swap of (v, v) one
// result holds the lane's own value and the other its partner's, so both
// partners add the same two values and every lane ends with the same sum.
__device__ __forceinline__ float aeth_sum_rows(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const float s = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ float aeth_max_rows(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const float s = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// v[l] + v[l ^ 32] (the two 32-lane halves), the same value in both partners.
__device__ __forceinline__ float aeth_add_halves(float v) {
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Sum / max over the wave, the same value in every lane (each step adds a
// lane's value to its partner's, and the partner adds the same pair).
__device__ __forceinline__ float aeth_wave_sum(float v) {
    v += aeth_dpp_xor1f(v);
    v += aeth_dpp_xor2f(v);
    v += aeth_dpp_mirror8f(v);
    v += aeth_dpp_mirror16f(v);
    return aeth_sum_rows(v);
}

__device__ __forceinline__ float aeth_wave_max(float v) {
    v = fmaxf(v, aeth_dpp_xor1f(v));
    v = fmaxf(v, aeth_dpp_xor2f(v));
    v = fmaxf(v, aeth_dpp_mirror8f(v));
    v = fmaxf(v, aeth_dpp_mirror16f(v));
    return aeth_max_rows(v);
}

static inline int64_t aeth_cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
