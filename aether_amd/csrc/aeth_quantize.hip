// f32 → GGUF blocks on the device: the load-time re-quantizers and the Q8_0
// activation quantizer, byte-exact with the reference.
//
//  * requantize_{q8_0,q4_k,q5_k,q6_k} (src/quant/matmul/dispatch.rs:149-184,
//    186-300, 302-429, 431-537): f32 rows → blocks, used by load_quant to transpose
//    quantized weights (model_loader.rs:330-386).
//  * quantize_q8_0_block / quantize_activations_q8_0[_batched]
//    (src/quant/matmul/neon.rs:45-155): the Q8_0 activation scheme.
//  * load_quant's transpose (model_loader.rs:372-385): dequantize the GGUF
//    [k][n] tensor, transpose to [n][k], re-quantize row by row.
//
// One thread per output block, in the reference's loop order: every step is a
// single f32 operation with IEEE rounding (contraction off, correctly rounded
// division), Rust's f32::round is C roundf (half away from zero), f32::max /
// f32::min ignore a NaN operand like fmaxf / fminf, and `as u8 / as i8` after
// the clamps is exact. The f16 scale bytes follow half::f16::from_f32:
// round-to-nearest-even, NaN keeps its sign and top payload bits with the
// quiet bit set.
#include "aeth_common.hpp"
#include "aeth_internal.hpp"

#pragma clang fp contract(off)

__device__ __forceinline__ uint32_t f16_bits(float f) { return aeth_f32_to_f16_bits(f); }

// requantize_q8_0, dispatch.rs:149-184: d = max|x|/127 (1 if the block is 0),
// q = clamp(round(x/d), −128, 127); a row's last block may be partial (its
// missing quants are 0).
__global__ void __launch_bounds__(256) k_requant_q8_0(const float* __restrict__ src, int64_t rows, int64_t cols,
                                                      int64_t bpr, uint8_t* __restrict__ out) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= rows * bpr) return;
    const int64_t r = b / bpr, blk = b - r * bpr;
    const float* x = src + r * cols + blk * 32;
    const int actual = (int)min((int64_t)32, cols - blk * 32);
    float mx = 0.0f;
    for (int i = 0; i < actual; i++) mx = fmaxf(mx, fabsf(x[i]));
    const float d = mx == 0.0f ? 1.0f : mx / 127.0f;
    uint8_t* o = out + b * 34;
    const uint32_t db = f16_bits(d);
    o[0] = (uint8_t)db;
    o[1] = (uint8_t)(db >> 8);
    for (int j = 0; j < 32; j++) {
        int8_t q = 0;
        if (j < actual) {
            float v = roundf(x[j] / d);
            v = fmaxf(v, -128.0f);
            v = fminf(v, 127.0f);
            q = (int8_t)v;
        }
        o[2 + j] = (uint8_t)q;
    }
}

// requantize_q4_k, dispatch.rs:186-300: per 32-element sub-block
// m_s = |min(min, 0)|, d_s = (max + m_s)/15; d = max_s d_s / 63,
// dmin = max_s m_s / 63 (1 when 0); sc, m = clamp(round(d_s/d)), clamp(round(m_s/dmin))
// in [0, 63], packed as get_scale_min_k4 reads them; q = clamp(round((x + dmin·m)/(d·sc)), 0, 15).
// Q5 = true: requantize_q5_k, dispatch.rs:302-429 — the same with 31 levels;
// the low nibbles fill qs (byte 48 on), the fifth bit of element e goes to
// bit e % 8 of qh[e / 8] (bytes 16..47).
template <bool Q5>
__global__ void __launch_bounds__(256) k_requant_qk(const float* __restrict__ src, int64_t rows, int64_t cols,
                                                    int64_t bpr, uint8_t* __restrict__ out) {
    constexpr float LV = Q5 ? 31.0f : 15.0f;
    constexpr int BB = Q5 ? Q5K_BLOCK_BYTES : Q4K_BLOCK_BYTES;
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= rows * bpr) return;
    const int64_t r = b / bpr, blk = b - r * bpr;
    const float* x = src + r * cols + blk * 256;
    const int actual = (int)min((int64_t)256, cols - blk * 256);
    float msub[8], dsub[8];
    for (int sb = 0; sb < 8; sb++) {
        float mn = 0.0f, mx = 0.0f;
        const int s0 = sb * 32;
        if (s0 < actual) {
            const int s1 = min(s0 + 32, actual);
            mn = x[s0];
            mx = x[s0];
            for (int i = s0; i < s1; i++) {
                mn = fminf(mn, x[i]);
                mx = fmaxf(mx, x[i]);
            }
        }
        msub[sb] = fabsf(fminf(mn, 0.0f));
        dsub[sb] = (mx + msub[sb]) / LV;
    }
    float maxd = 0.0f, maxm = 0.0f;
    for (int sb = 0; sb < 8; sb++) {
        maxd = fmaxf(maxd, dsub[sb]);
        maxm = fmaxf(maxm, msub[sb]);
    }
    const float d = maxd == 0.0f ? 1.0f : maxd / 63.0f;
    const float dmin = maxm == 0.0f ? 1.0f : maxm / 63.0f;
    uint8_t* o = out + b * BB;
    const uint32_t db = f16_bits(d), dmb = f16_bits(dmin);
    o[0] = (uint8_t)db;
    o[1] = (uint8_t)(db >> 8);
    o[2] = (uint8_t)dmb;
    o[3] = (uint8_t)(dmb >> 8);
    uint32_t sc[8], mm[8];
    for (int sb = 0; sb < 8; sb++) {
        sc[sb] = (uint32_t)fminf(fmaxf(roundf(dsub[sb] / d), 0.0f), 63.0f);
        mm[sb] = (uint32_t)fminf(fmaxf(roundf(msub[sb] / dmin), 0.0f), 63.0f);
    }
    for (int q = 0; q < 4; q++) {
        o[4 + q] = (uint8_t)((sc[q] & 63) | ((sc[q + 4] >> 4) << 6));
        o[8 + q] = (uint8_t)((mm[q] & 63) | ((mm[q + 4] >> 4) << 6));
        o[12 + q] = (uint8_t)((sc[q + 4] & 0x0F) | ((mm[q + 4] & 0x0F) << 4));
    }
    uint32_t qh[8] = {0, 0, 0, 0, 0, 0, 0, 0};  // Q5: the 256 fifth bits
    for (int ch = 0; ch < 4; ch++) {
        const int is = 2 * ch;
        const float d1 = d * (float)sc[is], m1 = dmin * (float)mm[is];
        const float d2 = d * (float)sc[is + 1], m2 = dmin * (float)mm[is + 1];
        for (int l = 0; l < 32; l++) {
            const int i0 = is * 32 + l, i1 = (is + 1) * 32 + l;
            uint32_t q0 = 0, q1 = 0;
            if (i0 < actual && d1 != 0.0f) q0 = (uint32_t)fminf(fmaxf(roundf((x[i0] + m1) / d1), 0.0f), LV);
            if (i1 < actual && d2 != 0.0f) q1 = (uint32_t)fminf(fmaxf(roundf((x[i1] + m2) / d2), 0.0f), LV);
            if (Q5) {
                o[48 + ch * 32 + l] = (uint8_t)((q0 & 0x0F) | ((q1 & 0x0F) << 4));
                qh[i0 >> 5] |= (q0 >> 4) << (i0 & 31);
                qh[i1 >> 5] |= (q1 >> 4) << (i1 & 31);
            } else {
                o[16 + ch * 32 + l] = (uint8_t)(q0 | (q1 << 4));
            }
        }
    }
    if (Q5)
        for (int j = 0; j < 32; j++) o[16 + j] = (uint8_t)(qh[j >> 2] >> (8 * (j & 3)));
}

// requantize_q6_k, dispatch.rs:431-537: per 16-element sub-block s_max = max|x|;
// d = max s_max / (32·127) (1 when 0); sc = clamp(round(s_max/(32·d)), 0, 127);
// q = clamp(round(x/(d·sc)), −32, 31) + 32 (0 + 32 where sc = 0), split into
// ql nibbles and qh 2-bit fields as dequant_q6_k reads them.
__global__ void __launch_bounds__(256) k_requant_q6_k(const float* __restrict__ src, int64_t rows, int64_t cols,
                                                      int64_t bpr, uint8_t* __restrict__ out) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= rows * bpr) return;
    const int64_t r = b / bpr, blk = b - r * bpr;
    const float* x = src + r * cols + blk * 256;
    const int actual = (int)min((int64_t)256, cols - blk * 256);
    float sub[16];
    for (int sb = 0; sb < 16; sb++) {
        float mx = 0.0f;
        const int s0 = sb * 16;
        if (s0 < actual) {
            const int s1 = min(s0 + 16, actual);
            mx = fabsf(x[s0]);
            for (int i = s0; i < s1; i++) mx = fmaxf(mx, fabsf(x[i]));
        }
        sub[sb] = mx;
    }
    float mv = 0.0f;
    for (int sb = 0; sb < 16; sb++) mv = fmaxf(mv, sub[sb]);
    const float d = mv == 0.0f ? 1.0f : mv / (32.0f * 127.0f);
    uint8_t* o = out + b * 210;
    uint32_t sc[16];
    for (int sb = 0; sb < 16; sb++) {
        sc[sb] = (uint32_t)fminf(fmaxf(roundf(sub[sb] / (32.0f * d)), 0.0f), 127.0f);
        o[192 + sb] = (uint8_t)sc[sb];
    }
    const uint32_t db = f16_bits(d);
    o[208] = (uint8_t)db;
    o[209] = (uint8_t)(db >> 8);
    for (int h = 0; h < 2; h++) {
        for (int l = 0; l < 32; l++) {
            const int is = l / 16;
            uint32_t u[4];
            for (int t = 0; t < 4; t++) {
                const float s = (float)sc[h * 8 + is + 2 * t];
                const int idx = h * 128 + l + 32 * t;
                int q = 0;
                if (idx < actual && s > 0.0f) q = (int)fminf(fmaxf(roundf(x[idx] / (d * s)), -32.0f), 31.0f);
                u[t] = (uint32_t)(q + 32);
            }
            o[h * 64 + l] = (uint8_t)((u[0] & 0x0F) | ((u[2] & 0x0F) << 4));
            o[h * 64 + l + 32] = (uint8_t)((u[1] & 0x0F) | ((u[3] & 0x0F) << 4));
            o[128 + h * 32 + l] = (uint8_t)((u[0] >> 4) | ((u[1] >> 4) << 2) | ((u[2] >> 4) << 4) | ((u[3] >> 4) << 6));
        }
    }
}

// quantize_q8_0_block, neon.rs:45-104, over rows of k (quantize_activations_q8_0
// [_batched], neon.rs:106-155: a partial last block is zero-padded).
// d = max|x|/127 with a NaN-propagating max (vmaxq_f32); stored as f16, while
// the quants use the f32 d: q = sat_i8(RNE(x·(1/d))) (vcvtnq_s32_f32 then two
// saturating narrows); d = 0 or NaN → zero quants. A block holding a NaN
// stores the quiet NaN 0x7E00 as its scale (the sign and payload that
// vmaxq_f32 would carry over from the input NaN are not reproduced).
__global__ void __launch_bounds__(256) k_quant_act_q8_0(const float* __restrict__ a, int64_t m, int64_t k,
                                                        int64_t bpr, uint8_t* __restrict__ out) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= m * bpr) return;
    const int64_t r = b / bpr, blk = b - r * bpr;
    const float* x = a + r * k + blk * 32;
    const int actual = (int)min((int64_t)32, k - blk * 32);
    float v[32];
    for (int i = 0; i < 32; i++) v[i] = i < actual ? x[i] : 0.0f;
    bool nan = false;
    float mx = 0.0f;
    for (int i = 0; i < 32; i++) {
        nan |= v[i] != v[i];
        mx = fmaxf(mx, fabsf(v[i]));
    }
    const float d = nan ? __uint_as_float(0x7FC00000u) : mx / 127.0f;
    uint8_t* o = out + b * 34;
    const uint32_t db = f16_bits(d);
    o[0] = (uint8_t)db;
    o[1] = (uint8_t)(db >> 8);
    if (d > 0.0f) {
        const float inv = 1.0f / d;
        for (int i = 0; i < 32; i++) {
            const float p = v[i] * inv;
            // RNE to integer with i32 saturation, NaN → 0 (vcvtnq_s32_f32), then clamp to i8
            int32_t q = p != p ? 0 : p >= 2147483648.0f ? INT32_MAX : p < -2147483648.0f ? INT32_MIN : (int32_t)rintf(p);
            q = max(-128, min(127, q));
            o[2 + i] = (uint8_t)(int8_t)q;
        }
    } else {
        for (int i = 0; i < 32; i++) o[2 + i] = 0;
    }
}

// [rows][cols] → [cols][rows] through 32 × 33 LDS tiles.
__global__ void __launch_bounds__(256) k_transpose_f32(const float* __restrict__ src, int64_t rows, int64_t cols,
                                                       float* __restrict__ dst) {
    __shared__ float t[32][33];
    const int64_t c0 = (int64_t)blockIdx.x * 32, r0 = (int64_t)blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 × 8
    for (int j = ty; j < 32; j += 8) {
        const int64_t r = r0 + j, c = c0 + tx;
        if (r < rows && c < cols) t[j][tx] = src[r * cols + c];
    }
    __syncthreads();
    for (int j = ty; j < 32; j += 8) {
        const int64_t c = c0 + j, r = r0 + tx;
        if (r < rows && c < cols) dst[c * rows + r] = t[tx][j];
    }
}

static int requant_launch(int dtype, const float* src, int64_t rows, int64_t cols, uint8_t* dst, hipStream_t s) {
    const int64_t bs = dtype == AETH_DTYPE_Q8_0 ? 32 : 256;
    const int64_t bpr = aeth_cdiv(cols, bs), nblk = rows * bpr;
    if (nblk == 0) return AETH_OK;
    if (aeth_cdiv(nblk, 256) > 0x7FFFFFFF) return aeth_set_error(AETH_EINVAL, "requantize: too many blocks");
    const dim3 grid((unsigned)aeth_cdiv(nblk, 256));
    if (dtype == AETH_DTYPE_Q8_0) hipLaunchKernelGGL(k_requant_q8_0, grid, dim3(256), 0, s, src, rows, cols, bpr, dst);
    else if (dtype == AETH_DTYPE_Q4_K) hipLaunchKernelGGL(k_requant_qk<false>, grid, dim3(256), 0, s, src, rows, cols, bpr, dst);
    else if (dtype == AETH_DTYPE_Q5_K) hipLaunchKernelGGL(k_requant_qk<true>, grid, dim3(256), 0, s, src, rows, cols, bpr, dst);
    else hipLaunchKernelGGL(k_requant_q6_k, grid, dim3(256), 0, s, src, rows, cols, bpr, dst);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}

static bool requant_dtype(int dtype) {
    return dtype == AETH_DTYPE_Q8_0 || dtype == AETH_DTYPE_Q4_K || dtype == AETH_DTYPE_Q5_K || dtype == AETH_DTYPE_Q6_K;
}

extern "C" AETH_API int aeth_requantize(int dtype, const float* d_src, int64_t rows, int64_t cols, void* d_dst,
                                        void* stream) {
    if (!requant_dtype(dtype)) return aeth_set_error(AETH_EUNSUPPORTED, "aeth_requantize: unsupported dtype %d", dtype);
    if (rows < 0 || cols <= 0 || (rows > 0 && (!d_src || !d_dst)))
        return aeth_set_error(AETH_EINVAL, "aeth_requantize: bad argument");
    return requant_launch(dtype, d_src, rows, cols, (uint8_t*)d_dst, (hipStream_t)stream);
}

extern "C" AETH_API int aeth_quantize_activations_q8_0(const float* d_a, int64_t m, int64_t k, void* d_dst,
                                                       void* stream) {
    if (m < 0 || k <= 0 || (m > 0 && (!d_a || !d_dst)))
        return aeth_set_error(AETH_EINVAL, "aeth_quantize_activations_q8_0: bad argument");
    const int64_t bpr = aeth_cdiv(k, 32), nblk = m * bpr;
    if (nblk == 0) return AETH_OK;
    hipLaunchKernelGGL(k_quant_act_q8_0, dim3((unsigned)aeth_cdiv(nblk, 256)), dim3(256), 0, (hipStream_t)stream, d_a,
                       m, k, bpr, (uint8_t*)d_dst);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}

extern "C" AETH_API int aeth_transpose_f32(const float* d_src, int64_t rows, int64_t cols, float* d_dst,
                                           void* stream) {
    if (rows < 0 || cols < 0 || (rows * cols > 0 && (!d_src || !d_dst)) || d_src == d_dst)
        return aeth_set_error(AETH_EINVAL, "aeth_transpose_f32: bad argument");
    if (rows == 0 || cols == 0) return AETH_OK;
    if (aeth_cdiv(rows, 32) > 65535) return aeth_set_error(AETH_EINVAL, "aeth_transpose_f32: rows=%lld too large", (long long)rows);
    hipLaunchKernelGGL(k_transpose_f32, dim3((unsigned)aeth_cdiv(cols, 32), (unsigned)aeth_cdiv(rows, 32)), dim3(256),
                       0, (hipStream_t)stream, d_src, rows, cols, d_dst);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}

extern "C" AETH_API int64_t aeth_load_quant_ws_bytes(int64_t k, int64_t n) {
    if (k <= 0 || n <= 0) return 0;
    int64_t kn = 0;
    if (!aeth_mul_ok(k, n, &kn) || kn > INT64_MAX / 8) return -1;  // too large for any device
    return 2 * kn * (int64_t)sizeof(float);
}

// load_quant for a 2-D quantized tensor, model_loader.rs:330-386: GGUF shape
// [k, n] (k·n elements, dequantized as one flat run of blocks and read as a
// row-major [k][n] matrix) → [n][k] f32 → requantized rows of k.
extern "C" AETH_API int aeth_load_quant(int dtype, const void* d_src, int64_t k, int64_t n, void* d_dst,
                                        void* d_ws, void* stream) {
    if (!requant_dtype(dtype)) return aeth_set_error(AETH_EUNSUPPORTED, "aeth_load_quant: unsupported dtype %d", dtype);
    if (k <= 0 || n <= 0 || !d_src || !d_dst || !d_ws) return aeth_set_error(AETH_EINVAL, "aeth_load_quant: bad argument");
    hipStream_t s = (hipStream_t)stream;
    float* flat = (float*)d_ws;
    float* tr = flat + k * n;
    // the K-quants dequantize whole blocks only; the reference's output starts zeroed
    AETH_HIP_CHECK(hipMemsetAsync(flat, 0, (size_t)k * n * sizeof(float), s));
    int rc = aeth_dequant(dtype, d_src, k * n, flat, stream);
    if (rc != AETH_OK) return rc;
    rc = aeth_transpose_f32(flat, k, n, tr, stream);
    if (rc != AETH_OK) return rc;
    return requant_launch(dtype, tr, n, k, (uint8_t*)d_dst, s);
}
