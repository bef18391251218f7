/*
 * oracle.c — CPU restatement of the reference's quantized-matmul hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the parity checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it. The
 * product library (aether_amd/libaether_hip.so) never links or calls it.
 *
 * The reference (theoxfaber/aether) is Rust and cannot be built here (no
 * rustc/cargo); every function below restates the Rust source text it
 * cites, keeping its floating-point operation order. Build with
 * -ffp-contract=off (Rust never contracts a*b+c into an FMA).
 *
 * Pinning (what checks each function against something other than itself):
 *   orc_f16_to_f32 / orc_f32_to_f16  exhaustive / 2^20-sample comparison with
 *                                    numpy float16 and F16C vcvtps2ph.
 *   orc_decode_d                     all 65536 patterns vs numpy + bits/65536 rule.
 *   orc_get_scale_min_k4             round trip with the packing of
 *                                    requantize_q4_k over all (sc,m) in [0,63]^2.
 *   dequant_*                        reference KATs (tests/gguf_loader.rs:180-221),
 *                                    closed-form per-element formula on random
 *                                    blocks, requantize round trips
 *                                    (tests/correctness.rs:1253-1316).
 *   avx2_matmul_*                    AVX2-intrinsic form == scalar op-order form
 *                                    bit for bit; f64 brute force of dequantized
 *                                    rows; reference tolerance vs scalar kernels
 *                                    (src/quant/matmul/tests.rs:386-508);
 *                                    requantize(1.0)/a=0.5 closed form
 *                                    (benches/quant_matmul.rs:11-14).
 *   quantize_q8_0_block / dotprod    integer-exact dot vs f64 brute force; hand
 *                                    cases (d=0, ties-to-even, saturation).
 *   rmsnorm / rope / attn / argmax   closed forms (constant vectors, pos 0
 *                                    identity, norm preservation, one-hot KV,
 *                                    ties → last index).
 *   decode step                      composed of the pinned pieces; checked
 *                                    against a numpy re-composition in tests.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>
#if defined(__AVX2__)
#include <immintrin.h>
#endif

#include "oracle.h"

/* ── f16 <-> f32 (third-party `half` 2.7.1, Cargo.lock:926-928) ─────────── */

/* Exact IEEE binary16 → binary32 (half::f16::to_f32). */
ORC_API float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: normalise */
            int e = -1;
            do { man <<= 1; e++; } while ((man & 0x400u) == 0);
            man &= 0x3FFu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13) | (man ? 0x400000u : 0u);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* binary32 → binary16, round-to-nearest-even (half::f16::from_f32). */
ORC_API uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (exp == 0xFF) {
        if (man) return (uint16_t)(sign | 0x7E00u | (man >> 13));
        return (uint16_t)(sign | 0x7C00u);
    }
    int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t mm = man | 0x800000u;
        int shift = 14 - e;
        uint32_t hm = mm >> shift;
        uint32_t rem = mm & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (hm & 1u))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t hm = man >> 13;
    uint32_t rem = man & 0x1FFFu;
    uint32_t r = sign | ((uint32_t)e << 10) | hm;
    if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) r++;
    return (uint16_t)r;
}

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* decode_f16_scale, src/quant/matmul/common.rs:19-27 (≡ decode_d,
 * src/loader/dequant.rs:161-168): NaN/Inf patterns decode to bits/65536. */
ORC_API float orc_decode_d(uint16_t bits) {
    float f = orc_f16_to_f32(bits);
    if (isnan(f) || isinf(f)) return (float)bits / 65536.0f;
    return f;
}

/* get_scale_min_k4, src/quant/matmul/common.rs:29-38. */
ORC_API void orc_get_scale_min_k4(int j, const uint8_t* s, uint8_t* sc, uint8_t* m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* ── Dequantization (src/loader/dequant.rs) ─────────────────────────────── */

/* dequant_q8_0, dequant.rs:103-127: plain f16 scale, out = q * d. */
ORC_API void orc_dequant_q8_0(const uint8_t* data, size_t data_len, size_t n, float* out) {
    size_t nb = (n + 31) / 32;
    memset(out, 0, n * sizeof(float));
    for (size_t b = 0; b < nb; b++) {
        size_t off = b * 34;
        if (off + 34 > data_len) break;
        float d = orc_f16_to_f32(rd16(data + off));
        for (size_t i = 0; i < 32; i++) {
            size_t idx = b * 32 + i;
            if (idx >= n) break;
            float q = (float)(int8_t)data[off + 2 + i];
            out[idx] = q * d;
        }
    }
}

/* dequant_q4_k_block, dequant.rs:516-541 (tensor form :195-227). */
ORC_API void orc_dequant_q4_k_block(const uint8_t* blk, float* out) {
    float d = orc_decode_d(rd16(blk));
    float dmin = orc_decode_d(rd16(blk + 2));
    const uint8_t* scales = blk + 4;
    const uint8_t* qs = blk + 16;
    for (int is = 0; is < 8; is += 2) {
        uint8_t sc0, m0, sc1, m1;
        orc_get_scale_min_k4(is, scales, &sc0, &m0);
        orc_get_scale_min_k4(is + 1, scales, &sc1, &m1);
        float d1 = d * (float)sc0, mm1 = dmin * (float)m0;
        float d2 = d * (float)sc1, mm2 = dmin * (float)m1;
        for (int l = 0; l < 32; l++) {
            out[is * 32 + l] = d1 * (float)(qs[l] & 0x0F) - mm1;
            out[(is + 1) * 32 + l] = d2 * (float)((qs[l] >> 4) & 0x0F) - mm2;
        }
        qs += 32;
    }
}

/* dequant_q4_k, dequant.rs:195-227: n/256 whole blocks (tail left zero). */
ORC_API void orc_dequant_q4_k(const uint8_t* data, size_t n, float* out) {
    memset(out, 0, n * sizeof(float));
    for (size_t b = 0; b < n / 256; b++) orc_dequant_q4_k_block(data + b * 144, out + b * 256);
}

/* dequant_q6_k_block, dequant.rs:585-623 (tensor form :301-348). */
ORC_API void orc_dequant_q6_k_block(const uint8_t* blk, float* out) {
    float d = orc_decode_d(rd16(blk + 208));
    const uint8_t* ql = blk;
    const uint8_t* qh = blk + 128;
    const uint8_t* sc = blk + 192;
    for (int h = 0; h < 2; h++) {
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            uint32_t a = ql[h * 64 + l], a32 = ql[h * 64 + l + 32], hb = qh[h * 32 + l];
            int q1 = (int)((a & 0x0F) | ((hb & 0x03) << 4)) - 32;
            int q2 = (int)((a32 & 0x0F) | ((hb & 0x0C) << 2)) - 32;
            int q3 = (int)((a >> 4) | (hb & 0x30)) - 32;
            int q4 = (int)((a32 >> 4) | ((hb & 0xC0) >> 2)) - 32;
            float s1 = (float)(int8_t)sc[h * 8 + is], s2 = (float)(int8_t)sc[h * 8 + is + 2];
            float s3 = (float)(int8_t)sc[h * 8 + is + 4], s4 = (float)(int8_t)sc[h * 8 + is + 6];
            float* o = out + h * 128;
            o[l] = d * s1 * (float)q1;
            o[l + 32] = d * s2 * (float)q2;
            o[l + 64] = d * s3 * (float)q3;
            o[l + 96] = d * s4 * (float)q4;
        }
    }
}

ORC_API void orc_dequant_q6_k(const uint8_t* data, size_t n, float* out) {
    memset(out, 0, n * sizeof(float));
    for (size_t b = 0; b < n / 256; b++) orc_dequant_q6_k_block(data + b * 210, out + b * 256);
}

/* ── AVX2 f32-pipeline matmuls (src/quant/avx2.rs) ─────────────────────────
 * c[row*n+col] = Σ_blk Σ_{i step 8} hsum_f32x8(a[i..i+8] * deq[i..i+8]).
 * hsum_f32x8 (avx2.rs:13-20): s_i = v_i + v_{i+4}; ((s0+s1)+(s2+s3)).
 * Each function has an intrinsic form (used when built with -mavx2) and a
 * scalar form with the identical operation order; tests check they agree
 * bit for bit. */

static inline float hsum8_scalar(const float* p) {
    float s0 = p[0] + p[4], s1 = p[1] + p[5], s2 = p[2] + p[6], s3 = p[3] + p[7];
    return (s0 + s1) + (s2 + s3);
}

typedef void (*orc_deq_block_fn)(const uint8_t*, float*);

static void kquant_avx2_order_scalar(orc_deq_block_fn deq_fn, size_t blk_bytes, const float* a,
                                     const uint8_t* b, size_t m, size_t n, size_t k, float* c) {
    size_t nb = k / 256;
    float deq[256], prod[8];
    for (size_t row = 0; row < m; row++) {
        for (size_t col = 0; col < n; col++) {
            float sum = 0.0f;
            for (size_t blk = 0; blk < nb; blk++) {
                deq_fn(b + (col * nb + blk) * blk_bytes, deq);
                const float* ad = a + row * k + blk * 256;
                float block_sum = 0.0f;
                for (int i = 0; i < 256; i += 8) {
                    for (int j = 0; j < 8; j++) prod[j] = ad[i + j] * deq[i + j];
                    block_sum += hsum8_scalar(prod);
                }
                sum += block_sum;
            }
            c[row * n + col] = sum;
        }
    }
}

#if defined(__AVX2__)
static inline float hsum8_avx(__m256 v) {
    __m128 hi = _mm256_extractf128_ps(v, 1);
    __m128 lo = _mm256_castps256_ps128(v);
    __m128 s = _mm_add_ps(lo, hi);
    s = _mm_hadd_ps(s, s);
    s = _mm_hadd_ps(s, s);
    return _mm_cvtss_f32(s);
}

static void kquant_avx2(orc_deq_block_fn deq_fn, size_t blk_bytes, const float* a, const uint8_t* b,
                        size_t m, size_t n, size_t k, float* c) {
    size_t nb = k / 256;
    float deq[256] __attribute__((aligned(32)));
    for (size_t row = 0; row < m; row++) {
        for (size_t col = 0; col < n; col++) {
            float sum = 0.0f;
            for (size_t blk = 0; blk < nb; blk++) {
                deq_fn(b + (col * nb + blk) * blk_bytes, deq);
                const float* ad = a + row * k + blk * 256;
                float block_sum = 0.0f;
                for (int i = 0; i < 256; i += 8) {
                    __m256 p = _mm256_mul_ps(_mm256_loadu_ps(ad + i), _mm256_load_ps(deq + i));
                    block_sum += hsum8_avx(p);
                }
                sum += block_sum;
            }
            c[row * n + col] = sum;
        }
    }
}
#endif

/* avx2::matmul_q4_k, avx2.rs:23-57. */
ORC_API void orc_avx2_matmul_q4_k(const float* a, const uint8_t* b, size_t m, size_t n, size_t k,
                                  float* c) {
#if defined(__AVX2__)
    kquant_avx2(orc_dequant_q4_k_block, 144, a, b, m, n, k, c);
#else
    kquant_avx2_order_scalar(orc_dequant_q4_k_block, 144, a, b, m, n, k, c);
#endif
}

/* avx2::matmul_q6_k, avx2.rs:60-94. */
ORC_API void orc_avx2_matmul_q6_k(const float* a, const uint8_t* b, size_t m, size_t n, size_t k,
                                  float* c) {
#if defined(__AVX2__)
    kquant_avx2(orc_dequant_q6_k_block, 210, a, b, m, n, k, c);
#else
    kquant_avx2_order_scalar(orc_dequant_q6_k_block, 210, a, b, m, n, k, c);
#endif
}

/* avx2::matmul_q5_k, avx2.rs:97-131 (dequant_q5_k_block, dequant.rs:542-584). */
ORC_API void orc_avx2_matmul_q5_k(const float* a, const uint8_t* b, size_t m, size_t n, size_t k,
                                  float* c) {
#if defined(__AVX2__)
    kquant_avx2(orc_dequant_q5_k_block, 176, a, b, m, n, k, c);
#else
    kquant_avx2_order_scalar(orc_dequant_q5_k_block, 176, a, b, m, n, k, c);
#endif
}

ORC_API void orc_avx2order_scalar_matmul_q5_k(const float* a, const uint8_t* b, size_t m, size_t n,
                                              size_t k, float* c) {
    kquant_avx2_order_scalar(orc_dequant_q5_k_block, 176, a, b, m, n, k, c);
}

ORC_API void orc_avx2order_scalar_matmul_q4_k(const float* a, const uint8_t* b, size_t m, size_t n,
                                              size_t k, float* c) {
    kquant_avx2_order_scalar(orc_dequant_q4_k_block, 144, a, b, m, n, k, c);
}

ORC_API void orc_avx2order_scalar_matmul_q6_k(const float* a, const uint8_t* b, size_t m, size_t n,
                                              size_t k, float* c) {
    kquant_avx2_order_scalar(orc_dequant_q6_k_block, 210, a, b, m, n, k, c);
}

/* avx2::matmul_q8_0, avx2.rs:134-207, restated WITH its addressing defect:
 * `ptr.add(1)` on a `*const __m128i` advances 16 bytes, so within each
 * 16-element step the second 8 products use quant bytes [i+16, i+24) of the
 * block instead of [i+8, i+16); at i=16 that is bytes 32..39 past the quant
 * start, i.e. the next block's scale and first quants. Bytes at or past
 * b_len (the last block's over-read, undefined in the reference) read as 0.
 * Kept only to document why the GPU Q8_0 path follows the scalar kernel. */
ORC_API void orc_avx2_matmul_q8_0(const float* a, const uint8_t* b, size_t b_len, size_t m, size_t n,
                                  size_t k, float* c) {
    size_t nb = k / 32;
    for (size_t row = 0; row < m; row++) {
        for (size_t col = 0; col < n; col++) {
            float sum = 0.0f;
            for (size_t blk = 0; blk < nb; blk++) {
                size_t off = (col * nb + blk) * 34;
                float d = orc_f16_to_f32(rd16(b + off));
                size_t qo = off + 2;
                float block_sum = 0.0f;
                for (size_t i = 0; i + 16 <= 32; i += 16) {
                    float p1[8], p2[8];
                    const float* ad = a + row * k + blk * 32 + i;
                    for (int j = 0; j < 8; j++) {
                        size_t i1 = qo + i + j, i2 = qo + i + 16 + j;
                        float q1 = (float)(int8_t)(i1 < b_len ? b[i1] : 0);
                        float q2 = (float)(int8_t)(i2 < b_len ? b[i2] : 0);
                        p1[j] = q1 * ad[j];
                        p2[j] = q2 * ad[8 + j];
                    }
                    block_sum += hsum8_scalar(p1) + hsum8_scalar(p2);
                }
                sum += block_sum * d;
            }
            c[row * n + col] = sum;
        }
    }
}

/* ── Scalar / rayon kernels (second oracle) ─────────────────────────────── */

/* matmul_q8_0_scalar + batched form, src/quant/matmul/q8_0.rs:5-89:
 * acc += d * Σ_i a_i q_i (sequential sums, plain f16 d). */
ORC_API void orc_scalar_matmul_q8_0(const float* a, const uint8_t* b, size_t b_len, size_t m, size_t n,
                                    size_t k, float* c) {
    size_t bpr = (k + 31) / 32;
    for (size_t row = 0; row < m; row++) {
        const float* act = a + row * k;
        for (size_t col = 0; col < n; col++) {
            float acc = 0.0f;
            size_t rs = col * bpr * 34;
            for (size_t blk = 0; blk < bpr; blk++) {
                size_t bo = rs + blk * 34;
                if (bo + 34 > b_len) break;
                float d = orc_f16_to_f32(rd16(b + bo));
                size_t base = blk * 32;
                size_t cnt = (k - base) < 32 ? (k - base) : 32;
                float s = 0.0f;
                for (size_t i = 0; i < cnt; i++) s += act[base + i] * (float)(int8_t)b[bo + 2 + i];
                acc += d * s;
            }
            c[row * n + col] = acc;
        }
    }
}

/* matmul_q4_k_scalar (m=1), q4_k.rs:5-63: per element acc += a*(d1*q - m1),
 * lo and hi interleaved; matmul_q4_k_batched_scalar (m>1), q4_k.rs:65-145:
 * results += d1*Σaq - m1*Σa per 32-element sub-block. */
ORC_API void orc_scalar_matmul_q4_k(const float* a, const uint8_t* b, size_t m, size_t n, size_t k,
                                    float* c) {
    size_t nb = k / 256;
    for (size_t row = 0; row < m; row++) {
        const float* act = a + row * k;
        for (size_t col = 0; col < n; col++) {
            float acc = 0.0f;
            for (size_t blk = 0; blk < nb; blk++) {
                const uint8_t* bo = b + (col * nb + blk) * 144;
                float d = orc_decode_d(rd16(bo)), dmin = orc_decode_d(rd16(bo + 2));
                const uint8_t* scales = bo + 4;
                const uint8_t* qs = bo + 16;
                size_t eb = blk * 256;
                for (int is = 0; is < 8; is += 2) {
                    uint8_t sc0, m0, sc1, m1;
                    orc_get_scale_min_k4(is, scales, &sc0, &m0);
                    orc_get_scale_min_k4(is + 1, scales, &sc1, &m1);
                    float d1 = d * (float)sc0, mm1 = dmin * (float)m0;
                    float d2 = d * (float)sc1, mm2 = dmin * (float)m1;
                    const uint8_t* q = qs + (is / 2) * 32;
                    if (m == 1) {
                        for (int l = 0; l < 32; l++) {
                            float qlo = (float)(q[l] & 0x0F), qhi = (float)((q[l] >> 4) & 0x0F);
                            acc += act[eb + is * 32 + l] * (d1 * qlo - mm1);
                            acc += act[eb + (is + 1) * 32 + l] * (d2 * qhi - mm2);
                        }
                    } else {
                        float aq_lo = 0, a_lo = 0, aq_hi = 0, a_hi = 0;
                        for (int l = 0; l < 32; l++) {
                            float vlo = act[eb + is * 32 + l], vhi = act[eb + (is + 1) * 32 + l];
                            aq_lo += vlo * (float)(q[l] & 0x0F);
                            a_lo += vlo;
                            aq_hi += vhi * (float)((q[l] >> 4) & 0x0F);
                            a_hi += vhi;
                        }
                        acc += d1 * aq_lo - mm1 * a_lo;
                        acc += d2 * aq_hi - mm2 * a_hi;
                    }
                }
            }
            c[row * n + col] = acc;
        }
    }
}

/* matmul_q6_k_scalar (m=1), q6_k.rs:5-92 and batched form q6_k.rs:94-190. */
ORC_API void orc_scalar_matmul_q6_k(const float* a, const uint8_t* b, size_t m, size_t n, size_t k,
                                    float* c) {
    size_t nb = k / 256;
    for (size_t row = 0; row < m; row++) {
        const float* act = a + row * k;
        for (size_t col = 0; col < n; col++) {
            float acc = 0.0f;
            for (size_t blk = 0; blk < nb; blk++) {
                const uint8_t* bo = b + (col * nb + blk) * 210;
                float d = orc_decode_d(rd16(bo + 208));
                const uint8_t *ql = bo, *qh = bo + 128, *sc = bo + 192;
                size_t eb = blk * 256;
                for (int h = 0; h < 2; h++) {
                    for (int l = 0; l < 32; l += 16) {
                        int is = l / 16;
                        float ds1 = d * (float)(int8_t)sc[h * 8 + is];
                        float ds2 = d * (float)(int8_t)sc[h * 8 + is + 2];
                        float ds3 = d * (float)(int8_t)sc[h * 8 + is + 4];
                        float ds4 = d * (float)(int8_t)sc[h * 8 + is + 6];
                        size_t hb = eb + h * 128 + l;
                        int8_t q1[16], q2[16], q3[16], q4[16];
                        for (int t = 0; t < 16; t++) {
                            uint8_t A = ql[h * 64 + l + t], B = ql[h * 64 + l + 32 + t], H = qh[h * 32 + l + t];
                            q1[t] = (int8_t)((A & 0x0F) | ((H & 0x03) << 4)) - 32;
                            q2[t] = (int8_t)((B & 0x0F) | ((H & 0x0C) << 2)) - 32;
                            q3[t] = (int8_t)((A >> 4) | (H & 0x30)) - 32;
                            q4[t] = (int8_t)((B >> 4) | ((H & 0xC0) >> 2)) - 32;
                        }
                        if (m == 1) {
                            for (int t = 0; t < 16; t++) {
                                acc += act[hb + t] * (ds1 * (float)q1[t]);
                                acc += act[hb + 32 + t] * (ds2 * (float)q2[t]);
                                acc += act[hb + 64 + t] * (ds3 * (float)q3[t]);
                                acc += act[hb + 96 + t] * (ds4 * (float)q4[t]);
                            }
                        } else {
                            float a1 = 0, a2 = 0, a3 = 0, a4 = 0;
                            for (int t = 0; t < 16; t++) {
                                a1 += act[hb + t] * (float)q1[t];
                                a2 += act[hb + 32 + t] * (float)q2[t];
                                a3 += act[hb + 64 + t] * (float)q3[t];
                                a4 += act[hb + 96 + t] * (float)q4[t];
                            }
                            acc += ds1 * a1 + ds2 * a2 + ds3 * a3 + ds4 * a4;
                        }
                    }
                }
            }
            c[row * n + col] = acc;
        }
    }
}

/* ── Re-quantizers (src/quant/matmul/dispatch.rs:149-184, 186-300, 431-537).
 * Rust f32::round is round-half-away-from-zero (C roundf). */

ORC_API void orc_requantize_q8_0(const float* data, size_t rows, size_t cols, uint8_t* out) {
    size_t bpr = (cols + 31) / 32;
    for (size_t r = 0; r < rows; r++) {
        for (size_t blk = 0; blk < bpr; blk++) {
            size_t start = r * cols + blk * 32;
            size_t end = start + 32 < r * cols + cols ? start + 32 : r * cols + cols;
            size_t actual = end - start;
            uint8_t* o = out + (r * bpr + blk) * 34;
            float mx = 0.0f;
            for (size_t i = 0; i < actual; i++) mx = fmaxf(mx, fabsf(data[start + i]));
            float d = mx == 0.0f ? 1.0f : mx / 127.0f;
            uint16_t db = orc_f32_to_f16(d);
            o[0] = db & 0xFF;
            o[1] = db >> 8;
            for (size_t j = 0; j < 32; j++) {
                int8_t q = 0;
                if (j < actual) {
                    float v = roundf(data[start + j] / d);
                    v = fmaxf(v, -128.0f);
                    v = fminf(v, 127.0f);
                    q = (int8_t)v;
                }
                o[2 + j] = (uint8_t)q;
            }
        }
    }
}

ORC_API void orc_requantize_q4_k(const float* data, size_t rows, size_t cols, uint8_t* out) {
    size_t bpr = (cols + 255) / 256;
    for (size_t r = 0; r < rows; r++) {
        for (size_t blk = 0; blk < bpr; blk++) {
            size_t start = r * cols + blk * 256;
            size_t end = start + 256 < r * cols + cols ? start + 256 : r * cols + cols;
            size_t actual = end - start;
            const float* block = data + start;
            uint8_t* o = out + (r * bpr + blk) * 144;
            float mins[8] = {0}, maxs[8] = {0}, msub[8], dsub[8];
            for (int sb = 0; sb < 8; sb++) {
                size_t s0 = (size_t)sb * 32;
                if (s0 < actual) {
                    size_t s1 = s0 + 32 < actual ? s0 + 32 : actual;
                    float mn = block[s0], mx = block[s0];
                    for (size_t i = s0; i < s1; i++) {
                        mn = fminf(mn, block[i]);
                        mx = fmaxf(mx, block[i]);
                    }
                    mins[sb] = mn;
                    maxs[sb] = mx;
                }
            }
            for (int sb = 0; sb < 8; sb++) {
                msub[sb] = fabsf(fminf(mins[sb], 0.0f));
                dsub[sb] = (maxs[sb] + msub[sb]) / 15.0f;
            }
            float maxd = 0.0f, maxm = 0.0f;
            for (int sb = 0; sb < 8; sb++) {
                maxd = fmaxf(maxd, dsub[sb]);
                maxm = fmaxf(maxm, msub[sb]);
            }
            float d = maxd == 0.0f ? 1.0f : maxd / 63.0f;
            float dmin = maxm == 0.0f ? 1.0f : maxm / 63.0f;
            uint16_t db = orc_f32_to_f16(d), dmb = orc_f32_to_f16(dmin);
            o[0] = db & 0xFF; o[1] = db >> 8; o[2] = dmb & 0xFF; o[3] = dmb >> 8;
            uint8_t sc[8], mm[8];
            for (int sb = 0; sb < 8; sb++) {
                sc[sb] = (uint8_t)fminf(fmaxf(roundf(dsub[sb] / d), 0.0f), 63.0f);
                mm[sb] = (uint8_t)fminf(fmaxf(roundf(msub[sb] / dmin), 0.0f), 63.0f);
            }
            for (int q = 0; q < 4; q++) {
                o[4 + q] = (uint8_t)((sc[q] & 63) | ((sc[q + 4] >> 4) << 6));
                o[8 + q] = (uint8_t)((mm[q] & 63) | ((mm[q + 4] >> 4) << 6));
                o[12 + q] = (uint8_t)((sc[q + 4] & 0x0F) | ((mm[q + 4] & 0x0F) << 4));
            }
            for (int ch = 0; ch < 4; ch++) {
                int is = ch * 2;
                float d1 = d * (float)sc[is], m1 = dmin * (float)mm[is];
                float d2 = d * (float)sc[is + 1], m2 = dmin * (float)mm[is + 1];
                for (int l = 0; l < 32; l++) {
                    size_t i0 = (size_t)is * 32 + l, i1 = (size_t)(is + 1) * 32 + l;
                    uint8_t q0 = 0, q1 = 0;
                    if (i0 < actual && d1 != 0.0f)
                        q0 = (uint8_t)fminf(fmaxf(roundf((block[i0] + m1) / d1), 0.0f), 15.0f);
                    if (i1 < actual && d2 != 0.0f)
                        q1 = (uint8_t)fminf(fmaxf(roundf((block[i1] + m2) / d2), 0.0f), 15.0f);
                    o[16 + ch * 32 + l] = (uint8_t)(q0 | (q1 << 4));
                }
            }
        }
    }
}

ORC_API void orc_requantize_q6_k(const float* data, size_t rows, size_t cols, uint8_t* out) {
    size_t bpr = (cols + 255) / 256;
    for (size_t r = 0; r < rows; r++) {
        for (size_t blk = 0; blk < bpr; blk++) {
            size_t start = r * cols + blk * 256;
            size_t end = start + 256 < r * cols + cols ? start + 256 : r * cols + cols;
            size_t actual = end - start;
            const float* block = data + start;
            uint8_t* o = out + (r * bpr + blk) * 210;
            float sub[16] = {0};
            for (int sb = 0; sb < 16; sb++) {
                size_t s0 = (size_t)sb * 16;
                if (s0 < actual) {
                    size_t s1 = s0 + 16 < actual ? s0 + 16 : actual;
                    float mx = fabsf(block[s0]);
                    for (size_t i = s0; i < s1; i++) mx = fmaxf(mx, fabsf(block[i]));
                    sub[sb] = mx;
                }
            }
            float mv = 0.0f;
            for (int sb = 0; sb < 16; sb++) mv = fmaxf(mv, sub[sb]);
            float d = mv == 0.0f ? 1.0f : mv / (32.0f * 127.0f);
            uint8_t sc[16];
            for (int sb = 0; sb < 16; sb++) {
                sc[sb] = (uint8_t)fminf(fmaxf(roundf(sub[sb] / (32.0f * d)), 0.0f), 127.0f);
                o[192 + sb] = sc[sb];
            }
            uint16_t db = orc_f32_to_f16(d);
            o[208] = db & 0xFF;
            o[209] = db >> 8;
            for (int h = 0; h < 2; h++) {
                for (int l = 0; l < 32; l++) {
                    int is = l / 16;
                    float s[4];
                    int q[4];
                    for (int t = 0; t < 4; t++) {
                        s[t] = (float)sc[h * 8 + is + 2 * t];
                        size_t idx = (size_t)h * 128 + (size_t)l + 32u * (size_t)t;
                        q[t] = 0;
                        if (idx < actual && s[t] > 0.0f)
                            q[t] = (int)fminf(fmaxf(roundf(block[idx] / (d * s[t])), -32.0f), 31.0f);
                    }
                    uint8_t u[4];
                    for (int t = 0; t < 4; t++) u[t] = (uint8_t)(q[t] + 32);
                    o[h * 64 + l] = (uint8_t)((u[0] & 0x0F) | ((u[2] & 0x0F) << 4));
                    o[h * 64 + l + 32] = (uint8_t)((u[1] & 0x0F) | ((u[3] & 0x0F) << 4));
                    o[128 + h * 32 + l] =
                        (uint8_t)((u[0] >> 4) | ((u[1] >> 4) << 2) | ((u[2] >> 4) << 4) | ((u[3] >> 4) << 6));
                }
            }
        }
    }
}

/* ── Q8_0 activation scheme (src/quant/matmul/neon.rs:45-155) ───────────── */

static inline float nan_max(float a, float b) { /* vmaxq_f32: NaN propagates */
    if (isnan(a) || isnan(b)) return NAN;
    return a > b ? a : b;
}

/* vcvtnq_s32_f32: round to nearest, ties to even, saturating; NaN → 0. */
static inline int32_t cvtn_s32(float v) {
    if (isnan(v)) return 0;
    if (v >= 2147483648.0f) return INT32_MAX;
    if (v < -2147483648.0f) return INT32_MIN;
    return (int32_t)nearbyintf(v); /* default FE_TONEAREST */
}

/* quantize_q8_0_block, neon.rs:45-104: d = max|x|/127 (f32), stored as f16;
 * q = sat_i8(sat_i16(RNE(x * (1/d)))) using the f32 d; d <= 0 or NaN → zeros. */
ORC_API void orc_quantize_q8_0_block(const float* src, uint8_t* dst) {
    float mx = fabsf(src[0]);
    for (int i = 1; i < 32; i++) mx = nan_max(mx, fabsf(src[i]));
    float d = mx / 127.0f;
    uint16_t db = orc_f32_to_f16(d);
    dst[0] = db & 0xFF;
    dst[1] = db >> 8;
    if (d > 0.0f) {
        float inv = 1.0f / d;
        for (int i = 0; i < 32; i++) {
            int32_t q = cvtn_s32(src[i] * inv);
            if (q > 32767) q = 32767;
            if (q < -32768) q = -32768;
            if (q > 127) q = 127;
            if (q < -128) q = -128;
            dst[2 + i] = (uint8_t)(int8_t)q;
        }
    } else {
        memset(dst + 2, 0, 32);
    }
}

/* quantize_activations_q8_0[_batched], neon.rs:106-155 (tail zero-padded). */
ORC_API void orc_quantize_activations_q8_0(const float* a, size_t m, size_t k, uint8_t* out) {
    size_t blocks = (k + 31) / 32;
    for (size_t r = 0; r < m; r++) {
        const float* src = a + r * k;
        uint8_t* dst = out + r * blocks * 34;
        size_t i = 0;
        for (; i + 32 <= k; i += 32) orc_quantize_q8_0_block(src + i, dst + (i / 32) * 34);
        if (i < k) {
            float buf[32] = {0};
            memcpy(buf, src + i, (k - i) * sizeof(float));
            orc_quantize_q8_0_block(buf, dst + (i / 32) * 34);
        }
    }
}

/* matmul_q4_k_dotprod_reference, src/quant/matmul/tests.rs:62-134:
 * exact i32 dots per 32-element sub-block against Q8_0 activation blocks,
 * acc += d_a * (d1*dot - m1*Σq_a). */
ORC_API void orc_dotprod_ref_q4_k(const uint8_t* aq, const uint8_t* b, size_t m, size_t n, size_t k,
                                  float* c) {
    size_t nb = k / 256;
    for (size_t row = 0; row < m; row++) {
        for (size_t col = 0; col < n; col++) {
            float acc = 0.0f;
            for (size_t blk = 0; blk < nb; blk++) {
                const uint8_t* bo = b + (col * nb + blk) * 144;
                float d = orc_decode_d(rd16(bo)), dmin = orc_decode_d(rd16(bo + 2));
                for (int is = 0; is < 8; is += 2) {
                    uint8_t sc0, m0, sc1, m1;
                    orc_get_scale_min_k4(is, bo + 4, &sc0, &m0);
                    orc_get_scale_min_k4(is + 1, bo + 4, &sc1, &m1);
                    float d1 = d * (float)sc0, mm1 = dmin * (float)m0;
                    float d2 = d * (float)sc1, mm2 = dmin * (float)m1;
                    const uint8_t* q = bo + 16 + (is / 2) * 32;
                    const uint8_t* alo = aq + (row * nb * 8 + blk * 8 + is) * 34;
                    const uint8_t* ahi = aq + (row * nb * 8 + blk * 8 + is + 1) * 34;
                    float da1 = orc_f16_to_f32(rd16(alo)), da2 = orc_f16_to_f32(rd16(ahi));
                    int32_t dlo = 0, slo = 0, dhi = 0, shi = 0;
                    for (int l = 0; l < 32; l++) {
                        int32_t vlo = (int8_t)alo[2 + l], vhi = (int8_t)ahi[2 + l];
                        dlo += (q[l] & 0x0F) * vlo;
                        slo += vlo;
                        dhi += ((q[l] >> 4) & 0x0F) * vhi;
                        shi += vhi;
                    }
                    acc += da1 * (d1 * (float)dlo - mm1 * (float)slo);
                    acc += da2 * (d2 * (float)dhi - mm2 * (float)shi);
                }
            }
            c[row * n + col] = acc;
        }
    }
}

/* matmul_q8_0_dotprod_reference, tests.rs:28-60. */
ORC_API void orc_dotprod_ref_q8_0(const uint8_t* aq, const uint8_t* b, size_t m, size_t n, size_t k,
                                  float* c) {
    size_t bpr = (k + 31) / 32;
    for (size_t row = 0; row < m; row++) {
        for (size_t col = 0; col < n; col++) {
            float acc = 0.0f;
            for (size_t blk = 0; blk < bpr; blk++) {
                const uint8_t* bo = b + (col * bpr + blk) * 34;
                const uint8_t* ao = aq + (row * bpr + blk) * 34;
                float dab = orc_f16_to_f32(rd16(ao)) * orc_f16_to_f32(rd16(bo));
                int32_t s = 0;
                for (int i = 0; i < 32; i++) s += (int32_t)(int8_t)ao[2 + i] * (int32_t)(int8_t)bo[2 + i];
                acc += (float)s * dab;
            }
            c[row * n + col] = acc;
        }
    }
}

/* ── Decode-step math (src/inference/runner.rs) ─────────────────────────── */

/* rmsnorm_inplace, runner.rs:1739-1746: ss = Σx² (sequential),
 * rms = sqrt(ss/n + eps), out = x / rms * w. */
ORC_API void orc_rmsnorm(const float* x, const float* w, size_t n, float eps, float* out) {
    float ss = 0.0f;
    for (size_t i = 0; i < n; i++) ss += x[i] * x[i];
    float rms = sqrtf(ss / (float)n + eps);
    for (size_t i = 0; i < n; i++) out[i] = x[i] / rms * w[i];
}

/* precompute_rope, runner.rs:1912-1924: θ = pos * base^(-2i/hd) (f32 powf). */
ORC_API void orc_precompute_rope(size_t max_seq, size_t head_dim, float base, float* sin_t,
                                 float* cos_t) {
    size_t half = head_dim / 2;
    for (size_t p = 0; p < max_seq; p++) {
        for (size_t i = 0; i < half; i++) {
            float theta = (float)p * powf(base, -2.0f * (float)i / (float)head_dim);
            sin_t[p * half + i] = sinf(theta);
            cos_t[p * half + i] = cosf(theta);
        }
    }
}

/* apply_rope_inplace, runner.rs:1886-1909: rotate halves (x_i, x_{i+hd/2});
 * pos clamped to max_seq-1. */
ORC_API void orc_apply_rope(float* x, size_t n_heads, size_t head_dim, size_t pos,
                            const float* sin_t, const float* cos_t, size_t max_seq) {
    size_t half = head_dim / 2;
    size_t p = pos < max_seq ? pos : (max_seq ? max_seq - 1 : 0);
    const float* s = sin_t + p * half;
    const float* c = cos_t + p * half;
    for (size_t h = 0; h < n_heads; h++) {
        float* hd = x + h * head_dim;
        for (size_t i = 0; i < half; i++) {
            float x0 = hd[i], x1 = hd[i + half];
            hd[i] = x0 * c[i] - x1 * s[i];
            hd[i + half] = x0 * s[i] + x1 * c[i];
        }
    }
}

/* attn_direct, runner.rs:1757-1801 (sliding window 0 = none). */
ORC_API void orc_attn_direct(const float* q, const float* k_st, const float* v_st, size_t seq,
                             size_t head_dim, size_t window, float* scores, float* out) {
    float scale = 1.0f / sqrtf((float)head_dim);
    size_t ws = (window && seq > window) ? seq - window : 0;
    for (size_t t = 0; t < ws; t++) scores[t] = -INFINITY;
    for (size_t t = ws; t < seq; t++) {
        float dot = 0.0f;
        for (size_t i = 0; i < head_dim; i++) dot += q[i] * k_st[t * head_dim + i];
        scores[t] = dot * scale;
    }
    float mx = -INFINITY;
    for (size_t t = 0; t < seq; t++) mx = fmaxf(mx, scores[t]);
    float sum = 0.0f;
    for (size_t t = 0; t < seq; t++) {
        scores[t] = expf(scores[t] - mx);
        sum += scores[t];
    }
    for (size_t t = 0; t < seq; t++) scores[t] /= sum;
    for (size_t i = 0; i < head_dim; i++) out[i] = 0.0f;
    for (size_t t = 0; t < seq; t++) {
        float w = scores[t];
        for (size_t i = 0; i < head_dim; i++) out[i] += w * v_st[t * head_dim + i];
    }
}

/* Greedy branch of sample(), runner.rs:1964-1973, and aether_argmax,
 * c_api.rs:384-396: Iterator::max_by keeps the LAST of equal maxima. */
ORC_API int32_t orc_argmax(const float* logits, size_t n) {
    size_t best = 0;
    for (size_t i = 1; i < n; i++)
        if (!(logits[i] < logits[best])) best = i;
    return (int32_t)best;
}

/* ── One decode step, CPU branch of forward_one_internal (runner.rs:1557-1646) */

/* LlamaConfig (model_loader.rs:71-84) as the runner uses it: max_seq is the
 * runner's cache length (min(max_seq_len, 4096), runner.rs:225 / :339);
 * sliding_window is ArchConfig::sliding_window (model_loader.rs:62-67, read
 * from attention.sliding_window_length :286), 0 for None. */
typedef struct {
    int32_t vocab, d_model, n_layers, n_heads, n_kv_heads, head_dim, d_ff, max_seq;
    float rope_base, eps;
    int32_t sliding_window;
} orc_llama_cfg;

enum { ORC_Q8_0 = 8, ORC_Q4_K = 12, ORC_Q5_K = 13, ORC_Q6_K = 14 };

/* quantized_matmul_impl's x86 route (dispatch.rs:98-135 → avx2_dispatch.rs), m rows:
 * Q4_K / Q5_K / Q6_K through the AVX2 f32 pipeline, Q8_0 through its scalar
 * kernel (the AVX2 one mis-addresses, above), every other format (F32, F16,
 * Q2_K, Q3_K: weights kept in GGUF [k][n] order) dequantized and multiplied
 * by matmul_f32_gguf. */
static void orc_qmatmul_m(int dtype, const float* a, size_t m, const uint8_t* w, size_t n, size_t k, float* c) {
    if (dtype == ORC_Q4_K) orc_avx2_matmul_q4_k(a, w, m, n, k, c);
    else if (dtype == ORC_Q5_K) orc_avx2_matmul_q5_k(a, w, m, n, k, c);
    else if (dtype == ORC_Q6_K) orc_avx2_matmul_q6_k(a, w, m, n, k, c);
    else if (dtype == ORC_Q8_0) orc_scalar_matmul_q8_0(a, w, n * ((k + 31) / 32) * 34, m, n, k, c);
    else if (orc_gguf_order_matmul(dtype, a, m, w, n, k, c) != 0) memset(c, 0, m * n * sizeof(float));
}

static void orc_qmatmul(int dtype, const float* a, const uint8_t* w, size_t n, size_t k, float* c) {
    orc_qmatmul_m(dtype, a, 1, w, n, k, c);
}

/* weights[l*7 + {0..6}] = q,k,v,o,gate,up,down: Q8_0/Q4_K/Q5_K/Q6_K as raw
 * row-major [out][in] blocks (load_quant's transposed form), F32/F16/Q2_K/Q3_K
 * as the file holds them, GGUF [in][out] order;
 * norms[l*2 + {0,1}] = attn_norm, ffn_norm; kv = StaticKVCache storage
 * [L][2][kv_heads][max_seq][hd] (kv_cache.rs:9-31); *seq_len is the cache's
 * fill and is advanced on return. x holds the token's embedding row. */
ORC_API int orc_decode_step_from(const orc_llama_cfg* cfg, const float* x_embed, int32_t pos, int32_t start_layer,
                                 const uint8_t* const* weights, const int32_t* wdtype,
                                 const float* const* norms, const float* final_norm,
                                 const uint8_t* lm_head, int32_t lm_dtype, const float* rope_sin,
                                 const float* rope_cos, float* kv, int32_t* seq_len, float* logits);

ORC_API int orc_decode_step(const orc_llama_cfg* cfg, const float* x_embed, int32_t pos,
                            const uint8_t* const* weights, const int32_t* wdtype,
                            const float* const* norms, const float* final_norm,
                            const uint8_t* lm_head, int32_t lm_dtype, const float* rope_sin,
                            const float* rope_cos, float* kv, int32_t* seq_len, float* logits) {
    return orc_decode_step_from(cfg, x_embed, pos, 0, weights, wdtype, norms, final_norm, lm_head, lm_dtype,
                                rope_sin, rope_cos, kv, seq_len, logits);
}

/* The same step entered at layer start_layer with x = the residual stream
 * after the layers before it: the resume of a budgeted decode
 * (forward_one_internal's start_layer = completed + 1 with the saved
 * partial.x, runner.rs:1201-1217). start_layer 0 is the plain step. */
ORC_API int orc_decode_step_from(const orc_llama_cfg* cfg, const float* x_embed, int32_t pos, int32_t start_layer,
                                 const uint8_t* const* weights, const int32_t* wdtype,
                                 const float* const* norms, const float* final_norm,
                                 const uint8_t* lm_head, int32_t lm_dtype, const float* rope_sin,
                                 const float* rope_cos, float* kv, int32_t* seq_len, float* logits) {
    size_t d = (size_t)cfg->d_model, hd = (size_t)cfg->head_dim, nh = (size_t)cfg->n_heads;
    size_t nkv = (size_t)cfg->n_kv_heads, dff = (size_t)cfg->d_ff, ms = (size_t)cfg->max_seq;
    size_t kvd = nkv * hd;
    /* the reference's append() refuses a full cache and attn_direct would then
     * index past max_seq (a panic in Rust); report it instead. */
    if (*seq_len < 0 || (size_t)*seq_len >= ms || start_layer < 0) return -2;
    float* x = malloc(d * 4);
    float* normed = malloc(d * 4);
    float* q = malloc(nh * hd * 4);
    float* kk = malloc(kvd * 4);
    float* vv = malloc(kvd * 4);
    float* attn = malloc(nh * hd * 4);
    float* proj = malloc(d * 4);
    float* gate = malloc(dff * 4);
    float* up = malloc(dff * 4);
    float* scores = malloc((ms + 1) * 4);
    if (!x || !normed || !q || !kk || !vv || !attn || !proj || !gate || !up || !scores) return -1;
    memcpy(x, x_embed, d * 4);
    size_t head_stride = ms * hd, layer_stride = 2 * nkv * head_stride;
    for (int32_t l = start_layer; l < cfg->n_layers; l++) {
        const uint8_t* const* W = weights + (size_t)l * 7;
        const int32_t* T = wdtype + (size_t)l * 7;
        orc_rmsnorm(x, norms[l * 2], d, cfg->eps, normed);
        orc_qmatmul(T[0], normed, W[0], nh * hd, d, q);
        orc_qmatmul(T[1], normed, W[1], kvd, d, kk);
        orc_qmatmul(T[2], normed, W[2], kvd, d, vv);
        orc_apply_rope(q, nh, hd, (size_t)pos, rope_sin, rope_cos, ms);
        orc_apply_rope(kk, nkv, hd, (size_t)pos, rope_sin, rope_cos, ms);
        float* lb = kv + (size_t)l * layer_stride;
        size_t slot = (size_t)*seq_len;
        if (slot < ms) { /* StaticKVCache::append, kv_cache.rs:40-65 */
            for (size_t h = 0; h < nkv; h++) {
                memcpy(lb + h * head_stride + slot * hd, kk + h * hd, hd * 4);
                memcpy(lb + nkv * head_stride + h * head_stride + slot * hd, vv + h * hd, hd * 4);
            }
        }
        size_t seq = slot + 1;
        size_t groups = nh / nkv;
        for (size_t h = 0; h < nh; h++) {
            size_t kvh = h / groups;
            orc_attn_direct(q + h * hd, lb + kvh * head_stride, lb + nkv * head_stride + kvh * head_stride,
                            seq, hd, (size_t)(cfg->sliding_window > 0 ? cfg->sliding_window : 0), scores,
                            attn + h * hd);
        }
        orc_qmatmul(T[3], attn, W[3], d, nh * hd, proj);
        for (size_t i = 0; i < d; i++) x[i] += proj[i];
        orc_rmsnorm(x, norms[l * 2 + 1], d, cfg->eps, normed);
        orc_qmatmul(T[4], normed, W[4], dff, d, gate);
        orc_qmatmul(T[5], normed, W[5], dff, d, up);
        for (size_t i = 0; i < dff; i++) gate[i] = gate[i] * (1.0f / (1.0f + expf(-gate[i]))) * up[i];
        orc_qmatmul(T[6], gate, W[6], d, dff, proj);
        for (size_t i = 0; i < d; i++) x[i] += proj[i];
    }
    if ((size_t)*seq_len < ms) (*seq_len)++; /* StaticKVCache::advance */
    orc_rmsnorm(x, final_norm, d, cfg->eps, normed);
    orc_qmatmul(lm_dtype, normed, lm_head, (size_t)cfg->vocab, d, logits);
    free(x); free(normed); free(q); free(kk); free(vv); free(attn); free(proj);
    free(gate); free(up); free(scores);
    return 0;
}

/* ── Batched prefill: forward_batch, CPU path (runner.rs:833-993) ─────────
 * All n prompt tokens in one pass: token i at position i, its K/V at cache
 * slot i (the cache is written from slot 0; LlamaRunner::prefill then sets
 * seq_len = n, runner.rs:695-704), batched matmuls with m = n, causal
 * attention_batch (runner.rs:1809-1883; with a sliding window w query i sees
 * keys max(0, i - w + 1) ..= i, :1825-1845), logits of the last token only.
 * x_embeds holds the n embedding rows. window 0 = none. */
static void orc_attention_batch(const float* q, const float* k, const float* v, size_t n, size_t nh, size_t nkv,
                                size_t hd, size_t window, float* out, float* scores) {
    float scale = 1.0f / sqrtf((float)hd);
    size_t groups = nh / nkv, q_stride = nh * hd, kv_stride = nkv * hd;
    if (window == 0) window = (size_t)-1; /* sliding_window.unwrap_or(usize::MAX) */
    for (size_t h = 0; h < nh; h++) {
        size_t kvh = h / groups;
        for (size_t i = 0; i < n; i++) {
            const float* qr = q + i * q_stride + h * hd;
            float* row = scores + i * n;
            size_t win_start = i >= window ? i - window + 1 : 0;
            for (size_t j = 0; j < win_start; j++) row[j] = -INFINITY;
            for (size_t j = win_start; j <= i; j++) {
                const float* kr = k + j * kv_stride + kvh * hd;
                float dot = 0.0f;
                for (size_t e = 0; e < hd; e++) dot += qr[e] * kr[e];
                row[j] = dot * scale;
            }
            for (size_t j = i + 1; j < n; j++) row[j] = -INFINITY;
        }
        for (size_t i = 0; i < n; i++) {
            float* row = scores + i * n;
            float mx = -INFINITY;
            for (size_t j = 0; j < n; j++) mx = fmaxf(mx, row[j]);
            float sum = 0.0f;
            for (size_t j = 0; j < n; j++)
                if (row[j] > -INFINITY / 2.0f) {
                    row[j] = expf(row[j] - mx);
                    sum += row[j];
                }
            for (size_t j = 0; j < n; j++)
                if (row[j] > 0.0f) row[j] /= sum;
        }
        for (size_t i = 0; i < n; i++) {
            const float* row = scores + i * n;
            float* o = out + i * q_stride + h * hd;
            for (size_t e = 0; e < hd; e++) o[e] = 0.0f;
            for (size_t j = 0; j <= i; j++) {
                float w = row[j];
                if (w <= 0.0f) continue;
                const float* vr = v + j * kv_stride + kvh * hd;
                for (size_t e = 0; e < hd; e++) o[e] += w * vr[e];
            }
        }
    }
}

ORC_API int orc_forward_batch(const orc_llama_cfg* cfg, const float* x_embeds, int32_t n_tokens,
                              const uint8_t* const* weights, const int32_t* wdtype, const float* const* norms,
                              const float* final_norm, const uint8_t* lm_head, int32_t lm_dtype,
                              const float* rope_sin, const float* rope_cos, float* kv, float* logits) {
    size_t d = (size_t)cfg->d_model, hd = (size_t)cfg->head_dim, nh = (size_t)cfg->n_heads;
    size_t nkv = (size_t)cfg->n_kv_heads, dff = (size_t)cfg->d_ff, ms = (size_t)cfg->max_seq;
    size_t kvd = nkv * hd, qd = nh * hd, n = (size_t)n_tokens;
    if (n_tokens <= 0 || n > ms) return -2; /* an empty prompt is an error; slots must fit */
    float* X = malloc(n * d * 4);
    float* N = malloc(n * d * 4);
    float* Q = malloc(n * qd * 4);
    float* K = malloc(n * kvd * 4);
    float* V = malloc(n * kvd * 4);
    float* A = malloc(n * qd * 4);
    float* P = malloc(n * d * 4);
    float* G = malloc(n * dff * 4);
    float* U = malloc(n * dff * 4);
    float* S = malloc(n * n * 4);
    if (!X || !N || !Q || !K || !V || !A || !P || !G || !U || !S) return -1;
    memcpy(X, x_embeds, n * d * 4);
    size_t head_stride = ms * hd, layer_stride = 2 * nkv * head_stride;
    for (int32_t l = 0; l < cfg->n_layers; l++) {
        const uint8_t* const* W = weights + (size_t)l * 7;
        const int32_t* T = wdtype + (size_t)l * 7;
        for (size_t i = 0; i < n; i++) orc_rmsnorm(X + i * d, norms[l * 2], d, cfg->eps, N + i * d);
        orc_qmatmul_m(T[0], N, n, W[0], qd, d, Q);
        orc_qmatmul_m(T[1], N, n, W[1], kvd, d, K);
        orc_qmatmul_m(T[2], N, n, W[2], kvd, d, V);
        for (size_t i = 0; i < n; i++) {
            orc_apply_rope(Q + i * qd, nh, hd, i, rope_sin, rope_cos, ms);
            orc_apply_rope(K + i * kvd, nkv, hd, i, rope_sin, rope_cos, ms);
        }
        float* lb = kv + (size_t)l * layer_stride;
        for (size_t i = 0; i < n; i++)
            for (size_t h = 0; h < nkv; h++) {
                memcpy(lb + h * head_stride + i * hd, K + (i * nkv + h) * hd, hd * 4);
                memcpy(lb + nkv * head_stride + h * head_stride + i * hd, V + (i * nkv + h) * hd, hd * 4);
            }
        orc_attention_batch(Q, K, V, n, nh, nkv, hd, (size_t)(cfg->sliding_window > 0 ? cfg->sliding_window : 0), A,
                            S);
        orc_qmatmul_m(T[3], A, n, W[3], d, qd, P);
        for (size_t i = 0; i < n * d; i++) X[i] += P[i];
        for (size_t i = 0; i < n; i++) orc_rmsnorm(X + i * d, norms[l * 2 + 1], d, cfg->eps, N + i * d);
        orc_qmatmul_m(T[4], N, n, W[4], dff, d, G);
        orc_qmatmul_m(T[5], N, n, W[5], dff, d, U);
        for (size_t i = 0; i < n * dff; i++) G[i] = G[i] * (1.0f / (1.0f + expf(-G[i]))) * U[i];
        orc_qmatmul_m(T[6], G, n, W[6], d, dff, P);
        for (size_t i = 0; i < n * d; i++) X[i] += P[i];
    }
    orc_rmsnorm(X + (n - 1) * d, final_norm, d, cfg->eps, N);
    orc_qmatmul(lm_dtype, N, lm_head, (size_t)cfg->vocab, d, logits);
    free(X); free(N); free(Q); free(K); free(V); free(A); free(P); free(G); free(U); free(S);
    return 0;
}
