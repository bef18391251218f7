/*
 * oracle_formats.c — CPU restatement of the reference's remaining weight
 * formats: Q5_K, Q2_K, Q3_K, F16 and F32, their matmuls, the Q5_K
 * re-quantizer, the Q5_K / Q6_K int8 dot-product references, and
 * quantized_matmul_impl's dequantize → GGUF-order f32 route.
 *
 * TEST INFRASTRUCTURE ONLY, like oracle.c (same library, liboracle.so): only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 * Built with -ffp-contract=off; where the reference uses an FMA
 * (_mm256_fmadd_ps, f32::mul_add) this file calls fmaf explicitly.
 *
 * Pinning (what checks each function against something other than itself):
 *   dequant_q5_k     a block whose qh is zero equals the Q4_K block with the
 *                    same header and quants (pinned Q4_K dequant); setting qh
 *                    bit e moves element e alone, by 16·d·sc(e/32);
 *                    requantize_q5_k round trip ≤ 0.15 (tests/correctness.rs:1309).
 *   dequant_q2_k     closed forms: q = 0 → −dmin·(sc >> 4); per-element
 *                    one-hot quant bytes; scale nibble order.
 *   dequant_q3_k     closed forms: the 6-bit scale unpack against hand-built
 *                    scale bytes; hmask bit set → q = ql, clear → ql − 4.
 *   dequant_f16/f32  numpy float16 / raw bytes.
 *   matmuls          the reference's own cross-checks (tests.rs:510-826):
 *                    dequantize + f32 matmul vs scalar vs AVX2 order vs
 *                    batched; plus an f64 brute force of the dequantized rows.
 *   f32_gguf route   test_asymmetric_gguf_order_f16 (tests.rs:704-760):
 *                    [k, n] F16 through the fallback equals the transposed
 *                    f32 product.
 *   dotprod q5/q6    integer-exact: equal to the f32 matmul of the
 *                    dequantized weights against the dequantized Q8_0
 *                    activations within f32 rounding; hand cases.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* hsum_f32x8 (avx2.rs:13-20): s_i = v_i + v_{i+4}; ((s0+s1)+(s2+s3)). */
static inline float hsum8(const float* p) {
    float s0 = p[0] + p[4], s1 = p[1] + p[5], s2 = p[2] + p[6], s3 = p[3] + p[7];
    return (s0 + s1) + (s2 + s3);
}

/* ── Dequantization (src/loader/dequant.rs) ─────────────────────────────── */

/* dequant_q5_k_block, dequant.rs:542-584 (tensor form :229-285): 176-byte
 * block [d f16][dmin f16][scales 12][qh 32][qs 128]; element e's fifth bit is
 * bit e % 8 of qh[e / 8]; q = ql | hbit << 4; out = d·sc·q − dmin·m. */
ORC_API void orc_dequant_q5_k_block(const uint8_t* blk, float* out) {
    float d = orc_decode_d(rd16(blk)), dmin = orc_decode_d(rd16(blk + 2));
    const uint8_t *scales = blk + 4, *qh = blk + 16, *qs = blk + 48;
    for (int is = 0; is < 8; is += 2) {
        uint8_t sc0, m0, sc1, m1;
        orc_get_scale_min_k4(is, scales, &sc0, &m0);
        orc_get_scale_min_k4(is + 1, scales, &sc1, &m1);
        float d1 = d * (float)sc0, mm1 = dmin * (float)m0;
        float d2 = d * (float)sc1, mm2 = dmin * (float)m1;
        for (int l = 0; l < 32; l++) {
            int elo = is * 32 + l, ehi = (is + 1) * 32 + l;
            uint8_t b = qs[(is / 2) * 32 + l];
            uint8_t qlo = (uint8_t)((b & 0x0F) | (((qh[elo / 8] >> (elo % 8)) & 1) << 4));
            uint8_t qhi = (uint8_t)(((b >> 4) & 0x0F) | (((qh[ehi / 8] >> (ehi % 8)) & 1) << 4));
            out[elo] = d1 * (float)qlo - mm1;
            out[ehi] = d2 * (float)qhi - mm2;
        }
    }
}

ORC_API void orc_dequant_q5_k(const uint8_t* data, size_t n, float* out) {
    memset(out, 0, n * sizeof(float));
    for (size_t b = 0; b < n / 256; b++) orc_dequant_q5_k_block(data + b * 176, out + b * 256);
}

/* dequant_q2_k, dequant.rs:350-398: 84-byte block [d][dmin][scales 16][qs 64];
 * 16 sub-blocks of 16, sub-block s = 8·half + 2·t + u (t = shift / 2) reads
 * bits 2t of qs[32·half + 16u + e]; out = d·(sc & 15)·q − dmin·(sc >> 4). */
ORC_API void orc_dequant_q2_k_block(const uint8_t* blk, float* out) {
    float d = orc_decode_d(rd16(blk)), dmin = orc_decode_d(rd16(blk + 2));
    const uint8_t *scales = blk + 4, *qs = blk + 20;
    int o = 0;
    for (int half = 0; half < 2; half++) {
        int is = half * 8;
        for (int shift = 0; shift < 8; shift += 2) {
            for (int u = 0; u < 2; u++) {
                uint8_t sc = scales[is];
                float dl = d * (float)(sc & 0xF), ml = dmin * (float)(sc >> 4);
                for (int l = 0; l < 16; l++) {
                    int q = (qs[half * 32 + 16 * u + l] >> shift) & 3;
                    out[o++] = dl * (float)q - ml;
                }
                is++;
            }
        }
    }
}

ORC_API void orc_dequant_q2_k(const uint8_t* data, size_t n, float* out) {
    memset(out, 0, n * sizeof(float));
    for (size_t b = 0; b < n / 256; b++) orc_dequant_q2_k_block(data + b * 84, out + b * 256);
}

/* Q3_K scale unpack (dequant.rs:412-425): 16 six-bit scales from 12 bytes,
 * low nibbles from sr[0..8], high pairs from sr[8..12], centred by −32. */
static void q3k_scales(const uint8_t* sr, int* sc) {
    for (int i = 0; i < 8; i++) {
        sc[i] = sr[i] & 0x0F;
        sc[i + 8] = sr[i] >> 4;
    }
    for (int i = 0; i < 4; i++) {
        int b = sr[i + 8];
        sc[i] |= (b & 0x03) << 4;
        sc[i + 4] |= ((b >> 2) & 0x03) << 4;
        sc[i + 8] |= ((b >> 4) & 0x03) << 4;
        sc[i + 12] |= ((b >> 6) & 0x03) << 4;
    }
    for (int i = 0; i < 16; i++) sc[i] -= 32;
}

/* dequant_q3_k, dequant.rs:400-451: 110-byte block [hmask 32][qs 64][scales 12][d];
 * sub-block s reads bits 2·((s/2) % 4) of qs[32·(s/8) + 16·(s%2) + e] and bit
 * s/2 of hmask[16·(s%2) + e]; q = ql − 4·(1 − hbit); out = d·sc_s·q. */
ORC_API void orc_dequant_q3_k_block(const uint8_t* blk, float* out) {
    const uint8_t *hmask = blk, *qs = blk + 32, *sr = blk + 96;
    float d = orc_decode_d(rd16(blk + 108));
    int sc[16];
    q3k_scales(sr, sc);
    for (int s = 0; s < 16; s++) {
        int qoff = (s / 8) * 32, shift = ((s / 2) % 4) * 2, hb = (s % 2) * 16, bit = s / 2;
        float dl = d * (float)sc[s];
        for (int e = 0; e < 16; e++) {
            int ql = (qs[qoff + hb + e] >> shift) & 3;
            int qhb = ((hmask[hb + e] >> bit) & 1) ^ 1;
            int q = ql - (qhb << 2);
            out[s * 16 + e] = dl * (float)q;
        }
    }
}

ORC_API void orc_dequant_q3_k(const uint8_t* data, size_t n, float* out) {
    memset(out, 0, n * sizeof(float));
    for (size_t b = 0; b < n / 256; b++) orc_dequant_q3_k_block(data + b * 110, out + b * 256);
}

/* dequant_f16, dequant.rs:79-95 (half::f16::to_f32 per element). */
ORC_API void orc_dequant_f16(const uint8_t* data, size_t n, float* out) {
    for (size_t i = 0; i < n; i++) out[i] = orc_f16_to_f32(rd16(data + 2 * i));
}

/* ── Scalar kernels on [n][k] row-major weights ─────────────────────────── */

/* matmul_q5_k_scalar (m = 1), q5_k.rs:5-83: per element acc += a·(d1·q − m1),
 * lo and hi interleaved; batched form (m > 1), q5_k.rs:85-160: per row
 * results += d1·Σaq − m1·Σa per 32-element sub-block. */
ORC_API void orc_scalar_matmul_q5_k(const float* a, const uint8_t* b, size_t m, size_t n, size_t k, float* c) {
    size_t nb = k / 256;
    for (size_t row = 0; row < m; row++) {
        const float* act = a + row * k;
        for (size_t col = 0; col < n; col++) {
            float acc = 0.0f;
            for (size_t blk = 0; blk < nb; blk++) {
                const uint8_t* bo = b + (col * nb + blk) * 176;
                float d = orc_decode_d(rd16(bo)), dmin = orc_decode_d(rd16(bo + 2));
                const uint8_t *scales = bo + 4, *qh = bo + 16, *qs = bo + 48;
                size_t eb = blk * 256;
                for (int is = 0; is < 8; is += 2) {
                    uint8_t sc0, m0, sc1, m1;
                    orc_get_scale_min_k4(is, scales, &sc0, &m0);
                    orc_get_scale_min_k4(is + 1, scales, &sc1, &m1);
                    float d1 = d * (float)sc0, mm1 = dmin * (float)m0;
                    float d2 = d * (float)sc1, mm2 = dmin * (float)m1;
                    float aq_lo = 0, a_lo = 0, aq_hi = 0, a_hi = 0;
                    for (int l = 0; l < 32; l++) {
                        int elo = is * 32 + l, ehi = (is + 1) * 32 + l;
                        uint8_t byte = qs[(is / 2) * 32 + l];
                        float qlo = (float)(byte & 0x0F) + (float)((qh[elo / 8] >> (elo % 8)) & 1) * 16.0f;
                        float qhi = (float)((byte >> 4) & 0x0F) + (float)((qh[ehi / 8] >> (ehi % 8)) & 1) * 16.0f;
                        if (m == 1) {
                            acc += act[eb + elo] * (d1 * qlo - mm1);
                            acc += act[eb + ehi] * (d2 * qhi - mm2);
                        } else {
                            aq_lo += act[eb + elo] * qlo;
                            a_lo += act[eb + elo];
                            aq_hi += act[eb + ehi] * qhi;
                            a_hi += act[eb + ehi];
                        }
                    }
                    if (m > 1) {
                        acc += d1 * aq_lo - mm1 * a_lo;
                        acc += d2 * aq_hi - mm2 * a_hi;
                    }
                }
            }
            c[row * n + col] = acc;
        }
    }
}

/* matmul_q2_k_scalar + batched form, q2_k.rs:4-108 (the same sums per row):
 * acc += dl·Σ a·q − ml·Σ a per 16-element sub-block. */
ORC_API void orc_scalar_matmul_q2_k(const float* a, const uint8_t* b, size_t m, size_t n, size_t k, float* c) {
    size_t nb = k / 256;
    for (size_t row = 0; row < m; row++) {
        const float* act = a + row * k;
        for (size_t col = 0; col < n; col++) {
            float acc = 0.0f;
            for (size_t blk = 0; blk < nb; blk++) {
                const uint8_t* bo = b + (col * nb + blk) * 84;
                float d = orc_decode_d(rd16(bo)), dmin = orc_decode_d(rd16(bo + 2));
                const uint8_t *scales = bo + 4, *qs = bo + 20;
                size_t eb = blk * 256;
                for (int s = 0; s < 16; s++) {
                    int qoff = (s / 8) * 32, shift = ((s / 2) % 4) * 2, bb = (s % 2) * 16;
                    float dl = d * (float)(scales[s] & 0xF), ml = dmin * (float)(scales[s] >> 4);
                    float aq = 0.0f, as = 0.0f;
                    for (int e = 0; e < 16; e++) {
                        float q = (float)((qs[qoff + bb + e] >> shift) & 3);
                        float v = act[eb + s * 16 + e];
                        aq += v * q;
                        as += v;
                    }
                    acc += dl * aq - ml * as;
                }
            }
            c[row * n + col] = acc;
        }
    }
}

/* matmul_q3_k_scalar + batched form, q3_k.rs:4-134: acc += dl·Σ a·q per
 * 16-element sub-block. */
ORC_API void orc_scalar_matmul_q3_k(const float* a, const uint8_t* b, size_t m, size_t n, size_t k, float* c) {
    size_t nb = k / 256;
    for (size_t row = 0; row < m; row++) {
        const float* act = a + row * k;
        for (size_t col = 0; col < n; col++) {
            float acc = 0.0f;
            for (size_t blk = 0; blk < nb; blk++) {
                const uint8_t* bo = b + (col * nb + blk) * 110;
                const uint8_t *hmask = bo, *qs = bo + 32;
                float d = orc_decode_d(rd16(bo + 108));
                int sc[16];
                q3k_scales(bo + 96, sc);
                size_t eb = blk * 256;
                for (int s = 0; s < 16; s++) {
                    int qoff = (s / 8) * 32, shift = ((s / 2) % 4) * 2, bb = (s % 2) * 16, bit = s / 2;
                    float dl = d * (float)sc[s];
                    float aq = 0.0f;
                    for (int e = 0; e < 16; e++) {
                        int ql = (qs[qoff + bb + e] >> shift) & 3;
                        int qhb = ((hmask[bb + e] >> bit) & 1) ^ 1;
                        aq += act[eb + s * 16 + e] * (float)(ql - (qhb << 2));
                    }
                    acc += dl * aq;
                }
            }
            c[row * n + col] = acc;
        }
    }
}

/* matmul_f16_scalar + batched form, f16.rs:3-56: sequential acc += a·w. */
ORC_API void orc_scalar_matmul_f16(const float* a, const uint8_t* b, size_t m, size_t n, size_t k, float* c) {
    for (size_t row = 0; row < m; row++)
        for (size_t col = 0; col < n; col++) {
            float acc = 0.0f;
            for (size_t i = 0; i < k; i++) acc += a[row * k + i] * orc_f16_to_f32(rd16(b + (col * k + i) * 2));
            c[row * n + col] = acc;
        }
}

/* ── AVX2 operation order (src/quant/avx2.rs), restated in scalar C ─────── */

/* avx2::matmul_q2_k, avx2.rs:241-309: per 8 lanes w = fma(dl, q, 0 − ml)
 * (one rounding), sub-block sum of hsum8(w·a); plain f16 d and dmin. */
ORC_API void orc_avx2order_matmul_q2_k(const float* a, const uint8_t* b, size_t m, size_t n, size_t k, float* c) {
    size_t nb = k / 256;
    float prod[8];
    for (size_t row = 0; row < m; row++)
        for (size_t col = 0; col < n; col++) {
            float sum = 0.0f;
            for (size_t blk = 0; blk < nb; blk++) {
                const uint8_t* bo = b + (col * nb + blk) * 84;
                float d = orc_f16_to_f32(rd16(bo)), dmin = orc_f16_to_f32(rd16(bo + 2));
                const uint8_t *scales = bo + 4, *qs = bo + 20;
                const float* ad = a + row * k + blk * 256;
                for (int s = 0; s < 16; s++) {
                    int qoff = (s / 8) * 32, shift = ((s / 2) % 4) * 2, bb = (s % 2) * 16;
                    float dl = d * (float)(scales[s] & 0xF), ml = dmin * (float)(scales[s] >> 4);
                    float bs = 0.0f;
                    for (int i = 0; i < 16; i += 8) {
                        for (int j = 0; j < 8; j++) {
                            float q = (float)((qs[qoff + bb + i + j] >> shift) & 3);
                            prod[j] = fmaf(dl, q, 0.0f - ml) * ad[s * 16 + i + j];
                        }
                        bs += hsum8(prod);
                    }
                    sum += bs;
                }
            }
            c[row * n + col] = sum;
        }
}

/* avx2::matmul_q3_k, avx2.rs:312-389: per 8 lanes (dl·q)·a, hsum8 per
 * sub-block; plain f16 d. */
ORC_API void orc_avx2order_matmul_q3_k(const float* a, const uint8_t* b, size_t m, size_t n, size_t k, float* c) {
    size_t nb = k / 256;
    float prod[8];
    for (size_t row = 0; row < m; row++)
        for (size_t col = 0; col < n; col++) {
            float sum = 0.0f;
            for (size_t blk = 0; blk < nb; blk++) {
                const uint8_t* bo = b + (col * nb + blk) * 110;
                const uint8_t *hmask = bo, *qs = bo + 32;
                float d = orc_f16_to_f32(rd16(bo + 108));
                int sc[16];
                q3k_scales(bo + 96, sc);
                const float* ad = a + row * k + blk * 256;
                for (int s = 0; s < 16; s++) {
                    int qoff = (s / 8) * 32, shift = ((s / 2) % 4) * 2, bb = (s % 2) * 16, bit = s / 2;
                    float dl = d * (float)sc[s];
                    float bs = 0.0f;
                    for (int i = 0; i < 16; i += 8) {
                        for (int j = 0; j < 8; j++) {
                            int ql = (qs[qoff + bb + i + j] >> shift) & 3;
                            int qhb = ((hmask[bb + i + j] >> bit) & 1) ^ 1;
                            prod[j] = (dl * (float)(ql - (qhb << 2))) * ad[s * 16 + i + j];
                        }
                        bs += hsum8(prod);
                    }
                    sum += bs;
                }
            }
            c[row * n + col] = sum;
        }
}

/* avx2::matmul_f16, avx2.rs:210-238: hsum8(a·w) per 8, then a sequential tail. */
ORC_API void orc_avx2order_matmul_f16(const float* a, const uint8_t* b, size_t m, size_t n, size_t k, float* c) {
    float prod[8];
    for (size_t row = 0; row < m; row++)
        for (size_t col = 0; col < n; col++) {
            const float* ar = a + row * k;
            const uint8_t* br = b + col * k * 2;
            float sum = 0.0f;
            size_t i = 0;
            for (; i + 8 <= k; i += 8) {
                for (int j = 0; j < 8; j++) prod[j] = ar[i + j] * orc_f16_to_f32(rd16(br + (i + j) * 2));
                sum += hsum8(prod);
            }
            for (; i < k; i++) sum += ar[i] * orc_f16_to_f32(rd16(br + i * 2));
            c[row * n + col] = sum;
        }
}

/* ── Re-quantizer (dispatch.rs:302-429) ───────────────────────────────────
 * requantize_q4_k with 31 levels; the fifth bit of element e goes to bit
 * e % 8 of qh[e / 8]. Rust f32::round = roundf; min/max ignore NaN. */
ORC_API void orc_requantize_q5_k(const float* data, size_t rows, size_t cols, uint8_t* out) {
    size_t bpr = (cols + 255) / 256;
    memset(out, 0, rows * bpr * 176);
    for (size_t r = 0; r < rows; r++) {
        for (size_t blk = 0; blk < bpr; blk++) {
            size_t start = r * cols + blk * 256;
            size_t end = start + 256 < r * cols + cols ? start + 256 : r * cols + cols;
            size_t actual = end - start;
            const float* block = data + start;
            uint8_t* o = out + (r * bpr + blk) * 176;
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
                dsub[sb] = (maxs[sb] + msub[sb]) / 31.0f;
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
                        q0 = (uint8_t)(int)fminf(fmaxf(roundf((block[i0] + m1) / d1), 0.0f), 31.0f);
                    if (i1 < actual && d2 != 0.0f)
                        q1 = (uint8_t)(int)fminf(fmaxf(roundf((block[i1] + m2) / d2), 0.0f), 31.0f);
                    o[48 + ch * 32 + l] = (uint8_t)((q0 & 0x0F) | ((q1 & 0x0F) << 4));
                    o[16 + i0 / 8] |= (uint8_t)((q0 >> 4) << (i0 % 8));
                    o[16 + i1 / 8] |= (uint8_t)((q1 >> 4) << (i1 % 8));
                }
            }
        }
    }
}

/* ── int8 dot-product references (Q8_0 activation blocks) ─────────────── */

/* matmul_q5_k_dotprod_reference, tests.rs:254-330: per 32-element
 * sub-block exact i32 dot and Σq_a, acc += d_a·(d1·dot − m1·Σq_a). The
 * activation block of sub-block is of super-block blk is 8·blk + is, as the
 * Q4_K and Q6_K dot-product kernels index it (neon.rs:392-393, tests.rs:99-103).
 * The reference's Q5_K test helper and its NEON kernel (neon.rs:1441-1446)
 * both drop the 8·blk term, so for k > 256 they read the first super-block's
 * activations for every super-block; at k = 256, the only size the reference
 * tests, the two forms agree. This restatement keeps the format's semantics. */
ORC_API void orc_dotprod_ref_q5_k(const uint8_t* aq, const uint8_t* b, size_t m, size_t n, size_t k, float* c) {
    size_t nb = k / 256;
    for (size_t row = 0; row < m; row++)
        for (size_t col = 0; col < n; col++) {
            float acc = 0.0f;
            for (size_t blk = 0; blk < nb; blk++) {
                const uint8_t* bo = b + (col * nb + blk) * 176;
                float d = orc_decode_d(rd16(bo)), dmin = orc_decode_d(rd16(bo + 2));
                const uint8_t *qh = bo + 16, *qs = bo + 48;
                for (int is = 0; is < 8; is += 2) {
                    uint8_t sc0, m0, sc1, m1;
                    orc_get_scale_min_k4(is, bo + 4, &sc0, &m0);
                    orc_get_scale_min_k4(is + 1, bo + 4, &sc1, &m1);
                    float d1 = d * (float)sc0, mm1 = dmin * (float)m0;
                    float d2 = d * (float)sc1, mm2 = dmin * (float)m1;
                    const uint8_t* alo = aq + (row * nb * 8 + blk * 8 + is) * 34;
                    const uint8_t* ahi = aq + (row * nb * 8 + blk * 8 + is + 1) * 34;
                    int32_t dlo = 0, slo = 0, dhi = 0, shi = 0;
                    for (int l = 0; l < 32; l++) {
                        int elo = is * 32 + l, ehi = (is + 1) * 32 + l;
                        uint8_t byte = qs[(is / 2) * 32 + l];
                        int32_t qlo = (byte & 0x0F) + (((qh[elo / 8] >> (elo % 8)) & 1) * 16);
                        int32_t qhi = ((byte >> 4) & 0x0F) + (((qh[ehi / 8] >> (ehi % 8)) & 1) * 16);
                        int32_t vlo = (int8_t)alo[2 + l], vhi = (int8_t)ahi[2 + l];
                        dlo += qlo * vlo;
                        slo += vlo;
                        dhi += qhi * vhi;
                        shi += vhi;
                    }
                    float dalo = orc_f16_to_f32(rd16(alo)), dahi = orc_f16_to_f32(rd16(ahi));
                    acc += dalo * (d1 * (float)dlo - mm1 * (float)slo);
                    acc += dahi * (d2 * (float)dhi - mm2 * (float)shi);
                }
            }
            c[row * n + col] = acc;
        }
}

/* matmul_q6_k_dotprod_reference, tests.rs:136-252: per 16 elements exact i32
 * dot of (q − 32) with the activation quants, acc += (d·sc·d_a)·dot. */
ORC_API void orc_dotprod_ref_q6_k(const uint8_t* aq, const uint8_t* b, size_t m, size_t n, size_t k, float* c) {
    size_t nb = k / 256;
    for (size_t row = 0; row < m; row++)
        for (size_t col = 0; col < n; col++) {
            float acc = 0.0f;
            for (size_t blk = 0; blk < nb; blk++) {
                const uint8_t* bo = b + (col * nb + blk) * 210;
                float d = orc_decode_d(rd16(bo + 208));
                const uint8_t *ql = bo, *qh = bo + 128, *sc = bo + 192;
                for (int h = 0; h < 2; h++)
                    for (int l = 0; l < 32; l += 16) {
                        int is = l / 16;
                        float sv[4];
                        int32_t dot[4] = {0, 0, 0, 0};
                        const uint8_t* ab[4];
                        for (int t = 0; t < 4; t++) {
                            sv[t] = (float)(int8_t)sc[h * 8 + is + 2 * t];
                            ab[t] = aq + (row * nb * 8 + blk * 8 + h * 4 + t) * 34;
                        }
                        for (int e = 0; e < 16; e++) {
                            uint8_t A = ql[h * 64 + l + e], B = ql[h * 64 + l + 32 + e], H = qh[h * 32 + l + e];
                            int32_t q[4] = {(int32_t)((A & 0x0F) | ((H & 0x03) << 4)) - 32,
                                            (int32_t)((B & 0x0F) | ((H & 0x0C) << 2)) - 32,
                                            (int32_t)((A >> 4) | (H & 0x30)) - 32,
                                            (int32_t)((B >> 4) | ((H & 0xC0) >> 2)) - 32};
                            for (int t = 0; t < 4; t++) dot[t] += (int32_t)(int8_t)ab[t][2 + l + e] * q[t];
                        }
                        for (int t = 0; t < 4; t++) {
                            float f = d * sv[t] * orc_f16_to_f32(rd16(ab[t]));
                            acc += f * (float)dot[t];
                        }
                    }
            }
            c[row * n + col] = acc;
        }
}

/* ── quantized_matmul_impl's fallback (dispatch.rs:98-135, 541-574) ───────
 * Formats without a fused kernel (F32, F16, Q2_K, Q3_K) are kept by
 * load_quant in GGUF [k][n] order (model_loader.rs:344-350) and multiplied by
 * dequantize(b, [k, n]) then matmul_f32_gguf: c[j] = fma(a_i, b[i·n + j], c[j])
 * over i in order, rows with a_i == 0 skipped. */
ORC_API int orc_dequant_any(int dtype, const uint8_t* data, size_t n, float* out) {
    switch (dtype) {
        case ORC_DT_F32: memcpy(out, data, n * 4); return 0;
        case ORC_DT_F16: orc_dequant_f16(data, n, out); return 0;
        case ORC_DT_Q2_K: orc_dequant_q2_k(data, n, out); return 0;
        case ORC_DT_Q3_K: orc_dequant_q3_k(data, n, out); return 0;
        case ORC_DT_Q5_K: orc_dequant_q5_k(data, n, out); return 0;
        default: return -1;
    }
}

ORC_API void orc_matmul_f32_gguf(const float* a, const float* b, size_t m, size_t n, size_t k, float* c) {
    memset(c, 0, m * n * sizeof(float));
    for (size_t i = 0; i < k; i++)
        for (size_t row = 0; row < m; row++) {
            float s = a[row * k + i];
            if (s != 0.0f)
                for (size_t j = 0; j < n; j++) c[row * n + j] = fmaf(s, b[i * n + j], c[row * n + j]);
        }
}

ORC_API int orc_gguf_order_matmul(int dtype, const float* a, size_t m, const uint8_t* b, size_t n, size_t k,
                                  float* c) {
    float* w = (float*)malloc(n * k * sizeof(float));
    if (!w) return -1;
    int rc = orc_dequant_any(dtype, b, n * k, w);
    if (rc == 0) orc_matmul_f32_gguf(a, w, m, n, k, c);
    free(w);
    return rc;
}
