/* CPU oracle, part 3: the two ops of the device trait Backend
 * (src/backend/mod.rs:12-218) that sit on the decode path, as the reference's
 * CpuBackend computes them. TEST INFRASTRUCTURE ONLY (see oracle.c): only
 * tests/ call it, as the checker of aeth_backend_rms_norm /
 * aeth_backend_causal_attention; the product library never links it.
 * Built with -ffp-contract=off: Rust never fuses a*b+c. */
#include <math.h>
#include <stddef.h>
#include <stdint.h>

#include "oracle.h"

/* Op::RmsNorm { epsilon } (src/backend/cpu.rs:514-545): per row of last_dim,
 * ssq = (sequential f32 sum of v*v) / last_dim, rms = sqrt(ssq + eps),
 * out = (x / rms) * w. */
ORC_API void orc_backend_rms_norm(const float* x, const float* w, size_t rows, size_t last_dim, float eps,
                                  float* out) {
    for (size_t r = 0; r < rows; r++) {
        const float* row = x + r * last_dim;
        float ssq = 0.0f;
        for (size_t c = 0; c < last_dim; c++) ssq += row[c] * row[c];
        ssq = ssq / (float)last_dim;
        const float rms = sqrtf(ssq + eps);
        for (size_t c = 0; c < last_dim; c++) out[r * last_dim + c] = (row[c] / rms) * w[c];
    }
}

/* Op::CausalAttention { scale, num_heads } (src/backend/cpu.rs:1660-1727):
 * q, k, v, out are [batch][seq][d]; head h owns columns [h·hd, (h+1)·hd) with
 * hd = d / num_heads (integer division: columns past num_heads·hd stay 0).
 * For query i: score_j = (sequential f32 dot of q_i, k_j) * scale for j <= i,
 * -inf after; max; e_j = exp(score_j - max), sum in j order; out = sum over j
 * of (e_j / sum) * v_j, in j order. score_row is `scratch` (seq floats). */
ORC_API int orc_causal_attention(const float* q, const float* k, const float* v, size_t batch, size_t seq, size_t d,
                                 size_t num_heads, float scale, float* scratch, float* out) {
    if (num_heads == 0) return -1; /* the reference divides by it (a panic) */
    const size_t hd = d / num_heads;
    for (size_t i = 0; i < batch * seq * d; i++) out[i] = 0.0f;
    for (size_t b = 0; b < batch; b++)
        for (size_t h = 0; h < num_heads; h++)
            for (size_t i = 0; i < seq; i++) {
                float* row = scratch;
                for (size_t j = 0; j < seq; j++) {
                    row[j] = -INFINITY;
                    if (j > i) continue;
                    float dot = 0.0f;
                    for (size_t e = 0; e < hd; e++)
                        dot += q[b * seq * d + i * d + h * hd + e] * k[b * seq * d + j * d + h * hd + e];
                    row[j] = dot * scale;
                }
                float mx = -INFINITY;
                for (size_t j = 0; j < seq; j++) mx = fmaxf(mx, row[j]);
                float sum = 0.0f;
                for (size_t j = 0; j < seq; j++)
                    if (row[j] != -INFINITY) {
                        row[j] = expf(row[j] - mx);
                        sum += row[j];
                    }
                for (size_t e = 0; e < hd; e++) {
                    float acc = 0.0f;
                    for (size_t j = 0; j < seq; j++)
                        if (row[j] != -INFINITY) acc += (row[j] / sum) * v[b * seq * d + j * d + h * hd + e];
                    out[b * seq * d + i * d + h * hd + e] = acc;
                }
            }
    return 0;
}
