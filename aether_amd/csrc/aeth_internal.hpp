// Internal (non-exported) declarations shared by the library's sources.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

// Device copy of one QuantWeight in per-field planes, rows in 16-row tiles
// (layouts in aeth_weights.hip).
struct aeth_weight {
    int dtype;
    int64_t n, k;         // out_features, in_features
    int64_t nb;           // blocks per row
    int64_t nblk;         // n * nb
    int64_t block_bytes;  // GGUF bytes per block
    int64_t bytes;        // nblk * block_bytes
    uint8_t* base;
    uint8_t *p0, *p1, *p2, *p3;
};

int aeth_num_cus();
int64_t aeth_blocks_per_row(int dtype, int64_t k);

// Q4_K device layout: rows are grouped in tiles of 16 (zero rows pad the last
// tile) so that one wave load covers 16 rows × 64 quant bytes contiguously.
//  p0 (headers d, dmin, scales[12]): [tile][block][16 rows][16 B]
//  p1 (quants): [tile][block][half h][lane n + 16·kg][16 B], lane (n, kg)
//               holding qs[64h + 16kg, +16) of row 16·tile + n.
__host__ __device__ inline int64_t aeth_q4k_hdr_off(int64_t row, int64_t b, int64_t nb) {
    return (((row >> 4) * nb + b) * 16 + (row & 15)) * 16;
}
// Address of qs byte q (0..127) of block b of `row`.
__host__ __device__ inline int64_t aeth_q4k_qs_off(int64_t row, int64_t b, int q, int64_t nb) {
    return ((((row >> 4) * nb + b) * 2 + (q >> 6)) * 64 + (row & 15) + 16 * ((q >> 4) & 3)) * 16 + (q & 15);
}

// Fusions around the GEMV (see k_gemv_mf in aeth_gemv.hip).
struct GemvEpi {
    unsigned flags = 0;                   // AETH_MM_ACCUMULATE
    const float* norm_w = nullptr;        // fused RMSNorm weight (length k)
    float eps = 0.0f;
    int swiglu = 0;                       // rows are (gate, up) pairs; y gets n/2 outputs
    unsigned long long* amax = nullptr;   // fused greedy argmax key
    int64_t ldc = 0;                      // output row stride for m > 1 (0: the output width)
};

// GEMV on one activation row per launch-row (a: [m][k] f32, c: [m][n]).
int aeth_gemv_launch_ex(const aeth_weight* w, const float* d_x, int64_t m, float* d_y, const GemvEpi& e,
                        hipStream_t s);
int aeth_gemv_launch(const aeth_weight* w, const float* d_x, int64_t m, float* d_y, unsigned flags,
                     hipStream_t s);
// Q4_K prefill GEMM (m > 1); ldc = output row stride (0: n).
int aeth_gemm_q4k_launch(const aeth_weight* w, const float* d_a, int64_t m, float* d_c, unsigned flags,
                         hipStream_t s, int64_t ldc = 0);
// aeth_qmatmul with an output row stride (rows of c are ldc floats apart).
int aeth_qmatmul_ld(const aeth_weight* w, const float* d_a, int64_t m, float* d_c, int64_t ldc, unsigned flags,
                    hipStream_t s);

// GGUF file → runner (aeth_gguf.cpp): LlamaModel::from_gguf on the device load path.
struct aeth_runner;
int aeth_gguf_load_runner(const char* path, aeth_runner** out, int* bos, int* eos);

