// Internal (non-exported) declarations shared by the library's sources.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <exception>
#include <new>

#include "../../include/aether_hip.h"

int aeth_set_error(int code, const char* fmt, ...);

// Runs an entry point's body so that no C++ exception crosses the C ABI: an
// allocation failure of the host containers becomes AETH_ENOMEM, anything
// else AETH_EINVAL, with the message in aeth_last_error().
template <class F>
int aeth_guard(const char* what, F&& body) noexcept {
    try {
        return body();
    } catch (const std::bad_alloc&) {
        return aeth_set_error(AETH_ENOMEM, "%s: out of host memory", what);
    } catch (const std::exception& e) {
        return aeth_set_error(AETH_EINVAL, "%s: %s", what, e.what());
    } catch (...) {
        return aeth_set_error(AETH_EINVAL, "%s: unexpected exception", what);
    }
}

// a·b for non-negative sizes; false (and *out untouched) on overflow of int64.
inline bool aeth_mul_ok(int64_t a, int64_t b, int64_t* out) {
    int64_t r;
    if (a < 0 || b < 0 || __builtin_mul_overflow(a, b, &r)) return false;
    *out = r;
    return true;
}

// How a weight's bytes are held on the device.
enum {
    AETH_ORDER_PLANAR = 0,  // Q8_0 / Q4_K / Q5_K / Q6_K: [n][k] row blocks re-laid in per-field planes
    AETH_ORDER_GGUF = 1,    // F32 / F16 / Q2_K / Q3_K as load_quant keeps them: GGUF [k][n], raw
    AETH_ORDER_ROWS = 2,    // F16 / Q2_K / Q3_K [n][k] row blocks, raw (matmul_f16 / _q2_k / _q3_k)
};

// The formats with a fused matrix-core kernel (is_quantized_type_supported,
// model_loader.rs:362-367): load_quant re-quantizes them into [n][k] rows.
inline bool aeth_dtype_fused(int dtype) {
    return dtype == AETH_DTYPE_Q8_0 || dtype == AETH_DTYPE_Q4_K || dtype == AETH_DTYPE_Q5_K || dtype == AETH_DTYPE_Q6_K;
}

// Device copy of one QuantWeight: planar (row tiles of 16, layouts in
// aeth_weights.hip) for the fused formats, the raw bytes otherwise.
struct aeth_weight {
    int dtype;
    int order;            // AETH_ORDER_*
    int64_t n, k;         // out_features, in_features
    int64_t nb;           // blocks per row
    int64_t nblk;         // n * nb
    int64_t block_bytes;  // GGUF bytes per block
    int64_t bytes;        // nblk * block_bytes
    uint8_t* base;
    uint8_t *p0, *p1, *p2, *p3;
    // planar weights: some block scale (Q8_0 d; Q4_K / Q5_K d or dmin; Q6_K d) has the f16
    // exponent 31 (NaN / infinity bits), found when the bytes are laid out
    int special_scales = 0;
};

int aeth_num_cus();
int64_t aeth_blocks_per_row(int dtype, int64_t k);
// Bytes of a weight's raw form: planar / rows: n·blocks_per_row·block_bytes;
// GGUF order: (n·k / block_elems)·block_bytes. < 0 on a bad dtype / shape.
int64_t aeth_weight_raw_bytes(int dtype, int order, int64_t n, int64_t k);
int aeth_weight_create_ex(int dtype, int order, int64_t n, int64_t k, const void* raw, int raw_is_device,
                          hipStream_t s, aeth_weight** out);

// Orderable 64-bit key of (value, row) for the fused greedy argmax: a larger
// value wins, ties go to the larger row (Iterator::max_by, runner.rs:1964-1973).
__device__ __forceinline__ unsigned long long aeth_amax_key(float v, int64_t row) {
    const uint32_t f = __float_as_uint(v);
    const uint32_t o = (f & 0x80000000u) ? ~f : (f | 0x80000000u);
    return ((unsigned long long)o << 32) | (unsigned long long)(uint32_t)row;
}

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
    float* ws = nullptr;                  // GGUF-order weights: scratch of ws_floats floats
    int64_t ws_floats = 0;                //   (NULL: the library's scratch of the launch stream)
};

// GEMV on one activation row per launch-row (a: [m][k] f32, c: [m][n]).
int aeth_gemv_launch_ex(const aeth_weight* w, const float* d_x, int64_t m, float* d_y, const GemvEpi& e,
                        hipStream_t s);
int aeth_gemv_launch(const aeth_weight* w, const float* d_x, int64_t m, float* d_y, unsigned flags,
                     hipStream_t s);
// VALU GEMV for GGUF-order and raw-row weights (aeth_gemv_ext.hip); the same
// epilogue except SwiGLU (GGUF order: RMSNorm through the scratch, argmax and
// accumulate in the reduction; raw rows: accumulate only).
int aeth_xgemv_launch(const aeth_weight* w, const float* d_x, int64_t m, float* d_y, const GemvEpi& e,
                      hipStream_t s);
// Scratch floats a GGUF-order GEMV of m rows needs at most.
int64_t aeth_xgemv_ws_floats(const aeth_weight* w, int64_t m);
// The op whose output the Q4_K GEMM takes as A, run inside its activation prep:
// A itself, the RMSNorm of A's rows with weight norm_w (k_rmsnorm_v's formula),
// or h = g·σ(g)·u over A's interleaved (g, u) pairs (A has 2k columns;
// k_silu_pairs's formula).
enum { PREP_PLAIN = 0, PREP_RMSNORM = 1, PREP_SWIGLU = 2 };
struct GemmIn {
    int mode = PREP_PLAIN;
    const float* norm_w = nullptr;
    float eps = 0.0f;
    // the output's columns are interleaved (g, u) pairs (the gate|up weight): C receives
    // h = g·σ(g)·u, n/2 columns per row (σ through the reciprocal instruction), instead of the pairs
    bool swiglu_out = false;
    // the stream's GEMM scratch already holds this A's prep (the same d_a, m, k, mode and
    // flags, run by the GEMM launched just before on the stream): the prep launch is skipped
    bool prepared = false;
};
// Whether m activation rows against planar Q4_K weight w go to the prefill GEMM
// (else the row-batched GEMV): from 16 rows, or from 5 once m · (weight bytes) reaches
// 150 MB. Below that the GEMM's near-constant cost (its 64-row tile idles most of its
// MFMA work) exceeds the GEMV's, which streams the weight once per row.
bool aeth_q4k_gemm_rows(const aeth_weight* w, int64_t m);
// The same for planar Q5_K weights (the K-split GEMM's Q5_K form): whole super-blocks, buffers
// within its 32-bit offsets, from 16 rows or from 5 once m · (weight bytes) reaches 150 MB.
bool aeth_q5k_gemm_rows(const aeth_weight* w, int64_t m);
// Whether aeth_gemm_q4k_launch runs producer `mode` for this weight and A (else
// the caller runs the producer itself): a planar Q4_K or Q5_K weight, m > 1, and for
// the RMSNorm and SwiGLU producers whole super-blocks, k ≤ 16384 and 16-byte
// aligned A (and norm weight).
bool aeth_gemm_fuses(const aeth_weight* w, int64_t m, int mode, const float* d_a, const float* norm_w);
// Whether aeth_gemm_q4k_launch can apply GemmIn::swiglu_out for this weight: a planar
// Q4_K or Q5_K weight of even n and whole super-blocks, m > 1 (no accumulate).
bool aeth_gemm_swiglu_out(const aeth_weight* w, int64_t m);
// Q4_K and Q5_K prefill GEMM (m > 1; Q5_K: where aeth_q5k_gemm_rows says so); ldc = output
// row stride (0: n); in = the fused producer (nullptr: plain A; any other mode must pass
// aeth_gemm_fuses).
int aeth_gemm_q4k_launch(const aeth_weight* w, const float* d_a, int64_t m, float* d_c, unsigned flags,
                         hipStream_t s, int64_t ldc = 0, void* ws = nullptr, size_t ws_bytes = 0,
                         const GemmIn* in = nullptr);
// Whether m activation rows against planar Q8_0 weight w take the Q8_0 GEMM (aeth_gemm_q80.hip):
// whole blocks (k = 32·nb) within the kernel's 32-bit buffer offsets, from 16 rows, or from 5
// once m · (weight bytes) reaches 150 MB.
bool aeth_q80_gemm_rows(const aeth_weight* w, int64_t m);
// aeth_gemm_fuses for the Q8_0 GEMM (its prep is the Q4_K GEMM's).
bool aeth_q80_gemm_fuses(const aeth_weight* w, int64_t m, int mode, const float* d_a, const float* norm_w);
// Q8_0 prefill GEMM (AETH_MM_ACCUMULATE, the Q8 activation blocks, the fused producers and the
// SwiGLU output as aeth_gemm_q4k_launch); requires aeth_q80_gemm_rows, and a producer in `in`
// aeth_q80_gemm_fuses.
int aeth_gemm_q80_launch(const aeth_weight* w, const float* d_a, int64_t m, float* d_c, unsigned flags,
                         hipStream_t s, int64_t ldc = 0, const GemmIn* in = nullptr);
// The runner's view of the three GEMMs: whether weight w takes producer `mode` in a GEMM
// (Q4_K, Q6_K, Q8_0), whether its GEMM writes the SwiGLU output (Q4_K, Q8_0), and the launch.
bool aeth_gemm_fused_ok(const aeth_weight* w, int64_t m, int mode, const float* d_a, const float* norm_w);
bool aeth_gemm_swo_ok(const aeth_weight* w, int64_t m);
int aeth_gemm_fused_launch(const aeth_weight* w, const float* d_a, int64_t m, float* d_c, unsigned flags,
                           hipStream_t s, int64_t ldc, const GemmIn* in);
// Whether m activation rows against Q6_K weight w take the Q6_K GEMM (aeth_gemm_q6k.hip):
// planar whole super-blocks within the kernel's 32-bit buffer offsets, once m · (weight
// bytes) reaches 200 MB (the row-batched GEMV below).
bool aeth_q6k_gemm_rows(const aeth_weight* w, int64_t m);
// aeth_gemm_fuses for the Q6_K GEMM (its prep is the Q4_K GEMM's).
bool aeth_q6k_gemm_fuses(const aeth_weight* w, int64_t m, int mode, const float* d_a, const float* norm_w);
// Q6_K prefill GEMM (the exact mode of the Q4_K GEMM; AETH_MM_ACCUMULATE and the Q8
// activation blocks as aeth_gemm_q4k_launch); requires aeth_q6k_gemm_rows, and a producer
// in `in` aeth_q6k_gemm_fuses (no SwiGLU output).
int aeth_gemm_q6k_launch(const aeth_weight* w, const float* d_a, int64_t m, float* d_c, unsigned flags,
                         hipStream_t s, int64_t ldc = 0, const GemmIn* in = nullptr);
// aeth_qmatmul with an output row stride (rows of c are ldc floats apart).
int aeth_qmatmul_ld(const aeth_weight* w, const float* d_a, int64_t m, float* d_c, int64_t ldc, unsigned flags,
                    hipStream_t s);

// Library scratch (aeth_host.cpp): a grow-only device buffer per (device,
// stream, use) for calls that bring no workspace of their own. Calls on one
// stream share it (their kernels run in order); a grow waits for the stream
// and is refused during graph capture.
enum {
    AETH_SCRATCH_GEMM = 0,
    AETH_SCRATCH_XGEMV = 1,
    AETH_SCRATCH_ATTN = 2,
    AETH_SCRATCH_ARGMAX = 3,
    AETH_SCRATCH_DEQ = 4,   // dequantized f32 weight of a batched product (aeth_blas.cpp)
    AETH_SCRATCH_QACT = 5,  // Q8_0 activation blocks and their f32 values (same)
    AETH_SCRATCH_SPLIT = 6, // partial output tiles of a GEMM split over K across workgroups (aeth_gemm.hip)
};
int aeth_stream_scratch(hipStream_t s, int use, size_t bytes, void** out);
// Frees every scratch buffer of stream s (before the stream is destroyed).
void aeth_stream_scratch_release(hipStream_t s);
// Resolves the device address of the no-allocation entry point's static
// scratch on device dev (current); called by aeth_init and on first use.
int aeth_noalloc_setup(int dev);
// Batched product (m > 1) through a dequantized f32 weight and one rocBLAS
// SGEMM (aeth_blas.cpp), for the formats without a matrix-core GEMM; rows of c
// are ldc floats apart (0: n). Handles are per (device, stream);
// aeth_blas_release_stream drops those of a stream.
int aeth_dequant_gemm_launch(const aeth_weight* w, const float* d_a, int64_t m, float* d_c, int64_t ldc,
                             unsigned flags, hipStream_t s);
void aeth_blas_release_stream(hipStream_t s);
// Bytes of GEMM scratch (A fragments, sub-block sums, row scales) for m rows of k.
int64_t aeth_gemm_ws_bytes(int64_t m, int64_t k);

// GGUF file → runner (aeth_gguf.cpp): LlamaModel::from_gguf on the device load path.
struct aeth_runner;
int aeth_gguf_load_runner(const char* path, aeth_runner** out, int* bos, int* eos);

