/*
 * aether_hip.h — C ABI of the MI355X (gfx950) quantized-matmul hot path.
 *
 * Plain pointers and sizes only. Every function returns an int status
 * (AETH_OK = 0, negative on error; the message is in aeth_last_error())
 * and never unwinds. "d_" arguments are device pointers; `stream` is a
 * hipStream_t (NULL = the null stream). Device-pointer entry points are
 * asynchronous on `stream`; host-slice entry points synchronise.
 *
 * Each entry point names the reference interface it replaces
 * (theoxfaber/aether, path:line).
 */
#ifndef AETHER_HIP_H
#define AETHER_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AETH_API __attribute__((visibility("default")))

#define AETH_OK 0
#define AETH_EINVAL (-1)
#define AETH_EHIP (-2)
#define AETH_ENOMEM (-3)
#define AETH_EUNSUPPORTED (-4)
#define AETH_ESTATE (-5)

/* GGUFDtype discriminants, src/loader/gguf.rs:92-110. */
#define AETH_DTYPE_F32 0
#define AETH_DTYPE_F16 1
#define AETH_DTYPE_Q8_0 8
#define AETH_DTYPE_Q2_K 10
#define AETH_DTYPE_Q3_K 11
#define AETH_DTYPE_Q4_K 12
#define AETH_DTYPE_Q5_K 13
#define AETH_DTYPE_Q6_K 14

/* aeth_qmatmul flags */
#define AETH_MM_ACCUMULATE 1u /* c += A·Wᵀ instead of c = A·Wᵀ (fused residual add,
                                 runner.rs:1609-1611, 1629-1631) */
#define AETH_MM_Q8_ACTIVATIONS 2u /* the int8 dot-product path of an aarch64 host with
                                     dotprod (avx2_dispatch.rs:9-44, dispatch.rs:21-22):
                                     activations quantized to Q8_0 blocks as
                                     quantize_activations_q8_0 (neon.rs:106-155) does,
                                     exact integer dots against the weight quants
                                     (matmul_q8_0 / q4_k / q5_k / q6_k_dotprod). Q8_0,
                                     Q4_K, Q5_K, Q6_K weights; ignored for the others,
                                     which have no such path. */

/* ── runtime ─────────────────────────────────────────────────────────────── */

/* Select the device and create the library's per-device state. */
AETH_API int aeth_init(int device);
/* Last error message of the calling thread ("" if none). */
AETH_API const char* aeth_last_error(void);
/* Block geometry, GGUFDtype::block_size/block_byte_size (gguf.rs:137-173). */
AETH_API int aeth_block_geometry(int dtype, int* block_elems, int* block_bytes);

/* ── device-resident weights ─────────────────────────────────────────────
 * A registered weight is the device copy of one QuantWeight
 * (src/inference/model_loader.rs:88-93) of shape [n, k] (out, in), with
 * `raw` exactly as QuantWeight.data holds it:
 *   Q8_0 / Q4_K / Q5_K / Q6_K — n rows of k/block_elems GGUF blocks (the
 *     form load_quant re-quantizes them into, model_loader.rs:344-347);
 *     re-laid on upload into per-field planes (scales / quants split so every
 *     wave load is 16-byte aligned and contiguous);
 *   F32 / F16 / Q2_K / Q3_K — the GGUF tensor as the file holds it, [k][n]
 *     read as one flat run of elements / blocks (model_loader.rs:348-350);
 *     kept as is (Q2_K / Q3_K need n % 256 == 0).
 * aeth_weight_export_raw reproduces the original bytes. The QuantKernel
 * host-slice path registers weights implicitly (see aeth_quantized_matmul_impl). */
typedef struct aeth_weight aeth_weight;

AETH_API int aeth_weight_create(int dtype, int64_t n, int64_t k, const void* raw, int raw_is_device,
                                void* stream, aeth_weight** out);
AETH_API int aeth_weight_free(aeth_weight* w);
/* Device bytes held by the weight's planes (== raw GGUF bytes). */
AETH_API int64_t aeth_weight_bytes(const aeth_weight* w);
AETH_API int aeth_weight_export_raw(const aeth_weight* w, void* dst, int dst_is_device, void* stream);

/* ── kernels ───────────────────────────────────────────────────────────── */

/* GGUF blocks → f32, bit-exact with src/loader/dequant.rs: dequant_f32 /
 * dequant_f16 (:57-95), dequant_q8_0 (:103-127), dequant_q4_k (:195-227),
 * dequant_q5_k (:229-285), dequant_q6_k (:301-348), dequant_q2_k (:350-398),
 * dequant_q3_k (:400-451). d_raw holds ceil(n/block_elems) raw blocks; n is
 * rounded down to whole blocks for the K-quants as the reference does (tail
 * left untouched). */
AETH_API int aeth_dequant(int dtype, const void* d_raw, int64_t n_elems, float* d_out, void* stream);

/* f32 [rows][cols] → GGUF blocks [rows][ceil(cols/block_elems)], byte-exact
 * with requantize_q8_0 / requantize_q4_k / requantize_q5_k / requantize_q6_k
 * (src/quant/matmul/dispatch.rs:149-184, 186-300, 302-429, 431-537; entry
 * `requantize` :139-147). d_dst holds rows·ceil(cols/bs)·block_bytes bytes. */
AETH_API int aeth_requantize(int dtype, const float* d_src, int64_t rows, int64_t cols, void* d_dst,
                             void* stream);

/* Q8_0 activation blocks, byte-exact with quantize_activations_q8_0[_batched]
 * (src/quant/matmul/neon.rs:106-155) over quantize_q8_0_block (:45-104):
 * m rows of k f32 → m·ceil(k/32) blocks of 34 bytes (a partial last block is
 * zero-padded). */
AETH_API int aeth_quantize_activations_q8_0(const float* d_a, int64_t m, int64_t k, void* d_dst, void* stream);

/* [rows][cols] f32 → [cols][rows] (the transpose inside transpose_quantized_bytes,
 * src/inference/model_loader.rs:372-385). d_src and d_dst must not overlap. */
AETH_API int aeth_transpose_f32(const float* d_src, int64_t rows, int64_t cols, float* d_dst, void* stream);

/* load_quant (src/inference/model_loader.rs:330-386) for a 2-D quantized
 * tensor on the device: GGUF bytes of shape [k, n] → dequantize → transpose
 * → requantize, giving [n][k] row blocks in d_dst (n·ceil(k/bs)·block_bytes
 * bytes, the layout aeth_weight_create takes). d_ws holds
 * aeth_load_quant_ws_bytes(k, n) bytes (-1 when k·n is too large to size).
 * Q8_0, Q4_K, Q5_K and Q6_K (the
 * formats is_quantized_type_supported names, model_loader.rs:362-367). */
AETH_API int64_t aeth_load_quant_ws_bytes(int64_t k, int64_t n);
AETH_API int aeth_load_quant(int dtype, const void* d_src, int64_t k, int64_t n, void* d_dst, void* d_ws,
                             void* stream);

/* C[m×n] = A[m×k] · Wᵀ on the device — QuantKernel::matmul
 * (src/quant/matmul/registry.rs:7-19) / quantized_matmul_impl
 * (src/quant/matmul/dispatch.rs:98-135) with device operands. Routing:
 *   - m == 1: the matrix-core decode GEMV (Q8_0, Q4_K, Q5_K, Q6_K rows);
 *   - m > 1, Q4_K / Q5_K / Q6_K / Q8_0 rows: the exact-mode fp16 MFMA GEMMs —
 *     Q4_K and Q5_K from 16 rows (from 5 once m · weight bytes reaches 150 MB),
 *     Q6_K once m · weight bytes reaches 200 MB, Q8_0 from 3 rows once it
 *     reaches 180 MB (380 MB for a weight up to 32 MiB) — the row-batched GEMV
 *     below that; Q5_K / Q6_K / Q8_0 products the GEMMs do not take (k not
 *     whole super-blocks / blocks, buffers past 32-bit offsets) run the
 *     row-batched GEMV up to 80 / 80 / 112 rows, then the DGEMM below;
 *   - m > 1, GGUF-order Q2_K / Q3_K: the row-batched GEMV up to a per-format
 *     row count (Q2_K 40, Q3_K 32), then the weight dequantized once and one
 *     rocBLAS f64 DGEMM (also every K-quant product of the dot-product mode
 *     with k not a multiple of 256);
 *   - F32 / F16 / Q2_K / Q3_K in GGUF order: the kernel of matmul_f32_gguf
 *     (dispatch.rs:541-574) for the rows not sent to the DGEMM.
 * Stream scratch: the GEMMs' activation fragments and split-K partials, the
 * GGUF-order kernel's partials, and the DGEMM's dequantized weight, f64
 * operands and partials live in buffers the library keeps per (device,
 * stream), as do the rocBLAS handles: calls on different streams never share
 * them, calls on one stream run in order. A buffer grows on first use of a
 * larger shape (a grow waits for the stream and fails with AETH_ESTATE during
 * graph capture: run every shape once before capturing). Several host
 * threads enqueueing on the same stream at once must serialise their calls. */
AETH_API int aeth_qmatmul(const aeth_weight* w, const float* d_a, int64_t m, float* d_c, unsigned flags,
                          void* stream);

/* Same, on GGUF bytes and host slices: quantized_matmul_impl
 * (dispatch.rs:98-106) with b_shape = [n, k] — every format above, with the
 * byte order of aeth_weight_create. The weight bytes are uploaded once and
 * cached (see aeth_weight_cache_clear); a and c are copied per call. Calls on
 * one device are serialised. Fails (no CPU fallback) if no device is usable. */
AETH_API int aeth_quantized_matmul_impl(const float* a, int64_t m, const uint8_t* b_raw, int64_t b_len,
                                        int64_t n, int64_t k, int dtype, float* c);
/* quantized_matmul_impl with its b_f32_cache argument (dispatch.rs:98-117):
 * when b_f32_cache is non-NULL it holds the weight dequantized to f32 in GGUF
 * [k][n] order (k·n floats) and c = matmul_f32_gguf(a, cache) — b_raw is then
 * not read; with NULL this is aeth_quantized_matmul_impl. Same caching. */
AETH_API int aeth_quantized_matmul_impl_cached(const float* a, int64_t m, const uint8_t* b_raw, int64_t b_len,
                                               int64_t n, int64_t k, int dtype, float* c, const float* b_f32_cache);
/* quantized_matmul_impl as an aarch64 host with dotprod runs it
 * (avx2_dispatch.rs:9-44, dispatch.rs:21-22): Q8_0 / Q4_K / Q5_K / Q6_K
 * through the int8 dot-product kernels (AETH_MM_Q8_ACTIVATIONS), the other
 * formats as aeth_quantized_matmul_impl. Same arguments and caching. */
AETH_API int aeth_quantized_matmul_dotprod(const float* a, int64_t m, const uint8_t* b_raw, int64_t b_len,
                                           int64_t n, int64_t k, int dtype, float* c);
/* matmul_q8_0 / matmul_q4_k / matmul_q6_k(a, b, m, n, k, c)
 * (src/quant/matmul/avx2_dispatch.rs:58-68): argument order as the reference. */
AETH_API int aeth_matmul_q8_0(const float* a, const uint8_t* b, int64_t b_len, int64_t m, int64_t n,
                              int64_t k, float* c);
AETH_API int aeth_matmul_q4_k(const float* a, const uint8_t* b, int64_t b_len, int64_t m, int64_t n,
                              int64_t k, float* c);
AETH_API int aeth_matmul_q6_k(const float* a, const uint8_t* b, int64_t b_len, int64_t m, int64_t n,
                              int64_t k, float* c);
/* matmul_q5_k (src/quant/matmul/dispatch.rs:15-34, x86: avx2.rs:97-131). */
AETH_API int aeth_matmul_q5_k(const float* a, const uint8_t* b, int64_t b_len, int64_t m, int64_t n,
                              int64_t k, float* c);
/* matmul_q2_k / matmul_q3_k / matmul_f16 (dispatch.rs:37-90; scalar forms
 * q2_k.rs, q3_k.rs, f16.rs; x86: avx2.rs:210-389): b holds n rows of
 * k/256 blocks (F16: n rows of k values), row-major [n][k] — unlike
 * quantized_matmul_impl, which reads these formats in GGUF order. */
AETH_API int aeth_matmul_q2_k(const float* a, const uint8_t* b, int64_t b_len, int64_t m, int64_t n,
                              int64_t k, float* c);
AETH_API int aeth_matmul_q3_k(const float* a, const uint8_t* b, int64_t b_len, int64_t m, int64_t n,
                              int64_t k, float* c);
AETH_API int aeth_matmul_f16(const float* a, const uint8_t* b, int64_t b_len, int64_t m, int64_t n,
                             int64_t k, float* c);
/* QuantKernel registry (registry.rs:33-63): registers the HIP kernels for
 * F32, F16, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K and Q6_K (bytes as
 * quantized_matmul_impl passes them); a second registration of a dtype fails with
 * AETH_ESTATE (the reference panics). aeth_dispatch_matmul returns 1 if a
 * registered kernel handled the call, 0 if none is registered for dtype, <0
 * on error. */
AETH_API int aeth_register_hip_kernels(void);
AETH_API int aeth_registered_kernel_name(int dtype, char* buf, int buf_len);
AETH_API int aeth_dispatch_matmul(const float* a, int64_t m, const uint8_t* b_raw, int64_t b_len, int64_t n,
                                  int64_t k, int dtype, float* c);
/* The host-slice weight cache (no counterpart in the reference, whose
 * QuantKernel::matmul reads b_raw on every call): entries are keyed by
 * (pointer, length, dtype, n, k, device) and every hit is re-checked against a
 * 64-bit fingerprint of the bytes, so a buffer rewritten in place or
 * reallocated at the same address is uploaded again. clear drops every entry;
 * set_limit bounds the device bytes held (least recently used entries go
 * first; default 32 GiB; a weight larger than the limit is not kept);
 * cache_bytes reports the bytes held. */
AETH_API int aeth_weight_cache_clear(void);
AETH_API int aeth_weight_cache_set_limit(int64_t max_bytes);
AETH_API int64_t aeth_weight_cache_bytes(void);
/* The fingerprint a host-slice call computes over the weight bytes (the
 * per-call cost of the check above; exported to time it). */
AETH_API int aeth_weight_fingerprint(const void* host, int64_t bytes, uint64_t* out);

/* rmsnorm_inplace (runner.rs:1739-1746) on `rows` rows of n: out = x/rms*w. */
AETH_API int aeth_rmsnorm(const float* d_x, const float* d_w, int64_t rows, int64_t n, float eps,
                          float* d_out, void* stream);
/* apply_rope_inplace (runner.rs:1886-1909), rotate-half, one position, with
 * the host-built table of precompute_rope (runner.rs:1912-1924) already on
 * the device ([max_seq][head_dim/2] each); pos is clamped to max_seq-1. */
AETH_API int aeth_rope(float* d_x, int64_t n_heads, int64_t head_dim, int64_t pos, const float* d_sin,
                       const float* d_cos, int64_t max_seq, void* stream);
/* StaticKVCache::append (kv_cache.rs:40-65) for one layer: copies k, v
 * ([kv_heads][head_dim]) into slot `slot` of the [2][kv_heads][max_seq][hd]
 * layer slice d_layer_kv. */
AETH_API int aeth_kv_append(float* d_layer_kv, const float* d_k, const float* d_v, int64_t kv_heads,
                            int64_t head_dim, int64_t max_seq, int64_t slot, void* stream);
/* GQA decode attention (runner.rs:1579-1603 with attn_direct :1757-1801)
 * over positions [0, seq) of one layer slice of the static cache. */
AETH_API int aeth_attn_decode(const float* d_q, const float* d_layer_kv, int64_t n_heads, int64_t kv_heads,
                              int64_t head_dim, int64_t max_seq, int64_t seq, float* d_out, void* stream);
/* No counterpart in the reference: aeth_attn_decode for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). Same arguments and results; the chunk partials go to a
 * static device array of 4 MiB (1,048,576 floats) per GPU instead of a
 * library allocation, so n_heads·ceil(max_seq/128)·(head_dim+2) must not exceed
 * 1,048,576 (AETH_EINVAL otherwise). Calls that overlap on one GPU share that
 * array and race: serialise them (one stream, or one caller at a time). */
AETH_API int aeth_attn_decode_noalloc(const float* d_q, const float* d_layer_kv, int64_t n_heads, int64_t kv_heads,
                                      int64_t head_dim, int64_t max_seq, int64_t seq, float* d_out, void* stream);
/* Causal GQA attention of a prompt batch (attention_batch, runner.rs:1809-1883):
 * query i (row i of d_q, [n][q_stride] with head h at column h*head_dim, RoPE
 * already applied) attends to cache slots 0..i of the layer slice d_layer_kv
 * ([2][kv_heads][max_seq][head_dim]); d_out is [n][n_heads*head_dim]. */
AETH_API int aeth_attn_prefill(const float* d_q, int64_t q_stride, const float* d_layer_kv, int64_t n,
                               int64_t n_heads, int64_t kv_heads, int64_t head_dim, int64_t max_seq, float* d_out,
                               void* stream);
/* SiLU-MLP glue (runner.rs:1617-1625): g = g * sigmoid(g) * up. */
AETH_API int aeth_silu_mul(float* d_gate, const float* d_up, int64_t n, void* stream);
/* Residual add (runner.rs:1609-1611): x += y. */
AETH_API int aeth_add(float* d_x, const float* d_y, int64_t n, void* stream);
/* Greedy sample (runner.rs:1964-1973; aether_argmax c_api.rs:384-396):
 * index of the maximum, the LAST one on ties; result written to d_out. */
AETH_API int aeth_argmax(const float* d_logits, int64_t n, int32_t* d_out, void* stream);

/* ── device trait Backend (src/backend/mod.rs:12-218) ─────────────────────
 * The decode-path ops of the reference's Backend, which a Rust
 * `impl Backend for HipBackend` binds (its execute() matches Op::RmsNorm and
 * Op::CausalAttention and returns an error for every other op — there is no
 * CPU fallback, unlike CudaBackend::execute, src/backend/cuda.rs:60-64).
 * Host slices in and out (Tensor data), synchronous. */
/* Backend::rms_norm → Op::RmsNorm { epsilon } (cpu.rs:514-545): x holds
 * rows·last_dim f32 ([..., last_dim] flattened), w last_dim; per row
 * out = (x / sqrt(Σx²/last_dim + eps)) · w. */
AETH_API int aeth_backend_rms_norm(const float* x, const float* w, int64_t rows, int64_t last_dim, float eps,
                                   float* out);
/* Backend::causal_attention → Op::CausalAttention { scale, num_heads }
 * (mod.rs:209-218, cpu.rs:1660-1727): q, k, v, out are [batch][seq][d] f32;
 * head h owns columns [h·hd, (h+1)·hd), hd = d / num_heads (columns past
 * num_heads·hd are 0); query i attends to keys 0..i with softmax((q·k)·scale).
 * head_dim up to 256; num_heads == 0 is AETH_EINVAL (the reference panics). */
AETH_API int aeth_backend_causal_attention(const float* q, const float* k, const float* v, int64_t batch,
                                           int64_t seq, int64_t d, int64_t num_heads, float scale, float* out);
/* The same attention on device pointers, asynchronous on `stream`. */
AETH_API int aeth_causal_attention(const float* d_q, const float* d_k, const float* d_v, int64_t batch, int64_t seq,
                                   int64_t d, int64_t num_heads, float scale, float* d_out, void* stream);

/* ── synthetic inputs (generated on the device, counter-based, seeded) ───
 * Raw GGUF blocks as the benchmark configs describe them:
 *   Q8_0: d = f16(|N(0,1)|*0.01), q uniform int in [-127,127];
 *   Q4_K: d, dmin = f16(|N(0,1)|*0.01), scales[12] and qs[128] uniform bytes;
 *   Q6_K: d = f16(|N(0,1)|*0.01), sc uniform int in [-64,63], ql/qh uniform bytes.
 * The same (seed, block index) always yields the same bytes. */
AETH_API int aeth_fill_synthetic_raw(int dtype, uint64_t seed, void* d_raw, int64_t n_blocks, void* stream);
/* out[i] = mean + std * N(0,1) from (seed, i). */
AETH_API int aeth_fill_normal_f32(uint64_t seed, float* d_out, int64_t n, float mean, float std, void* stream);

/* Measurement kernel, no counterpart in the reference: reads `bytes`
 * (a multiple of 16, 16-byte aligned) once with streaming loads, the plain
 * HBM read a single launch of that size achieves (the benchmark's floor for
 * the GEMVs). d_sink holds sink_words >= 256 words (256 per workgroup used,
 * up to 2048 workgroups); a word is written only if the fold of the input
 * hits one fixed value. */
AETH_API int aeth_stream_read(const void* d_src, int64_t bytes, uint32_t* d_sink, int64_t sink_words, void* stream);
/* Measurement kernel, no counterpart in the reference: `workgroups` × 4 waves
 * each issue iters × 8 independent matrix-core instructions on register
 * operands — kind 0: v_mfma_f32_32x32x16_f16 (32768 flops each), kind 1:
 * v_mfma_i32_32x32x32_i8 (65536 ops each): the rate the box sustains (the
 * GEMM's second roofline). d_sink holds workgroups × 256 floats; a value is
 * written only if a fold of the results hits one fixed value. */
AETH_API int aeth_mfma_rate(int kind, int iters, int workgroups, float* d_sink, void* stream);

/* ── LlamaRunner (src/inference/runner.rs) on the device ─────────────────
 * Model shape = LlamaConfig (model_loader.rs:71-84). sliding_window is
 * ArchConfig::sliding_window (model_loader.rs:62-67; 0 = None): decode and
 * prefill attention see the last sliding_window positions only
 * (runner.rs:1768-1777, :1825-1845). As LlamaRunner::new / new_streaming do
 * (runner.rs:225, :339), the runner's cache and RoPE table hold
 * min(max_seq_len, 4096) positions; flags AETH_CFG_FULL_CONTEXT keeps
 * max_seq_len instead (up to 8192, the decode attention's limit) — an
 * opt-in with no counterpart in the reference. */
typedef struct aeth_llama_config {
    int32_t vocab_size, d_model, num_layers, num_heads, num_kv_heads, head_dim, d_ff, max_seq_len;
    float rope_base, rms_norm_eps;
    int32_t sliding_window;
    int32_t flags;
} aeth_llama_config;
#define AETH_CFG_FULL_CONTEXT 1
#define AETH_RUNNER_MAX_SEQ 4096

typedef struct aeth_runner aeth_runner;

/* Creates a runner with device weights and a zeroed StaticKVCache of
 * min(max_seq_len, 4096) positions (max_seq_len with AETH_CFG_FULL_CONTEXT). Host buffers: per layer l, layer_weights[l*7+j]
 * for j = q,k,v,o,gate,up,down (each as its QuantWeight holds it: [out][in]
 * row blocks for Q8_0 / Q4_K / Q5_K / Q6_K, the GGUF [in][out] tensor for
 * F32 / F16 / Q2_K / Q3_K — see aeth_weight_create), layer_dtypes likewise; norms[l*2+{0,1}] = attn_norm, ffn_norm (f32);
 * final_norm (f32, d_model); lm_head (raw, dtype lm_dtype); embeddings
 * f32 [vocab][d_model]. Any pointer may be NULL when `synthetic_seed` is
 * nonzero: the runner then generates that tensor on the device (weights as
 * aeth_fill_synthetic_raw with the dtypes given, norms 1+N(0,0.02),
 * embeddings N(0,1)). */
AETH_API int aeth_runner_create(const aeth_llama_config* cfg, const void* const* layer_weights,
                                const int32_t* layer_dtypes, const float* const* norms, const float* final_norm,
                                const void* lm_head, int32_t lm_dtype, const float* embeddings,
                                uint64_t synthetic_seed, aeth_runner** out);
AETH_API int aeth_runner_free(aeth_runner* r);
/* Fills the first `seq_len` cache positions of every layer with N(0,1) from
 * `seed` and sets the cache fill (prefilled-context benchmark setup). */
AETH_API int aeth_runner_fill_kv(aeth_runner* r, uint64_t seed, int32_t seq_len);
/* Copies KV storage [L][2][kv_heads][max_seq][hd] to/from the host and sets the fill. */
AETH_API int aeth_runner_kv_to_host(aeth_runner* r, float* host, int32_t* seq_len);
AETH_API int aeth_runner_kv_from_host(aeth_runner* r, const float* host, int32_t seq_len);
AETH_API int aeth_runner_seq_len(const aeth_runner* r);
/* One decode step (forward_one_internal, runner.rs:1175-1649): token's
 * embedding → L layers → final norm → LM head. logits (host, vocab floats)
 * may be NULL; next_token (host) receives the greedy argmax if non-NULL. */
AETH_API int aeth_runner_decode(aeth_runner* r, int32_t token, int32_t pos, float* logits, int32_t* next_token);
/* Batched prefill (LlamaRunner::prefill, runner.rs:695-704 → forward_batch,
 * :833-993): the n prompt tokens (host) are placed at positions 0..n-1 in
 * one pass (GEMM projections, causal attention_batch :1809-1883), K/V written
 * to cache slots 0..n-1, and the cache fill becomes n. logits (host, vocab
 * floats) receive the last token's logits and next_token its greedy argmax;
 * either may be NULL. 1 <= n <= max_seq_len. */
AETH_API int aeth_runner_prefill(aeth_runner* r, const int32_t* tokens, int32_t n, float* logits,
                                 int32_t* next_token);
/* Greedy decode of n_steps tokens starting from `token` at `pos`; tokens
 * (host, n_steps) receive each step's argmax (fed back as the next input).
 * Uses a captured HIP graph per step when use_graph != 0. */
AETH_API int aeth_runner_generate(aeth_runner* r, int32_t token, int32_t pos, int32_t n_steps, int32_t* tokens,
                                  int use_graph);
/* Copies device tensors back for checking: which = 0..6 layer weight j of
 * layer l (raw GGUF bytes), 7 attn_norm, 8 ffn_norm, 9 final_norm, 10 lm_head
 * (raw), 11 embedding row `l`, 12 rope sin table, 13 rope cos table. */
AETH_API int aeth_runner_export(const aeth_runner* r, int which, int32_t l, void* host, int64_t host_bytes);
/* The stream the runner launches on (hipStream_t). */
AETH_API void* aeth_runner_stream(const aeth_runner* r);

#ifdef __cplusplus
}
#endif

#endif /* AETHER_HIP_H */
