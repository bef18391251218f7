// Internal launchers of the decode-step kernels (aeth_decode_ops.hip).
// Scalars given as (device pointer, value): the pointer wins when non-NULL.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

int aeth_rmsnorm_launch(const float* x, const float* w, int64_t rows, int64_t n, float eps, float* out,
                        hipStream_t s);
int aeth_rope_launch(float* x, int64_t n_heads, int64_t head_dim, const int* d_pos, int64_t pos,
                     const float* sin_t, const float* cos_t, int64_t max_seq, hipStream_t s);
int aeth_kv_append_launch(float* layer_kv, const float* k, const float* v, int64_t kv_heads, int64_t head_dim,
                          int64_t max_seq, const int* d_slot, int64_t slot, hipStream_t s);
// Attention workspace (floats): the chunk softmax partials.
int64_t aeth_attn_ws_floats(int64_t n_heads, int64_t head_dim, int64_t max_seq);
// Decode attention over one layer slice of the cache. Either q (rotated, with
// seq given) or qkv (fused projection output: RoPE of q/k and the KV append
// of the new token happen here, scalars from d_st = {token, pos, fill}).
// window > 0: sliding-window attention over the last `window` positions.
int aeth_attn_launch(const float* q, const float* qkv, float* layer_kv, const float* sin_t, const float* cos_t,
                     const int* d_st, int64_t seq, int64_t n_heads, int64_t kv_heads, int64_t head_dim,
                     int64_t max_seq, int64_t window, float* ws, float* out, hipStream_t s);
int aeth_silu_mul_launch(float* g, const float* up, int64_t n, hipStream_t s);
int aeth_add_launch(float* x, const float* y, int64_t n, hipStream_t s);
int64_t aeth_argmax_ws_bytes();
int aeth_argmax_launch(const float* x, int64_t n, int* out, int* next_token, void* ws, hipStream_t s);
int aeth_embed_launch(const float* table, const int* d_token, int64_t token, int64_t d, int64_t vocab, float* x,
                      hipStream_t s);
// After a step: token = argmax key's row (key reset to 0), pos += 1, fill
// advanced (StaticKVCache::advance).
int aeth_state_advance_launch(int* st, unsigned long long* amax, int* hist, int64_t max_seq, hipStream_t s);
// Batched prefill glue (aeth_prefill.hip).
int aeth_embed_rows_launch(const float* table, const int* d_tokens, int64_t n, int64_t d, float* x, hipStream_t s);
int aeth_prefill_rope_kv_launch(float* qkv, int64_t n, int64_t nh, int64_t nkv, int64_t hd, const float* sin_t,
                                const float* cos_t, int64_t max_seq, float* layer_kv, hipStream_t s);
// q rows of q_stride floats (the fused projection: (nh + 2·nkv)·hd), head h at column h·hd;
// window > 0: query i sees keys max(0, i - window + 1) ..= i
int aeth_attn_prefill_launch(const float* q, int64_t q_stride, const float* layer_kv, int64_t n, int64_t nh,
                             int64_t nkv, int64_t hd, int64_t max_seq, int64_t window, float* out, hipStream_t s);
int aeth_silu_pairs_launch(const float* gu, int64_t total, float* h, hipStream_t s);
