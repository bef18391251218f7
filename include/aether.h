/*
 * aether.h — the reference's C ABI (theoxfaber/aether aether.h:28-81,
 * implemented in src/c_api.rs), served by the gfx950 device runner.
 *
 * Same functions, argument meaning and return codes as the reference:
 * 0 = AETHER_OK, -1 = AETHER_ERR, -2 = AETHER_TIMEOUT; logits buffers hold
 * aether_vocab_size() floats. Differences of this build:
 *   - aether_load / aether_load_streaming read a GGUF v3 file (gguf.rs:297-397,
 *     model_loader.rs:159-386) into the device runner: layer and LM-head
 *     weights F32 / F16 / Q8_0 / Q2_K..Q6_K (any mix across tensors, as in
 *     Q4_K_M / Q5_K_M / Q3_K_M files; F32 / F16 / Q2_K / Q3_K need
 *     out_features % 4 == 0), norms F32 / F16, head_dim 128, at most 8 query heads per KV
 *     head, no partial RoPE; attention.sliding_window_length is honoured
 *     (ArchConfig::sliding_window) and the cache holds min(context_length,
 *     4096) positions, as LlamaRunner::new sizes it (runner.rs:225), and
 *     aether_context_len reports that. max_hot is ignored: every layer
 *     stays in HBM. Other files return NULL with the reason in
 *     aether_last_error. Models can also be created with
 *     aeth_runner_create (aether_hip.h) and wrapped by
 *     aether_model_from_runner — no counterpart in the reference.
 *   - aether_encode / aether_decode_token: no tokenizer (NULL).
 *   - aether_sample: greedy only (temperature <= 1e-6 or top_p <= 1e-6).
 *   - aether_prefill runs the batched device prefill (aeth_runner_prefill:
 *     positions 0..n-1, cache slots 0..n-1), returning the last logits.
 */
#ifndef AETHER_H
#define AETHER_H

#define AETHER_API __attribute__((visibility("default")))

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct aether_model aether_model;

#define AETHER_OK 0
#define AETHER_ERR -1
#define AETHER_TIMEOUT -2

/* model lifecycle (aether.h:28-30; c_api.rs:53-95) */
AETHER_API aether_model* aether_load(const char* path);
AETHER_API aether_model* aether_load_streaming(const char* path, int max_hot);
AETHER_API void aether_free(aether_model* model);

/* no counterpart in the reference: wraps a device runner (aether_hip.h);
 * the model owns it afterwards and aether_free releases it. */
struct aeth_runner;
AETHER_API aether_model* aether_model_from_runner(struct aeth_runner* runner);

/* config queries (aether.h:34-41) */
AETHER_API int aether_vocab_size(const aether_model* model);
AETHER_API int aether_context_len(const aether_model* model);
AETHER_API int aether_num_layers(const aether_model* model);
AETHER_API int aether_d_model(const aether_model* model);
AETHER_API int aether_eos_id(const aether_model* model);
AETHER_API int aether_bos_id(const aether_model* model);
AETHER_API int aether_num_gpu_layers(const aether_model* model);
AETHER_API int aether_num_cpu_layers(const aether_model* model);

/* frame budget (aether.h:52-53) */
AETHER_API void aether_set_frame_budget(aether_model* model, float max_ms);
AETHER_API float aether_frame_budget(const aether_model* model);

/* tokenization (aether.h:57-60) */
AETHER_API int* aether_encode(const aether_model* model, const char* text, int* out_len);
AETHER_API char* aether_decode_token(const aether_model* model, int token);
AETHER_API void aether_free_string(char* s);
AETHER_API void aether_free_tokens(int* tokens);

/* inference (aether.h:72-74) */
AETHER_API int aether_prefill(aether_model* model, const int* tokens, int n_tokens, float* logits_out);
AETHER_API int aether_decode(aether_model* model, int token, int pos, float* logits_out);
AETHER_API int aether_decode_budgeted(aether_model* model, int token, int pos, float* logits_out);

/* sampling (aether.h:78-79) */
AETHER_API int aether_sample(const aether_model* model, const float* logits, float temperature, float top_p);
AETHER_API int aether_argmax(const aether_model* model, const float* logits);

/* error (aether.h:83); free with aether_free_string */
AETHER_API char* aether_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* AETHER_H */
