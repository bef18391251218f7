/* Shared declarations of the CPU oracle (test infrastructure only; the
 * product library never includes or links this). */
#ifndef AETHER_ORACLE_H
#define AETHER_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#define ORC_API __attribute__((visibility("default")))

/* GGUF ggml type ids (src/loader/gguf.rs:92-110). */
enum { ORC_DT_F32 = 0, ORC_DT_F16 = 1, ORC_DT_Q8_0 = 8, ORC_DT_Q2_K = 10, ORC_DT_Q3_K = 11, ORC_DT_Q4_K = 12,
       ORC_DT_Q5_K = 13, ORC_DT_Q6_K = 14 };

ORC_API float orc_f16_to_f32(uint16_t h);
ORC_API uint16_t orc_f32_to_f16(float f);
ORC_API float orc_decode_d(uint16_t bits);
ORC_API void orc_get_scale_min_k4(int j, const uint8_t* s, uint8_t* sc, uint8_t* m);

ORC_API void orc_dequant_q5_k_block(const uint8_t* blk, float* out);
ORC_API int orc_gguf_order_matmul(int dtype, const float* a, size_t m, const uint8_t* b, size_t n, size_t k,
                                  float* c);
#endif
