// Prefill GEMM for Q4_K weights (m > 1): placeholder routing to the
// row-batched GEMV until the MFMA kernel lands.
#include "aeth_common.hpp"
#include "aeth_internal.hpp"

int aeth_gemm_q4k_launch(const aeth_weight* w, const float* d_a, int64_t m, float* d_c, unsigned flags,
                         hipStream_t s) {
    return aeth_gemv_launch(w, d_a, m, d_c, flags, s);
}
