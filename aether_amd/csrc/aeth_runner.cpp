// LlamaRunner on the device (src/inference/runner.rs) and the aether_* C ABI
// (aether.h:28-81, src/c_api.rs).
//
// Every tensor of a decode step stays in HBM: token id in, logits / next
// token out. The step reads its scalars {token, pos, cache fill} from a
// device int[3], so one step is captured once as a HIP graph and replayed
// for greedy generation without host round trips.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <chrono>
#include <mutex>
#include <vector>

#include "../../include/aether.h"
#include "aeth_common.hpp"
#include "aeth_internal.hpp"
#include "aeth_ops_internal.hpp"

struct aeth_runner {
    aeth_llama_config cfg;
    hipStream_t stream = nullptr;
    // weights
    // per layer: q|k|v rows concatenated; gate and up rows interleaved
    // (row 2i = gate_i, row 2i+1 = up_i) for the fused SwiGLU epilogue
    std::vector<aeth_weight*> wqkv, wo, wgu, wdown;
    // per layer, set when q/k/v (gate/up) do not share a dtype: the fused weight is then NULL
    std::vector<aeth_weight*> wq, wk, wv, wg, wu;
    // per layer, set when q and k share a fused dtype and v does not (llama.cpp's Q4_K_M keeps
    // attn_v in Q6_K): q|k rows concatenated, v in wv, wq / wk NULL
    std::vector<aeth_weight*> wqk;
    std::vector<int> dtypes;                         // per layer x 7
    aeth_weight* lm_head = nullptr;
    float* norms = nullptr;       // [L][2][d]
    float* final_norm = nullptr;  // [d]
    float* emb = nullptr;         // [vocab][d]
    float* rope_sin = nullptr;    // [max_seq][hd/2]
    float* rope_cos = nullptr;
    float* kv = nullptr;          // [L][2][kvh][max_seq][hd]
    // activations
    float *x = nullptr, *normed = nullptr, *qkv = nullptr, *attn = nullptr, *gu = nullptr, *logits = nullptr;
    float* attn_ws = nullptr;
    void* am_ws = nullptr;
    float* xws = nullptr;    // scratch of the GGUF-order GEMVs (F32 / F16 / Q2_K / Q3_K weights)
    int64_t xws_floats = 0;
    int* st = nullptr;       // device {token, pos, fill, next token}
    unsigned long long* amax = nullptr;  // fused LM-head argmax key (reset by the state kernel)
    int* tok_out = nullptr;  // [max_seq] greedy tokens of the current generate call, by step
    int fill = 0;           // host mirror of the cache fill
    hipGraphExec_t graph = nullptr;
    // batched prefill buffers (grow-only): rows of x, normed x, q|k|v, attention
    // output, interleaved gate|up, SiLU product; prompt token ids
    float *p_x = nullptr, *p_n = nullptr, *p_qkv = nullptr, *p_att = nullptr, *p_gu = nullptr, *p_h = nullptr;
    int* p_tok = nullptr;
    int64_t p_cap = 0;
    // frame budget / partial decode (runner.rs:1201-1282, c_api.rs:313-355)
    float frame_budget_ms = 0.0f;
    bool partial_valid = false;
    int partial_token = 0, partial_pos = 0, partial_layer = 0;
    std::mutex mu;
};

namespace {

const int64_t kKvd(const aeth_llama_config& c) { return (int64_t)c.num_kv_heads * c.head_dim; }

int64_t kv_layer_floats(const aeth_llama_config& c) {
    return 2LL * c.num_kv_heads * (int64_t)c.max_seq_len * c.head_dim;
}

// precompute_rope (runner.rs:1912-1924) with the host libm (f32 powf/sinf/cosf).
void precompute_rope(int max_seq, int head_dim, float base, std::vector<float>& s, std::vector<float>& c) {
    int half = head_dim / 2;
    s.resize((size_t)max_seq * half);
    c.resize((size_t)max_seq * half);
    for (int p = 0; p < max_seq; p++)
        for (int i = 0; i < half; i++) {
            float theta = (float)p * powf(base, -2.0f * (float)i / (float)head_dim);
            s[(size_t)p * half + i] = sinf(theta);
            c[(size_t)p * half + i] = cosf(theta);
        }
}

int make_weight(int dtype, int64_t n, int64_t k, const void* host_raw, uint64_t seed, hipStream_t s,
                aeth_weight** out) {
    int be, bb;
    int rc = aeth_block_geometry(dtype, &be, &bb);
    if (rc) return rc;
    if (host_raw) return aeth_weight_create(dtype, n, k, host_raw, 0, s, out);
    const int order = aeth_dtype_fused(dtype) ? AETH_ORDER_PLANAR : AETH_ORDER_GGUF;
    const int64_t nblk = aeth_weight_raw_bytes(dtype, order, n, k) / bb;
    void* raw = nullptr;
    AETH_HIP_CHECK(hipMalloc(&raw, (size_t)(nblk * bb)));
    rc = aeth_fill_synthetic_raw(dtype, seed, raw, nblk, s);
    if (!rc) rc = aeth_weight_create(dtype, n, k, raw, 1, s, out);
    hipError_t e = hipStreamSynchronize(s);
    hipFree(raw);
    if (!rc && e != hipSuccess) rc = aeth_set_error(AETH_EHIP, "make_weight sync: %s", hipGetErrorString(e));
    return rc;
}

// Rows of several host weights concatenated (same dtype and k) into one
// device weight: row-major [out][in] blocks concatenate byte-wise.
int make_concat(int dtype, const std::vector<int64_t>& ns, int64_t k, const std::vector<const void*>& hosts,
                uint64_t seed, hipStream_t s, aeth_weight** out) {
    int be, bb;
    int rc = aeth_block_geometry(dtype, &be, &bb);
    if (rc) return rc;
    int64_t rowb = aeth_blocks_per_row(dtype, k) * bb, ntot = 0;
    for (auto n : ns) ntot += n;
    bool any_host = false, all_host = true;
    for (auto h : hosts) { any_host |= h != nullptr; all_host &= h != nullptr; }
    if (any_host && !all_host) return aeth_set_error(AETH_EINVAL, "runner: partial host weights for a fused group");
    if (!all_host) return make_weight(dtype, ntot, k, nullptr, seed, s, out);
    std::vector<uint8_t> cat((size_t)(ntot * rowb));
    size_t off = 0;
    for (size_t i = 0; i < ns.size(); i++) {
        memcpy(cat.data() + off, hosts[i], (size_t)(ns[i] * rowb));
        off += (size_t)(ns[i] * rowb);
    }
    return aeth_weight_create(dtype, ntot, k, cat.data(), 0, s, out);
}

// gate (rows 0..dff) and up interleaved row by row: row 2i = gate_i, 2i+1 = up_i.
int make_interleaved(int dtype, int64_t dff, int64_t k, const void* gate, const void* up, uint64_t seed,
                     hipStream_t s, aeth_weight** out) {
    if (!gate && !up) return make_weight(dtype, 2 * dff, k, nullptr, seed, s, out);
    if (!gate || !up) return aeth_set_error(AETH_EINVAL, "runner: gate/up must both be given");
    int be, bb;
    int rc = aeth_block_geometry(dtype, &be, &bb);
    if (rc) return rc;
    const int64_t rowb = aeth_blocks_per_row(dtype, k) * bb;
    std::vector<uint8_t> cat((size_t)(2 * dff * rowb));
    for (int64_t i = 0; i < dff; i++) {
        memcpy(cat.data() + (size_t)(2 * i) * rowb, (const uint8_t*)gate + i * rowb, (size_t)rowb);
        memcpy(cat.data() + (size_t)(2 * i + 1) * rowb, (const uint8_t*)up + i * rowb, (size_t)rowb);
    }
    return aeth_weight_create(dtype, 2 * dff, k, cat.data(), 0, s, out);
}

template <typename T>
int dmalloc(T** p, int64_t count) {
    AETH_HIP_CHECK(hipMalloc((void**)p, sizeof(T) * (size_t)(count > 0 ? count : 1)));
    return AETH_OK;
}

uint64_t mix(uint64_t seed, uint64_t a, uint64_t b) {
    uint64_t z = seed ^ (a * 0x9E3779B97F4A7C15ull) ^ (b * 0xC2B2AE3D27D4EB4Full);
    z = (z ^ (z >> 31)) * 0xBF58476D1CE4E5B9ull;
    return z ^ (z >> 29);
}

void runner_release(aeth_runner* r) {
    if (!r) return;
    if (r->stream) hipStreamSynchronize(r->stream);  // nothing in flight reads what is freed below
    if (r->graph) hipGraphExecDestroy(r->graph);
    for (auto* w : r->wqkv) aeth_weight_free(w);
    for (auto* w : r->wo) aeth_weight_free(w);
    for (auto* w : r->wgu) aeth_weight_free(w);
    for (auto* v : {&r->wq, &r->wk, &r->wv, &r->wg, &r->wu, &r->wqk})
        for (auto* w : *v) aeth_weight_free(w);
    for (auto* w : r->wdown) aeth_weight_free(w);
    aeth_weight_free(r->lm_head);
    void* bufs[] = {r->norms, r->final_norm, r->emb, r->rope_sin, r->rope_cos, r->kv, r->x, r->normed, r->qkv,
                    r->attn, r->gu, r->logits, r->attn_ws, r->am_ws, r->st, r->tok_out, r->amax, r->xws,
                    r->p_x, r->p_n, r->p_qkv, r->p_att, r->p_gu, r->p_h, r->p_tok};
    for (void* b : bufs)
        if (b) hipFree(b);
    if (r->stream) {
        aeth_stream_scratch_release(r->stream);  // the GEMM / GGUF-order scratch of this runner's stream
        hipStreamDestroy(r->stream);
    }
    delete r;
}

// Enqueues layers [l0, l1) of one decode step on r->stream; scalars come
// from r->st = {token, pos, fill, next token, generate step}. Per layer (runner.rs:1557-1632):
//   qkv  = rmsnorm(x, attn_norm) · Wqkvᵀ          (norm fused into the GEMV)
//   attn = GQA attention with RoPE + KV append   (one kernel)
//   x   += attn · Woᵀ                              (residual fused)
//   h    = silu(g)·u, [g|u] = rmsnorm(x, ffn_norm) · Wguᵀ (norm + SwiGLU fused)
//   x   += h · Wdownᵀ                              (residual fused)
// A decode-step epilogue carrying the runner's GGUF-order scratch (so no
// launch allocates, as graph capture requires).
GemvEpi step_epi(const aeth_runner* r) {
    GemvEpi e;
    e.ws = r->xws;
    e.ws_floats = r->xws_floats;
    return e;
}

int enqueue_layers(aeth_runner* r, int l0, int l1) {
    const aeth_llama_config& c = r->cfg;
    hipStream_t s = r->stream;
    const int64_t d = c.d_model, hd = c.head_dim, nh = c.num_heads, nkv = c.num_kv_heads;
    int rc;
    for (int l = l0; l < l1; l++) {
        float* lkv = r->kv + (int64_t)l * kv_layer_floats(c);
        GemvEpi e1 = step_epi(r);
        e1.norm_w = r->norms + (int64_t)l * 2 * d;
        e1.eps = c.rms_norm_eps;
        if (r->wqkv[l]) {
            if ((rc = aeth_gemv_launch_ex(r->wqkv[l], r->x, 1, r->qkv, e1, s))) return rc;
        } else if (r->wqk[l]) {  // q|k, then v of another format
            if ((rc = aeth_gemv_launch_ex(r->wqk[l], r->x, 1, r->qkv, e1, s)) ||
                (rc = aeth_gemv_launch_ex(r->wv[l], r->x, 1, r->qkv + (nh + nkv) * hd, e1, s)))
                return rc;
        } else {  // q, k, v of different formats: three GEMVs into the q|k|v vector
            const int64_t qd = nh * hd, kvd = nkv * hd;
            if ((rc = aeth_gemv_launch_ex(r->wq[l], r->x, 1, r->qkv, e1, s)) ||
                (rc = aeth_gemv_launch_ex(r->wk[l], r->x, 1, r->qkv + qd, e1, s)) ||
                (rc = aeth_gemv_launch_ex(r->wv[l], r->x, 1, r->qkv + qd + kvd, e1, s)))
                return rc;
        }
        if ((rc = aeth_attn_launch(nullptr, r->qkv, lkv, r->rope_sin, r->rope_cos, r->st, 0, nh, nkv, hd,
                                   c.max_seq_len, c.sliding_window, r->attn_ws, r->attn, s)))
            return rc;
        GemvEpi e2 = step_epi(r);
        e2.flags = AETH_MM_ACCUMULATE;
        if ((rc = aeth_gemv_launch_ex(r->wo[l], r->attn, 1, r->x, e2, s))) return rc;
        GemvEpi e3 = step_epi(r);
        e3.norm_w = r->norms + (int64_t)l * 2 * d + d;
        e3.eps = c.rms_norm_eps;
        if (r->wgu[l]) {
            e3.swiglu = 1;
            if ((rc = aeth_gemv_launch_ex(r->wgu[l], r->x, 1, r->gu, e3, s))) return rc;
        } else {  // gate and up of different formats: g, u, then g·σ(g)·u in place
            const int64_t dff = c.d_ff;
            if ((rc = aeth_gemv_launch_ex(r->wg[l], r->x, 1, r->gu, e3, s)) ||
                (rc = aeth_gemv_launch_ex(r->wu[l], r->x, 1, r->gu + dff, e3, s)) ||
                (rc = aeth_silu_mul_launch(r->gu, r->gu + dff, dff, s)))
                return rc;
        }
        if ((rc = aeth_gemv_launch_ex(r->wdown[l], r->gu, 1, r->x, e2, s))) return rc;
    }
    return AETH_OK;
}

// Final norm + LM head with the greedy argmax fused, then the state update
// (StaticKVCache::advance, runner.rs:1639; next token = argmax).
int enqueue_head(aeth_runner* r) {
    const aeth_llama_config& c = r->cfg;
    hipStream_t s = r->stream;
    int rc;
    GemvEpi e = step_epi(r);
    e.norm_w = r->final_norm;
    e.eps = c.rms_norm_eps;
    e.amax = r->amax;
    if ((rc = aeth_gemv_launch_ex(r->lm_head, r->x, 1, r->logits, e, s))) return rc;
    return aeth_state_advance_launch(r->st, r->amax, r->tok_out, c.max_seq_len, s);
}

int enqueue_step(aeth_runner* r) {
    int rc = aeth_embed_launch(r->emb, r->st, 0, r->cfg.d_model, r->cfg.vocab_size, r->x, r->stream);
    if (rc) return rc;
    if ((rc = enqueue_layers(r, 0, r->cfg.num_layers))) return rc;
    return enqueue_head(r);
}

int set_state(aeth_runner* r, int token, int pos);

// Batched prefill (forward_batch, runner.rs:833-993; LlamaRunner::prefill :695-704):
// tokens at positions 0..n-1, K/V at cache slots 0..n-1, per layer
//   xn = rmsnorm(x, attn_norm); qkv = xn · Wqkvᵀ (GEMM, m = n); RoPE + cache write;
//   att = causal attention; x += att · Woᵀ; xn = rmsnorm(x, ffn_norm);
//   [g|u] = xn · Wguᵀ; h = g·σ(g)·u; x += h · Wdownᵀ
// then the decode head on the last row (final norm, LM head, greedy argmax).
int ensure_prefill_buffers(aeth_runner* r, int64_t n) {
    if (n <= r->p_cap) return AETH_OK;
    const aeth_llama_config& c = r->cfg;
    const int64_t d = c.d_model, qd = (int64_t)c.num_heads * c.head_dim, kvd = kKvd(c), dff = c.d_ff;
    AETH_HIP_CHECK(hipStreamSynchronize(r->stream));
    float** bufs[] = {&r->p_x, &r->p_n, &r->p_qkv, &r->p_att, &r->p_gu, &r->p_h};
    const int64_t sizes[] = {n * d, n * (d > dff ? d : dff), n * (qd + 2 * kvd), n * qd, n * 2 * dff, n * dff};
    for (int i = 0; i < 6; i++) {
        if (*bufs[i]) AETH_HIP_CHECK(hipFree(*bufs[i]));
        *bufs[i] = nullptr;
    }
    if (r->p_tok) AETH_HIP_CHECK(hipFree(r->p_tok));
    r->p_tok = nullptr;
    r->p_cap = 0;
    for (int i = 0; i < 6; i++) {
        int rc = dmalloc(bufs[i], sizes[i]);
        if (rc) return rc;
    }
    int rc = dmalloc(&r->p_tok, n);
    if (rc) return rc;
    r->p_cap = n;
    return AETH_OK;
}

int runner_prefill_locked(aeth_runner* r, const int32_t* tokens, int32_t n, float* logits, int32_t* next_token) {
    const aeth_llama_config& c = r->cfg;
    if (!tokens || n <= 0) return aeth_set_error(AETH_EINVAL, "prefill: empty prompt");
    if (n > c.max_seq_len)
        return aeth_set_error(AETH_EINVAL, "prefill: %d tokens exceed max_seq %d", n, c.max_seq_len);
    for (int32_t i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= c.vocab_size)
            return aeth_set_error(AETH_EINVAL, "prefill: token %d out of range [0, %d)", tokens[i], c.vocab_size);
    int rc = ensure_prefill_buffers(r, n);
    if (rc) return rc;
    r->partial_valid = false;
    hipStream_t s = r->stream;
    const int64_t d = c.d_model, hd = c.head_dim, nh = c.num_heads, nkv = c.num_kv_heads, dff = c.d_ff;
    AETH_HIP_CHECK(hipMemcpyAsync(r->p_tok, tokens, sizeof(int32_t) * n, hipMemcpyHostToDevice, s));
    if ((rc = aeth_embed_rows_launch(r->emb, r->p_tok, n, d, r->p_x, s))) return rc;
    for (int l = 0; l < c.num_layers; l++) {
        float* lkv = r->kv + (int64_t)l * kv_layer_floats(c);
        const float* attn_norm = r->norms + (int64_t)l * 2 * d;
        const float* ffn_norm = attn_norm + d;
        // the Q4_K, Q6_K and Q8_0 GEMMs take the RMSNorm inside their activation prep (the SwiGLU: below)
        GemmIn nin;
        nin.mode = PREP_RMSNORM;
        nin.eps = c.rms_norm_eps;
        nin.norm_w = attn_norm;
        {
            // each projection into its columns of the [n][q|k|v] rows: a Q4_K or Q6_K GEMM that
            // takes the RMSNorm in its prep reads x; any other reads rmsnorm(x), formed once
            const int64_t qd = nh * hd, kvd = nkv * hd, ld = qd + 2 * kvd;
            bool normed = false;
            GemmIn pin = nin;  // after the first fused GEMM the stream's scratch holds the prep of x
            auto proj = [&](const aeth_weight* w, float* out) -> int {
                int e;
                if (aeth_gemm_fused_ok(w, n, PREP_RMSNORM, r->p_x, attn_norm)) {
                    e = aeth_gemm_fused_launch(w, r->p_x, n, out, 0, s, ld, &pin);
                } else {
                    if (!normed) {
                        if ((e = aeth_rmsnorm_launch(r->p_x, attn_norm, n, d, c.rms_norm_eps, r->p_n, s))) return e;
                        normed = true;
                    }
                    return aeth_qmatmul_ld(w, r->p_n, n, out, ld, 0, s);
                }
                pin.prepared = e == AETH_OK;
                return e;
            };
            if (r->wqkv[l]) {
                if ((rc = proj(r->wqkv[l], r->p_qkv))) return rc;
            } else if (r->wqk[l]) {
                if ((rc = proj(r->wqk[l], r->p_qkv)) || (rc = proj(r->wv[l], r->p_qkv + qd + kvd))) return rc;
            } else if ((rc = proj(r->wq[l], r->p_qkv)) || (rc = proj(r->wk[l], r->p_qkv + qd)) ||
                       (rc = proj(r->wv[l], r->p_qkv + qd + kvd))) {
                return rc;
            }
        }
        if ((rc = aeth_prefill_rope_kv_launch(r->p_qkv, n, nh, nkv, hd, r->rope_sin, r->rope_cos, c.max_seq_len,
                                              lkv, s)))
            return rc;
        if ((rc = aeth_attn_prefill_launch(r->p_qkv, (nh + 2 * nkv) * hd, lkv, n, nh, nkv, hd, c.max_seq_len,
                                           c.sliding_window, r->p_att, s)))
            return rc;
        if ((rc = aeth_qmatmul(r->wo[l], r->p_att, n, r->p_x, AETH_MM_ACCUMULATE, s))) return rc;
        const float* h = r->p_h;
        GemmIn din;  // the down GEMM's producer
        if (r->wgu[l]) {
            // a Q4_K or Q8_0 gate|up GEMM writes h = g·σ(g)·u from its epilogue (n·d_ff floats instead of the
            // 2·n·d_ff pairs); otherwise the pairs go to p_gu and the down GEMM's prep (or
            // k_silu_pairs) gates them
            GemmIn gin = nin;
            gin.norm_w = ffn_norm;
            gin.swiglu_out = aeth_gemm_swo_ok(r->wgu[l], n);
            float* gu = gin.swiglu_out ? r->p_h : r->p_gu;
            if (aeth_gemm_fused_ok(r->wgu[l], n, PREP_RMSNORM, r->p_x, ffn_norm)) {
                if ((rc = aeth_gemm_fused_launch(r->wgu[l], r->p_x, n, gu, 0, s, 0, &gin))) return rc;
            } else {
                if ((rc = aeth_rmsnorm_launch(r->p_x, ffn_norm, n, d, c.rms_norm_eps, r->p_n, s))) return rc;
                gin.mode = PREP_PLAIN;
                rc = gin.swiglu_out ? aeth_gemm_fused_launch(r->wgu[l], r->p_n, n, gu, 0, s, 0, &gin)
                                    : aeth_qmatmul(r->wgu[l], r->p_n, n, gu, 0, s);
                if (rc) return rc;
            }
            if (gin.swiglu_out) {
                h = r->p_h;
            } else if (aeth_gemm_fused_ok(r->wdown[l], n, PREP_SWIGLU, r->p_gu, nullptr)) {  // in the down prep
                din.mode = PREP_SWIGLU;
                h = r->p_gu;
            } else if ((rc = aeth_silu_pairs_launch(r->p_gu, n * dff, r->p_h, s))) {
                return rc;
            }
        } else {  // g [n][dff], u [n][dff], then g·σ(g)·u in place
            if ((rc = aeth_rmsnorm_launch(r->p_x, ffn_norm, n, d, c.rms_norm_eps, r->p_n, s)) ||
                (rc = aeth_qmatmul(r->wg[l], r->p_n, n, r->p_gu, 0, s)) ||
                (rc = aeth_qmatmul(r->wu[l], r->p_n, n, r->p_gu + n * dff, 0, s)) ||
                (rc = aeth_silu_mul_launch(r->p_gu, r->p_gu + n * dff, n * dff, s)))
                return rc;
            h = r->p_gu;
        }
        rc = din.mode == PREP_SWIGLU ? aeth_gemm_fused_launch(r->wdown[l], h, n, r->p_x, AETH_MM_ACCUMULATE, s, 0, &din)
                                     : aeth_qmatmul(r->wdown[l], h, n, r->p_x, AETH_MM_ACCUMULATE, s);
        if (rc) return rc;
    }
    // head on the last row; the state update then leaves pos = fill = n
    AETH_HIP_CHECK(hipMemcpyAsync(r->x, r->p_x + (int64_t)(n - 1) * d, sizeof(float) * d, hipMemcpyDeviceToDevice, s));
    r->fill = n - 1;
    if ((rc = set_state(r, tokens[n - 1], n - 1))) return rc;
    if ((rc = enqueue_head(r))) return rc;
    if (logits)
        AETH_HIP_CHECK(hipMemcpyAsync(logits, r->logits, sizeof(float) * c.vocab_size, hipMemcpyDeviceToHost, s));
    int tok = 0;
    AETH_HIP_CHECK(hipMemcpyAsync(&tok, r->st + 3, sizeof(int), hipMemcpyDeviceToHost, s));
    AETH_HIP_CHECK(hipStreamSynchronize(s));
    r->fill = n;
    if (next_token) *next_token = tok;
    return AETH_OK;
}

int set_state(aeth_runner* r, int token, int pos) {
    int h[5] = {token, pos, r->fill, token, 0};  // + the generate step counter
    AETH_HIP_CHECK(hipMemcpyAsync(r->st, h, sizeof(h), hipMemcpyHostToDevice, r->stream));
    return AETH_OK;
}

int check_step_args(aeth_runner* r, int token, int pos) {
    if (token < 0 || token >= r->cfg.vocab_size)
        return aeth_set_error(AETH_EINVAL, "decode: token %d out of range [0, %d)", token, r->cfg.vocab_size);
    if (pos < 0) return aeth_set_error(AETH_EINVAL, "decode: negative pos");
    if (r->fill >= r->cfg.max_seq_len)
        return aeth_set_error(AETH_ESTATE, "decode: KV cache full (%d positions)", r->cfg.max_seq_len);
    return AETH_OK;
}

}  // namespace

namespace {
// Releases a half-built runner on every early return or exception.
struct RunnerHold {
    aeth_runner* r = nullptr;
    ~RunnerHold() {
        if (r) runner_release(r);
    }
};

int runner_create_impl(const aeth_llama_config* cfg, const void* const* layer_weights, const int32_t* layer_dtypes,
                       const float* const* norms, const float* final_norm, const void* lm_head, int32_t lm_dtype,
                       const float* embeddings, uint64_t seed, aeth_runner** out) {
    if (!cfg || !out || !layer_dtypes) return aeth_set_error(AETH_EINVAL, "aeth_runner_create: NULL argument");
    *out = nullptr;
    aeth_llama_config c = *cfg;
    if (c.num_layers <= 0 || c.d_model <= 0 || c.num_heads <= 0 || c.num_kv_heads <= 0 || c.head_dim <= 0 ||
        c.d_ff <= 0 || c.vocab_size <= 0 || c.max_seq_len <= 0 || c.num_heads % c.num_kv_heads != 0 ||
        c.head_dim % 2 != 0)
        return aeth_set_error(AETH_EINVAL, "aeth_runner_create: invalid config");
    if (c.head_dim != 128 || c.num_heads / c.num_kv_heads > 8)
        return aeth_set_error(AETH_EUNSUPPORTED, "aeth_runner_create: the attention kernel needs head_dim 128 and "
                                                 "at most 8 query heads per KV head");
    if (c.sliding_window < 0 || (c.flags & ~AETH_CFG_FULL_CONTEXT))
        return aeth_set_error(AETH_EINVAL, "aeth_runner_create: sliding_window %d / flags %d", c.sliding_window, c.flags);
    // LlamaRunner::new and new_streaming size the cache and the RoPE table at
    // min(max_seq_len, 4096) (runner.rs:225, :339); a longer cache is an opt-in
    const int32_t eff_seq = (c.flags & AETH_CFG_FULL_CONTEXT) ? c.max_seq_len
                                                             : std::min<int32_t>(c.max_seq_len, AETH_RUNNER_MAX_SEQ);
    if (eff_seq > 8192)
        return aeth_set_error(AETH_EUNSUPPORTED, "aeth_runner_create: a cache of %d positions (the decode attention "
                                                 "holds up to 8192)", eff_seq);
    c.max_seq_len = eff_seq;
    bool need_seed = !lm_head || !embeddings || !final_norm || !layer_weights || !norms;
    if (need_seed && seed == 0)
        return aeth_set_error(AETH_EINVAL, "aeth_runner_create: missing tensors need a nonzero synthetic_seed");
    RunnerHold hold;
    aeth_runner* r = hold.r = new aeth_runner();
    r->cfg = c;
    int rc = AETH_OK;
#define RC(expr)                        \
    do {                                \
        if ((rc = (expr)) != AETH_OK) { \
            return rc;                  \
        }                               \
    } while (0)
    if (hipStreamCreateWithFlags(&r->stream, hipStreamNonBlocking) != hipSuccess)
        return aeth_set_error(AETH_EHIP, "aeth_runner_create: stream creation failed");
    hipStream_t s = r->stream;
    (void)aeth_num_cus();  // cache the device query outside any graph capture
    const int64_t d = c.d_model, qd = (int64_t)c.num_heads * c.head_dim, kvd = kKvd(c), dff = c.d_ff;
    r->dtypes.assign(layer_dtypes, layer_dtypes + (size_t)c.num_layers * 7);
    for (int l = 0; l < c.num_layers; l++) {
        const int32_t* T = layer_dtypes + (size_t)l * 7;
        const void* const* W = layer_weights ? layer_weights + (size_t)l * 7 : nullptr;
        auto hw = [&](int j) -> const void* { return W ? W[j] : nullptr; };
        aeth_weight* w = nullptr;
        // q|k|v rows fused into one weight, gate/up rows interleaved (SwiGLU epilogue),
        // when they share a fused format; separate weights otherwise (mixed-format
        // files; GGUF-order F32 / F16 / Q2_K / Q3_K weights, whose rows are not [out] rows)
        for (auto* v : {&r->wqkv, &r->wq, &r->wk, &r->wv, &r->wgu, &r->wg, &r->wu, &r->wqk}) v->push_back(nullptr);
        if (T[0] == T[1] && T[0] == T[2] && aeth_dtype_fused(T[0])) {
            RC(make_concat(T[0], {qd, kvd, kvd}, d, {hw(0), hw(1), hw(2)}, mix(seed, l, 1), s, &r->wqkv[l]));
        } else if (T[0] == T[1] && aeth_dtype_fused(T[0])) {
            RC(make_concat(T[0], {qd, kvd}, d, {hw(0), hw(1)}, mix(seed, l, 1), s, &r->wqk[l]));
            RC(make_weight(T[2], kvd, d, hw(2), mix(seed, l, 3), s, &r->wv[l]));
        } else {
            RC(make_weight(T[0], qd, d, hw(0), mix(seed, l, 1), s, &r->wq[l]));
            RC(make_weight(T[1], kvd, d, hw(1), mix(seed, l, 2), s, &r->wk[l]));
            RC(make_weight(T[2], kvd, d, hw(2), mix(seed, l, 3), s, &r->wv[l]));
        }
        RC(make_weight(T[3], d, qd, hw(3), mix(seed, l, 4), s, &w));
        r->wo.push_back(w);
        if (T[4] == T[5] && aeth_dtype_fused(T[4])) {
            RC(make_interleaved(T[4], dff, d, hw(4), hw(5), mix(seed, l, 5), s, &r->wgu[l]));
        } else {
            RC(make_weight(T[4], dff, d, hw(4), mix(seed, l, 5), s, &r->wg[l]));
            RC(make_weight(T[5], dff, d, hw(5), mix(seed, l, 6), s, &r->wu[l]));
        }
        RC(make_weight(T[6], d, dff, hw(6), mix(seed, l, 7), s, &w));
        r->wdown.push_back(w);
    }
    RC(make_weight(lm_dtype, c.vocab_size, d, lm_head, mix(seed, 1000003, 9), s, &r->lm_head));
    {  // scratch for the GGUF-order weights' decode GEMVs (one row)
        int64_t need = aeth_xgemv_ws_floats(r->lm_head, 1);
        for (auto* v : {&r->wq, &r->wk, &r->wv, &r->wo, &r->wg, &r->wu, &r->wdown})
            for (auto* w : *v) need = std::max(need, aeth_xgemv_ws_floats(w, 1));
        if (need > 0) {
            RC(dmalloc(&r->xws, need));
            r->xws_floats = need;
        }
    }
    RC(dmalloc(&r->norms, (int64_t)c.num_layers * 2 * d));
    RC(dmalloc(&r->final_norm, d));
    RC(dmalloc(&r->emb, (int64_t)c.vocab_size * d));
    if (norms) {
        for (int l = 0; l < c.num_layers; l++)
            for (int j = 0; j < 2; j++)
                if (hipMemcpy(r->norms + ((int64_t)l * 2 + j) * d, norms[l * 2 + j], sizeof(float) * d,
                              hipMemcpyHostToDevice) != hipSuccess) {
                    return aeth_set_error(AETH_EHIP, "runner: norm upload failed");
                }
    } else {
        RC(aeth_fill_normal_f32(mix(seed, 2, 2), r->norms, (int64_t)c.num_layers * 2 * d, 1.0f, 0.02f, s));
    }
    if (final_norm) {
        if (hipMemcpy(r->final_norm, final_norm, sizeof(float) * d, hipMemcpyHostToDevice) != hipSuccess) {
            return aeth_set_error(AETH_EHIP, "runner: final norm upload failed");
        }
    } else {
        RC(aeth_fill_normal_f32(mix(seed, 3, 3), r->final_norm, d, 1.0f, 0.02f, s));
    }
    if (embeddings) {
        if (hipMemcpy(r->emb, embeddings, sizeof(float) * (size_t)c.vocab_size * d, hipMemcpyHostToDevice) !=
            hipSuccess) {
            return aeth_set_error(AETH_EHIP, "runner: embedding upload failed");
        }
    } else {
        RC(aeth_fill_normal_f32(mix(seed, 4, 4), r->emb, (int64_t)c.vocab_size * d, 0.0f, 1.0f, s));
    }
    std::vector<float> rs, rcs;
    precompute_rope(c.max_seq_len, c.head_dim, c.rope_base, rs, rcs);
    RC(dmalloc(&r->rope_sin, (int64_t)rs.size()));
    RC(dmalloc(&r->rope_cos, (int64_t)rcs.size()));
    if (hipMemcpy(r->rope_sin, rs.data(), rs.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(r->rope_cos, rcs.data(), rcs.size() * 4, hipMemcpyHostToDevice) != hipSuccess) {
        return aeth_set_error(AETH_EHIP, "runner: rope upload failed");
    }
    RC(dmalloc(&r->kv, (int64_t)c.num_layers * kv_layer_floats(c)));
    if (hipMemsetAsync(r->kv, 0, sizeof(float) * (size_t)c.num_layers * kv_layer_floats(c), s) != hipSuccess) {
        return aeth_set_error(AETH_EHIP, "runner: kv clear failed");
    }
    RC(dmalloc(&r->x, d));
    RC(dmalloc(&r->normed, d > dff ? d : dff));
    RC(dmalloc(&r->qkv, qd + 2 * kvd));
    RC(dmalloc(&r->attn, qd));
    RC(dmalloc(&r->gu, 2 * dff));  // h, or g | u when gate and up are separate
    RC(dmalloc(&r->logits, c.vocab_size));
    RC(dmalloc(&r->attn_ws, aeth_attn_ws_floats(c.num_heads, c.head_dim, c.max_seq_len)));
    if (hipMemset(r->attn_ws, 0, sizeof(float) * aeth_attn_ws_floats(c.num_heads, c.head_dim, c.max_seq_len)) !=
        hipSuccess) {
        return aeth_set_error(AETH_EHIP, "runner: workspace clear failed");
    }
    RC(dmalloc(&r->amax, 1));
    if (hipMemset(r->amax, 0, sizeof(unsigned long long)) != hipSuccess) {
        return aeth_set_error(AETH_EHIP, "runner: argmax slot clear failed");
    }
    RC(dmalloc((uint8_t**)&r->am_ws, aeth_argmax_ws_bytes()));
    RC(dmalloc(&r->st, 5));
    RC(dmalloc(&r->tok_out, c.max_seq_len));
    if (hipStreamSynchronize(s) != hipSuccess) {
        return aeth_set_error(AETH_EHIP, "runner: setup sync failed");
    }
#undef RC
    hold.r = nullptr;
    *out = r;
    return AETH_OK;
}
}  // namespace

extern "C" AETH_API int aeth_runner_create(const aeth_llama_config* cfg, const void* const* layer_weights,
                                           const int32_t* layer_dtypes, const float* const* norms,
                                           const float* final_norm, const void* lm_head, int32_t lm_dtype,
                                           const float* embeddings, uint64_t seed, aeth_runner** out) {
    return aeth_guard("aeth_runner_create", [&] {
        return runner_create_impl(cfg, layer_weights, layer_dtypes, norms, final_norm, lm_head, lm_dtype, embeddings,
                                  seed, out);
    });
}

extern "C" AETH_API int aeth_runner_free(aeth_runner* r) {
    runner_release(r);
    return AETH_OK;
}

extern "C" AETH_API void* aeth_runner_stream(const aeth_runner* r) { return r ? (void*)r->stream : nullptr; }

extern "C" AETH_API int aeth_runner_seq_len(const aeth_runner* r) { return r ? r->fill : -1; }

extern "C" AETH_API int aeth_runner_fill_kv(aeth_runner* r, uint64_t seed, int32_t seq_len) {
    if (!r || seq_len < 0 || seq_len > r->cfg.max_seq_len)
        return aeth_set_error(AETH_EINVAL, "aeth_runner_fill_kv: bad argument");
    std::lock_guard<std::mutex> lk(r->mu);
    const aeth_llama_config& c = r->cfg;
    // N(0,1) over the whole storage, then the unfilled tail cleared per head.
    int64_t tot = (int64_t)c.num_layers * kv_layer_floats(c);
    int rc = aeth_fill_normal_f32(seed, r->kv, tot, 0.0f, 1.0f, r->stream);
    if (rc) return rc;
    int64_t rows = (int64_t)c.num_layers * 2 * c.num_kv_heads;
    int64_t tail = (int64_t)(c.max_seq_len - seq_len) * c.head_dim;
    if (tail > 0)
        for (int64_t i = 0; i < rows; i++)
            AETH_HIP_CHECK(hipMemsetAsync(r->kv + i * c.max_seq_len * c.head_dim + (int64_t)seq_len * c.head_dim, 0,
                                          sizeof(float) * tail, r->stream));
    AETH_HIP_CHECK(hipStreamSynchronize(r->stream));
    r->fill = seq_len;
    r->partial_valid = false;
    return AETH_OK;
}

extern "C" AETH_API int aeth_runner_kv_to_host(aeth_runner* r, float* host, int32_t* seq_len) {
    if (!r || !host) return aeth_set_error(AETH_EINVAL, "aeth_runner_kv_to_host: NULL");
    std::lock_guard<std::mutex> lk(r->mu);
    int64_t tot = (int64_t)r->cfg.num_layers * kv_layer_floats(r->cfg);
    AETH_HIP_CHECK(hipStreamSynchronize(r->stream));
    AETH_HIP_CHECK(hipMemcpy(host, r->kv, sizeof(float) * tot, hipMemcpyDeviceToHost));
    if (seq_len) *seq_len = r->fill;
    return AETH_OK;
}

extern "C" AETH_API int aeth_runner_kv_from_host(aeth_runner* r, const float* host, int32_t seq_len) {
    if (!r || !host || seq_len < 0 || seq_len > r->cfg.max_seq_len)
        return aeth_set_error(AETH_EINVAL, "aeth_runner_kv_from_host: bad argument");
    std::lock_guard<std::mutex> lk(r->mu);
    int64_t tot = (int64_t)r->cfg.num_layers * kv_layer_floats(r->cfg);
    AETH_HIP_CHECK(hipStreamSynchronize(r->stream));
    AETH_HIP_CHECK(hipMemcpy(r->kv, host, sizeof(float) * tot, hipMemcpyHostToDevice));
    r->fill = seq_len;
    r->partial_valid = false;
    return AETH_OK;
}

static int runner_decode_locked(aeth_runner* r, int32_t token, int32_t pos, float* logits, int32_t* next_token) {
    int rc = check_step_args(r, token, pos);
    if (rc) return rc;
    r->partial_valid = false;
    if ((rc = set_state(r, token, pos))) return rc;
    if ((rc = enqueue_step(r))) return rc;
    if (logits)
        AETH_HIP_CHECK(hipMemcpyAsync(logits, r->logits, sizeof(float) * r->cfg.vocab_size, hipMemcpyDeviceToHost,
                                      r->stream));
    int tok = 0;
    AETH_HIP_CHECK(hipMemcpyAsync(&tok, r->st + 3, sizeof(int), hipMemcpyDeviceToHost, r->stream));
    AETH_HIP_CHECK(hipStreamSynchronize(r->stream));
    if (r->fill < r->cfg.max_seq_len) r->fill++;
    if (next_token) *next_token = tok;
    return AETH_OK;
}

extern "C" AETH_API int aeth_runner_decode(aeth_runner* r, int32_t token, int32_t pos, float* logits,
                                           int32_t* next_token) {
    if (!r) return aeth_set_error(AETH_EINVAL, "aeth_runner_decode: NULL runner");
    std::lock_guard<std::mutex> lk(r->mu);
    return runner_decode_locked(r, token, pos, logits, next_token);
}

extern "C" AETH_API int aeth_runner_prefill(aeth_runner* r, const int32_t* tokens, int32_t n, float* logits,
                                            int32_t* next_token) {
    if (!r) return aeth_set_error(AETH_EINVAL, "aeth_runner_prefill: NULL runner");
    std::lock_guard<std::mutex> lk(r->mu);
    return runner_prefill_locked(r, tokens, n, logits, next_token);
}

extern "C" AETH_API int aeth_runner_generate(aeth_runner* r, int32_t token, int32_t pos, int32_t n_steps,
                                             int32_t* tokens, int use_graph) {
    if (!r || n_steps < 0 || (n_steps > 0 && !tokens))
        return aeth_set_error(AETH_EINVAL, "aeth_runner_generate: bad argument");
    std::lock_guard<std::mutex> lk(r->mu);
    int rc = check_step_args(r, token, pos);
    if (rc) return rc;
    if (r->fill + n_steps > r->cfg.max_seq_len)
        return aeth_set_error(AETH_ESTATE, "generate: %d steps overflow the KV cache (%d of %d used)", n_steps, r->fill,
                              r->cfg.max_seq_len);
    r->partial_valid = false;
    if ((rc = set_state(r, token, pos))) return rc;
    if (use_graph && !r->graph) {
        hipGraph_t g = nullptr;
        AETH_HIP_CHECK(hipStreamBeginCapture(r->stream, hipStreamCaptureModeThreadLocal));
        rc = enqueue_step(r);
        hipError_t e = hipStreamEndCapture(r->stream, &g);
        if (rc) {
            if (g) hipGraphDestroy(g);
            return rc;
        }
        if (e != hipSuccess) return aeth_set_error(AETH_EHIP, "graph capture failed: %s", hipGetErrorString(e));
        e = hipGraphInstantiate(&r->graph, g, nullptr, nullptr, 0);
        hipGraphDestroy(g);
        if (e != hipSuccess) {
            r->graph = nullptr;
            return aeth_set_error(AETH_EHIP, "graph instantiate failed: %s", hipGetErrorString(e));
        }
    }
    for (int i = 0; i < n_steps; i++) {  // each step appends its token to tok_out on the device
        if (use_graph) AETH_HIP_CHECK(hipGraphLaunch(r->graph, r->stream));
        else if ((rc = enqueue_step(r))) return rc;
    }
    if (n_steps > 0)
        AETH_HIP_CHECK(hipMemcpyAsync(tokens, r->tok_out, sizeof(int32_t) * n_steps, hipMemcpyDeviceToHost, r->stream));
    AETH_HIP_CHECK(hipStreamSynchronize(r->stream));
    r->fill += n_steps;
    return AETH_OK;
}

static int runner_export_impl(const aeth_runner* r, int which, int32_t l, void* host, int64_t host_bytes) {
    if (!r || !host) return aeth_set_error(AETH_EINVAL, "aeth_runner_export: NULL");
    const aeth_llama_config& c = r->cfg;
    const int64_t d = c.d_model, qd = (int64_t)c.num_heads * c.head_dim, kvd = kKvd(c), dff = c.d_ff;
    (void)dff;
    AETH_HIP_CHECK(hipStreamSynchronize(r->stream));
    if (which >= 0 && which <= 6) {
        if (l < 0 || l >= c.num_layers) return aeth_set_error(AETH_EINVAL, "export: layer out of range");
        const aeth_weight* sep[7] = {r->wq[l], r->wk[l], r->wv[l], r->wo[l], r->wg[l], r->wu[l], r->wdown[l]};
        if (sep[which] && ((which != 3 && which != 6) || sep[which]->order != AETH_ORDER_PLANAR)) {
            // a separately stored weight (or a raw-order one): its bytes as they are
            if (host_bytes < sep[which]->bytes) return aeth_set_error(AETH_EINVAL, "export: buffer too small");
            return aeth_weight_export_raw(sep[which], host, 0, r->stream);
        }
        const aeth_weight* w = which <= 2 ? (r->wqkv[l] ? r->wqkv[l] : r->wqk[l])
                               : which == 3 ? r->wo[l] : which <= 5 ? r->wgu[l] : r->wdown[l];
        std::vector<uint8_t> all((size_t)w->bytes);
        int rc = aeth_weight_export_raw(w, all.data(), 0, r->stream);
        if (rc) return rc;
        int64_t rowb = w->bytes / w->n, r0 = 0, nr = w->n;
        if (which == 0) { r0 = 0; nr = qd; }
        else if (which == 1) { r0 = qd; nr = kvd; }
        else if (which == 2) { r0 = qd + kvd; nr = kvd; }
        else if (which == 4 || which == 5) { r0 = which - 4; nr = dff; }
        if (host_bytes < nr * rowb) return aeth_set_error(AETH_EINVAL, "export: buffer too small");
        if (which == 4 || which == 5) {  // de-interleave gate (even rows) / up (odd rows)
            for (int64_t i = 0; i < dff; i++)
                memcpy((uint8_t*)host + i * rowb, all.data() + (2 * i + r0) * rowb, (size_t)rowb);
        } else {
            memcpy(host, all.data() + r0 * rowb, (size_t)(nr * rowb));
        }
        return AETH_OK;
    }
    const void* src = nullptr;
    int64_t bytes = 0;
    switch (which) {
        case 7: src = r->norms + (int64_t)l * 2 * d; bytes = d * 4; break;
        case 8: src = r->norms + (int64_t)l * 2 * d + d; bytes = d * 4; break;
        case 9: src = r->final_norm; bytes = d * 4; break;
        case 10: {
            if (host_bytes < r->lm_head->bytes) return aeth_set_error(AETH_EINVAL, "export: buffer too small");
            return aeth_weight_export_raw(r->lm_head, host, 0, r->stream);
        }
        case 11:
            if (l < 0 || l >= c.vocab_size) return aeth_set_error(AETH_EINVAL, "export: token out of range");
            src = r->emb + (int64_t)l * d; bytes = d * 4; break;
        case 12: src = r->rope_sin; bytes = (int64_t)c.max_seq_len * (c.head_dim / 2) * 4; break;
        case 13: src = r->rope_cos; bytes = (int64_t)c.max_seq_len * (c.head_dim / 2) * 4; break;
        default: return aeth_set_error(AETH_EINVAL, "export: unknown tensor %d", which);
    }
    if (host_bytes < bytes) return aeth_set_error(AETH_EINVAL, "export: buffer too small");
    AETH_HIP_CHECK(hipMemcpy(host, src, (size_t)bytes, hipMemcpyDeviceToHost));
    return AETH_OK;
}

extern "C" AETH_API int aeth_runner_export(const aeth_runner* r, int which, int32_t l, void* host, int64_t host_bytes) {
    return aeth_guard("aeth_runner_export", [&] { return runner_export_impl(r, which, l, host, host_bytes); });
}

// ── aether.h C ABI (src/c_api.rs) over the device runner ─────────────────

struct aether_model {
    aeth_runner* runner;
    float frame_budget_ms;
    int bos_id, eos_id;
};

extern "C" AETHER_API aether_model* aether_model_from_runner(aeth_runner* r) {
    if (!r) return nullptr;
    aether_model* m = new (std::nothrow) aether_model{r, 0.0f, 1, 2};
    if (!m) aeth_set_error(AETH_ENOMEM, "aether_model_from_runner: out of host memory");
    return m;
}

// aether_load (c_api.rs:41-74): GGUF file → device runner (aeth_gguf.cpp);
// NULL with aether_last_error set on failure.
extern "C" AETHER_API aether_model* aether_load(const char* path) {
    aeth_runner* r = nullptr;
    int bos = 1, eos = 2;
    if (aeth_guard("aether_load", [&] { return aeth_gguf_load_runner(path, &r, &bos, &eos); }) != AETH_OK)
        return nullptr;
    aether_model* m = new (std::nothrow) aether_model{r, 0.0f, bos, eos};
    if (!m) {
        aeth_runner_free(r);
        aeth_set_error(AETH_ENOMEM, "aether_load: out of host memory");
    }
    return m;
}

// aether_load_streaming (c_api.rs:76-102) keeps max_hot decoder layers resident on
// the reference's CPU path; with 288 GB of HBM every layer stays on the device.
extern "C" AETHER_API aether_model* aether_load_streaming(const char* path, int max_hot) {
    (void)max_hot;
    return aether_load(path);
}

extern "C" AETHER_API void aether_free(aether_model* m) {
    if (!m) return;
    aeth_runner_free(m->runner);
    delete m;
}

extern "C" AETHER_API int aether_vocab_size(const aether_model* m) { return m ? m->runner->cfg.vocab_size : 0; }
extern "C" AETHER_API int aether_context_len(const aether_model* m) { return m ? m->runner->cfg.max_seq_len : 0; }
extern "C" AETHER_API int aether_num_layers(const aether_model* m) { return m ? m->runner->cfg.num_layers : 0; }
extern "C" AETHER_API int aether_d_model(const aether_model* m) { return m ? m->runner->cfg.d_model : 0; }
// tokenizer.ggml.{eos,bos}_token_id of a loaded file (tokenizer/mod.rs:65-66);
// the conventional LLaMA ids 2 / 1 otherwise.
extern "C" AETHER_API int aether_eos_id(const aether_model* m) { return m ? m->eos_id : -1; }
extern "C" AETHER_API int aether_bos_id(const aether_model* m) { return m ? m->bos_id : -1; }
extern "C" AETHER_API int aether_num_gpu_layers(const aether_model* m) { return m ? m->runner->cfg.num_layers : 0; }
extern "C" AETHER_API int aether_num_cpu_layers(const aether_model* m) { return m ? 0 : 0; }

extern "C" AETHER_API void aether_set_frame_budget(aether_model* m, float max_ms) {
    if (m) m->frame_budget_ms = max_ms;
}
extern "C" AETHER_API float aether_frame_budget(const aether_model* m) { return m ? m->frame_budget_ms : 0.0f; }

// Tokenization needs GGUF tokenizer metadata, which synthetic models lack.
extern "C" AETHER_API int* aether_encode(const aether_model* m, const char* text, int* out_len) {
    (void)m;
    (void)text;
    if (out_len) *out_len = 0;
    aeth_set_error(AETH_EUNSUPPORTED, "aether_encode: no tokenizer in this build");
    return nullptr;
}
extern "C" AETHER_API char* aether_decode_token(const aether_model* m, int token) {
    (void)m;
    (void)token;
    aeth_set_error(AETH_EUNSUPPORTED, "aether_decode_token: no tokenizer in this build");
    return nullptr;
}
extern "C" AETHER_API void aether_free_string(char* s) { free(s); }
extern "C" AETHER_API void aether_free_tokens(int* t) { free(t); }

// aether_prefill (c_api.rs:257-278 → LlamaRunner::prefill, runner.rs:695):
// the batched device prefill; token i at position i / cache slot i, the
// logits of the last token are returned.
extern "C" AETHER_API int aether_prefill(aether_model* m, const int* tokens, int n_tokens, float* logits_out) {
    if (!m || !tokens || n_tokens <= 0 || !logits_out) return AETHER_ERR;
    aeth_runner* r = m->runner;
    std::lock_guard<std::mutex> lk(r->mu);
    if (n_tokens > r->cfg.max_seq_len) {
        aeth_set_error(AETH_EINVAL, "prefill: %d tokens exceed max_seq %d", n_tokens, r->cfg.max_seq_len);
        return AETHER_ERR;
    }
    return runner_prefill_locked(r, (const int32_t*)tokens, n_tokens, logits_out, nullptr) == AETH_OK ? AETHER_OK
                                                                                                : AETHER_ERR;
}

extern "C" AETHER_API int aether_decode(aether_model* m, int token, int pos, float* logits_out) {
    if (!m || !logits_out) return AETHER_ERR;
    return aeth_runner_decode(m->runner, token, pos, logits_out, nullptr) == AETH_OK ? AETHER_OK : AETHER_ERR;
}

// aether_decode_budgeted (c_api.rs:324-355, runner.rs:1201-1282): the
// deadline is checked before each layer; on expiry the layers done so far
// are kept (x stays on the device) and AETHER_TIMEOUT is returned without
// logits; a retry with the same (token, pos) resumes after the last
// completed layer. The resume index follows the reference exactly,
// including its saturating_sub: a budget that expires before layer 0
// records completed_layer = 0 and the retry starts at layer 1.
extern "C" AETHER_API int aether_decode_budgeted(aether_model* m, int token, int pos, float* logits_out) {
    if (!m || !logits_out) return AETHER_ERR;
    aeth_runner* r = m->runner;
    std::lock_guard<std::mutex> lk(r->mu);
    if (m->frame_budget_ms <= 0.0f) {
        return runner_decode_locked(r, token, pos, logits_out, nullptr) == AETH_OK ? AETHER_OK : AETHER_ERR;
    }
    if (check_step_args(r, token, pos)) return AETHER_ERR;
    int start = 0;
    if (r->partial_valid && r->partial_token == token && r->partial_pos == pos) {
        start = r->partial_layer + 1;
    } else {
        r->partial_valid = false;
        if (set_state(r, token, pos)) return AETHER_ERR;
        if (aeth_embed_launch(r->emb, r->st, 0, r->cfg.d_model, r->cfg.vocab_size, r->x, r->stream)) return AETHER_ERR;
    }
    auto deadline = std::chrono::steady_clock::now() +
                    std::chrono::duration_cast<std::chrono::steady_clock::duration>(
                        std::chrono::duration<double, std::milli>(m->frame_budget_ms));
    for (int l = start; l < r->cfg.num_layers; l++) {
        if (std::chrono::steady_clock::now() >= deadline) {
            if (hipStreamSynchronize(r->stream) != hipSuccess) return AETHER_ERR;
            r->partial_valid = true;
            r->partial_token = token;
            r->partial_pos = pos;
            r->partial_layer = l > 0 ? l - 1 : 0;
            return AETHER_TIMEOUT;
        }
        if (enqueue_layers(r, l, l + 1)) return AETHER_ERR;
        if (hipStreamSynchronize(r->stream) != hipSuccess) return AETHER_ERR;
    }
    r->partial_valid = false;
    if (enqueue_head(r)) return AETHER_ERR;
    if (hipMemcpyAsync(logits_out, r->logits, sizeof(float) * r->cfg.vocab_size, hipMemcpyDeviceToHost, r->stream) !=
            hipSuccess ||
        hipStreamSynchronize(r->stream) != hipSuccess)
        return AETHER_ERR;
    if (r->fill < r->cfg.max_seq_len) r->fill++;
    return AETHER_OK;
}

// Greedy only (temperature ≤ 1e-6, runner.rs:1946-1973); stochastic
// sampling is not on the measured path.
extern "C" AETHER_API int aether_sample(const aether_model* m, const float* logits, float temperature, float top_p) {
    if (!m || !logits) return -1;
    if (temperature > 1e-6f && top_p > 1e-6f) {
        aeth_set_error(AETH_EUNSUPPORTED, "aether_sample: only greedy sampling is built");
        return -1;
    }
    return aether_argmax(m, logits);
}

extern "C" AETHER_API int aether_argmax(const aether_model* m, const float* logits) {
    if (!m || !logits) return -1;
    int n = m->runner->cfg.vocab_size, best = 0;
    for (int i = 1; i < n; i++)
        if (!(logits[i] < logits[best])) best = i;
    return best;
}

extern "C" AETHER_API char* aether_last_error(void) {
    const char* e = aeth_last_error();
    size_t len = strlen(e);
    char* s = (char*)malloc(len + 1);
    if (s) memcpy(s, e, len + 1);
    return s;
}
