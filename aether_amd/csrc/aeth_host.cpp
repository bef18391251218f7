// Host side of the quantized-matmul path: the device-pointer entry points,
// the QuantKernel plugin registry (src/quant/matmul/registry.rs:7-63) with its
// HIP kernels, and quantized_matmul_impl / matmul_q* over host slices
// (src/quant/matmul/dispatch.rs:98-135, avx2_dispatch.rs:58-68).
#include <hip/hip_runtime.h>

#include <string.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <tuple>
#include <vector>

#include "aeth_common.hpp"
#include "aeth_internal.hpp"
#include "aeth_ops_internal.hpp"

// ── library scratch: one grow-only buffer per (device, stream, use) ───────
// Work enqueued on one stream runs in order, so calls on the same stream can
// share a buffer; calls on different streams (runners, host threads) get
// their own. A grow first waits for the stream (the old buffer may still be
// read by its kernels) and is refused while the stream is being captured.
namespace {
struct Scratch {
    void* ptr = nullptr;
    size_t bytes = 0;
};
std::mutex g_scratch_mu;
std::map<std::tuple<int, hipStream_t, int>, Scratch> g_scratch;
}  // namespace

int aeth_stream_scratch(hipStream_t s, int use, size_t bytes, void** out) {
    int dev = 0;
    AETH_HIP_CHECK(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    Scratch& w = g_scratch[std::make_tuple(dev, s, use)];
    if (w.bytes < bytes) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        AETH_HIP_CHECK(hipStreamIsCapturing(s, &cs));
        if (cs != hipStreamCaptureStatusNone)
            return aeth_set_error(AETH_ESTATE, "scratch of %zu bytes would have to be allocated during graph capture "
                                               "(run the call once before capturing)", bytes);
        if (w.ptr) {
            AETH_HIP_CHECK(hipStreamSynchronize(s));
            AETH_HIP_CHECK(hipFree(w.ptr));
        }
        w.ptr = nullptr;
        w.bytes = 0;
        AETH_HIP_CHECK(hipMalloc(&w.ptr, bytes));
        w.bytes = bytes;
    }
    *out = w.ptr;
    return AETH_OK;
}

void aeth_stream_scratch_release(hipStream_t s) {
    aeth_blas_release_stream(s);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    for (auto it = g_scratch.begin(); it != g_scratch.end();) {
        if (std::get<1>(it->first) == s) {
            if (it->second.ptr) hipFree(it->second.ptr);
            it = g_scratch.erase(it);
        } else {
            ++it;
        }
    }
}

namespace {
// Rows from which a block format's product is dequantized once and run as one DGEMM
// (aeth_blas.cpp, its K range split over batches until the tiles fill the chip) instead
// of the row-batched GEMV: the DGEMM costs about the same for any m up to a few hundred
// (4096 × 4096: 0.15 ms, 4096 × 14336: 0.73 ms), the GEMV grows with m (≈ 2 µs per row
// at 4096 × 4096). Measured crossovers (HIP events, rotated weight copies): Q6_K 4096 ×
// 4096 ≈ 64 rows, 4096 × 14336 ≈ 80, 1024 × 4096 ≈ 136; Q8_0 ≈ 112; Q5_K ≈ 80; Q2_K ≈ 40
// and Q3_K ≈ 32 (GGUF order). Q6_K rows of whole super-blocks and Q8_0 rows of whole blocks take
// the Q6_K / Q8_0 GEMMs (aeth_gemm_q6k.hip, aeth_gemm_q80.hip) instead, from the row counts
// aeth_q6k_gemm_rows / aeth_q80_gemm_rows give.
int64_t dequant_gemm_rows(int dtype) {
    switch (dtype) {
        case AETH_DTYPE_Q8_0: return 112;
        case AETH_DTYPE_Q2_K: return 40;
        case AETH_DTYPE_Q3_K: return 32;
        default: return 80;  // Q5_K, Q6_K
    }
}
}  // namespace

int aeth_qmatmul_ld(const aeth_weight* w, const float* d_a, int64_t m, float* d_c, int64_t ldc, unsigned flags,
                    hipStream_t s) {
    const bool kquant = w->dtype == AETH_DTYPE_Q4_K || w->dtype == AETH_DTYPE_Q5_K || w->dtype == AETH_DTYPE_Q6_K;
    // the dot-product mode's batched K-quant kernels index activation rows (k/256)·8 blocks
    // apart; for k % 256 != 0 only the dequantized product reproduces that (aeth_blas.cpp)
    if (m > 1 && (flags & AETH_MM_Q8_ACTIVATIONS) && kquant && (w->k % 256) != 0)
        return aeth_dequant_gemm_launch(w, d_a, m, d_c, ldc, flags, s);
    if (m > 1 && w->dtype == AETH_DTYPE_Q4_K && w->order == AETH_ORDER_PLANAR && aeth_q4k_gemm_rows(w, m))
        return aeth_gemm_q4k_launch(w, d_a, m, d_c, flags, s, ldc);
    if (m > 1 && aeth_q5k_gemm_rows(w, m)) return aeth_gemm_q4k_launch(w, d_a, m, d_c, flags, s, ldc);  // Q5_K
    if (m > 1 && aeth_q6k_gemm_rows(w, m)) return aeth_gemm_q6k_launch(w, d_a, m, d_c, flags, s, ldc);  // Q6_K
    if (m > 1 && aeth_q80_gemm_rows(w, m)) return aeth_gemm_q80_launch(w, d_a, m, d_c, flags, s, ldc);  // Q8_0
    // the other block formats from a few hundred rows on: dequantized once, one DGEMM (instead
    // of the weight streamed once per row by the batched GEMV). Their dequantized
    // weights are finite (K-quant scales go through decode_d), so the SGEMM's
    // 0·w terms equal matmul_f32_gguf's skipped rows; F32 / F16 weights, which may
    // hold infinities, keep the kernels that skip zero activations as the reference does.
    // (a Q8_0 weight with a NaN or infinite block scale stays on the GEMV: dequantized, its
    // q = 0 entries become 0·Inf = NaN, where q8_0.rs multiplies the block's sum by d)
    if (m >= dequant_gemm_rows(w->dtype) && w->dtype != AETH_DTYPE_F32 && w->dtype != AETH_DTYPE_F16 &&
        !(w->dtype == AETH_DTYPE_Q8_0 && w->special_scales))
        return aeth_dequant_gemm_launch(w, d_a, m, d_c, ldc, flags, s);
    GemvEpi e;
    e.flags = flags;
    e.ldc = ldc;
    return aeth_gemv_launch_ex(w, d_a, m, d_c, e, s);
}

extern "C" AETH_API int aeth_qmatmul(const aeth_weight* w, const float* d_a, int64_t m, float* d_c, unsigned flags,
                                     void* stream) {
    if (!w || !d_a || !d_c || m <= 0) return aeth_set_error(AETH_EINVAL, "aeth_qmatmul: bad argument");
    return aeth_qmatmul_ld(w, d_a, m, d_c, 0, flags, (hipStream_t)stream);
}

extern "C" AETH_API int aeth_rmsnorm(const float* d_x, const float* d_w, int64_t rows, int64_t n, float eps,
                                     float* d_out, void* stream) {
    if (!d_x || !d_w || !d_out || rows < 0 || n < 0) return aeth_set_error(AETH_EINVAL, "aeth_rmsnorm: bad argument");
    return aeth_rmsnorm_launch(d_x, d_w, rows, n, eps, d_out, (hipStream_t)stream);
}

extern "C" AETH_API int aeth_rope(float* d_x, int64_t n_heads, int64_t head_dim, int64_t pos, const float* d_sin,
                                  const float* d_cos, int64_t max_seq, void* stream) {
    if (!d_x || !d_sin || !d_cos || max_seq <= 0 || head_dim % 2 || pos < 0)
        return aeth_set_error(AETH_EINVAL, "aeth_rope: bad argument");
    return aeth_rope_launch(d_x, n_heads, head_dim, nullptr, pos, d_sin, d_cos, max_seq, (hipStream_t)stream);
}

extern "C" AETH_API int aeth_kv_append(float* d_layer_kv, const float* d_k, const float* d_v, int64_t kv_heads,
                                       int64_t head_dim, int64_t max_seq, int64_t slot, void* stream) {
    if (!d_layer_kv || !d_k || !d_v || slot < 0) return aeth_set_error(AETH_EINVAL, "aeth_kv_append: bad argument");
    if (slot >= max_seq) return aeth_set_error(AETH_EINVAL, "aeth_kv_append: cache full (slot %lld)", (long long)slot);
    return aeth_kv_append_launch(d_layer_kv, d_k, d_v, kv_heads, head_dim, max_seq, nullptr, slot,
                                 (hipStream_t)stream);
}

extern "C" AETH_API int aeth_attn_decode(const float* d_q, const float* d_layer_kv, int64_t n_heads, int64_t kv_heads,
                                         int64_t head_dim, int64_t max_seq, int64_t seq, float* d_out, void* stream) {
    if (!d_q || !d_layer_kv || !d_out || seq <= 0 || seq > max_seq)
        return aeth_set_error(AETH_EINVAL, "aeth_attn_decode: bad argument (seq %lld, max_seq %lld)", (long long)seq,
                              (long long)max_seq);
    void* ws = nullptr;
    int rc = aeth_stream_scratch((hipStream_t)stream, AETH_SCRATCH_ATTN,
                                 sizeof(float) * aeth_attn_ws_floats(n_heads, head_dim, max_seq), &ws);
    if (rc) return rc;
    return aeth_attn_launch(d_q, nullptr, (float*)d_layer_kv, nullptr, nullptr, nullptr, seq, n_heads, kv_heads,
                            head_dim, max_seq, 0, (float*)ws, d_out, (hipStream_t)stream);
}

// ── decode attention without allocation ───────────────────────────────────
// For callers that cannot allocate (code under HIP graph capture, tight serving
// loops): the chunk partials live in a file-scope device array, `scratch`, of
// kNoAllocFloats floats (4 MiB) that every GPU the library runs on holds until
// the process ends. Host code never passes the array's name (a host-side
// stand-in): it uses the per-device address hipGetSymbolAddress returns.
// Nothing in it has to start at zero (each chunk's partial is written before the
// merge reads it). Calls that overlap on one GPU share the array and race.
namespace {
constexpr int64_t kNoAllocFloats = (int64_t)1 << 20;
constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mu;
float* g_noalloc_ptr[kMaxDevices] = {};
}  // namespace

static __device__ __align__(256) float scratch[kNoAllocFloats];

// Resolves this device's copy of `scratch` (the device must be current).
int aeth_noalloc_setup(int dev) {
    if (dev < 0 || dev >= kMaxDevices) return aeth_set_error(AETH_EINVAL, "no-alloc scratch: device %d", dev);
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    if (g_noalloc_ptr[dev]) return AETH_OK;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
        return aeth_set_error(AETH_EHIP, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                              hipGetErrorString(e));
    g_noalloc_ptr[dev] = (float*)p;
    return AETH_OK;
}

extern "C" AETH_API int aeth_attn_decode_noalloc(const float* d_q, const float* d_layer_kv, int64_t n_heads,
                                                 int64_t kv_heads, int64_t head_dim, int64_t max_seq, int64_t seq,
                                                 float* d_out, void* stream) {
    if (!d_q || !d_layer_kv || !d_out || seq <= 0 || seq > max_seq || n_heads <= 0 || head_dim <= 0 ||
        n_heads > 65536 || head_dim > 65536 || max_seq > INT32_MAX)
        return aeth_set_error(AETH_EINVAL, "aeth_attn_decode_noalloc: bad argument (seq %lld, max_seq %lld)",
                              (long long)seq, (long long)max_seq);
    const int64_t need = aeth_attn_ws_floats(n_heads, head_dim, max_seq);
    if (need > kNoAllocFloats)
        return aeth_set_error(AETH_EINVAL,
                              "aeth_attn_decode_noalloc: %lld scratch floats needed (n_heads x ceil(max_seq/128) x "
                              "(head_dim+2)), more than the %lld the library holds",
                              (long long)need, (long long)kNoAllocFloats);
    int dev = 0;
    AETH_HIP_CHECK(hipGetDevice(&dev));
    int rc = aeth_noalloc_setup(dev);
    if (rc) return rc;
    return aeth_attn_launch(d_q, nullptr, (float*)d_layer_kv, nullptr, nullptr, nullptr, seq, n_heads, kv_heads,
                            head_dim, max_seq, 0, g_noalloc_ptr[dev], d_out, (hipStream_t)stream);
}

extern "C" AETH_API int aeth_attn_prefill(const float* d_q, int64_t q_stride, const float* d_layer_kv, int64_t n,
                                          int64_t n_heads, int64_t kv_heads, int64_t head_dim, int64_t max_seq,
                                          float* d_out, void* stream) {
    if (!d_q || !d_layer_kv || !d_out || n <= 0 || n > max_seq || kv_heads <= 0 || n_heads <= 0 ||
        n_heads % kv_heads != 0 || q_stride < n_heads * head_dim || (q_stride & 3))
        return aeth_set_error(AETH_EINVAL, "aeth_attn_prefill: bad argument (n %lld, max_seq %lld)", (long long)n,
                              (long long)max_seq);
    return aeth_attn_prefill_launch(d_q, q_stride, d_layer_kv, n, n_heads, kv_heads, head_dim, max_seq, 0, d_out,
                                    (hipStream_t)stream);
}

extern "C" AETH_API int aeth_silu_mul(float* d_gate, const float* d_up, int64_t n, void* stream) {
    if (!d_gate || !d_up || n < 0) return aeth_set_error(AETH_EINVAL, "aeth_silu_mul: bad argument");
    return aeth_silu_mul_launch(d_gate, d_up, n, (hipStream_t)stream);
}

extern "C" AETH_API int aeth_add(float* d_x, const float* d_y, int64_t n, void* stream) {
    if (!d_x || !d_y || n < 0) return aeth_set_error(AETH_EINVAL, "aeth_add: bad argument");
    return aeth_add_launch(d_x, d_y, n, (hipStream_t)stream);
}

extern "C" AETH_API int aeth_argmax(const float* d_logits, int64_t n, int32_t* d_out, void* stream) {
    if (!d_logits || !d_out) return aeth_set_error(AETH_EINVAL, "aeth_argmax: bad argument");
    void* ws = nullptr;
    int rc = aeth_stream_scratch((hipStream_t)stream, AETH_SCRATCH_ARGMAX, (size_t)aeth_argmax_ws_bytes(), &ws);
    if (rc) return rc;
    return aeth_argmax_launch(d_logits, n, d_out, nullptr, ws, (hipStream_t)stream);
}

// ── host-slice path: QuantWeight bytes → cached device weight ────────────
// A host-slice call (QuantKernel::matmul semantics: borrowed slices, c fully
// written) uploads the weight once and keeps the device copy in a cache keyed
// by (pointer, length, dtype, n, k, device, layout). Every call re-checks the
// bytes against a 64-bit content fingerprint, so a buffer rewritten in place,
// or freed and reallocated at the same address, is uploaded again. The cache
// holds at most aeth_weight_cache_set_limit() device bytes (least recently
// used weights are dropped first). Calls on one device are serialised; they
// run on a library stream with reused staging buffers for a and c.
namespace {
using WKey = std::tuple<const void*, int64_t, int, int64_t, int64_t, int, int>;  // ptr, len, dtype, n, k, device, order

// Content fingerprint: four multiply-rotate lanes over 32-byte steps (a
// 64-bit mix in the style of the xxHash family), the tail byte-wise, then the
// length. Buffers past 8 MiB are split into 1 MiB chunks hashed by a
// persistent pool of host threads (the caller and up to 7 workers, started
// once) and the chunk digests folded in order.
inline uint64_t rotl64(uint64_t x, int r) { return (x << r) | (x >> (64 - r)); }
const uint64_t kP1 = 0x9E3779B185EBCA87ull, kP2 = 0xC2B2AE3D27D4EB4Full, kP3 = 0x165667B19E3779F9ull;

uint64_t fp_chunk(const uint8_t* p, size_t n, uint64_t seed) {
    uint64_t v[4] = {seed + kP1 + kP2, seed + kP2, seed, seed - kP1};
    size_t i = 0;
    for (; i + 32 <= n; i += 32)
        for (int l = 0; l < 4; l++) {
            uint64_t w;
            memcpy(&w, p + i + 8 * l, 8);
            v[l] = rotl64(v[l] + w * kP2, 31) * kP1;
        }
    uint64_t h = rotl64(v[0], 1) + rotl64(v[1], 7) + rotl64(v[2], 12) + rotl64(v[3], 18);
    for (; i < n; i++) h = rotl64(h ^ (p[i] * kP3), 11) * kP1;
    h ^= (uint64_t)n;
    h ^= h >> 33;
    h *= kP2;
    h ^= h >> 29;
    h *= kP3;
    return h ^ (h >> 32);
}

// Workers that hash the chunks of one buffer at a time: a job is published
// under the pool lock with a generation number, chunks are claimed through an
// atomic counter (the caller claims too), and the caller waits until every
// worker has left the job. The pool lives for the process (never destroyed,
// so no thread is joined during static destruction); one job at a time.
class HashPool {
  public:
    static HashPool& get() {
        static HashPool* pool = new HashPool();
        return *pool;
    }
    void run(const uint8_t* p, size_t n, size_t chunk, uint64_t* d) {
        std::lock_guard<std::mutex> job(job_mu_);
        const size_t nc = (n + chunk - 1) / chunk;
        {
            std::lock_guard<std::mutex> lk(mu_);
            p_ = p;
            n_ = n;
            chunk_ = chunk;
            d_ = d;
            nc_ = nc;
            next_.store(0);
            busy_ = (int)workers_.size();
            gen_++;
        }
        cv_.notify_all();
        work();
        std::unique_lock<std::mutex> lk(mu_);
        done_cv_.wait(lk, [&] { return busy_ == 0; });
    }

  private:
    HashPool() {
        const unsigned hc = std::thread::hardware_concurrency();
        const unsigned nw = std::min(7u, hc > 1 ? hc - 1 : 0u);
        for (unsigned i = 0; i < nw; i++) workers_.emplace_back([this] { loop(); });
    }
    void work() {
        for (size_t c; (c = next_.fetch_add(1)) < nc_;)
            d_[c] = fp_chunk(p_ + c * chunk_, std::min(chunk_, n_ - c * chunk_), c);
    }
    void loop() {
        uint64_t seen = 0;
        for (;;) {
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_.wait(lk, [&] { return gen_ != seen; });
                seen = gen_;
            }
            work();
            std::lock_guard<std::mutex> lk(mu_);
            if (--busy_ == 0) done_cv_.notify_one();
        }
    }
    std::mutex job_mu_, mu_;
    std::condition_variable cv_, done_cv_;
    std::vector<std::thread> workers_;
    const uint8_t* p_ = nullptr;
    size_t n_ = 0, chunk_ = 1, nc_ = 0;
    uint64_t* d_ = nullptr;
    std::atomic<size_t> next_{0};
    int busy_ = 0;
    uint64_t gen_ = 0;
};

uint64_t fingerprint(const uint8_t* p, size_t n) {
    const size_t chunk = 1 << 20;
    if (n <= ((size_t)8 << 20)) return fp_chunk(p, n, 0);
    const size_t nc = (n + chunk - 1) / chunk;
    std::vector<uint64_t> d(nc);
    HashPool::get().run(p, n, chunk, d.data());
    return fp_chunk((const uint8_t*)d.data(), nc * 8, (uint64_t)n);
}

struct CacheEntry {
    std::shared_ptr<aeth_weight> w;
    uint64_t fp = 0;
    uint64_t tick = 0;
};
std::mutex g_wc_mu;
std::map<WKey, CacheEntry> g_wcache;
int64_t g_wc_bytes = 0;                  // device bytes held by the cache
int64_t g_wc_limit = (int64_t)32 << 30;  // eviction bound
uint64_t g_wc_tick = 0;

std::shared_ptr<aeth_weight> share(aeth_weight* w) {
    return std::shared_ptr<aeth_weight>(w, [](aeth_weight* p) { aeth_weight_free(p); });
}

// Drops least recently used entries until `incoming` more bytes fit (a weight in
// use by another call stays alive until that call releases it).
void evict_for(int64_t incoming) {
    while (!g_wcache.empty() && g_wc_bytes + incoming > g_wc_limit) {
        auto lru = g_wcache.begin();
        for (auto it = g_wcache.begin(); it != g_wcache.end(); ++it)
            if (it->second.tick < lru->second.tick) lru = it;
        g_wc_bytes -= lru->second.w->bytes;
        g_wcache.erase(lru);
    }
}

int cached_weight(const uint8_t* b_raw, int64_t b_len, int dtype, int order, int64_t n, int64_t k,
                  std::shared_ptr<aeth_weight>* out) {
    int be, bb;
    int rc = aeth_block_geometry(dtype, &be, &bb);
    if (rc) return rc;
    int64_t need = aeth_weight_raw_bytes(dtype, order, n, k);
    if (need < 0)
        return aeth_set_error(AETH_EINVAL, "matmul: bad weight shape [%lld, %lld]", (long long)n, (long long)k);
    if (b_len < need)
        return aeth_set_error(AETH_EINVAL, "weight bytes %lld < %lld needed for [%lld, %lld] dtype %d",
                              (long long)b_len, (long long)need, (long long)n, (long long)k, dtype);
    int dev = 0;
    AETH_HIP_CHECK(hipGetDevice(&dev));
    const WKey key{b_raw, b_len, dtype, n, k, dev, order};
    const uint64_t fp = fingerprint(b_raw, (size_t)need);
    {
        std::lock_guard<std::mutex> lk(g_wc_mu);
        auto it = g_wcache.find(key);
        if (it != g_wcache.end()) {
            if (it->second.fp == fp) {
                it->second.tick = ++g_wc_tick;
                *out = it->second.w;
                return AETH_OK;
            }
            g_wc_bytes -= it->second.w->bytes;  // the bytes changed: upload again
            g_wcache.erase(it);
        }
    }
    aeth_weight* w = nullptr;
    rc = aeth_weight_create_ex(dtype, order, n, k, b_raw, 0, nullptr, &w);
    if (rc) return rc;
    std::shared_ptr<aeth_weight> sw = share(w);
    std::lock_guard<std::mutex> lk(g_wc_mu);
    auto it = g_wcache.find(key);
    if (it != g_wcache.end()) {  // another thread uploaded the same bytes meanwhile
        g_wc_bytes -= it->second.w->bytes;
        g_wcache.erase(it);
    }
    evict_for(sw->bytes);
    if (sw->bytes <= g_wc_limit) {
        g_wcache[key] = CacheEntry{sw, fp, ++g_wc_tick};
        g_wc_bytes += sw->bytes;
    }
    *out = sw;
    return AETH_OK;
}

// Per-device state of the host-slice calls: a lock, a non-blocking stream and
// grow-only staging for a and c.
struct HostDev {
    std::mutex mu;
    hipStream_t s = nullptr;
    float *da = nullptr, *dc = nullptr;
    int64_t a_cap = 0, c_cap = 0;
};
std::mutex g_hd_mu;
std::map<int, std::unique_ptr<HostDev>> g_hostdev;

HostDev& host_dev(int dev) {
    std::lock_guard<std::mutex> lk(g_hd_mu);
    auto& p = g_hostdev[dev];
    if (!p) p.reset(new HostDev());
    return *p;
}

int grow(float** p, int64_t* cap, int64_t floats) {
    if (floats <= *cap) return AETH_OK;
    if (*p) AETH_HIP_CHECK(hipFree(*p));
    *p = nullptr;
    *cap = 0;
    AETH_HIP_CHECK(hipMalloc((void**)p, sizeof(float) * (size_t)floats));
    *cap = floats;
    return AETH_OK;
}

// One host-slice matmul: H2D a, launch, D2H c. order: how b_raw is laid out —
// the QuantWeight form (planar for the fused formats, GGUF [k][n] for the
// others) or [n][k] rows.
int host_matmul_impl(const float* a, int64_t m, const uint8_t* b_raw, int64_t b_len, int64_t n, int64_t k, int dtype,
                     float* c, int order, unsigned flags) {
    if (order < 0) order = aeth_dtype_fused(dtype) ? AETH_ORDER_PLANAR : AETH_ORDER_GGUF;
    int64_t mk = 0, mn = 0;
    if (!a || !b_raw || !c || m <= 0 || n <= 0 || k <= 0 || !aeth_mul_ok(m, k, &mk) || !aeth_mul_ok(m, n, &mn))
        return aeth_set_error(AETH_EINVAL, "matmul: bad argument (m=%lld n=%lld k=%lld)", (long long)m, (long long)n,
                              (long long)k);
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0)
        return aeth_set_error(AETH_EHIP, "matmul: no HIP device available (no CPU fallback in this library)");
    std::shared_ptr<aeth_weight> w;
    int rc = cached_weight(b_raw, b_len, dtype, order, n, k, &w);
    if (rc) return rc;
    int dev = 0;
    AETH_HIP_CHECK(hipGetDevice(&dev));
    HostDev& h = host_dev(dev);
    std::lock_guard<std::mutex> lk(h.mu);
    if (!h.s) AETH_HIP_CHECK(hipStreamCreateWithFlags(&h.s, hipStreamNonBlocking));
    if ((rc = grow(&h.da, &h.a_cap, mk)) || (rc = grow(&h.dc, &h.c_cap, mn))) return rc;
    AETH_HIP_CHECK(hipMemcpyAsync(h.da, a, sizeof(float) * (size_t)mk, hipMemcpyHostToDevice, h.s));
    if ((rc = aeth_qmatmul(w.get(), h.da, m, h.dc, flags, h.s))) {
        hipStreamSynchronize(h.s);
        return rc;
    }
    AETH_HIP_CHECK(hipMemcpyAsync(c, h.dc, sizeof(float) * (size_t)mn, hipMemcpyDeviceToHost, h.s));
    AETH_HIP_CHECK(hipStreamSynchronize(h.s));
    return AETH_OK;
}

int host_matmul(const float* a, int64_t m, const uint8_t* b_raw, int64_t b_len, int64_t n, int64_t k, int dtype,
                float* c, int order = -1, unsigned flags = 0) {
    return aeth_guard("matmul", [&] { return host_matmul_impl(a, m, b_raw, b_len, n, k, dtype, c, order, flags); });
}
}  // namespace

extern "C" AETH_API int aeth_weight_fingerprint(const void* host, int64_t bytes, uint64_t* out) {
    if (!host || bytes < 0 || !out) return aeth_set_error(AETH_EINVAL, "aeth_weight_fingerprint: bad argument");
    *out = fingerprint((const uint8_t*)host, (size_t)bytes);
    return AETH_OK;
}

extern "C" AETH_API int aeth_weight_cache_clear(void) {
    std::lock_guard<std::mutex> lk(g_wc_mu);
    g_wcache.clear();  // weights still in use by a running call are freed when it ends
    g_wc_bytes = 0;
    return AETH_OK;
}

extern "C" AETH_API int aeth_weight_cache_set_limit(int64_t max_bytes) {
    if (max_bytes < 0) return aeth_set_error(AETH_EINVAL, "aeth_weight_cache_set_limit: negative limit");
    std::lock_guard<std::mutex> lk(g_wc_mu);
    g_wc_limit = max_bytes;
    evict_for(0);
    return AETH_OK;
}

extern "C" AETH_API int64_t aeth_weight_cache_bytes(void) {
    std::lock_guard<std::mutex> lk(g_wc_mu);
    return g_wc_bytes;
}

// ── QuantKernel registry (registry.rs:7-63) ──────────────────────────────
namespace aeth {

// trait QuantKernel: Send + Sync { fn matmul(&self, a, m, b_raw, n, k, c);
// fn dtype(&self) -> GGUFDtype; fn name(&self) -> &'static str; }
class QuantKernel {
  public:
    virtual ~QuantKernel() = default;
    virtual int matmul(const float* a, int64_t m, const uint8_t* b_raw, int64_t b_len, int64_t n, int64_t k,
                       float* c) const = 0;
    virtual int dtype() const = 0;
    virtual const char* name() const = 0;
};

class HipQuantKernel final : public QuantKernel {
  public:
    explicit HipQuantKernel(int dtype) : dtype_(dtype) {}
    int matmul(const float* a, int64_t m, const uint8_t* b_raw, int64_t b_len, int64_t n, int64_t k,
               float* c) const override {
        return host_matmul(a, m, b_raw, b_len, n, k, dtype_, c);
    }
    int dtype() const override { return dtype_; }
    const char* name() const override {
        switch (dtype_) {
            case AETH_DTYPE_F32: return "F32 (hip gfx950)";
            case AETH_DTYPE_F16: return "F16 (hip gfx950)";
            case AETH_DTYPE_Q2_K: return "Q2_K (hip gfx950)";
            case AETH_DTYPE_Q3_K: return "Q3_K (hip gfx950)";
            case AETH_DTYPE_Q8_0: return "Q8_0 (hip gfx950)";
            case AETH_DTYPE_Q4_K: return "Q4_K (hip gfx950)";
            case AETH_DTYPE_Q5_K: return "Q5_K (hip gfx950)";
            default: return "Q6_K (hip gfx950)";
        }
    }

  private:
    int dtype_;
};

std::mutex g_reg_mu;  // RwLock in the reference; lookups are short
std::map<int, std::unique_ptr<QuantKernel>> g_registry;

// register_kernel: a duplicate dtype is an error (the reference panics).
int register_kernel(std::unique_ptr<QuantKernel> k) {
    std::lock_guard<std::mutex> lk(g_reg_mu);
    int dt = k->dtype();
    if (g_registry.count(dt))
        return aeth_set_error(AETH_ESTATE, "QuantKernel for dtype %d already registered", dt);
    g_registry[dt] = std::move(k);
    return AETH_OK;
}

// dispatch_matmul: 1 if a registered kernel ran, 0 if none for dtype.
int dispatch_matmul(const float* a, int64_t m, const uint8_t* b_raw, int64_t b_len, int64_t n, int64_t k, int dtype,
                    float* c) {
    const QuantKernel* kern = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_reg_mu);
        auto it = g_registry.find(dtype);
        if (it != g_registry.end()) kern = it->second.get();
    }
    if (!kern) return 0;
    int rc = kern->matmul(a, m, b_raw, b_len, n, k, c);
    return rc ? rc : 1;
}

}  // namespace aeth

extern "C" AETH_API int aeth_register_hip_kernels(void) {
    return aeth_guard("aeth_register_hip_kernels", [] {
        for (int dt : {AETH_DTYPE_F32, AETH_DTYPE_F16, AETH_DTYPE_Q8_0, AETH_DTYPE_Q2_K, AETH_DTYPE_Q3_K,
                       AETH_DTYPE_Q4_K, AETH_DTYPE_Q5_K, AETH_DTYPE_Q6_K}) {
            int rc = aeth::register_kernel(std::unique_ptr<aeth::QuantKernel>(new aeth::HipQuantKernel(dt)));
            if (rc) return rc;
        }
        return (int)AETH_OK;
    });
}

extern "C" AETH_API int aeth_registered_kernel_name(int dtype, char* buf, int buf_len) {
    std::lock_guard<std::mutex> lk(aeth::g_reg_mu);
    auto it = aeth::g_registry.find(dtype);
    if (it == aeth::g_registry.end()) return 0;
    if (buf && buf_len > 0) snprintf(buf, (size_t)buf_len, "%s", it->second->name());
    return 1;
}

extern "C" AETH_API int aeth_dispatch_matmul(const float* a, int64_t m, const uint8_t* b_raw, int64_t b_len, int64_t n,
                                             int64_t k, int dtype, float* c) {
    return aeth_guard("aeth_dispatch_matmul", [&] { return aeth::dispatch_matmul(a, m, b_raw, b_len, n, k, dtype, c); });
}

// quantized_matmul_impl (dispatch.rs:98-135): registered kernel first; with
// none registered the supported dtypes still run on the HIP kernels directly
// (this library has no CPU path). F32 / F16 / Q2_K / Q3_K bytes are GGUF
// [k][n], as load_quant leaves them and the reference's dequantize fallback
// reads them (dispatch.rs:126-133).
extern "C" AETH_API int aeth_quantized_matmul_impl(const float* a, int64_t m, const uint8_t* b_raw, int64_t b_len,
                                                   int64_t n, int64_t k, int dtype, float* c) {
    int rc = aeth_guard("quantized_matmul_impl", [&] { return aeth::dispatch_matmul(a, m, b_raw, b_len, n, k, dtype, c); });
    if (rc == 1) return AETH_OK;
    if (rc < 0) return rc;
    int be, bb;
    if (aeth_block_geometry(dtype, &be, &bb) != AETH_OK)
        return aeth_set_error(AETH_EUNSUPPORTED, "quantized_matmul_impl: dtype %d not on the HIP path", dtype);
    return host_matmul(a, m, b_raw, b_len, n, k, dtype, c);
}

// quantized_matmul_impl with b_f32_cache (dispatch.rs:113-117): the cached f32
// weight, GGUF [k][n], multiplied by the F32 GGUF-order kernel of matmul_f32_gguf.
extern "C" AETH_API int aeth_quantized_matmul_impl_cached(const float* a, int64_t m, const uint8_t* b_raw,
                                                          int64_t b_len, int64_t n, int64_t k, int dtype, float* c,
                                                          const float* b_f32_cache) {
    if (!b_f32_cache) return aeth_quantized_matmul_impl(a, m, b_raw, b_len, n, k, dtype, c);
    int64_t kn = 0;
    if (!aeth_mul_ok(k, n, &kn) || kn > INT64_MAX / 4)
        return aeth_set_error(AETH_EINVAL, "quantized_matmul_impl: bad shape [%lld, %lld]", (long long)n, (long long)k);
    return host_matmul(a, m, (const uint8_t*)b_f32_cache, kn * 4, n, k, AETH_DTYPE_F32, c, AETH_ORDER_GGUF);
}

// quantized_matmul_impl on an aarch64 host with dotprod: Q8_0 / Q4_K / Q5_K /
// Q6_K through the int8 dot-product kernels, the other formats as on x86.
extern "C" AETH_API int aeth_quantized_matmul_dotprod(const float* a, int64_t m, const uint8_t* b_raw, int64_t b_len,
                                                      int64_t n, int64_t k, int dtype, float* c) {
    int be, bb;
    if (aeth_block_geometry(dtype, &be, &bb) != AETH_OK)
        return aeth_set_error(AETH_EUNSUPPORTED, "quantized_matmul_dotprod: dtype %d not on the HIP path", dtype);
    return host_matmul(a, m, b_raw, b_len, n, k, dtype, c, -1, AETH_MM_Q8_ACTIVATIONS);
}

extern "C" AETH_API int aeth_matmul_q8_0(const float* a, const uint8_t* b, int64_t b_len, int64_t m, int64_t n,
                                         int64_t k, float* c) {
    return host_matmul(a, m, b, b_len, n, k, AETH_DTYPE_Q8_0, c);
}
extern "C" AETH_API int aeth_matmul_q4_k(const float* a, const uint8_t* b, int64_t b_len, int64_t m, int64_t n,
                                         int64_t k, float* c) {
    return host_matmul(a, m, b, b_len, n, k, AETH_DTYPE_Q4_K, c);
}
extern "C" AETH_API int aeth_matmul_q5_k(const float* a, const uint8_t* b, int64_t b_len, int64_t m, int64_t n,
                                         int64_t k, float* c) {
    return host_matmul(a, m, b, b_len, n, k, AETH_DTYPE_Q5_K, c);
}
extern "C" AETH_API int aeth_matmul_q2_k(const float* a, const uint8_t* b, int64_t b_len, int64_t m, int64_t n,
                                         int64_t k, float* c) {
    return host_matmul(a, m, b, b_len, n, k, AETH_DTYPE_Q2_K, c, AETH_ORDER_ROWS);
}
extern "C" AETH_API int aeth_matmul_q3_k(const float* a, const uint8_t* b, int64_t b_len, int64_t m, int64_t n,
                                         int64_t k, float* c) {
    return host_matmul(a, m, b, b_len, n, k, AETH_DTYPE_Q3_K, c, AETH_ORDER_ROWS);
}
extern "C" AETH_API int aeth_matmul_f16(const float* a, const uint8_t* b, int64_t b_len, int64_t m, int64_t n,
                                        int64_t k, float* c) {
    return host_matmul(a, m, b, b_len, n, k, AETH_DTYPE_F16, c, AETH_ORDER_ROWS);
}
extern "C" AETH_API int aeth_matmul_q6_k(const float* a, const uint8_t* b, int64_t b_len, int64_t m, int64_t n,
                                         int64_t k, float* c) {
    return host_matmul(a, m, b, b_len, n, k, AETH_DTYPE_Q6_K, c);
}
