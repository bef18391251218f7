// GGUF file → device LlamaRunner: the reader of src/loader/gguf.rs:297-397
// (v3 layout: header, typed metadata, tensor infos, aligned data) and the
// LlamaModel / LlamaConfig construction of src/inference/model_loader.rs:
// 159-300 (config keys with the architecture prefix, tensor names, the
// token-embedding transpose) and 312-386 (load_f32_norm, load_quant).
//
// Quantized 2-D weights go through the device load path (aeth_load_quant:
// dequantize → transpose → requantize on the GPU, byte-exact with the
// reference's transpose_quantized_bytes); the file itself is memory-mapped.
// Supported as the runner needs them: layer and LM-head weights Q8_0, Q4_K,
// Q6_K; norms F32 / F16; token embeddings F32, F16, Q8_0, Q4_K, Q6_K.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <string.h>
#include <unistd.h>

#include <algorithm>
#include <map>
#include <string>
#include <vector>

#include "aeth_common.hpp"
#include "aeth_internal.hpp"

namespace {

const uint32_t kGgufMagic = 0x46554747u;  // "GGUF", gguf.rs:33

// GGUFDtype block geometry as the reference tabulates it (gguf.rs:137-173),
// used only to size each tensor's byte range. Returns false for unknown ids.
bool dtype_geometry(uint32_t t, uint64_t* elems, uint64_t* bytes) {
    struct G { uint32_t id; uint32_t e, b; };
    static const G tab[] = {{0, 1, 4},    {1, 1, 2},     {2, 32, 18},   {3, 32, 20},  {6, 32, 22},
                            {7, 32, 24},  {8, 32, 34},   {9, 32, 34},   {10, 256, 84}, {11, 256, 110},
                            {12, 256, 144}, {13, 256, 176}, {14, 256, 210}, {15, 256, 136}, {16, 1, 1},
                            {17, 1, 2},   {18, 1, 4}};
    for (const G& g : tab)
        if (g.id == t) {
            *elems = g.e;
            *bytes = g.b;
            return true;
        }
    return false;
}

struct MetaVal {
    int kind = 0;  // 1 unsigned, 2 signed, 3 float, 4 string, 5 other (bool, array)
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0.0;
    std::string s;
};

struct TensorInfo {
    std::vector<uint64_t> shape;
    uint32_t dtype = 0;
    uint64_t offset = 0;
    uint64_t bytes = 0;
    const uint8_t* data = nullptr;
};

struct Gguf {
    uint8_t* map = nullptr;
    size_t len = 0;
    std::map<std::string, MetaVal> meta;
    std::map<std::string, TensorInfo> tensors;
    ~Gguf() {
        if (map) munmap(map, len);
    }
};

struct Reader {
    const uint8_t* p;
    size_t n, pos = 0;
    bool bad = false;
    bool take(void* dst, size_t k) {
        if (bad || k > n - pos) {
            bad = true;
            return false;
        }
        memcpy(dst, p + pos, k);
        pos += k;
        return true;
    }
    template <class T>
    T get() {
        T v{};
        take(&v, sizeof(T));
        return v;
    }
    std::string str() {
        const uint64_t k = get<uint64_t>();
        if (bad || k > n - pos) {
            bad = true;
            return std::string();
        }
        std::string s((const char*)p + pos, (size_t)k);
        pos += (size_t)k;
        return s;
    }
};

// read_value, gguf.rs:490-517 (value types :36-51); arrays are walked and dropped
bool read_value(Reader& r, uint32_t type, MetaVal* out, int depth = 0) {
    MetaVal v;
    switch (type) {
        case 0: v.kind = 1; v.u = r.get<uint8_t>(); break;
        case 1: v.kind = 2; v.i = r.get<int8_t>(); break;
        case 2: v.kind = 1; v.u = r.get<uint16_t>(); break;
        case 3: v.kind = 2; v.i = r.get<int16_t>(); break;
        case 4: v.kind = 1; v.u = r.get<uint32_t>(); break;
        case 5: v.kind = 2; v.i = r.get<int32_t>(); break;
        case 6: v.kind = 3; v.f = r.get<float>(); break;
        case 7: v.kind = 5; v.u = r.get<uint8_t>(); break;
        case 8: v.kind = 4; v.s = r.str(); break;
        case 9: {
            const uint32_t et = r.get<uint32_t>();
            const uint64_t cnt = r.get<uint64_t>();
            if (depth > 4) return false;
            for (uint64_t e = 0; e < cnt && !r.bad; e++)
                if (!read_value(r, et, nullptr, depth + 1)) return false;
            v.kind = 5;
            break;
        }
        case 10: v.kind = 1; v.u = r.get<uint64_t>(); break;
        case 11: v.kind = 2; v.i = r.get<int64_t>(); break;
        case 12: v.kind = 3; v.f = r.get<double>(); break;
        default: return false;
    }
    if (out) *out = v;
    return !r.bad;
}

int gguf_open(const char* path, Gguf& g) {
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return aeth_set_error(AETH_EINVAL, "Failed to open GGUF file: %s", path);
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) {
        close(fd);
        return aeth_set_error(AETH_EINVAL, "GGUF file %s is too short", path);
    }
    g.len = (size_t)st.st_size;
    void* m = mmap(nullptr, g.len, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) return aeth_set_error(AETH_EINVAL, "Failed to mmap GGUF file: %s", path);
    g.map = (uint8_t*)m;
    Reader r{g.map, g.len};
    const uint32_t magic = r.get<uint32_t>();
    if (magic != kGgufMagic) return aeth_set_error(AETH_EINVAL, "Invalid GGUF magic: %#x", magic);
    (void)r.get<uint32_t>();  // version: parsed with the v3 layout (gguf.rs:321-327 warns otherwise)
    const uint64_t n_tensors = r.get<uint64_t>(), n_kv = r.get<uint64_t>();
    for (uint64_t i = 0; i < n_kv && !r.bad; i++) {
        std::string key = r.str();
        const uint32_t type = r.get<uint32_t>();
        MetaVal v;
        if (!read_value(r, type, &v)) return aeth_set_error(AETH_EINVAL, "GGUF metadata %s: bad value", key.c_str());
        g.meta[key] = v;
    }
    std::vector<std::pair<std::string, TensorInfo>> infos;
    for (uint64_t i = 0; i < n_tensors && !r.bad; i++) {
        TensorInfo t;
        std::string name = r.str();
        const uint32_t nd = r.get<uint32_t>();
        if (nd > 8) return aeth_set_error(AETH_EINVAL, "GGUF tensor %s: %u dims", name.c_str(), nd);
        for (uint32_t d = 0; d < nd; d++) t.shape.push_back(r.get<uint64_t>());
        t.dtype = r.get<uint32_t>();
        t.offset = r.get<uint64_t>();
        infos.emplace_back(std::move(name), t);
    }
    if (r.bad) return aeth_set_error(AETH_EINVAL, "GGUF header of %s is truncated", path);
    uint64_t align = 32;  // general.alignment, any integer type (gguf.rs:345-356)
    auto al = g.meta.find("general.alignment");
    if (al != g.meta.end() && (al->second.kind == 1 || al->second.kind == 2))
        align = al->second.kind == 1 ? al->second.u : (uint64_t)al->second.i;
    if (align == 0) return aeth_set_error(AETH_EINVAL, "GGUF alignment 0");
    const uint64_t start = (r.pos + align - 1) / align * align;
    for (auto& it : infos) {
        TensorInfo& t = it.second;
        uint64_t be, bb, ne = 1;
        if (!dtype_geometry(t.dtype, &be, &bb))
            return aeth_set_error(AETH_EINVAL, "Unknown tensor dtype: %u (%s)", t.dtype, it.first.c_str());
        // every dimension within int32 and the element and byte counts within uint64:
        // a wrapped product would let a crafted header pass the bounds check below
        for (uint64_t d : t.shape)
            if (d > (uint64_t)INT32_MAX || __builtin_mul_overflow(ne, d, &ne))
                return aeth_set_error(AETH_EINVAL, "Tensor '%s': shape overflows", it.first.c_str());
        if (__builtin_mul_overflow((ne + be - 1) / be, bb, &t.bytes))  // compute_tensor_byte_size, gguf.rs:539-551
            return aeth_set_error(AETH_EINVAL, "Tensor '%s': byte size overflows", it.first.c_str());
        const uint64_t off = start + t.offset;
        if (off > g.len || t.bytes > g.len - off)
            return aeth_set_error(AETH_EINVAL, "Tensor '%s' offset out of bounds", it.first.c_str());
        t.data = g.map + off;
        g.tensors[it.first] = t;
    }
    return AETH_OK;
}

bool meta_usize(const Gguf& g, const std::string& k, int64_t* v) {  // gguf_usize, model_loader.rs:408-416
    auto it = g.meta.find(k);
    if (it == g.meta.end()) return false;
    if (it->second.kind == 1 && it->second.u <= (uint64_t)INT64_MAX) *v = (int64_t)it->second.u;
    else if (it->second.kind == 2) *v = it->second.i;
    else return false;
    return true;
}
bool meta_f32(const Gguf& g, const std::string& k, float* v) {  // gguf_f32, :418-424
    auto it = g.meta.find(k);
    if (it == g.meta.end() || it->second.kind != 3) return false;
    *v = (float)it->second.f;
    return true;
}

// f16 → f32, exact (the half crate's to_f32)
float half_to_float(uint16_t h) {
    const uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu, bits;
    if (e == 0) {
        if (m == 0) {
            bits = s;
        } else {
            int sh = 0;
            while (!(m & 0x400u)) {
                m <<= 1;
                sh++;
            }
            bits = s | ((uint32_t)(113 - sh) << 23) | ((m & 0x3FFu) << 13);
        }
    } else if (e == 31) {
        bits = s | 0x7F800000u | (m << 13);
    } else {
        bits = s | ((e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

// Device staging for the load path, grown to the largest tensor.
struct Staging {
    void *src = nullptr, *ws = nullptr, *dst = nullptr;
    size_t src_b = 0, ws_b = 0, dst_b = 0;
    hipStream_t s = nullptr;
    ~Staging() {
        if (src) hipFree(src);
        if (ws) hipFree(ws);
        if (dst) hipFree(dst);
        if (s) hipStreamDestroy(s);
    }
    static int grow(void** p, size_t* cap, size_t need) {
        if (need <= *cap) return AETH_OK;
        if (*p) hipFree(*p);
        *p = nullptr;
        *cap = 0;
        AETH_HIP_CHECK(hipMalloc(p, need));
        *cap = need;
        return AETH_OK;
    }
};

// load_quant (model_loader.rs:330-359): GGUF shape [k, n] → QuantWeight bytes (host): [n][k]
// re-quantized rows for the fused formats, the GGUF bytes for the others
int load_quant(const Gguf& g, const std::string& name, Staging& st, std::vector<uint8_t>& out, int* dtype,
               int64_t* n_out, int64_t* k_out) {
    auto it = g.tensors.find(name);
    if (it == g.tensors.end()) return aeth_set_error(AETH_EINVAL, "Missing tensor: %s", name.c_str());
    const TensorInfo& t = it->second;
    if (t.shape.size() != 2) return aeth_set_error(AETH_EUNSUPPORTED, "tensor %s is not 2-D", name.c_str());
    const int64_t k = (int64_t)t.shape[0], n = (int64_t)t.shape[1];  // each <= INT32_MAX (gguf_open)
    if (k < 1 || n < 1) return aeth_set_error(AETH_EINVAL, "tensor %s has an empty dimension", name.c_str());
    int be, bb;
    if (aeth_block_geometry((int)t.dtype, &be, &bb) != AETH_OK)
        return aeth_set_error(AETH_EUNSUPPORTED,
                              "tensor %s: dtype %u is not a format this build runs (F32, F16, Q8_0, Q2_K..Q6_K)",
                              name.c_str(), t.dtype);
    int rc;
    if (!aeth_dtype_fused((int)t.dtype)) {  // F32 / F16 / Q2_K / Q3_K: the bytes as the file holds them (:348-350)
        const int64_t need = aeth_weight_raw_bytes((int)t.dtype, AETH_ORDER_GGUF, n, k);
        if (need < 0 || (uint64_t)need > t.bytes)
            return aeth_set_error(AETH_EINVAL, "tensor %s: %llu bytes for [%lld, %lld]", name.c_str(),
                                  (unsigned long long)t.bytes, (long long)k, (long long)n);
        out.assign(t.data, t.data + need);
        *dtype = (int)t.dtype;
        *n_out = n;
        *k_out = k;
        return AETH_OK;
    }
    int64_t out_b = 0, kn = 0;
    const int64_t ws_b = aeth_load_quant_ws_bytes(k, n);
    if (!aeth_mul_ok(n, aeth_cdiv(k, be) * bb, &out_b) || !aeth_mul_ok(k, n, &kn) || ws_b < 0)
        return aeth_set_error(AETH_EINVAL, "tensor %s: [%lld, %lld] is too large", name.c_str(), (long long)k,
                              (long long)n);
    if ((uint64_t)kn / (uint64_t)be * (uint64_t)bb > t.bytes)
        return aeth_set_error(AETH_EINVAL, "tensor %s: %llu bytes for [%lld, %lld]", name.c_str(),
                              (unsigned long long)t.bytes, (long long)k, (long long)n);
    if ((rc = Staging::grow(&st.src, &st.src_b, t.bytes)) || (rc = Staging::grow(&st.dst, &st.dst_b, (size_t)out_b)) ||
        (rc = Staging::grow(&st.ws, &st.ws_b, (size_t)ws_b)))
        return rc;
    AETH_HIP_CHECK(hipMemcpyAsync(st.src, t.data, t.bytes, hipMemcpyHostToDevice, st.s));
    if ((rc = aeth_load_quant((int)t.dtype, st.src, k, n, st.dst, st.ws, st.s))) return rc;
    out.resize((size_t)out_b);
    AETH_HIP_CHECK(hipMemcpyAsync(out.data(), st.dst, (size_t)out_b, hipMemcpyDeviceToHost, st.s));
    AETH_HIP_CHECK(hipStreamSynchronize(st.s));
    *dtype = (int)t.dtype;
    *n_out = n;
    *k_out = k;
    return AETH_OK;
}

// dequantize of an F32 / F16 / Q8_0 / Q2_K..Q6_K tensor to f32 (loader/dequant.rs entry `dequantize`)
int dequantize(const TensorInfo& t, const std::string& name, Staging& st, std::vector<float>& out) {
    uint64_t ne = 1;
    for (uint64_t d : t.shape) ne *= d;
    out.assign(ne, 0.0f);
    if (t.dtype == 0) {
        memcpy(out.data(), t.data, ne * 4);
    } else if (t.dtype == 1) {
        for (uint64_t i = 0; i < ne; i++) {
            uint16_t h;
            memcpy(&h, t.data + 2 * i, 2);
            out[i] = half_to_float(h);
        }
    } else if (t.dtype == AETH_DTYPE_Q8_0 || (t.dtype >= AETH_DTYPE_Q2_K && t.dtype <= AETH_DTYPE_Q6_K)) {
        int rc;
        if ((rc = Staging::grow(&st.src, &st.src_b, t.bytes)) || (rc = Staging::grow(&st.ws, &st.ws_b, ne * 4)))
            return rc;
        AETH_HIP_CHECK(hipMemcpyAsync(st.src, t.data, t.bytes, hipMemcpyHostToDevice, st.s));
        AETH_HIP_CHECK(hipMemsetAsync(st.ws, 0, ne * 4, st.s));  // whole blocks only; the tail stays 0
        if ((rc = aeth_dequant((int)t.dtype, st.src, (int64_t)ne, (float*)st.ws, st.s))) return rc;
        AETH_HIP_CHECK(hipMemcpyAsync(out.data(), st.ws, ne * 4, hipMemcpyDeviceToHost, st.s));
        AETH_HIP_CHECK(hipStreamSynchronize(st.s));
    } else {
        return aeth_set_error(AETH_EUNSUPPORTED, "tensor %s: dtype %u cannot be dequantized by this build", name.c_str(),
                              t.dtype);
    }
    return AETH_OK;
}

}  // namespace

// LlamaModel::from_gguf + LlamaConfig::from_gguf (model_loader.rs:159-300) into a
// device runner. bos/eos from tokenizer.ggml.{bos,eos}_token_id (defaults 1, 2:
// tokenizer/mod.rs:65-66).
int aeth_gguf_load_runner(const char* path, aeth_runner** out, int* bos, int* eos) {
    if (!path || !out) return aeth_set_error(AETH_EINVAL, "aether_load: null argument");
    *out = nullptr;
    Gguf g;
    int rc = gguf_open(path, g);
    if (rc) return rc;
    // key(): arch-specific prefix, then "llama.", then the bare key (model_loader.rs:240-252)
    std::string prefix = "llama.";
    auto ar = g.meta.find("general.architecture");
    if (ar != g.meta.end() && ar->second.kind == 4) {
        const std::string& a = ar->second.s;
        if (a == "mistral" || a == "phi3" || a == "qwen2" || a == "gemma2" || a == "deepseek2") prefix = a + ".";
    }
    auto key = [&](const char* k) {
        const std::string ak = prefix + k, lk = std::string("llama.") + k;
        if (g.meta.count(ak)) return ak;
        if (g.meta.count(lk)) return lk;
        return std::string(k);
    };
    int64_t d = 0, nl = 0, nh = 0, nkv = 0, dff = 0, ctx = 2048, rope_dim = 0, sw = 0;
    if (!meta_usize(g, key("embedding_length"), &d)) return aeth_set_error(AETH_EINVAL, "Missing embedding_length");
    if (!meta_usize(g, key("block_count"), &nl)) return aeth_set_error(AETH_EINVAL, "Missing block_count");
    if (!meta_usize(g, key("attention.head_count"), &nh)) return aeth_set_error(AETH_EINVAL, "Missing attention.head_count");
    if (!meta_usize(g, key("attention.head_count_kv"), &nkv)) nkv = nh;
    if (!meta_usize(g, key("feed_forward_length"), &dff)) return aeth_set_error(AETH_EINVAL, "Missing feed_forward_length");
    meta_usize(g, key("context_length"), &ctx);
    float rope_base = 10000.0f, eps = 1e-5f;
    meta_f32(g, key("rope.freq_base"), &rope_base);
    meta_f32(g, key("attention.layer_norm_rms_epsilon"), &eps);
    auto te = g.tensors.find("token_embd.weight");
    if (te == g.tensors.end() || te->second.shape.size() < 2) return aeth_set_error(AETH_EINVAL, "Cannot determine vocab size");
    const int64_t vocab = (int64_t)te->second.shape[1];
    // every dimension positive and within int32, so that the products below cannot wrap
    const int64_t dims[] = {d, nl, nh, nkv, dff, vocab};
    for (int64_t v : dims)
        if (v <= 0 || v > INT32_MAX)
            return aeth_set_error(AETH_EINVAL, "GGUF config: a dimension (%lld) is not in [1, 2^31)", (long long)v);
    if (nl > 65536 || (d % nh)) return aeth_set_error(AETH_EINVAL, "GGUF config: %lld layers, d %lld, %lld heads",
                                                       (long long)nl, (long long)d, (long long)nh);
    int64_t vd = 0;
    if (!aeth_mul_ok(vocab, d, &vd) || vd > (1LL << 40))
        return aeth_set_error(AETH_EINVAL, "GGUF config: vocab %lld x d %lld is too large", (long long)vocab,
                              (long long)d);
    const int64_t hd = d / nh;
    if (meta_usize(g, key("rope.dimension_count"), &rope_dim) && rope_dim != hd)
        return aeth_set_error(AETH_EUNSUPPORTED, "partial RoPE (rope.dimension_count %lld of head_dim %lld) is not built",
                              (long long)rope_dim, (long long)hd);
    // ArchConfig::sliding_window (model_loader.rs:286): None when the key is absent
    const bool has_sw = meta_usize(g, key("attention.sliding_window_length"), &sw);
    if (has_sw && sw < 1)  // attn_direct would mask every position (NaN logits); refused instead
        return aeth_set_error(AETH_EUNSUPPORTED, "attention.sliding_window_length %lld masks every position",
                              (long long)sw);
    if (ctx < 1) return aeth_set_error(AETH_EINVAL, "GGUF config: context_length %lld", (long long)ctx);
    // LlamaConfig::max_seq_len = context_length (default 2048, model_loader.rs:280); the runner then
    // holds min(max_seq_len, 4096) positions (runner.rs:225, :339)
    const int64_t max_seq = ctx > INT32_MAX ? INT32_MAX : ctx;
    int64_t bv = 1, ev = 2;
    meta_usize(g, "tokenizer.ggml.bos_token_id", &bv);
    meta_usize(g, "tokenizer.ggml.eos_token_id", &ev);
    if (bos) *bos = (int)bv;
    if (eos) *eos = (int)ev;

    aeth_llama_config cfg{(int32_t)vocab, (int32_t)d, (int32_t)nl, (int32_t)nh, (int32_t)nkv, (int32_t)hd,
                          (int32_t)dff, (int32_t)max_seq, rope_base, eps,
                          has_sw ? (int32_t)std::min<int64_t>(sw, INT32_MAX) : 0, 0};
    Staging st;
    AETH_HIP_CHECK(hipStreamCreate(&st.s));
    // token embeddings: [d_model][vocab] as the reference reads them → [vocab][d_model] (model_loader.rs:174-188)
    std::vector<float> emb_raw, emb;
    if ((rc = dequantize(te->second, "token_embd.weight", st, emb_raw))) return rc;
    if ((int64_t)emb_raw.size() != vocab * d)
        return aeth_set_error(AETH_EINVAL, "token_embd.weight has %zu elements, expected %lld", emb_raw.size(),
                              (long long)(vocab * d));
    emb.resize(emb_raw.size());
    {
        int rc2;
        float *dsrc = nullptr, *ddst = nullptr;
        AETH_HIP_CHECK(hipMalloc(&dsrc, emb_raw.size() * 4));
        if (hipMalloc(&ddst, emb_raw.size() * 4) != hipSuccess) {
            hipFree(dsrc);
            return aeth_set_error(AETH_ENOMEM, "token embeddings: device memory");
        }
        rc2 = hipMemcpy(dsrc, emb_raw.data(), emb_raw.size() * 4, hipMemcpyHostToDevice) == hipSuccess ? AETH_OK : AETH_EHIP;
        if (!rc2) rc2 = aeth_transpose_f32(dsrc, d, vocab, ddst, st.s);
        if (!rc2 && hipMemcpyAsync(emb.data(), ddst, emb.size() * 4, hipMemcpyDeviceToHost, st.s) != hipSuccess) rc2 = AETH_EHIP;
        if (!rc2 && hipStreamSynchronize(st.s) != hipSuccess) rc2 = AETH_EHIP;
        hipFree(dsrc);
        hipFree(ddst);
        if (rc2) return rc2 == AETH_EHIP ? aeth_set_error(AETH_EHIP, "token embeddings: transpose failed") : rc2;
    }
    emb_raw = std::vector<float>();
    auto load_norm = [&](const std::string& name, std::vector<float>& v) {  // load_f32_norm, :312-328
        auto it = g.tensors.find(name);
        if (it == g.tensors.end()) return aeth_set_error(AETH_EINVAL, "Missing norm tensor: %s", name.c_str());
        int r2 = dequantize(it->second, name, st, v);
        if (r2) return r2;
        if ((int64_t)v.size() != d)
            return aeth_set_error(AETH_EINVAL, "Norm tensor %s has %zu elements, expected %lld", name.c_str(), v.size(),
                                  (long long)d);
        return AETH_OK;
    };
    static const char* names[7] = {"attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"};
    const int64_t want[7][2] = {{nh * hd, d}, {nkv * hd, d}, {nkv * hd, d}, {d, nh * hd}, {dff, d}, {dff, d}, {d, dff}};
    std::vector<std::vector<uint8_t>> wbuf((size_t)(nl * 7));
    std::vector<std::vector<float>> nbuf((size_t)(nl * 2));
    std::vector<const void*> wp((size_t)(nl * 7));
    std::vector<int32_t> wdt((size_t)(nl * 7));
    std::vector<const float*> np((size_t)(nl * 2));
    for (int64_t l = 0; l < nl; l++) {
        const std::string pre = "blk." + std::to_string(l) + ".";
        if ((rc = load_norm(pre + "attn_norm.weight", nbuf[l * 2])) || (rc = load_norm(pre + "ffn_norm.weight", nbuf[l * 2 + 1])))
            return rc;
        np[l * 2] = nbuf[l * 2].data();
        np[l * 2 + 1] = nbuf[l * 2 + 1].data();
        for (int j = 0; j < 7; j++) {
            int dt;
            int64_t n, k;
            const std::string nm = pre + names[j] + ".weight";
            if ((rc = load_quant(g, nm, st, wbuf[l * 7 + j], &dt, &n, &k))) return rc;
            if (n != want[j][0] || k != want[j][1])
                return aeth_set_error(AETH_EINVAL, "%s is [%lld, %lld] (GGUF order), expected [%lld, %lld]", nm.c_str(),
                                      (long long)k, (long long)n, (long long)want[j][1], (long long)want[j][0]);
            wp[l * 7 + j] = wbuf[l * 7 + j].data();
            wdt[l * 7 + j] = dt;
        }
    }
    std::vector<float> fnorm;
    if ((rc = load_norm("output_norm.weight", fnorm))) return rc;
    std::vector<uint8_t> lm;
    int lm_dt;
    int64_t ln, lk;
    if ((rc = load_quant(g, "output.weight", st, lm, &lm_dt, &ln, &lk))) return rc;
    if (ln != vocab || lk != d)
        return aeth_set_error(AETH_EINVAL, "output.weight is [%lld, %lld], expected [%lld, %lld]", (long long)lk,
                              (long long)ln, (long long)d, (long long)vocab);
    return aeth_runner_create(&cfg, wp.data(), wdt.data(), np.data(), fnorm.data(), lm.data(), lm_dt, emb.data(), 0,
                              out);
}
