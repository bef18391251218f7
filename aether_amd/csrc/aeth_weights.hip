// Runtime state, error reporting, device-resident weights (planar re-layout
// of GGUF blocks) and the seeded synthetic-input generators.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>

#include "aeth_common.hpp"
#include "aeth_internal.hpp"

static thread_local char g_err[1024];

int aeth_set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

extern "C" AETH_API const char* aeth_last_error(void) { return g_err; }

static int g_num_cus[64];

int aeth_num_cus() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (g_num_cus[dev] == 0) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
        g_num_cus[dev] = v;
    }
    return g_num_cus[dev];
}

extern "C" AETH_API int aeth_init(int device) {
    int count = 0;
    AETH_HIP_CHECK(hipGetDeviceCount(&count));
    if (device < 0 || device >= count)
        return aeth_set_error(AETH_EINVAL, "aeth_init: device %d out of range (%d devices)", device, count);
    AETH_HIP_CHECK(hipSetDevice(device));
    (void)aeth_num_cus();
    return aeth_noalloc_setup(device);
}

extern "C" AETH_API int aeth_block_geometry(int dtype, int* block_elems, int* block_bytes) {
    int e, b;
    switch (dtype) {
        case AETH_DTYPE_F32: e = 1; b = 4; break;
        case AETH_DTYPE_F16: e = 1; b = 2; break;
        case AETH_DTYPE_Q2_K: e = QK_BLOCK_ELEMS; b = Q2K_BLOCK_BYTES; break;
        case AETH_DTYPE_Q3_K: e = QK_BLOCK_ELEMS; b = Q3K_BLOCK_BYTES; break;
        case AETH_DTYPE_Q8_0: e = Q8_BLOCK_ELEMS; b = Q8_BLOCK_BYTES; break;
        case AETH_DTYPE_Q4_K: e = QK_BLOCK_ELEMS; b = Q4K_BLOCK_BYTES; break;
        case AETH_DTYPE_Q5_K: e = QK_BLOCK_ELEMS; b = Q5K_BLOCK_BYTES; break;
        case AETH_DTYPE_Q6_K: e = QK_BLOCK_ELEMS; b = Q6K_BLOCK_BYTES; break;
        default: return aeth_set_error(AETH_EUNSUPPORTED, "unsupported dtype %d", dtype);
    }
    if (block_elems) *block_elems = e;
    if (block_bytes) *block_bytes = b;
    return AETH_OK;
}

// Blocks per row as the reference counts them: Q8_0 rows hold ceil(k/32)
// blocks (q8_0.rs:16, requantize_q8_0); K-quant kernels read k/256 blocks
// (avx2.rs:26, q4_k.rs:16, q2_k.rs:16); F16 / F32 rows hold k elements.
int64_t aeth_blocks_per_row(int dtype, int64_t k) {
    if (dtype == AETH_DTYPE_Q8_0) return (k + 31) / 32;
    if (dtype == AETH_DTYPE_F16 || dtype == AETH_DTYPE_F32) return k;
    return k / 256;
}

int64_t aeth_weight_raw_bytes(int dtype, int order, int64_t n, int64_t k) {
    int be, bb;
    // n, k within int32 (the kernels index rows and columns in 32 bits) and no product past int64
    if (aeth_block_geometry(dtype, &be, &bb) != AETH_OK || n <= 0 || k <= 0 || n > INT32_MAX || k > INT32_MAX)
        return -1;
    if (order == AETH_ORDER_GGUF) return (n * k / be) * bb;  // dequantize's flat run of whole blocks
    return n * aeth_blocks_per_row(dtype, k) * bb;
}

// ── device layout ────────────────────────────────────────────────────────
// Rows are grouped in tiles of 16 (zero rows pad the last tile) so that each
// wave load of the matrix-core GEMV (aeth_gemv.hip) covers 16 rows
// contiguously; lane (n, kg) = lane n + 16·kg of a 64-lane wave.
//  Q4_K: p0 = headers [tile][b][16 rows][16 B]; p1 = quants [tile][b][half h][lane][16 B],
//        lane (n, kg) = qs[64h + 16kg, +16) of row n (aeth_q4k_*_off).
//  Q5_K: p0, p1 as Q4_K (header bytes 0..15; qs = bytes 48..175 in Q4_K's qs
//        order); p2 = fifth bits [tile][b][lane][8 B], lane (n, kg) holding, per
//        half h, the 16-bit runs of qh for its low-nibble elements
//        (128h + 64(kg/2) + 16(kg%2) + [0,16)) and high-nibble elements (+32);
//        p3 = the same bits again for the GEMM (aeth_gemm_kq.hip), [tile][b][J 4][kg 2]
//        [row 16][half 2] 16-bit words (k_q5_gemm_bits).
//  Q6_K: p0 = [tile][b][part][lane][16 B], lane (n, kg = 2h + g'): part 0 =
//        ql[64h + 16g', +16), part 1 = ql[64h + 32 + 16g', +16), part 2 =
//        qh[32h + 16g', +16); p1 = sc [tile][b][16 rows][16 B]; p2 = d [tile][b][16 rows].
//  Q8_0: blocks in groups of 4 (zero blocks pad the row to whole groups);
//        p0 = quants [tile][group][j][lane][16 B], lane (n, kg) = bytes
//        [16(kg & 1), +16) of block 4·group + 2j + (kg ≥ 2); p1 = d [tile][group][4][16 rows].

static int64_t align256(int64_t v) { return (v + 255) & ~(int64_t)255; }

// Maps raw GGUF byte i (block-major over all rows) to its device address.
__device__ __forceinline__ uint8_t* planar_addr(int dtype, int64_t i, int64_t nb, uint8_t* p0, uint8_t* p1,
                                                uint8_t* p2, uint8_t* p3) {
    (void)p3;
    if (dtype == AETH_DTYPE_Q4_K) {
        const int64_t blk = i / Q4K_BLOCK_BYTES;
        const int off = (int)(i - blk * Q4K_BLOCK_BYTES);
        const int64_t row = blk / nb, b = blk - row * nb;
        if (off < 16) return p0 + aeth_q4k_hdr_off(row, b, nb) + off;
        return p1 + aeth_q4k_qs_off(row, b, off - 16, nb);
    }
    if (dtype == AETH_DTYPE_Q5_K) {
        const int64_t blk = i / Q5K_BLOCK_BYTES;
        const int off = (int)(i - blk * Q5K_BLOCK_BYTES);
        const int64_t row = blk / nb, b = blk - row * nb;
        if (off < 16) return p0 + aeth_q4k_hdr_off(row, b, nb) + off;
        if (off >= 48) return p1 + aeth_q4k_qs_off(row, b, off - 48, nb);
        // qh byte q: half q/16, r = q%16 → lane group kg = 2(r/8) + (r/2)%2,
        // byte 4h + 2·(high nibble: (r%8)/4) + r%2 of the lane's 8
        const int q = off - 16, h = q >> 4, r = q & 15;
        const int kg = 2 * (r >> 3) + ((r >> 1) & 1), j = 4 * h + 2 * ((r & 7) >> 2) + (r & 1);
        return p2 + ((((row >> 4) * nb + b) * 64 + (row & 15) + 16 * kg) * 8 + j);
    }
    if (dtype == AETH_DTYPE_Q6_K) {
        const int64_t blk = i / Q6K_BLOCK_BYTES;
        const int off = (int)(i - blk * Q6K_BLOCK_BYTES);
        const int64_t row = blk / nb, b = blk - row * nb;
        const int64_t tb = (row >> 4) * nb + b, n = row & 15;
        if (off < 128) {  // ql
            const int h = off >> 6, r = off & 63, part = r >> 5, kg = 2 * h + ((r >> 4) & 1);
            return p0 + ((tb * 3 + part) * 64 + n + 16 * kg) * 16 + (r & 15);
        }
        if (off < 192) {  // qh
            const int q = off - 128, kg = 2 * (q >> 5) + ((q >> 4) & 1);
            return p0 + ((tb * 3 + 2) * 64 + n + 16 * kg) * 16 + (q & 15);
        }
        if (off < 208) return p1 + (tb * 16 + n) * 16 + (off - 192);
        return p2 + (tb * 16 + n) * 2 + (off - 208);
    }
    const int64_t blk = i / Q8_BLOCK_BYTES;
    const int off = (int)(i - blk * Q8_BLOCK_BYTES);
    const int64_t row = blk / nb, b = blk - row * nb, ngr = (nb + 3) / 4;
    const int64_t tg = (row >> 4) * ngr + (b >> 2), n = row & 15;
    const int s = (int)(b & 3);
    if (off < 2) return p1 + ((tg * 4 + s) * 16 + n) * 2 + off;
    const int p = off - 2, kg = 2 * (s & 1) + (p >> 4);
    return p0 + ((tg * 2 + (s >> 1)) * 64 + n + 16 * kg) * 16 + (p & 15);
}

// True when raw byte i is the high byte of an f16 block scale: Q8_0 d (bytes 0-1), Q4_K / Q5_K
// d and dmin (0-3), Q6_K d (208-209).
__device__ __forceinline__ bool scale_high_byte(int dtype, int64_t i) {
    if (dtype == AETH_DTYPE_Q4_K) { const int o = (int)(i % Q4K_BLOCK_BYTES); return o == 1 || o == 3; }
    if (dtype == AETH_DTYPE_Q5_K) { const int o = (int)(i % Q5K_BLOCK_BYTES); return o == 1 || o == 3; }
    if (dtype == AETH_DTYPE_Q6_K) return i % Q6K_BLOCK_BYTES == 209;
    return i % Q8_BLOCK_BYTES == 1;
}

// to_planar: raw → planes, and *special set if a block scale has the f16 exponent 31
// (bits 2-6 of its high byte all set); otherwise planes → raw.
__global__ void k_relayout(int dtype, int64_t nb, uint8_t* __restrict__ raw, uint8_t* __restrict__ p0,
                           uint8_t* __restrict__ p1, uint8_t* __restrict__ p2, uint8_t* __restrict__ p3,
                           int64_t total_bytes, int to_planar, int* special) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total_bytes) return;
    uint8_t* dst = planar_addr(dtype, i, nb, p0, p1, p2, p3);
    if (to_planar) {
        const uint8_t b = raw[i];
        *dst = b;
        if ((b & 0x7C) == 0x7C && scale_high_byte(dtype, i)) atomicOr(special, 1);
    } else {
        raw[i] = *dst;
    }
}

static int relayout(aeth_weight* w, uint8_t* d_raw, int to_planar, hipStream_t s, int* d_special = nullptr) {
    int64_t total = w->nblk * w->block_bytes;
    if (total == 0) return AETH_OK;
    int64_t grid = aeth_cdiv(total, 256);
    hipLaunchKernelGGL(k_relayout, dim3((unsigned)grid), dim3(256), 0, s, w->dtype, w->nb, d_raw, w->p0, w->p1,
                       w->p2, w->p3, total, to_planar, d_special);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}

// The Q5_K GEMM's fifth-bit words (aeth_gemm_kq.hip). GEMM lane half h of slice pair (J, kg)
// takes elements l = 16kg + 8h + p (p = 0..7) of sub-blocks 2J and 2J + 1, whose fifth bits
// (bit 32·s + l of qh) are bits p of qh bytes 8J + 2kg + h and 8J + 4 + 2kg + h. The word holds
// them in the order of the MFMA operand's halves: bits 0-3 the low sub-block's p = 0, 1, 4, 5,
// bits 4-7 the high sub-block's, bits 8-11 and 12-15 the same for p = 2, 3, 6, 7. One thread
// per (row, super-block) of the raw [n][nb] blocks; the padding rows stay zero.
__device__ __forceinline__ uint32_t q5_pick(uint32_t v, int a, int b, int c, int d) {
    return ((v >> a) & 1u) | (((v >> b) & 1u) << 1) | (((v >> c) & 1u) << 2) | (((v >> d) & 1u) << 3);
}
__global__ void k_q5_gemm_bits(const uint8_t* __restrict__ raw, int64_t n, int64_t nb, uint8_t* __restrict__ p3) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n * nb) return;
    const int64_t row = i / nb, b = i - row * nb;
    const uint8_t* qh = raw + i * Q5K_BLOCK_BYTES + 16;
    uint16_t* dst = (uint16_t*)(p3 + ((row >> 4) * nb + b) * 512) + (row & 15) * 2;
    for (int J = 0; J < 4; J++)
        for (int kg = 0; kg < 2; kg++)
            for (int h = 0; h < 2; h++) {
                const uint32_t lo = qh[8 * J + 2 * kg + h], hi = qh[8 * J + 4 + 2 * kg + h];
                const uint32_t w = q5_pick(lo, 0, 1, 4, 5) | (q5_pick(hi, 0, 1, 4, 5) << 4) |
                                   (q5_pick(lo, 2, 3, 6, 7) << 8) | (q5_pick(hi, 2, 3, 6, 7) << 12);
                dst[(J * 2 + kg) * 32 + h] = (uint16_t)w;
            }
}

// Raw (GGUF-order or row) weights: the bytes as given, one allocation.
static int create_raw(int dtype, int order, int64_t n, int64_t k, const void* raw, int raw_is_device, hipStream_t s,
                      aeth_weight** out) {
    const int64_t bytes = aeth_weight_raw_bytes(dtype, order, n, k);
    const bool kq = dtype == AETH_DTYPE_Q2_K || dtype == AETH_DTYPE_Q3_K;
    // the GEMV lanes read 4 consecutive elements of one row (and one block)
    if (order == AETH_ORDER_GGUF && n % 4)
        return aeth_set_error(AETH_EUNSUPPORTED, "GGUF-order weights need out_features %% 4 == 0 (n=%lld)", (long long)n);
    if (order == AETH_ORDER_GGUF && kq && (n * k) % 256)
        return aeth_set_error(AETH_EINVAL, "GGUF-order Q2_K/Q3_K weights need whole blocks (n·k = %lld)",
                              (long long)(n * k));
    if (order == AETH_ORDER_ROWS && kq && k < 256)
        return aeth_set_error(AETH_EINVAL, "aeth_weight_create: K-quant needs k >= 256 (k=%lld)", (long long)k);
    if (order == AETH_ORDER_ROWS && dtype == AETH_DTYPE_F16 && k % 4)
        return aeth_set_error(AETH_EUNSUPPORTED, "row-order F16 weights need k %% 4 == 0 (k=%lld)", (long long)k);
    if (order == AETH_ORDER_ROWS && dtype == AETH_DTYPE_F32)
        return aeth_set_error(AETH_EUNSUPPORTED, "row-order F32 weights are not a kernel of this build");
    if (bytes < 0) return aeth_set_error(AETH_EINVAL, "aeth_weight_create: bad shape n=%lld k=%lld", (long long)n,
                                         (long long)k);
    aeth_weight* w = new (std::nothrow) aeth_weight();
    if (!w) return aeth_set_error(AETH_ENOMEM, "aeth_weight_create: out of host memory");
    w->dtype = dtype;
    w->order = order;
    w->n = n;
    w->k = k;
    w->nb = aeth_blocks_per_row(dtype, k);
    int be, bb;
    aeth_block_geometry(dtype, &be, &bb);
    w->block_bytes = bb;
    w->nblk = bytes / bb;
    w->bytes = bytes;
    hipError_t e = hipMalloc((void**)&w->base, (size_t)(bytes > 0 ? bytes : 256));
    if (e != hipSuccess) {
        delete w;
        return aeth_set_error(AETH_ENOMEM, "aeth_weight_create: hipMalloc(%lld) failed: %s", (long long)bytes,
                              hipGetErrorString(e));
    }
    e = hipMemcpyAsync(w->base, raw, (size_t)bytes, raw_is_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, s);
    if (e == hipSuccess && !raw_is_device) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
        hipFree(w->base);
        delete w;
        return aeth_set_error(AETH_EHIP, "aeth_weight_create: copy failed: %s", hipGetErrorString(e));
    }
    w->p0 = w->base;
    *out = w;
    return AETH_OK;
}

int aeth_weight_create_ex(int dtype, int order, int64_t n, int64_t k, const void* raw, int raw_is_device,
                          hipStream_t s, aeth_weight** out) {
    if (!out) return aeth_set_error(AETH_EINVAL, "aeth_weight_create: out is NULL");
    *out = nullptr;
    int be, bb;
    int rc = aeth_block_geometry(dtype, &be, &bb);
    if (rc) return rc;
    if (n <= 0 || k <= 0) return aeth_set_error(AETH_EINVAL, "aeth_weight_create: bad shape n=%lld k=%lld",
                                                (long long)n, (long long)k);
    if (!raw) return aeth_set_error(AETH_EINVAL, "aeth_weight_create: raw is NULL");
    if (order != AETH_ORDER_PLANAR) return create_raw(dtype, order, n, k, raw, raw_is_device, s, out);
    if (!aeth_dtype_fused(dtype))
        return aeth_set_error(AETH_EUNSUPPORTED, "aeth_weight_create: dtype %d has no planar layout", dtype);
    if (dtype != AETH_DTYPE_Q8_0 && k < 256)
        return aeth_set_error(AETH_EINVAL, "aeth_weight_create: K-quant needs k >= 256 (k=%lld)", (long long)k);
    if (n > INT32_MAX || k > INT32_MAX)
        return aeth_set_error(AETH_EINVAL, "aeth_weight_create: shape n=%lld k=%lld beyond int32", (long long)n,
                              (long long)k);
    aeth_weight* w = new (std::nothrow) aeth_weight();
    if (!w) return aeth_set_error(AETH_ENOMEM, "aeth_weight_create: out of host memory");
    w->dtype = dtype;
    w->order = AETH_ORDER_PLANAR;
    w->n = n;
    w->k = k;
    w->nb = aeth_blocks_per_row(dtype, k);
    w->nblk = n * w->nb;
    w->block_bytes = bb;
    int64_t sz[4] = {0, 0, 0, 0};
    const int64_t prow = aeth_cdiv(n, 16) * 16;  // whole 16-row tiles
    if (dtype == AETH_DTYPE_Q4_K) { sz[0] = prow * w->nb * 16; sz[1] = prow * w->nb * 128; }
    else if (dtype == AETH_DTYPE_Q5_K) {
        sz[0] = prow * w->nb * 16;
        sz[1] = prow * w->nb * 128;
        sz[2] = prow * w->nb * 32;
        sz[3] = prow * w->nb * 32;
    }
    else if (dtype == AETH_DTYPE_Q6_K) { sz[0] = prow * w->nb * 192; sz[1] = prow * w->nb * 16; sz[2] = prow * w->nb * 2; }
    else { const int64_t pb = aeth_cdiv(w->nb, 4) * 4; sz[0] = prow * pb * 32; sz[1] = prow * pb * 2; }
    int64_t off[4], tot = 0;
    for (int i = 0; i < 4; i++) { off[i] = tot; tot += align256(sz[i]); }
    w->bytes = w->nblk * bb;
    const int64_t flag_off = tot;  // one int after the planes: the special-scale flag
    tot += 256;
    hipError_t e = hipMalloc((void**)&w->base, (size_t)tot);
    if (e != hipSuccess) {
        delete w;
        return aeth_set_error(AETH_ENOMEM, "aeth_weight_create: hipMalloc(%lld) failed: %s", (long long)tot,
                              hipGetErrorString(e));
    }
    {
        e = hipMemsetAsync(w->base, 0, (size_t)tot, s);  // padding rows / blocks read as zero
        if (e != hipSuccess) {
            hipFree(w->base);
            delete w;
            return aeth_set_error(AETH_EHIP, "aeth_weight_create: memset failed: %s", hipGetErrorString(e));
        }
    }
    w->p0 = w->base + off[0];
    w->p1 = w->base + off[1];
    w->p2 = sz[2] ? w->base + off[2] : nullptr;
    w->p3 = sz[3] ? w->base + off[3] : nullptr;
    uint8_t* staging = nullptr;
    if (raw_is_device) {
        staging = (uint8_t*)raw;
    } else {
        e = hipMalloc((void**)&staging, (size_t)w->bytes);
        if (e != hipSuccess) {
            hipFree(w->base);
            delete w;
            return aeth_set_error(AETH_ENOMEM, "aeth_weight_create: staging hipMalloc failed: %s",
                                  hipGetErrorString(e));
        }
        e = hipMemcpyAsync(staging, raw, (size_t)w->bytes, hipMemcpyHostToDevice, s);
        if (e != hipSuccess) {
            hipFree(staging);
            hipFree(w->base);
            delete w;
            return aeth_set_error(AETH_EHIP, "aeth_weight_create: H2D copy failed: %s", hipGetErrorString(e));
        }
    }
    rc = relayout(w, staging, 1, s, (int*)(w->base + flag_off));
    if (rc == AETH_OK && dtype == AETH_DTYPE_Q5_K) {
        hipLaunchKernelGGL(k_q5_gemm_bits, dim3((unsigned)aeth_cdiv(n * w->nb, 256)), dim3(256), 0, s, staging, n,
                           w->nb, w->p3);
        const hipError_t le = hipGetLastError();
        if (le != hipSuccess) rc = aeth_set_error(AETH_EHIP, "aeth_weight_create: launch failed: %s", hipGetErrorString(le));
    }
    int special = 0;
    if (rc == AETH_OK) {
        hipError_t e2 = hipMemcpyAsync(&special, w->base + flag_off, sizeof(int), hipMemcpyDeviceToHost, s);
        if (e2 == hipSuccess) e2 = hipStreamSynchronize(s);
        if (e2 != hipSuccess)
            rc = aeth_set_error(AETH_EHIP, "aeth_weight_create: sync failed: %s", hipGetErrorString(e2));
    }
    w->special_scales = special;
    if (!raw_is_device) hipFree(staging);
    if (rc) {
        hipFree(w->base);
        delete w;
        return rc;
    }
    *out = w;
    return AETH_OK;
}

extern "C" AETH_API int aeth_weight_create(int dtype, int64_t n, int64_t k, const void* raw, int raw_is_device,
                                           void* stream, aeth_weight** out) {
    return aeth_weight_create_ex(dtype, aeth_dtype_fused(dtype) ? AETH_ORDER_PLANAR : AETH_ORDER_GGUF, n, k, raw,
                                 raw_is_device, (hipStream_t)stream, out);
}

extern "C" AETH_API int aeth_weight_free(aeth_weight* w) {
    if (!w) return AETH_OK;
    if (w->base) AETH_HIP_CHECK(hipFree(w->base));
    delete w;
    return AETH_OK;
}

extern "C" AETH_API int64_t aeth_weight_bytes(const aeth_weight* w) { return w ? w->bytes : 0; }

extern "C" AETH_API int aeth_weight_export_raw(const aeth_weight* w, void* dst, int dst_is_device, void* stream) {
    if (!w || !dst) return aeth_set_error(AETH_EINVAL, "aeth_weight_export_raw: NULL argument");
    hipStream_t s = (hipStream_t)stream;
    if (w->order != AETH_ORDER_PLANAR) {
        AETH_HIP_CHECK(hipMemcpyAsync(dst, w->base, (size_t)w->bytes,
                                      dst_is_device ? hipMemcpyDeviceToDevice : hipMemcpyDeviceToHost, s));
        if (!dst_is_device) AETH_HIP_CHECK(hipStreamSynchronize(s));
        return AETH_OK;
    }
    uint8_t* tmp = (uint8_t*)dst;
    if (!dst_is_device) AETH_HIP_CHECK(hipMalloc((void**)&tmp, (size_t)w->bytes));
    int rc = relayout((aeth_weight*)w, tmp, 0, s);
    if (!dst_is_device) {
        if (rc == AETH_OK) {
            hipError_t e = hipMemcpyAsync(dst, tmp, (size_t)w->bytes, hipMemcpyDeviceToHost, s);
            if (e == hipSuccess) e = hipStreamSynchronize(s);
            if (e != hipSuccess) rc = aeth_set_error(AETH_EHIP, "export copy failed: %s", hipGetErrorString(e));
        }
        hipFree(tmp);
    }
    return rc;
}

// ── seeded synthetic inputs ──────────────────────────────────────────────

__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// N(0,1) by Box-Muller from the counter (key, idx).
__device__ __forceinline__ float normal_at(uint64_t key, uint64_t idx) {
    uint64_t h1 = splitmix64(key ^ (idx * 2 + 0x51ull));
    uint64_t h2 = splitmix64(key ^ (idx * 2 + 0x52ull) ^ 0xD1B54A32D192ED03ull);
    float u1 = ((float)(h1 >> 40) + 1.0f) * (1.0f / 16777216.0f);  // (0, 1]
    float u2 = (float)(h2 >> 40) * (1.0f / 16777216.0f);           // [0, 1)
    return sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
}

__device__ __forceinline__ uint32_t scale_f16_bits(uint64_t key, uint64_t blk, int which) {
    float v = fabsf(normal_at(key ^ (0xABCDull + (uint64_t)which), blk)) * 0.01f;
    return (uint32_t)__half_as_ushort(__float2half_rn(v));
}

__global__ void k_fill_synthetic(int dtype, uint64_t seed, uint8_t* __restrict__ raw, int64_t total_bytes) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total_bytes) return;
    uint64_t key = splitmix64(seed);
    uint8_t v;
    if (dtype == AETH_DTYPE_Q4_K || dtype == AETH_DTYPE_Q5_K) {
        const int bb = dtype == AETH_DTYPE_Q4_K ? Q4K_BLOCK_BYTES : Q5K_BLOCK_BYTES;
        int64_t blk = i / bb;
        int off = (int)(i - blk * bb);
        if (off < 4) {
            uint32_t b = scale_f16_bits(key, (uint64_t)blk, off >> 1);
            v = (uint8_t)((off & 1) ? (b >> 8) : b);
        } else {
            v = (uint8_t)splitmix64(key ^ ((uint64_t)i * 0x9E37ull + 0x1234567ull));
        }
    } else if (dtype == AETH_DTYPE_Q2_K || dtype == AETH_DTYPE_Q3_K) {
        const int bb = dtype == AETH_DTYPE_Q2_K ? Q2K_BLOCK_BYTES : Q3K_BLOCK_BYTES;
        const int d0 = dtype == AETH_DTYPE_Q2_K ? 0 : 108;  // Q2_K: d, dmin lead; Q3_K: d last
        const int nd = dtype == AETH_DTYPE_Q2_K ? 4 : 2;
        int64_t blk = i / bb;
        int off = (int)(i - blk * bb);
        if (off >= d0 && off < d0 + nd) {
            uint32_t b = scale_f16_bits(key, (uint64_t)blk, (off - d0) >> 1);
            v = (uint8_t)(((off - d0) & 1) ? (b >> 8) : b);
        } else {
            v = (uint8_t)splitmix64(key ^ ((uint64_t)i * 0x9E37ull + 0x2718281ull));
        }
    } else if (dtype == AETH_DTYPE_F16 || dtype == AETH_DTYPE_F32) {
        const int eb = dtype == AETH_DTYPE_F16 ? 2 : 4;
        const int64_t el = i / eb;
        const float x = 0.02f * normal_at(key ^ 0xF16F32ull, (uint64_t)el);
        const uint32_t bits = dtype == AETH_DTYPE_F16 ? (uint32_t)__half_as_ushort(__float2half_rn(x)) : __float_as_uint(x);
        v = (uint8_t)(bits >> (8 * (int)(i - el * eb)));
    } else if (dtype == AETH_DTYPE_Q6_K) {
        int64_t blk = i / Q6K_BLOCK_BYTES;
        int off = (int)(i - blk * Q6K_BLOCK_BYTES);
        uint64_t h = splitmix64(key ^ ((uint64_t)i * 0x9E37ull + 0x7654321ull));
        if (off < 192) v = (uint8_t)h;
        else if (off < 208) v = (uint8_t)(int8_t)((int)(h & 127) - 64);
        else {
            uint32_t b = scale_f16_bits(key, (uint64_t)blk, 0);
            v = (uint8_t)((off & 1) ? (b >> 8) : b);
        }
    } else {
        int64_t blk = i / Q8_BLOCK_BYTES;
        int off = (int)(i - blk * Q8_BLOCK_BYTES);
        if (off < 2) {
            uint32_t b = scale_f16_bits(key, (uint64_t)blk, 0);
            v = (uint8_t)((off & 1) ? (b >> 8) : b);
        } else {
            uint64_t h = splitmix64(key ^ ((uint64_t)i * 0x9E37ull + 0x3141592ull));
            v = (uint8_t)(int8_t)((int)(h % 255ull) - 127);
        }
    }
    raw[i] = v;
}

extern "C" AETH_API int aeth_fill_synthetic_raw(int dtype, uint64_t seed, void* d_raw, int64_t n_blocks,
                                                void* stream) {
    int be, bb;
    int rc = aeth_block_geometry(dtype, &be, &bb);
    if (rc) return rc;
    if (!d_raw || n_blocks < 0) return aeth_set_error(AETH_EINVAL, "aeth_fill_synthetic_raw: bad argument");
    int64_t total = n_blocks * bb;
    if (total == 0) return AETH_OK;
    hipLaunchKernelGGL(k_fill_synthetic, dim3((unsigned)aeth_cdiv(total, 256)), dim3(256), 0,
                       (hipStream_t)stream, dtype, seed, (uint8_t*)d_raw, total);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}

__global__ void k_fill_normal(uint64_t seed, float* __restrict__ out, int64_t n, float mean, float stdv) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    out[i] = mean + stdv * normal_at(splitmix64(seed ^ 0x6E6F726D616CULL), (uint64_t)i);
}

extern "C" AETH_API int aeth_fill_normal_f32(uint64_t seed, float* d_out, int64_t n, float mean, float stdv,
                                             void* stream) {
    if (!d_out || n < 0) return aeth_set_error(AETH_EINVAL, "aeth_fill_normal_f32: bad argument");
    if (n == 0) return AETH_OK;
    hipLaunchKernelGGL(k_fill_normal, dim3((unsigned)aeth_cdiv(n, 256)), dim3(256), 0, (hipStream_t)stream, seed,
                       d_out, n, mean, stdv);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}

// ── measurement: a plain streaming read ──────────────────────────────────
// Reads every 16-byte word of [src, src + bytes) once (non-temporal loads,
// four in flight per thread before any is used) and folds them into one word
// per thread, stored only if it equals a value no input makes likely, so the
// loads cannot be dropped. The benchmark times it on the GEMV's weight copies:
// the HBM floor a single launch of that size can show. Shape (a sweep of 256 /
// 512 / 1024 threads, 4 / 8 / 16 loads per thread, 256 … 26307 workgroups,
// non-temporal or plain loads, measured on the headline's 33 MB and the LM
// head's 431 MB): 256 threads × 4 loads, one workgroup per 16 KiB up to 2048
// workgroups, else 512 workgroups looping over the buffer — 6.10 µs for 33 MB,
// 61.5 µs for 431 MB (7.0 TB/s); non-temporal loads beat plain ones by 4-9 %.
typedef uint32_t sr_u4 __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(256) k_stream_read(const sr_u4* __restrict__ src, int64_t n16,
                                                     uint32_t* __restrict__ sink) {
    constexpr int U = 4;
    const int64_t per_block = (int64_t)256 * U;
    uint32_t acc = 0;
    for (int64_t base = (int64_t)blockIdx.x * per_block; base < n16; base += (int64_t)gridDim.x * per_block) {
        sr_u4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int64_t i = base + (int64_t)u * 256 + threadIdx.x;
            v[u] = i < n16 ? __builtin_nontemporal_load(src + i) : sr_u4{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x9E3779B9u) sink[blockIdx.x * 256 + threadIdx.x] = acc;
}

extern "C" AETH_API int aeth_stream_read(const void* d_src, int64_t bytes, uint32_t* d_sink, int64_t sink_words,
                                         void* stream) {
    if (!d_src || !d_sink || bytes < 16 || (bytes & 15) || ((uintptr_t)d_src & 15))
        return aeth_set_error(AETH_EINVAL, "aeth_stream_read: bad argument");
    const int64_t n16 = bytes / 16, per_block = 256 * 4, full = aeth_cdiv(n16, per_block);
    const int64_t blocks = std::min<int64_t>(full <= 2048 ? full : 512, sink_words / 256);
    if (blocks <= 0) return aeth_set_error(AETH_EINVAL, "aeth_stream_read: sink of %lld words < 256",
                                           (long long)sink_words);
    hipLaunchKernelGGL(k_stream_read, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, (const sr_u4*)d_src,
                       n16, d_sink);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}

// Matrix-core rate of this GPU (measurement kernel): every wave issues `iters`
// rounds of 8 independent MFMAs — kind 0: v_mfma_f32_32x32x16_f16 (32768
// flops each), kind 1: v_mfma_i32_32x32x32_i8 (65536 ops each) — on register
// operands, one wave per SIMD (256 threads per workgroup). The MFMA peak the
// GEMM's fraction is quoted against, as the box sustains it.
typedef _Float16 mr_h8 __attribute__((ext_vector_type(8)));
typedef float mr_f16x __attribute__((ext_vector_type(16)));
typedef int mr_i16x __attribute__((ext_vector_type(16)));
typedef int mr_i4 __attribute__((ext_vector_type(4)));
template <int KIND>
__global__ void __launch_bounds__(256) k_mfma_rate(int iters, float* __restrict__ sink) {
    mr_h8 a, b;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        a[i] = (_Float16)(threadIdx.x * 0.001f + i);
        b[i] = (_Float16)(i * 0.5f);
    }
    const mr_i4 ai = {(int)threadIdx.x, 1, 2, 3}, bi = {3, 2, 1, (int)threadIdx.x};
    mr_f16x acc[8];
    mr_i16x iacc[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        acc[j] = (mr_f16x){};
        iacc[j] = (mr_i16x){};
    }
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            if (KIND == 0) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[j], 0, 0, 0);
            else iacc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ai, bi, iacc[j], 0, 0, 0);
        }
    }
    float t = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) t += acc[j][0] + (float)iacc[j][0];
    if (t == 12345.0f) sink[blockIdx.x * 256 + threadIdx.x] = t;
}

extern "C" AETH_API int aeth_mfma_rate(int kind, int iters, int workgroups, float* d_sink, void* stream) {
    if ((kind != 0 && kind != 1) || iters <= 0 || workgroups <= 0 || !d_sink)
        return aeth_set_error(AETH_EINVAL, "aeth_mfma_rate: bad argument");
    if (kind == 0)
        hipLaunchKernelGGL(k_mfma_rate<0>, dim3((unsigned)workgroups), dim3(256), 0, (hipStream_t)stream, iters, d_sink);
    else
        hipLaunchKernelGGL(k_mfma_rate<1>, dim3((unsigned)workgroups), dim3(256), 0, (hipStream_t)stream, iters, d_sink);
    AETH_LAUNCH_CHECK();
    return AETH_OK;
}
