// contiguous.hip -- the reference's contiguous-cache attention call
// (cpu_backend.c:40-51 -> attention_ref.c:7-88) served by the paged kernels.
//
// A VspecKVCache holds [T][H][D] keys and values in host memory: fp32 rows (also the fp32
// mirror when the reference's int3 codec is on, kv_cache.c:198-215), or, for a cache whose
// codec runs without a mirror, 3-bit codes with per-block fp32 scales that the reference's
// accessors decode on every read (kv_cache.c:296-362).  Rows are uploaded as they are;
// codes and scales are uploaded and decoded to fp32 on the device, bit for bit as the
// reference decodes them.  For head_dim 64 / 128 the rows then go through the append
// kernel into a temporary f32 paged pool with an identity block table and the decode
// kernel runs with Hq == Hkv (MHA); other head sizes run a generic
// one-workgroup-per-head kernel over the rows.
#include <hip/hip_runtime.h>

#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "vspec_rocm.h"

extern "C" void vspec_rocm_set_error_(const char* msg);

namespace {

constexpr int kThreads = 256;
constexpr float kLog2e = 1.4426950408889634f;

struct ContigParams {
    const float* q;    // [H][D]
    const float* k;    // [T][H][D]
    const float* v;    // [T][H][D]
    float* out;        // [H][D]
    float* scores;     // [H][T] scratch
    uint32_t tokens, heads, head_dim;
    float qscale;      // softmax scale * log2(e)
    float alpha;       // std-clamp alpha
    float logit_clip;  // +-24*log2(e) in 3-bit mode, +inf otherwise
    float input_clip;  // 16 in 3-bit mode, +inf otherwise
};

__device__ float block_sum(float x, float* red) {
    red[threadIdx.x] = x;
    __syncthreads();
    for (int s = kThreads / 2; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
        __syncthreads();
    }
    const float r = red[0];
    __syncthreads();
    return r;
}

__device__ float block_max(float x, float* red) {
    red[threadIdx.x] = x;
    __syncthreads();
    for (int s = kThreads / 2; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + s]);
        __syncthreads();
    }
    const float r = red[0];
    __syncthreads();
    return r;
}

// Attention of one head over a contiguous [T][H][D] fp32 cache for any head_dim: the
// reference single-query path (attention_ref.c:7-88) with its std clamp of q and of every
// key (three_bit_runtime_modules.c:175-203) and the 3-bit clips.  One workgroup per head;
// threads take keys for the scores and output elements for P.V.
__global__ __launch_bounds__(kThreads) void attention_contig(ContigParams p) {
    extern __shared__ float sm[];
    float* red = sm;                // [kThreads]
    float* qs = sm + kThreads;      // [D]
    const uint32_t h = blockIdx.x, D = p.head_dim, T = p.tokens, H = p.heads;
    const float* qrow = p.q + (size_t)h * D;

    float part = 0.f;
    for (uint32_t d = threadIdx.x; d < D; d += kThreads) part += qrow[d];
    const float qmean = block_sum(part, red) / (float)D;
    part = 0.f;
    for (uint32_t d = threadIdx.x; d < D; d += kThreads) part = fmaf(qrow[d] - qmean, qrow[d] - qmean, part);
    const float qth = fminf(fmaxf(1e-6f, p.alpha * sqrtf(block_sum(part, red) / (float)D)), p.input_clip);
    for (uint32_t d = threadIdx.x; d < D; d += kThreads) qs[d] = fminf(fmaxf(qrow[d], -qth), qth) * p.qscale;
    __syncthreads();

    float* sc = p.scores + (size_t)h * T;
    float mx = -INFINITY;
    for (uint32_t t = threadIdx.x; t < T; t += kThreads) {
        const float* k = p.k + ((size_t)t * H + h) * D;
        float m = 0.f;
        for (uint32_t d = 0; d < D; ++d) m += k[d];
        m /= (float)D;
        float var = 0.f;
        for (uint32_t d = 0; d < D; ++d) var = fmaf(k[d] - m, k[d] - m, var);
        const float th = fminf(fmaxf(1e-6f, p.alpha * sqrtf(var / (float)D)), p.input_clip);
        float dot = 0.f;
        for (uint32_t d = 0; d < D; ++d) dot = fmaf(qs[d], fminf(fmaxf(k[d], -th), th), dot);
        const float s = fminf(fmaxf(dot, -p.logit_clip), p.logit_clip);
        sc[t] = s;
        mx = fmaxf(mx, s);
    }
    const float M = block_max(mx, red);
    float l = 0.f;
    for (uint32_t t = threadIdx.x; t < T; t += kThreads) {
        const float e = exp2f(sc[t] - M);
        sc[t] = e;
        l += e;
    }
    const float L = block_sum(l, red);  // the barriers in the sum also publish sc[]
    for (uint32_t d = threadIdx.x; d < D; d += kThreads) {
        float a = 0.f;
        for (uint32_t t = 0; t < T; ++t) a = fmaf(sc[t], p.v[((size_t)t * H + h) * D + d], a);
        p.out[(size_t)h * D + d] = L > 0.f ? a / L : 0.f;
    }
}

// int3 rows to fp32: the reference's dequantize_head_int3 (kv_cache.c:109-126) with the
// bit reader of pack.c:56-76 -- 3-bit two's-complement codes packed LSB first, a code
// that starts at bit 6 or 7 of a byte continuing into the next one -- times the scale of
// its block of block_size elements.  Row r = token * heads + head has its codes at
// r * packed_head_bytes and its scales at r * blocks_per_head, as the cache stores them.
struct Int3Rows {
    const uint8_t* codes;
    const float* scales;
    float* out;  // [rows][head_dim]
    size_t rows, packed_head_bytes, blocks_per_head;
    uint32_t head_dim, block_size;
};

__global__ __launch_bounds__(kThreads) void int3_rows_to_f32(Int3Rows p) {
    const size_t n = p.rows * p.head_dim;
    const size_t step = (size_t)gridDim.x * kThreads;
    for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += step) {
        const size_t r = i / p.head_dim;
        const uint32_t e = (uint32_t)(i - r * p.head_dim);
        const uint8_t* c = p.codes + r * p.packed_head_bytes;
        const uint32_t bit = e * 3u, at = bit >> 3, sh = bit & 7u;
        uint32_t code = (uint32_t)c[at] >> sh;
        if (sh > 5u) code |= (uint32_t)c[at + 1] << (8u - sh);
        code &= 7u;
        const int qv = (code & 4u) ? (int)code - 8 : (int)code;
        p.out[i] = (float)qv * p.scales[r * p.blocks_per_head + e / p.block_size];
    }
}

// Attention over [T][H][D] fp32 rows already in device memory, q and out in host memory.
// head_dim 64 / 128: the rows go through the append kernel into a temporary f32 paged
// pool (identity block table) and the decode kernel runs with Hq == Hkv; other head sizes
// take the generic kernel above.
int attention_rows(const float* q, const float* d_k, const float* d_v, size_t tokens, size_t heads,
                   size_t head_dim, int32_t numerics, float* out) {
    const size_t q_bytes = heads * head_dim * sizeof(float);
    if (head_dim != 64 && head_dim != 128) {
        void *d_q = nullptr, *d_o = nullptr, *d_s = nullptr;
        int ok = hipMalloc(&d_q, q_bytes) == hipSuccess && hipMalloc(&d_o, q_bytes) == hipSuccess &&
                 hipMalloc(&d_s, tokens * heads * sizeof(float)) == hipSuccess &&
                 hipMemcpy(d_q, q, q_bytes, hipMemcpyHostToDevice) == hipSuccess;
        if (!ok) vspec_rocm_set_error_("attention: device allocation or upload failed");
        if (ok) {
            const bool three = numerics == VSPEC_NUMERICS_3BIT;
            float scale = 1.0f / sqrtf((float)head_dim);
            if (three) scale = fminf(fmaxf(scale, 1e-4f), 32.0f);
            ContigParams p = {(const float*)d_q, d_k, d_v, (float*)d_o, (float*)d_s,
                              (uint32_t)tokens, (uint32_t)heads, (uint32_t)head_dim, scale * kLog2e, 4.5f,
                              three ? 24.0f * kLog2e : INFINITY, three ? 16.0f : INFINITY};
            const size_t smem = (kThreads + head_dim) * sizeof(float);
            hipLaunchKernelGGL(attention_contig, dim3((unsigned)heads), dim3(kThreads), smem, nullptr, p);
            ok = hipGetLastError() == hipSuccess &&
                 hipMemcpy(out, d_o, q_bytes, hipMemcpyDeviceToHost) == hipSuccess;
            if (!ok) vspec_rocm_set_error_("attention: launch or download failed");
        }
        (void)hipFree(d_q);
        (void)hipFree(d_o);
        (void)hipFree(d_s);
        return ok;
    }
    const uint32_t P = 16;
    const uint32_t nblk = (uint32_t)((tokens + P - 1) / P);
    VspecPagedKV kv;
    if (!vspec_rocm_kv_pool_create(&kv, VSPEC_KV_F32, nblk, P, (uint32_t)heads, (uint32_t)head_dim)) {
        return 0;
    }
    int32_t* h_tab = (int32_t*)malloc(nblk * sizeof(int32_t));
    void *d_q = nullptr, *d_o = nullptr, *d_tab = nullptr, *d_misc = nullptr;
    int ok = h_tab != nullptr;
    if (ok) {
        for (uint32_t i = 0; i < nblk; ++i) h_tab[i] = (int32_t)i;
    }
    ok = ok && hipMalloc(&d_q, q_bytes) == hipSuccess && hipMalloc(&d_o, q_bytes) == hipSuccess &&
         hipMalloc(&d_tab, nblk * sizeof(int32_t)) == hipSuccess &&
         hipMalloc(&d_misc, 2 * sizeof(int32_t)) == hipSuccess;
    int32_t misc[2] = {0, (int32_t)tokens};  // start_pos, ctx_len
    ok = ok && hipMemcpy(d_q, q, q_bytes, hipMemcpyHostToDevice) == hipSuccess &&
         hipMemcpy(d_tab, h_tab, nblk * sizeof(int32_t), hipMemcpyHostToDevice) == hipSuccess &&
         hipMemcpy(d_misc, misc, sizeof(misc), hipMemcpyHostToDevice) == hipSuccess;
    if (!ok) vspec_rocm_set_error_("attention: device allocation or upload failed");
    ok = ok && vspec_rocm_kv_append(&kv, 1, (const int32_t*)d_tab, nblk, (const int32_t*)d_misc,
                                    (uint32_t)tokens, d_k, d_v, VSPEC_KV_F32, nullptr);
    if (ok) {
        VspecPagedAttnDesc d;
        memset(&d, 0, sizeof(d));
        d.kv = kv;
        d.batch = 1;
        d.num_q_heads = (uint32_t)heads;
        d.block_tables = (const int32_t*)d_tab;
        d.max_blocks_per_seq = nblk;
        d.ctx_lens = (const int32_t*)d_misc + 1;
        d.max_ctx_len = (uint32_t)tokens;
        d.q = (const float*)d_q;
        d.out = (float*)d_o;
        d.numerics = numerics;
        ok = vspec_rocm_paged_decode_attention(&d);
    }
    if (ok && hipMemcpy(out, d_o, q_bytes, hipMemcpyDeviceToHost) != hipSuccess) {
        vspec_rocm_set_error_("attention: download failed");
        ok = 0;
    }
    (void)hipFree(d_q);
    (void)hipFree(d_o);
    (void)hipFree(d_tab);
    (void)hipFree(d_misc);
    free(h_tab);
    vspec_rocm_kv_pool_destroy(&kv);
    return ok;
}

// Where the reference's accessors read one side (key or value) of a cache from
// (kv_cache.c:296-362): the fp32 rows whenever they exist (the plain cache, or the int3
// codec's fp32 mirror), otherwise the int3 codes and scales when the codec is on.
struct CacheSide {
    const float* rows;
    const uint8_t* codes;
    const float* scales;
};

CacheSide cache_side(const VspecKVCache* c, bool value) {
    CacheSide s = {value ? c->value : c->key, nullptr, nullptr};
    if (!s.rows && c->int3_compressed) {
        s.codes = value ? c->value_int3 : c->key_int3;
        s.scales = value ? c->value_scales : c->key_scales;
    }
    return s;
}

// One side of the cache as device fp32 rows: an upload of the rows, or an upload of the
// codes and scales followed by the decode kernel.
int side_to_device(const VspecKVCache* c, const CacheSide& s, float* d_rows) {
    const size_t tokens = c->current_tokens, rows = tokens * c->num_heads;
    if (s.rows) {
        if (hipMemcpy(d_rows, s.rows, rows * c->head_dim * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) {
            vspec_rocm_set_error_("attention: upload of the cache rows failed");
            return 0;
        }
        return 1;
    }
    const size_t code_bytes = rows * c->packed_head_bytes;
    const size_t scale_bytes = rows * c->blocks_per_head * sizeof(float);
    void *d_codes = nullptr, *d_scales = nullptr;
    int ok = hipMalloc(&d_codes, code_bytes) == hipSuccess && hipMalloc(&d_scales, scale_bytes) == hipSuccess &&
             hipMemcpy(d_codes, s.codes, code_bytes, hipMemcpyHostToDevice) == hipSuccess &&
             hipMemcpy(d_scales, s.scales, scale_bytes, hipMemcpyHostToDevice) == hipSuccess;
    if (!ok) vspec_rocm_set_error_("attention: upload of the int3 codes failed");
    if (ok) {
        Int3Rows p = {(const uint8_t*)d_codes, (const float*)d_scales, d_rows, rows, c->packed_head_bytes,
                      c->blocks_per_head, (uint32_t)c->head_dim, (uint32_t)c->block_size};
        const size_t n = rows * c->head_dim;
        const unsigned grid = (unsigned)((n + kThreads - 1) / kThreads < 8192 ? (n + kThreads - 1) / kThreads : 8192);
        hipLaunchKernelGGL(int3_rows_to_f32, dim3(grid), dim3(kThreads), 0, nullptr, p);
        ok = hipGetLastError() == hipSuccess && hipStreamSynchronize(nullptr) == hipSuccess;
        if (!ok) vspec_rocm_set_error_("attention: int3 decode failed");
    }
    (void)hipFree(d_codes);
    (void)hipFree(d_scales);
    return ok;
}

}  // namespace

extern "C" int vspec_rocm_attention_cache_host(const float* q, const VspecKVCache* cache,
                                               int32_t numerics, float* out) {
    if (!q || !cache || !out || cache->current_tokens == 0 || cache->num_heads == 0 || cache->head_dim == 0) {
        vspec_rocm_set_error_("attention: bad arguments");
        return 0;
    }
    const size_t tokens = cache->current_tokens, heads = cache->num_heads, head_dim = cache->head_dim;
    const CacheSide ks = cache_side(cache, false), vs = cache_side(cache, true);
    if ((!ks.rows && (!ks.codes || !ks.scales)) || (!vs.rows && (!vs.codes || !vs.scales))) {
        vspec_rocm_set_error_("attention: cache has neither fp32 rows nor int3 codes with scales");
        return 0;
    }
    if (!ks.rows || !vs.rows) {
        const size_t bs = cache->block_size;
        if (bs == 0 || head_dim > UINT32_MAX || bs > UINT32_MAX ||
            cache->blocks_per_head < (head_dim + bs - 1) / bs ||
            cache->packed_head_bytes < (3 * head_dim + 7) / 8) {
            vspec_rocm_set_error_("attention: int3 cache geometry (block_size, blocks_per_head, "
                                  "packed_head_bytes) does not cover head_dim");
            return 0;
        }
    }
    if (head_dim == 64 || head_dim == 128) {
        if (tokens > (size_t)INT32_MAX / 2 || heads > (size_t)UINT32_MAX) {
            vspec_rocm_set_error_("attention: too many tokens");
            return 0;
        }
    } else {
        // other head sizes (the reference demo uses 4) take the generic kernel
        if (tokens > (size_t)UINT32_MAX || heads > (size_t)UINT32_MAX) {
            vspec_rocm_set_error_("attention: cache too large");
            return 0;
        }
        if ((kThreads + head_dim) * sizeof(float) > 64 * 1024) {
            vspec_rocm_set_error_("attention: head_dim too large for the contiguous path");
            return 0;
        }
    }
    const size_t kv_bytes = tokens * heads * head_dim * sizeof(float);
    void *d_k = nullptr, *d_v = nullptr;
    int ok = hipMalloc(&d_k, kv_bytes) == hipSuccess && hipMalloc(&d_v, kv_bytes) == hipSuccess;
    if (!ok) vspec_rocm_set_error_("attention: device allocation failed");
    ok = ok && side_to_device(cache, ks, (float*)d_k) && side_to_device(cache, vs, (float*)d_v) &&
         attention_rows(q, (const float*)d_k, (const float*)d_v, tokens, heads, head_dim, numerics, out);
    (void)hipFree(d_k);
    (void)hipFree(d_v);
    return ok;
}
