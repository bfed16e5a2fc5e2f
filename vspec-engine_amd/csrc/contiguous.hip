// contiguous.hip -- the reference's contiguous-cache attention call
// (cpu_backend.c:40-51 -> attention_ref.c:7-88) served by the paged kernels.
//
// A VspecKVCache holds fp32 [T][H][D] in host memory (the fp32 mirror when the
// reference's int3 codec is on, kv_cache.c:198-215).  For head_dim 64 / 128 the rows are
// uploaded into a temporary f32 paged pool through the append kernel with an identity
// block table, and the decode kernel runs with Hq == Hkv (MHA); other head sizes run a
// generic one-workgroup-per-head kernel over the uploaded rows.
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

// Any head_dim: upload, one launch, download.
int attention_contig_host(const float* q, const float* key, const float* value, size_t tokens,
                          size_t heads, size_t head_dim, int32_t numerics, float* out) {
    const size_t kv_bytes = tokens * heads * head_dim * sizeof(float);
    const size_t q_bytes = heads * head_dim * sizeof(float);
    const size_t smem = (kThreads + head_dim) * sizeof(float);
    if (smem > 64 * 1024) {
        vspec_rocm_set_error_("attention: head_dim too large for the contiguous path");
        return 0;
    }
    void *d_k = nullptr, *d_v = nullptr, *d_q = nullptr, *d_o = nullptr, *d_s = nullptr;
    int ok = hipMalloc(&d_k, kv_bytes) == hipSuccess && hipMalloc(&d_v, kv_bytes) == hipSuccess &&
             hipMalloc(&d_q, q_bytes) == hipSuccess && hipMalloc(&d_o, q_bytes) == hipSuccess &&
             hipMalloc(&d_s, tokens * heads * sizeof(float)) == hipSuccess;
    ok = ok && hipMemcpy(d_k, key, kv_bytes, hipMemcpyHostToDevice) == hipSuccess &&
         hipMemcpy(d_v, value, kv_bytes, hipMemcpyHostToDevice) == hipSuccess &&
         hipMemcpy(d_q, q, q_bytes, hipMemcpyHostToDevice) == hipSuccess;
    if (!ok) vspec_rocm_set_error_("attention: device allocation or upload failed");
    if (ok) {
        const bool three = numerics == VSPEC_NUMERICS_3BIT;
        float scale = 1.0f / sqrtf((float)head_dim);
        if (three) scale = fminf(fmaxf(scale, 1e-4f), 32.0f);
        ContigParams p = {(const float*)d_q, (const float*)d_k, (const float*)d_v, (float*)d_o, (float*)d_s,
                          (uint32_t)tokens, (uint32_t)heads, (uint32_t)head_dim, scale * kLog2e, 4.5f,
                          three ? 24.0f * kLog2e : INFINITY, three ? 16.0f : INFINITY};
        hipLaunchKernelGGL(attention_contig, dim3((unsigned)heads), dim3(kThreads), smem, nullptr, p);
        ok = hipGetLastError() == hipSuccess && hipMemcpy(out, d_o, q_bytes, hipMemcpyDeviceToHost) == hipSuccess;
        if (!ok) vspec_rocm_set_error_("attention: launch or download failed");
    }
    (void)hipFree(d_k);
    (void)hipFree(d_v);
    (void)hipFree(d_q);
    (void)hipFree(d_o);
    (void)hipFree(d_s);
    return ok;
}

}  // namespace

extern "C" int vspec_rocm_attention_contiguous_host(const float* q, const float* key,
                                                    const float* value, size_t tokens, size_t heads,
                                                    size_t head_dim, int32_t numerics, float* out) {
    if (!q || !key || !value || !out || tokens == 0 || heads == 0) {
        vspec_rocm_set_error_("attention: bad arguments");
        return 0;
    }
    if (head_dim != 64 && head_dim != 128) {
        // other head sizes (the reference demo uses 4) take the generic kernel
        if (tokens > (size_t)UINT32_MAX || heads > (size_t)UINT32_MAX) {
            vspec_rocm_set_error_("attention: cache too large");
            return 0;
        }
        return attention_contig_host(q, key, value, tokens, heads, head_dim, numerics, out);
    }
    if (tokens > (size_t)INT32_MAX / 2) {
        vspec_rocm_set_error_("attention: too many tokens");
        return 0;
    }
    const uint32_t P = 16;
    const uint32_t nblk = (uint32_t)((tokens + P - 1) / P);
    VspecPagedKV kv;
    if (!vspec_rocm_kv_pool_create(&kv, VSPEC_KV_F32, nblk, P, (uint32_t)heads, (uint32_t)head_dim)) {
        return 0;
    }
    const size_t kv_bytes = tokens * heads * head_dim * sizeof(float);
    const size_t q_bytes = heads * head_dim * sizeof(float);
    int32_t* h_tab = (int32_t*)malloc(nblk * sizeof(int32_t));
    void *d_k = nullptr, *d_v = nullptr, *d_q = nullptr, *d_o = nullptr, *d_tab = nullptr, *d_misc = nullptr;
    int ok = h_tab != nullptr;
    if (ok) {
        for (uint32_t i = 0; i < nblk; ++i) h_tab[i] = (int32_t)i;
    }
    ok = ok && hipMalloc(&d_k, kv_bytes) == hipSuccess && hipMalloc(&d_v, kv_bytes) == hipSuccess &&
         hipMalloc(&d_q, q_bytes) == hipSuccess && hipMalloc(&d_o, q_bytes) == hipSuccess &&
         hipMalloc(&d_tab, nblk * sizeof(int32_t)) == hipSuccess &&
         hipMalloc(&d_misc, 2 * sizeof(int32_t)) == hipSuccess;
    int32_t misc[2] = {0, (int32_t)tokens};  // start_pos, ctx_len
    ok = ok && hipMemcpy(d_k, key, kv_bytes, hipMemcpyHostToDevice) == hipSuccess &&
         hipMemcpy(d_v, value, kv_bytes, hipMemcpyHostToDevice) == hipSuccess &&
         hipMemcpy(d_q, q, q_bytes, hipMemcpyHostToDevice) == hipSuccess &&
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
    (void)hipFree(d_k);
    (void)hipFree(d_v);
    (void)hipFree(d_q);
    (void)hipFree(d_o);
    (void)hipFree(d_tab);
    (void)hipFree(d_misc);
    free(h_tab);
    vspec_rocm_kv_pool_destroy(&kv);
    return ok;
}
