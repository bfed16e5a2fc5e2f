// contiguous.hip -- the reference's contiguous-cache attention call
// (cpu_backend.c:40-51 -> attention_ref.c:7-88) served by the paged kernels.
//
// A VspecKVCache holds fp32 [T][H][D] in host memory (the fp32 mirror when the
// reference's int3 codec is on, kv_cache.c:198-215).  The rows are uploaded into a
// temporary f32 paged pool through the append kernel with an identity block table,
// and the decode kernel runs with Hq == Hkv (MHA).
#include <hip/hip_runtime.h>

#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "vspec_rocm.h"

extern "C" void vspec_rocm_set_error_(const char* msg);

extern "C" int vspec_rocm_attention_contiguous_host(const float* q, const float* key,
                                                    const float* value, size_t tokens, size_t heads,
                                                    size_t head_dim, int32_t numerics, float* out) {
    if (!q || !key || !value || !out || tokens == 0 || heads == 0) {
        vspec_rocm_set_error_("attention: bad arguments");
        return 0;
    }
    if (head_dim != 64 && head_dim != 128) {
        vspec_rocm_set_error_("attention: head_dim must be 64 or 128 on the ROCm backend");
        return 0;
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
