// py_handles.hip -- the paged-KV section of the reference Python C-API
// (capi.h:46-57, capi.c:2188-2299) over an HBM pool.
//
// Handle ids are 1..16 as in the reference (capi.c:29, :135-143).  Page placement is
// decided by VspecRocmPagedMeta (the reference allocator policy); token data lives in
// an f32 VspecPagedKV pool and moves with the append and row-gather kernels.  Calls are
// synchronous with respect to the host, like the reference functions they replace.
// The reference accepts any head_dim; the pool's rows are padded to a multiple of 8
// floats (the append kernel's vector width) and the padding never reaches the caller.
#include <hip/hip_runtime.h>

#include <stdlib.h>
#include <string.h>

#include "vspec_rocm_paged.h"

extern "C" void vspec_rocm_set_error_(const char* msg);

namespace {

constexpr int kMaxHandles = 16;

struct Handle {
    int active = 0;
    size_t page_tokens = 0, max_pages = 0, num_heads = 0, head_dim = 0;
    size_t pool_dim = 0;  // head_dim rounded up to a multiple of 8
    float* host_row = nullptr;  // padded [H][pool_dim] K then V staging on the host
    VspecRocmPagedMeta* meta = nullptr;
    VspecPagedKV pool{};
    // grow-only device staging: [page, slot] + K + V for appends; row lists + outputs for reads
    void* stage = nullptr;
    size_t stage_bytes = 0;
};

Handle g_handles[kMaxHandles];

Handle* get(int id) {
    if (id <= 0 || id > kMaxHandles) return nullptr;
    return g_handles[id - 1].active ? &g_handles[id - 1] : nullptr;
}

void* stage(Handle* h, size_t bytes) {
    if (h->stage_bytes >= bytes) return h->stage;
    if (h->stage) (void)hipFree(h->stage);
    h->stage = nullptr;
    h->stage_bytes = 0;
    if (hipMalloc(&h->stage, bytes) != hipSuccess) return nullptr;
    h->stage_bytes = bytes;
    return h->stage;
}

void release(Handle* h) {
    if (h->stage) (void)hipFree(h->stage);
    free(h->host_row);
    vspec_rocm_kv_pool_destroy(&h->pool);
    vspec_rocm_paged_meta_destroy(h->meta);
    *h = Handle();
}

// [n][H][pool_dim] device rows -> [n][H][head_dim] host rows
bool download(const Handle* h, float* dst, const void* src, size_t n) {
    const size_t rows = n * h->num_heads;
    if (h->pool_dim == h->head_dim) {
        return hipMemcpy(dst, src, rows * h->head_dim * sizeof(float), hipMemcpyDeviceToHost) == hipSuccess;
    }
    return hipMemcpy2D(dst, h->head_dim * sizeof(float), src, h->pool_dim * sizeof(float),
                       h->head_dim * sizeof(float), rows, hipMemcpyDeviceToHost) == hipSuccess;
}

}  // namespace

extern "C" {

int vspec_py_kv_cache_create(size_t page_tokens, size_t max_pages, size_t num_heads, size_t head_dim) {
    if (page_tokens == 0 || max_pages == 0 || num_heads == 0 || head_dim == 0 ||
        page_tokens > UINT32_MAX || max_pages > UINT32_MAX || num_heads > UINT32_MAX ||
        head_dim > UINT32_MAX) {
        vspec_rocm_set_error_("kv_cache_create: bad geometry");
        return 0;
    }
    for (int i = 0; i < kMaxHandles; ++i) {
        Handle* h = &g_handles[i];
        if (h->active) continue;
        *h = Handle();
        h->pool_dim = (head_dim + 7) / 8 * 8;
        h->meta = vspec_rocm_paged_meta_create(page_tokens, max_pages, 0, 0);
        h->host_row = (float*)calloc(2 * num_heads * h->pool_dim, sizeof(float));
        if (!h->meta || !h->host_row ||
            !vspec_rocm_kv_pool_create(&h->pool, VSPEC_KV_F32, (uint32_t)max_pages,
                                       (uint32_t)page_tokens, (uint32_t)num_heads,
                                       (uint32_t)h->pool_dim)) {
            release(h);
            return 0;
        }
        h->page_tokens = page_tokens;
        h->max_pages = max_pages;
        h->num_heads = num_heads;
        h->head_dim = head_dim;
        h->active = 1;
        return i + 1;
    }
    vspec_rocm_set_error_("kv_cache_create: all 16 handles in use");
    return 0;
}

void vspec_py_kv_cache_destroy(int handle_id) {
    Handle* h = get(handle_id);
    if (h) release(h);
}

int vspec_py_kv_cache_reset(int handle_id) {
    Handle* h = get(handle_id);
    if (!h) return 0;
    vspec_rocm_paged_meta_reset(h->meta);  // token data is left in place, as in capi.c
    return 1;
}

int vspec_py_kv_cache_append(int handle_id, uint64_t session_id, const float* key_token,
                             const float* value_token) {
    Handle* h = get(handle_id);
    if (!h || !key_token || !value_token) return 0;
    uint32_t page = 0, slot = 0;
    if (!vspec_rocm_paged_reserve(h->meta, session_id, &page, &slot)) return 0;
    const size_t row = h->num_heads * h->pool_dim * sizeof(float);
    char* d = (char*)stage(h, 256 + 2 * row);
    if (!d) {
        vspec_rocm_set_error_("kv_cache_append: staging allocation failed");
        return 0;
    }
    const int32_t idx[2] = {(int32_t)page, (int32_t)slot};
    const float* src_k = key_token;
    const float* src_v = value_token;
    if (h->pool_dim != h->head_dim) {  // pad each head's row with zeros
        float* pk = h->host_row;
        float* pv = h->host_row + h->num_heads * h->pool_dim;
        for (size_t i = 0; i < h->num_heads; ++i) {
            memcpy(pk + i * h->pool_dim, key_token + i * h->head_dim, h->head_dim * sizeof(float));
            memcpy(pv + i * h->pool_dim, value_token + i * h->head_dim, h->head_dim * sizeof(float));
        }
        src_k = pk;
        src_v = pv;
    }
    if (hipMemcpy(d, idx, sizeof(idx), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(d + 256, src_k, row, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(d + 256 + row, src_v, row, hipMemcpyHostToDevice) != hipSuccess) {
        vspec_rocm_set_error_("kv_cache_append: upload failed");
        return 0;
    }
    // one token at slot `slot` of page `page`: a one-entry block table and start position
    if (!vspec_rocm_kv_append(&h->pool, 1, (const int32_t*)d, 1, (const int32_t*)d + 1, 1, d + 256,
                              d + 256 + row, VSPEC_KV_F32, nullptr)) {
        return 0;
    }
    return hipStreamSynchronize(nullptr) == hipSuccess ? 1 : 0;
}

size_t vspec_py_kv_cache_session_tokens(int handle_id, uint64_t session_id) {
    Handle* h = get(handle_id);
    return h ? vspec_rocm_paged_session_tokens(h->meta, session_id) : 0u;
}

size_t vspec_py_kv_cache_read(int handle_id, uint64_t session_id, float* out_keys,
                              float* out_values, size_t max_tokens) {
    Handle* h = get(handle_id);
    if (!h || !out_keys || !out_values) return 0u;
    size_t total = vspec_rocm_paged_session_tokens(h->meta, session_id);
    if (max_tokens > 0u && total > max_tokens) total = max_tokens;
    if (total == 0u) return 0u;
    if (total > (size_t)INT32_MAX) return 0u;
    // token -> (page, slot) in one walk of the page list (get_token_ptr's walk, :335-347)
    int32_t* rows = (int32_t*)malloc(2 * total * sizeof(int32_t));
    const size_t npages = vspec_rocm_paged_session_pages(h->meta, session_id, nullptr, 0);
    uint32_t* pages = (uint32_t*)malloc((npages ? npages : 1) * sizeof(uint32_t));
    if (!rows || !pages) {
        free(rows);
        free(pages);
        return 0u;
    }
    vspec_rocm_paged_session_pages(h->meta, session_id, pages, npages);
    size_t t = 0;
    for (size_t i = 0; i < npages && t < total; ++i) {
        uint32_t allocated = 0, used = 0, refc = 0;
        vspec_rocm_paged_page_info(h->meta, pages[i], &allocated, &used, &refc);
        for (uint32_t s = 0; s < used && t < total; ++s, ++t) {
            rows[t] = (int32_t)pages[i];
            rows[total + t] = (int32_t)s;
        }
    }
    // tokens a walk cannot reach read page 0, slot 0 (:333-334)
    for (; t < total; ++t) {
        rows[t] = 0;
        rows[total + t] = 0;
    }
    free(pages);
    const size_t out_bytes = total * h->num_heads * h->pool_dim * sizeof(float);
    const size_t idx_bytes = (2 * total * sizeof(int32_t) + 255) / 256 * 256;
    char* d = (char*)stage(h, idx_bytes + 2 * out_bytes);
    size_t copied = 0u;
    if (d && hipMemcpy(d, rows, 2 * total * sizeof(int32_t), hipMemcpyHostToDevice) == hipSuccess &&
        vspec_rocm_kv_gather_rows(&h->pool, (uint32_t)total, (const int32_t*)d, (const int32_t*)d + total,
                                  (float*)(d + idx_bytes), (float*)(d + idx_bytes + out_bytes), nullptr) &&
        download(h, out_keys, d + idx_bytes, total) && download(h, out_values, d + idx_bytes + out_bytes, total)) {
        copied = total;
    } else {
        vspec_rocm_set_error_("kv_cache_read: device gather failed");
    }
    free(rows);
    return copied;
}

VspecRocmPagedMeta* vspec_py_kv_cache_meta(int handle_id) {
    Handle* h = get(handle_id);
    return h ? h->meta : nullptr;
}

const VspecPagedKV* vspec_py_kv_cache_pool(int handle_id) {
    Handle* h = get(handle_id);
    return h ? &h->pool : nullptr;
}

}  // extern "C"
