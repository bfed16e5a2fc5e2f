/*
 * vspec_rocm_paged.h -- session/page bookkeeping of the paged KV cache and the
 * GPU-resident handle API that Vspec's Python runtime binds with ctypes.
 *
 * 1. VspecRocmPagedMeta: the reference allocator (kv_paged_cache.c) restated on the
 *    host with its exact policy -- first-fit page allocation, whole-session LRU
 *    eviction on exhaustion, reference-counted prefix sharing, per-page used counts,
 *    the clock -- but with the caps lifted (page ids are uint32, limits are chosen at
 *    creation; 0 selects the reference's 128 sessions / 1024 pages per session).
 *    It only decides where tokens live; the data lives in a VspecPagedKV pool.
 *
 * 2. vspec_py_kv_cache_*: the paged-KV section of the reference's Python C-API
 *    (capi.h:46-57, capi.c:2188-2299) with identical signatures, backed by an HBM f32
 *    pool.  A ctypes loader that points at libvspec_rocm.so instead of
 *    libvspec_engine_capi runs CorePagedKVCache (runtime_core_bridge.py:479-549)
 *    unchanged.
 */
#ifndef VSPEC_ROCM_PAGED_H
#define VSPEC_ROCM_PAGED_H

#include <stddef.h>
#include <stdint.h>

#include "vspec_rocm.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Same fields and order as VspecKVPagedStats (kv_paged_cache.h:11-18). */
typedef struct VspecRocmPagedStats {
    uint64_t page_alloc_count;
    uint64_t page_reuse_count;
    uint64_t evict_session_count;
    uint64_t append_token_count;
    size_t free_pages;
    size_t active_sessions;
} VspecRocmPagedStats;

typedef struct VspecRocmPagedMeta VspecRocmPagedMeta; /* opaque */

/* vspec_kv_paged_cache_init (kv_paged_cache.c:124-149); returns NULL on bad arguments. */
VspecRocmPagedMeta* vspec_rocm_paged_meta_create(size_t page_tokens, size_t max_pages,
                                                 size_t max_sessions,
                                                 size_t max_pages_per_session);
void vspec_rocm_paged_meta_destroy(VspecRocmPagedMeta* m);
/* Back to the state right after creation (capi.c:2237-2245 reset). */
void vspec_rocm_paged_meta_reset(VspecRocmPagedMeta* m);

int vspec_rocm_paged_open_session(VspecRocmPagedMeta* m, uint64_t session_id);   /* :151-174 */
int vspec_rocm_paged_close_session(VspecRocmPagedMeta* m, uint64_t session_id);  /* :176-183 */
int vspec_rocm_paged_reuse_prefix(VspecRocmPagedMeta* m, uint64_t target_session_id,
                                  uint64_t source_session_id, size_t max_tokens);  /* :185-241 */
/* The bookkeeping of vspec_kv_paged_append (:243-310): reserves the next token of the
 * session and returns its physical page and slot; the caller writes the data. */
int vspec_rocm_paged_reserve(VspecRocmPagedMeta* m, uint64_t session_id, uint32_t* page,
                             uint32_t* slot);
/* vspec_kv_paged_get_token_ptr addressing (:312-356): page and slot of token_idx. */
int vspec_rocm_paged_locate(const VspecRocmPagedMeta* m, uint64_t session_id, size_t token_idx,
                            uint32_t* page, uint32_t* slot);
size_t vspec_rocm_paged_session_tokens(const VspecRocmPagedMeta* m, uint64_t session_id);
void vspec_rocm_paged_stats(const VspecRocmPagedMeta* m, VspecRocmPagedStats* out);  /* :366-384 */
/* The session's page list (physical page ids in order); returns the page count. */
size_t vspec_rocm_paged_session_pages(const VspecRocmPagedMeta* m, uint64_t session_id,
                                      uint32_t* out, size_t cap);
/* Page metadata: allocated flag, used tokens, reference count. */
int vspec_rocm_paged_page_info(const VspecRocmPagedMeta* m, size_t page, uint32_t* allocated,
                               uint32_t* used_tokens, uint32_t* ref_count);
/* Block table for the decode kernel: pages in order when every page but the last is
 * full (then *ctx_len = session tokens); returns 0 otherwise (prefix reuse left a
 * partly filled page in the middle: use vspec_rocm_paged_block_layout). */
int vspec_rocm_paged_block_table(const VspecRocmPagedMeta* m, uint64_t session_id, int32_t* out,
                                 size_t cap, uint32_t* ctx_len);
/* Any session as the decode kernel's (block table, block_used, span): blocks[i] = the
 * i-th page, used[i] = its used tokens (the counts get_token_ptr walks,
 * kv_paged_cache.c:335-347), *span = (pages - 1) * page_tokens + last page's used count
 * (the ctx_lens entry when VspecPagedAttnDesc.block_used is set), *tokens = the
 * session's token count.  Returns 0 for an unknown session or cap < pages. */
int vspec_rocm_paged_block_layout(const VspecRocmPagedMeta* m, uint64_t session_id, int32_t* blocks,
                                  int32_t* used, size_t cap, uint32_t* span, uint32_t* tokens);

/* A continuous-batching work item: same fields and layout as VspecContinuousBatchItem
 * (continuous_batch.h:15-20).  request_id doubles as the paged-cache session id;
 * phase is 1 (prefill) or 2 (decode); token_quota new tokens enter the cache. */
typedef struct VspecRocmStepItem {
    uint64_t request_id;
    uint32_t phase;
    size_t token_quota;
    size_t prompt_cursor;
} VspecRocmStepItem;

/* Plan one step of continuous batching: reserve each item's token_quota tokens and
 * emit, per item i, its block table row (block_tables[i*max_blocks ..], -1 padded), its
 * context after the step (ctx_lens[i]) and the position of its first new token
 * (start_pos[i]); and, per packed new token t (items in order, quota tokens each), its
 * item (token_item[t]) and position (token_pos[t]) -- the inputs of
 * vspec_rocm_kv_append_tokens and of the decode descriptor.  Positions are in
 * table-slot space (page index * page_tokens + slot), the token index while every page
 * but the last is full.  block_used (optional, [n_items][max_blocks]) receives each
 * entry's used count, and ctx_lens the span (see VspecPagedAttnDesc.block_used): every
 * session can then be decoded, partly filled middle pages included.  Without it a
 * session with such a page fails the step.  Returns 0 on a repeated request, a failed
 * reservation, an eviction of an earlier item's session by a later one, or outputs that
 * are too small; reservations made before the failure stay made. */
int vspec_rocm_paged_plan_step(VspecRocmPagedMeta* m, const VspecRocmStepItem* items,
                               size_t n_items, int32_t* block_tables, int32_t* block_used,
                               size_t max_blocks, int32_t* ctx_lens, int32_t* start_pos,
                               int32_t* token_item, int32_t* token_pos, size_t max_tokens,
                               size_t* n_tokens);
/* vspec_rocm_paged_plan_step for a serving loop that keeps its host tables between steps:
 * pass the same block_tables / block_used buffers (and max_blocks) every step and leave
 * their contents as the previous call wrote them.  A row that the previous call wrote for
 * the same session (not evicted and reopened since) only gets the entries that changed:
 * the former last entry's used count and the pages opened since; other rows are written
 * whole.  Outputs and failures are those of vspec_rocm_paged_plan_step; on a failure the
 * rows written so far stay consistent with what the next call assumes.  No counterpart in
 * the reference (its callers append token by token, kv_paged_cache.c:243-310). */
int vspec_rocm_paged_plan_step_update(VspecRocmPagedMeta* m, const VspecRocmStepItem* items,
                                      size_t n_items, int32_t* block_tables, int32_t* block_used,
                                      size_t max_blocks, int32_t* ctx_lens, int32_t* start_pos,
                                      int32_t* token_item, int32_t* token_pos, size_t max_tokens,
                                      size_t* n_tokens);

/* Append packed new tokens (device pointers): token t of k_new/v_new ([n][H][D] in
 * src_dtype) goes to position token_pos[t] of the sequence whose block table is row
 * token_item[t] of block_tables ([n_items][max_blocks_per_seq]); tokens whose item is
 * negative or not below n_items are skipped.  Mixed chunked-prefill and decode steps
 * append in one launch; quantises on write for int4 pools. */
int vspec_rocm_kv_append_tokens(const VspecPagedKV* kv, uint32_t n_tokens, const int32_t* token_item,
                                const int32_t* token_pos, const int32_t* block_tables, uint32_t n_items,
                                uint32_t max_blocks_per_seq, const void* k_new, const void* v_new,
                                int32_t src_dtype, void* stream);

/* ---- GPU-resident handles with the reference Python C-API signatures ---- */
int vspec_py_kv_cache_create(size_t page_tokens, size_t max_pages, size_t num_heads, size_t head_dim);
void vspec_py_kv_cache_destroy(int handle_id);
int vspec_py_kv_cache_reset(int handle_id);
int vspec_py_kv_cache_append(int handle_id, uint64_t session_id, const float* key_token,
                             const float* value_token);
size_t vspec_py_kv_cache_session_tokens(int handle_id, uint64_t session_id);
size_t vspec_py_kv_cache_read(int handle_id, uint64_t session_id, float* out_keys,
                              float* out_values, size_t max_tokens);

/* The handle's metadata and device pool, for callers that batch on the GPU. */
VspecRocmPagedMeta* vspec_py_kv_cache_meta(int handle_id);
const VspecPagedKV* vspec_py_kv_cache_pool(int handle_id);

/* Gather explicit rows: token i of the output is (pages[i], slots[i]) of every head,
 * written in [n][H][D] order as f32 (device pointers). */
int vspec_rocm_kv_gather_rows(const VspecPagedKV* kv, uint32_t n, const int32_t* pages,
                              const int32_t* slots, float* out_k, float* out_v, void* stream);

#ifdef __cplusplus
}
#endif

#endif
