/*
 * ref_shim.c -- harness linked with the reference's own hot-path sources
 * (compiled in place from the reference tree by oracle/Makefile) into
 * oracle/_ref/libvspec_ref.so.
 *
 * TEST INFRASTRUCTURE ONLY.  It gives Python (ctypes) opaque handles to the
 * reference's structs and restates the two reference call sites that do not
 * compile standalone:
 *   - the paged gather loop of vspec_py_kv_cache_read (capi.c:2263-2299), which
 *     lives in a 2.8k-line file with many dependencies;
 *   - the GQA head mapping of the Python runtime (runtime_inference.py:151,1419:
 *     kv_h = h // group), which calls the MHA-only attention_ref per head.
 * Everything numeric is done by the reference's functions.
 */
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "vspec/attention/attention.h"
#include "vspec/attention/kv_cache.h"
#include "vspec/attention/kv_paged_cache.h"
#include "vspec/kernel/backend.h"
#include "vspec/kernel/context.h"

/* ---- paged cache handles ---- */
VspecKVPagedCache* vr_paged_new(size_t page_tokens, size_t max_pages, size_t num_heads,
                                size_t head_dim) {
    VspecKVPagedCache* c = (VspecKVPagedCache*)calloc(1, sizeof(VspecKVPagedCache));
    const size_t n = page_tokens * max_pages * num_heads * head_dim;
    float* k = (float*)calloc(n ? n : 1, sizeof(float));
    float* v = (float*)calloc(n ? n : 1, sizeof(float));
    if (!c || !k || !v || !vspec_kv_paged_cache_init(c, k, v, page_tokens, max_pages, num_heads, head_dim)) {
        free(c);
        free(k);
        free(v);
        return NULL;
    }
    return c;
}

void vr_paged_free(VspecKVPagedCache* c) {
    if (!c) return;
    free(c->key_pages);
    free(c->value_pages);
    free(c);
}

const float* vr_paged_key_pages(const VspecKVPagedCache* c) { return c->key_pages; }
const float* vr_paged_value_pages(const VspecKVPagedCache* c) { return c->value_pages; }

/* Session page list (uint16 page ids as stored by the reference). */
size_t vr_paged_session_pages(const VspecKVPagedCache* c, uint64_t session_id, uint32_t* out,
                              size_t cap) {
    for (size_t i = 0; i < VSPEC_KV_PAGED_MAX_SESSIONS; ++i) {
        if (c->sessions[i].active && c->sessions[i].session_id == session_id) {
            size_t n = c->sessions[i].page_count;
            for (size_t j = 0; j < n && j < cap; ++j) out[j] = c->sessions[i].pages[j];
            return n;
        }
    }
    return 0;
}

/* Per-page metadata: used tokens and ref count. */
void vr_paged_page_meta(const VspecKVPagedCache* c, size_t page, uint32_t* allocated,
                        uint32_t* used, uint32_t* refc) {
    *allocated = c->page_meta[page].allocated;
    *used = c->page_meta[page].used_tokens;
    *refc = c->page_meta[page].ref_count;
}

void vr_paged_stats(const VspecKVPagedCache* c, uint64_t* out6) {
    VspecKVPagedStats s;
    vspec_kv_paged_stats(c, &s);
    out6[0] = s.page_alloc_count;
    out6[1] = s.page_reuse_count;
    out6[2] = s.evict_session_count;
    out6[3] = s.append_token_count;
    out6[4] = s.free_pages;
    out6[5] = s.active_sessions;
}

/* capi.c:2263-2299 gather loop over vspec_kv_paged_get_token_ptr. */
size_t vr_paged_read(const VspecKVPagedCache* c, uint64_t session_id, float* out_keys,
                     float* out_values, size_t max_tokens) {
    const size_t stride = c->num_heads * c->head_dim;
    size_t total = vspec_kv_paged_session_tokens(c, session_id);
    if (max_tokens > 0u && total > max_tokens) total = max_tokens;
    for (size_t t = 0; t < total; ++t) {
        for (size_t h = 0; h < c->num_heads; ++h) {
            const float* kp = NULL;
            const float* vp = NULL;
            if (!vspec_kv_paged_get_token_ptr(c, session_id, t, h, &kp, &vp)) return t;
            for (size_t d = 0; d < c->head_dim; ++d) {
                const size_t base = t * stride + h * c->head_dim + d;
                out_keys[base] = kp[d];
                out_values[base] = vp[d];
            }
        }
    }
    return total;
}

/* ---- contiguous cache + attention through the CPU backend ---- */

/* attention_ref over a contiguous [T][H][D] fp32 cache via the registered CPU
 * backend (cpu_backend.c:40-51 -> attention_ref.c:7-88). */
void vr_attention_mha(const float* q, const float* key, const float* value, size_t tokens,
                      size_t heads, size_t head_dim, float* out) {
    VspecKVCache cache;
    if (!vspec_kv_cache_init(&cache, (float*)key, (float*)value, tokens ? tokens : 1, heads, head_dim)) {
        return;
    }
    cache.current_tokens = tokens;
    VspecBackend be = vspec_make_cpu_backend();
    VspecKernelContext ctx;
    memset(&ctx, 0, sizeof(ctx));
    ctx.input = (void*)q;
    ctx.weight = &cache;
    ctx.output = out;
    be.launch_attention(&ctx);
}

/* GQA decode for one sequence: q/out [Hq][D], key/value [T][Hkv][D].
 * The runtime maps query head h to kv head h / G.  For each group slot g the
 * sub-query collects heads h = kv_h*G + g (kv_h = 0..Hkv-1), which the MHA
 * attention_ref then pairs with kv head kv_h. */
void vr_attention_gqa(const float* q, const float* key, const float* value, size_t tokens,
                      size_t hq, size_t hkv, size_t head_dim, float* out) {
    const size_t group = hq / hkv;
    float* qs = (float*)malloc(hkv * head_dim * sizeof(float));
    float* os = (float*)malloc(hkv * head_dim * sizeof(float));
    if (!qs || !os) { free(qs); free(os); return; }
    for (size_t g = 0; g < group; ++g) {
        for (size_t k = 0; k < hkv; ++k) {
            memcpy(qs + k * head_dim, q + (k * group + g) * head_dim, head_dim * sizeof(float));
        }
        vr_attention_mha(qs, key, value, tokens, hkv, head_dim, os);
        for (size_t k = 0; k < hkv; ++k) {
            memcpy(out + (k * group + g) * head_dim, os + k * head_dim, head_dim * sizeof(float));
        }
    }
    free(qs);
    free(os);
}

/* ---- int3 KV codec through the reference's contiguous cache ---- */
int vr_int3_append_and_dump(const float* key_tokens, const float* value_tokens, size_t tokens,
                            size_t heads, size_t head_dim, size_t block_size, uint8_t* out_kq,
                            float* out_ks, float* out_kmirror) {
    float* kb = (float*)calloc(tokens * heads * head_dim, sizeof(float));
    float* vb = (float*)calloc(tokens * heads * head_dim, sizeof(float));
    VspecKVCache cache;
    int ok = kb && vb && vspec_kv_cache_init(&cache, kb, vb, tokens, heads, head_dim) &&
             vspec_kv_cache_enable_int3_compression(&cache, block_size);
    if (ok) {
        for (size_t t = 0; t < tokens; ++t) {
            vspec_kv_cache_append(&cache, key_tokens + t * heads * head_dim,
                                  value_tokens + t * heads * head_dim);
        }
        memcpy(out_kq, cache.key_int3, tokens * heads * cache.packed_head_bytes);
        memcpy(out_ks, cache.key_scales, tokens * heads * cache.blocks_per_head * sizeof(float));
        memcpy(out_kmirror, kb, tokens * heads * head_dim * sizeof(float));
        vspec_kv_cache_disable_int3_compression(&cache);
    }
    free(kb);
    free(vb);
    return ok;
}

/* Monotonic clock for the CPU baseline (CLOCK_MONOTONIC, seconds). */
double vr_now(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

/* ---- CPU baseline: the reference decode step for a batch of sequences ----
 * Per sequence (the reference's own path, one layer):
 *   setup (untimed): a fresh paged cache with T-1 tokens appended
 *   timed: append the decode-step token (kv_paged_cache.c:243-310), gather all T
 *          tokens through get_token_ptr (capi.c:2263-2299 loop), then GQA
 *          attention_ref (cpu_backend.c:40-51 per head group).
 * Sequences are split over nthreads POSIX threads.  Returns the timed wall seconds. */
#include <pthread.h>

typedef struct VrJob {
    size_t first, last, T, hq, hkv, d, p;
    const float *k, *v, *q;
    float* out;
    VspecKVPagedCache** caches;
    float *gk, *gv; /* per-thread gather buffers */
    int ok;
} VrJob;

static void* vr_job_setup(void* arg) {
    VrJob* j = (VrJob*)arg;
    const size_t row = j->hkv * j->d;
    for (size_t s = j->first; s < j->last; ++s) {
        VspecKVPagedCache* c = vr_paged_new(j->p, (j->T + j->p - 1) / j->p, j->hkv, j->d);
        j->caches[s] = c;
        if (!c) { j->ok = 0; return NULL; }
        const float* ks = j->k + s * j->T * row;
        const float* vs = j->v + s * j->T * row;
        for (size_t t = 0; t + 1 < j->T; ++t) {
            if (!vspec_kv_paged_append(c, 1u, ks + t * row, vs + t * row)) { j->ok = 0; return NULL; }
        }
    }
    return NULL;
}

static void* vr_job_run(void* arg) {
    VrJob* j = (VrJob*)arg;
    const size_t row = j->hkv * j->d;
    for (size_t s = j->first; s < j->last; ++s) {
        VspecKVPagedCache* c = j->caches[s];
        const size_t t = j->T - 1;
        if (!vspec_kv_paged_append(c, 1u, j->k + (s * j->T + t) * row, j->v + (s * j->T + t) * row)) {
            j->ok = 0;
            return NULL;
        }
        if (vr_paged_read(c, 1u, j->gk, j->gv, 0) != j->T) { j->ok = 0; return NULL; }
        vr_attention_gqa(j->q + s * j->hq * j->d, j->gk, j->gv, j->T, j->hq, j->hkv, j->d,
                         j->out + s * j->hq * j->d);
    }
    return NULL;
}

double vr_baseline_decode(int nthreads, size_t nseq, size_t T, size_t hq, size_t hkv, size_t d,
                          size_t p, const float* k, const float* v, const float* q, float* out) {
    if (nthreads < 1) nthreads = 1;
    if ((size_t)nthreads > nseq) nthreads = (int)nseq;
    VspecKVPagedCache** caches = (VspecKVPagedCache**)calloc(nseq, sizeof(*caches));
    VrJob* jobs = (VrJob*)calloc((size_t)nthreads, sizeof(VrJob));
    pthread_t* th = (pthread_t*)calloc((size_t)nthreads, sizeof(pthread_t));
    double elapsed = -1.0;
    int ok = caches && jobs && th;
    for (int i = 0; ok && i < nthreads; ++i) {
        VrJob* j = &jobs[i];
        j->first = nseq * (size_t)i / (size_t)nthreads;
        j->last = nseq * (size_t)(i + 1) / (size_t)nthreads;
        j->T = T; j->hq = hq; j->hkv = hkv; j->d = d; j->p = p;
        j->k = k; j->v = v; j->q = q; j->out = out; j->caches = caches; j->ok = 1;
        j->gk = (float*)malloc(T * hkv * d * sizeof(float));
        j->gv = (float*)malloc(T * hkv * d * sizeof(float));
        if (!j->gk || !j->gv) ok = 0;
    }
    if (ok) {
        for (int i = 0; i < nthreads; ++i) pthread_create(&th[i], NULL, vr_job_setup, &jobs[i]);
        for (int i = 0; i < nthreads; ++i) pthread_join(th[i], NULL);
        for (int i = 0; i < nthreads; ++i) ok = ok && jobs[i].ok;
    }
    if (ok) {
        const double t0 = vr_now();
        for (int i = 0; i < nthreads; ++i) pthread_create(&th[i], NULL, vr_job_run, &jobs[i]);
        for (int i = 0; i < nthreads; ++i) pthread_join(th[i], NULL);
        elapsed = vr_now() - t0;
        for (int i = 0; i < nthreads; ++i) ok = ok && jobs[i].ok;
        if (!ok) elapsed = -1.0;
    }
    for (size_t s = 0; caches && s < nseq; ++s) vr_paged_free(caches[s]);
    for (int i = 0; jobs && i < nthreads; ++i) { free(jobs[i].gk); free(jobs[i].gv); }
    free(caches);
    free(jobs);
    free(th);
    return elapsed;
}

/* ---- continuous-batching scheduler (continuous_batch.c) behind an opaque pointer ---- */
#include "vspec/runtime/continuous_batch.h"

VspecContinuousBatcher* vr_batcher_new(size_t total_vram_bytes, size_t max_active, size_t max_batch_items,
                                       size_t max_batch_tokens, size_t prefill_quantum, size_t decode_quantum) {
    VspecContinuousBatcher* b = (VspecContinuousBatcher*)calloc(1, sizeof(VspecContinuousBatcher));
    if (b) {
        vspec_continuous_batch_init(b, total_vram_bytes, max_active, max_batch_items, max_batch_tokens,
                                    prefill_quantum, decode_quantum);
    }
    return b;
}

void vr_batcher_free(VspecContinuousBatcher* b) { free(b); }

size_t vr_batch_item_size(void) { return sizeof(VspecContinuousBatchItem); }
