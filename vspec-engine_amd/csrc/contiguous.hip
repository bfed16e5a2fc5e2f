// contiguous.hip -- the reference's contiguous-cache attention call
// (cpu_backend.c:40-51 -> attention_ref.c:7-88) served by the paged kernels.
//
// A VspecKVCache holds [T][H][D] keys and values in host memory: fp32 rows (also the fp32
// mirror when the reference's int3 codec is on, kv_cache.c:198-215), or, for a cache whose
// codec runs without a mirror, 3-bit codes with per-block fp32 scales that the reference's
// accessors decode on every read (kv_cache.c:296-362).  Each cache gets a persistent device
// mirror (below): a call uploads only the rows appended since the previous call (codes and
// scales are decoded to fp32 on the device, bit for bit as the reference decodes them).
// For head_dim 64 / 128 the mirror is an f32 paged pool with an identity block table that
// the decode kernels read with Hq == Hkv (MHA); other head sizes run a generic
// one-workgroup-per-head kernel over device rows.
#include <hip/hip_runtime.h>

#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <strings.h>

#include <mutex>

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

// ---------------------------------------------------------------------------
// Persistent device mirror of a host VspecKVCache.
//
// The reference uploads the whole host cache on every attention call, and its caller owns
// those rows; so by default every call uploads every row again into a mirror keyed by the
// cache (device memory kept between calls).  A caller whose caches only grow between calls
// (kv_cache.c:160-226: rows go to current_tokens and the count increments) can opt in to
// uploading only the rows appended since the previous call (VSPEC_ROCM_MIRROR_APPEND_ONLY,
// vspec_rocm_cache_mirror_append_only).  head_dim 64 / 128: the rows are appended into a persistent f32 paged pool
// (identity block table, capacity max_tokens) and decoded by the paged kernels (Hq == Hkv);
// other head sizes keep device [max_tokens][H][D] rows for the generic kernel.  Per call:
// one upload of (q, the new rows or their int3 codes and scales) through pinned staging,
// the int3 decode when needed, the append, the attention launches and one download of the
// output; after a mirror's first call no device memory is allocated or freed unless the
// new rows outgrow the staging buffers.
//
// In append-only mode the uploaded rows are kept when the cache pointer, its buffer
// pointers and geometry are the same, current_tokens did not shrink, and fingerprints of
// the first token's rows and of the last synced token's rows still match; anything else
// resyncs from token 0.  A caller in that mode that rewrites rows in place keeps the
// contract by calling vspec_rocm_release_cache_mirror (which also frees the device memory
// with the cache).
// ---------------------------------------------------------------------------
struct Mirror {
    const VspecKVCache* cache = nullptr;
    VspecKVCache shape;  // the cache fields at the last sync (pointers and geometry)
    size_t synced = 0;   // tokens on the device
    uint64_t fp_first = 0, fp_last = 0;
    uint64_t last_use = 0;
    bool paged = false;
    VspecPagedKV kv;       // paged: persistent f32 pool
    int32_t* d_tab = nullptr;
    float* d_k = nullptr;  // generic: device rows [max_tokens][H][D]
    float* d_v = nullptr;
    float* d_scores = nullptr;
    uint8_t* d_stage = nullptr;  // q, ctx/start, new rows (or codes + scales), decoded rows
    size_t stage_bytes = 0;
    uint8_t* h_stage = nullptr;  // pinned
    size_t h_stage_bytes = 0;
    float* d_out = nullptr;
};

constexpr int kMirrors = 16;
Mirror g_mirror[kMirrors];
uint64_t g_mirror_clock = 0;
std::mutex g_mirror_mu;
// Upload policy of the mirror: -1 follows VSPEC_ROCM_MIRROR_APPEND_ONLY (unset, "0", "false",
// "off", "no": whole cache), 0 uploads every row on every call, 1 only the rows appended
// since the previous call (vspec_rocm_cache_mirror_append_only)
int g_append_only = -1;

bool append_only_mode() {
    if (g_append_only >= 0) return g_append_only != 0;
    const char* e = getenv("VSPEC_ROCM_MIRROR_APPEND_ONLY");
    if (!e || !*e) return false;
    return strcmp(e, "0") != 0 && strcasecmp(e, "false") != 0 && strcasecmp(e, "off") != 0 &&
           strcasecmp(e, "no") != 0;
}

void mirror_free(Mirror& m) {
    if (m.paged) vspec_rocm_kv_pool_destroy(&m.kv);
    (void)hipFree(m.d_tab);
    (void)hipFree(m.d_k);
    (void)hipFree(m.d_v);
    (void)hipFree(m.d_scores);
    (void)hipFree(m.d_stage);
    (void)hipFree(m.d_out);
    if (m.h_stage) (void)hipHostFree(m.h_stage);
    m = Mirror();
}

uint64_t fnv(uint64_t h, const void* p, size_t n) {
    const uint8_t* b = (const uint8_t*)p;
    for (size_t i = 0; i < n; ++i) h = (h ^ b[i]) * 1099511628211ull;
    return h;
}

// fingerprint of token t's rows (both sides, every head; fp32 rows, or codes + scales)
uint64_t token_fingerprint(const VspecKVCache* c, const CacheSide& ks, const CacheSide& vs, size_t t) {
    uint64_t h = 1469598103934665603ull;
    const size_t H = c->num_heads, D = c->head_dim;
    for (const CacheSide* s : {&ks, &vs}) {
        if (s->rows) {
            h = fnv(h, s->rows + t * H * D, H * D * sizeof(float));
        } else {
            h = fnv(h, s->codes + t * H * c->packed_head_bytes, H * c->packed_head_bytes);
            h = fnv(h, s->scales + t * H * c->blocks_per_head, H * c->blocks_per_head * sizeof(float));
        }
    }
    return h;
}

bool same_shape(const VspecKVCache& a, const VspecKVCache& b) {
    return a.key == b.key && a.value == b.value && a.max_tokens == b.max_tokens && a.num_heads == b.num_heads &&
           a.head_dim == b.head_dim && a.int3_compressed == b.int3_compressed && a.key_int3 == b.key_int3 &&
           a.value_int3 == b.value_int3 && a.key_scales == b.key_scales && a.value_scales == b.value_scales &&
           a.block_size == b.block_size && a.blocks_per_head == b.blocks_per_head &&
           a.packed_head_bytes == b.packed_head_bytes;
}

// device allocations that depend only on the cache's geometry (made once per mirror)
int mirror_setup(Mirror& m, const VspecKVCache* c) {
    const size_t T = c->max_tokens, H = c->num_heads, D = c->head_dim;
    m.paged = D == 64 || D == 128;
    const size_t qb = H * D * sizeof(float);
    if (hipMalloc((void**)&m.d_out, qb) != hipSuccess) return 0;
    if (m.paged) {
        const uint32_t P = 16, nblk = (uint32_t)((T + P - 1) / P);
        if (!vspec_rocm_kv_pool_create(&m.kv, VSPEC_KV_F32, nblk, P, (uint32_t)H, (uint32_t)D)) return 0;
        int32_t* h_tab = (int32_t*)malloc(nblk * sizeof(int32_t));
        if (!h_tab) return 0;
        for (uint32_t i = 0; i < nblk; ++i) h_tab[i] = (int32_t)i;
        const int ok = hipMalloc((void**)&m.d_tab, nblk * sizeof(int32_t)) == hipSuccess &&
                       hipMemcpy(m.d_tab, h_tab, nblk * sizeof(int32_t), hipMemcpyHostToDevice) == hipSuccess;
        free(h_tab);
        return ok;
    }
    const size_t kvb = T * H * D * sizeof(float);
    return hipMalloc((void**)&m.d_k, kvb) == hipSuccess && hipMalloc((void**)&m.d_v, kvb) == hipSuccess &&
           hipMalloc((void**)&m.d_scores, T * H * sizeof(float)) == hipSuccess;
}

int grow(uint8_t** d, size_t* have, size_t need, bool pinned) {
    if (*have >= need) return 1;
    const size_t n = need + need / 4;
    if (pinned) {
        if (*d) (void)hipHostFree(*d);
        *d = nullptr;
        *have = 0;
        if (hipHostMalloc((void**)d, n, hipHostMallocDefault) != hipSuccess) return 0;
    } else {
        if (*d) (void)hipFree(*d);
        *d = nullptr;
        *have = 0;
        if (hipMalloc((void**)d, n) != hipSuccess) return 0;
    }
    *have = n;
    return 1;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

Mirror* mirror_for(const VspecKVCache* c) {
    Mirror* slot = nullptr;
    for (Mirror& m : g_mirror) {
        if (m.cache == c) {
            slot = &m;
            break;
        }
    }
    if (slot && !same_shape(slot->shape, *c)) {
        mirror_free(*slot);  // another cache (or other buffers) at this address
        slot = nullptr;
    }
    if (!slot) {
        for (Mirror& m : g_mirror) {
            if (!m.cache && !slot) slot = &m;
        }
        if (!slot) {  // evict the least recently used
            slot = &g_mirror[0];
            for (Mirror& m : g_mirror) {
                if (m.last_use < slot->last_use) slot = &m;
            }
            mirror_free(*slot);
        }
        if (!mirror_setup(*slot, c)) {
            mirror_free(*slot);
            vspec_rocm_set_error_("attention: device allocation for the cache mirror failed");
            return nullptr;
        }
        slot->cache = c;
        slot->shape = *c;
        slot->synced = 0;
    }
    slot->last_use = ++g_mirror_clock;
    return slot;
}

}  // namespace

extern "C" int vspec_rocm_cache_mirror_append_only(int enable) {
    std::lock_guard<std::mutex> lock(g_mirror_mu);
    const int was = append_only_mode() ? 1 : 0;
    g_append_only = enable < 0 ? -1 : (enable ? 1 : 0);
    return was;
}

extern "C" int vspec_rocm_release_cache_mirror(const VspecKVCache* cache) {
    std::lock_guard<std::mutex> lock(g_mirror_mu);
    for (Mirror& m : g_mirror) {
        if (m.cache && (cache == nullptr || m.cache == cache)) mirror_free(m);
    }
    return 1;
}

extern "C" int vspec_rocm_attention_cache_host(const float* q, const VspecKVCache* cache,
                                               int32_t numerics, float* out) {
    if (!q || !cache || !out || cache->current_tokens == 0 || cache->num_heads == 0 || cache->head_dim == 0) {
        vspec_rocm_set_error_("attention: bad arguments");
        return 0;
    }
    const size_t tokens = cache->current_tokens, heads = cache->num_heads, head_dim = cache->head_dim;
    if (tokens > cache->max_tokens) {
        vspec_rocm_set_error_("attention: current_tokens exceeds max_tokens");
        return 0;
    }
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
        if (cache->max_tokens > (size_t)INT32_MAX / 2 || heads > (size_t)UINT32_MAX) {
            vspec_rocm_set_error_("attention: too many tokens");
            return 0;
        }
    } else {
        // other head sizes (the reference demo uses 4) take the generic kernel
        if (cache->max_tokens > (size_t)UINT32_MAX || heads > (size_t)UINT32_MAX) {
            vspec_rocm_set_error_("attention: cache too large");
            return 0;
        }
        if ((kThreads + head_dim) * sizeof(float) > 64 * 1024) {
            vspec_rocm_set_error_("attention: head_dim too large for the contiguous path");
            return 0;
        }
    }
    std::lock_guard<std::mutex> lock(g_mirror_mu);
    Mirror* m = mirror_for(cache);
    if (!m) return 0;
    // Every row is uploaded again unless the caller promised appends only; even then the
    // mirror resyncs from token 0 when the cache shrank or its first or last synced row changed.
    if (!append_only_mode() || m->synced > tokens ||
        (m->synced && (token_fingerprint(cache, ks, vs, 0) != m->fp_first ||
                       token_fingerprint(cache, ks, vs, m->synced - 1) != m->fp_last))) {
        m->synced = 0;
    }
    const size_t t0 = m->synced, n = tokens - t0, H = heads, D = head_dim;
    const size_t qb = H * D * sizeof(float), row_b = H * D * sizeof(float);
    // staging layout: q | (start, ctx) | per side: rows (fp32 side) or codes + scales
    // (int3 side) of the new tokens | per int3 side: decoded rows
    size_t off_side[2], sz_side[2], off_dec[2];
    size_t up = align256(qb) + 256;
    const CacheSide* sides[2] = {&ks, &vs};
    for (int w = 0; w < 2; ++w) {
        off_side[w] = up;
        sz_side[w] = sides[w]->rows ? n * row_b
                                    : align256(n * H * cache->packed_head_bytes) + n * H * cache->blocks_per_head * sizeof(float);
        up += align256(sz_side[w]);
    }
    size_t dev_total = up;
    for (int w = 0; w < 2; ++w) {
        off_dec[w] = dev_total;
        if (!sides[w]->rows) dev_total += align256(n * row_b);
    }
    if (!grow(&m->h_stage, &m->h_stage_bytes, up, true) || !grow(&m->d_stage, &m->stage_bytes, dev_total, false)) {
        vspec_rocm_set_error_("attention: staging allocation failed");
        mirror_free(*m);
        return 0;
    }
    uint8_t* hs = m->h_stage;
    memcpy(hs, q, qb);
    const int32_t misc[2] = {(int32_t)t0, (int32_t)tokens};
    memcpy(hs + align256(qb), misc, sizeof(misc));
    for (int w = 0; w < 2; ++w) {
        const CacheSide& sd = *sides[w];
        if (sd.rows) {
            memcpy(hs + off_side[w], sd.rows + t0 * H * D, n * row_b);
        } else {
            memcpy(hs + off_side[w], sd.codes + t0 * H * cache->packed_head_bytes, n * H * cache->packed_head_bytes);
            memcpy(hs + off_side[w] + align256(n * H * cache->packed_head_bytes), sd.scales + t0 * H * cache->blocks_per_head,
                   n * H * cache->blocks_per_head * sizeof(float));
        }
    }
    hipStream_t s = nullptr;
    int ok = hipMemcpyAsync(m->d_stage, hs, up, hipMemcpyHostToDevice, s) == hipSuccess;
    const float* d_q = (const float*)m->d_stage;
    const int32_t* d_misc = (const int32_t*)(m->d_stage + align256(qb));
    const float* new_rows[2];
    for (int w = 0; ok && w < 2; ++w) {
        const CacheSide& sd = *sides[w];
        if (sd.rows) {
            new_rows[w] = (const float*)(m->d_stage + off_side[w]);
            continue;
        }
        float* dec = (float*)(m->d_stage + off_dec[w]);
        Int3Rows p = {m->d_stage + off_side[w],
                      (const float*)(m->d_stage + off_side[w] + align256(n * H * cache->packed_head_bytes)), dec, n * H,
                      cache->packed_head_bytes, cache->blocks_per_head, (uint32_t)D, (uint32_t)cache->block_size};
        const size_t elems = n * H * D;
        if (elems) {
            const unsigned grid = (unsigned)((elems + kThreads - 1) / kThreads < 8192 ? (elems + kThreads - 1) / kThreads : 8192);
            hipLaunchKernelGGL(int3_rows_to_f32, dim3(grid), dim3(kThreads), 0, s, p);
            ok = hipGetLastError() == hipSuccess;
        }
        new_rows[w] = dec;
    }
    if (!ok) vspec_rocm_set_error_("attention: upload or int3 decode failed");
    if (ok && m->paged) {
        const uint32_t nblk = m->kv.num_blocks;
        ok = vspec_rocm_kv_append(&m->kv, 1, m->d_tab, nblk, d_misc, (uint32_t)n, new_rows[0], new_rows[1], VSPEC_KV_F32, s);
        if (ok) {
            VspecPagedAttnDesc d;
            memset(&d, 0, sizeof(d));
            d.kv = m->kv;
            d.batch = 1;
            d.num_q_heads = (uint32_t)H;
            d.block_tables = m->d_tab;
            d.max_blocks_per_seq = nblk;
            d.ctx_lens = d_misc + 1;
            d.max_ctx_len = (uint32_t)tokens;
            d.q = d_q;
            d.out = m->d_out;
            d.numerics = numerics;
            d.stream = s;
            ok = vspec_rocm_paged_decode_attention(&d);
        }
    } else if (ok) {
        if (n && (hipMemcpyAsync(m->d_k + t0 * H * D, new_rows[0], n * row_b, hipMemcpyDeviceToDevice, s) != hipSuccess ||
                  hipMemcpyAsync(m->d_v + t0 * H * D, new_rows[1], n * row_b, hipMemcpyDeviceToDevice, s) != hipSuccess)) {
            vspec_rocm_set_error_("attention: row copy failed");
            ok = 0;
        }
        if (ok) {
            const bool three = numerics == VSPEC_NUMERICS_3BIT;
            float scale = 1.0f / sqrtf((float)D);
            if (three) scale = fminf(fmaxf(scale, 1e-4f), 32.0f);
            ContigParams p = {d_q, m->d_k, m->d_v, m->d_out, m->d_scores, (uint32_t)tokens, (uint32_t)H, (uint32_t)D,
                              scale * kLog2e, 4.5f, three ? 24.0f * kLog2e : INFINITY, three ? 16.0f : INFINITY};
            const size_t smem = (kThreads + D) * sizeof(float);
            hipLaunchKernelGGL(attention_contig, dim3((unsigned)H), dim3(kThreads), smem, s, p);
            ok = hipGetLastError() == hipSuccess;
            if (!ok) vspec_rocm_set_error_("attention: launch failed");
        }
    }
    if (ok && (hipMemcpyAsync(out, m->d_out, qb, hipMemcpyDeviceToHost, s) != hipSuccess ||
               hipStreamSynchronize(s) != hipSuccess)) {
        vspec_rocm_set_error_("attention: download failed");
        ok = 0;
    }
    if (!ok) {
        mirror_free(*m);
        return 0;
    }
    m->synced = tokens;
    m->fp_first = token_fingerprint(cache, ks, vs, 0);
    m->fp_last = token_fingerprint(cache, ks, vs, tokens - 1);
    return 1;
}
