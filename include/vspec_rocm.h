/*
 * vspec_rocm.h -- C-ABI of the MI355X (gfx950) paged KV-cache decode path.
 *
 * Plain C: device pointers, sizes and a hipStream_t passed as void*.  No C++ or
 * torch types cross this boundary.  Conventions follow the reference:
 *   - cache operations return 1 on success and 0 on failure (kv_paged_cache.c);
 *     the reason is kept per thread and read with vspec_rocm_last_error();
 *   - the caller owns every buffer; nothing is retained past a call except the
 *     pools made by vspec_rocm_kv_pool_create;
 *   - no internal locking: calls that touch one pool are serialised by the caller
 *     (one stream per pool), as the reference's structs are unsynchronised.
 *
 * HBM layout, element (block b, kv head h, slot s, dim d):
 *   K, and V of f32 pools  data[((b*H + h)*P + s)*D + d]          (token-major rows)
 *   V of f16 pools         data[(b*H + h)*D*P + (s/4)*4*D + 4*d + s%4]  (groups of 4 tokens,
 *                          d-major inside a group: the matrix-core operand of P.V needs 4
 *                          consecutive tokens of one d per lane, and one token's row then
 *                          spans 4*D halves instead of D*P)
 *   int4 K codes           byte ((b*H + h)*P + s)*(D/2) + d/2, nibble d&1 (even = low)
 *   int4 K scales          ((b*H + h)*(D/32) + d/32)*P + s, fp16 bits (group-major)
 *   int4 V codes           16-token tiles of 8*D bytes, lane chunk (g, n) at (16g + n)*(D/8)
 *                          holds tokens 4g..4g+3 of d = 16j + n (two d-tiles per byte)
 *   int4 V scales          ((b*H + h)*P + s)*(D/32) + d/32, fp16 bits
 * so one (block, head) tile of P tokens is contiguous (4 KB at P=16, D=128, f16).
 *
 * int4 codec: per (token, kv head) groups of 32 elements;
 *   rep   = 2nd-largest |x| of the group (kv_cache.c:32-59, percentile 99.5 at n=32)
 *   scale = rep > 0 ? rep/8 : 1, floored at 1e-6, rounded to fp16 (RNE, max 65504)
 *   code  = clip(rint(x / float(scale16)), -8, 7) with saturation (NaN -> -8)
 *   value = code * float(scale16)                 (exact in fp32)
 *
 * Attention numerics follow attention_ref.c:7-88: q and every k are
 * clipped to +-max(1e-6, alpha*std) (three_bit_runtime_modules.c:175-203); with
 * VSPEC_NUMERICS_3BIT also to +-16 (:138-173), logits to +-24 (:205-250) and the
 * scale to [1e-4, 32] (:344-361).  GQA maps query head h to kv head h / (Hq/Hkv)
 * (runtime_inference.py:151).
 */
#ifndef VSPEC_ROCM_H
#define VSPEC_ROCM_H

#include <stddef.h>
#include <stdint.h>

#include "vspec_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

enum { VSPEC_KV_F32 = 0, VSPEC_KV_F16 = 1, VSPEC_KV_INT4 = 2 };
enum { VSPEC_NUMERICS_PLAIN = 0, VSPEC_NUMERICS_3BIT = 1 };
enum { VSPEC_GATHER_RAW = 0, VSPEC_GATHER_F32 = 1 };

/* VspecKernelContext.config.flags bit: ctx->weight is a VspecPagedAttnDesc*. */
#define VSPEC_KCTX_FLAG_PAGED ((size_t)1u)

typedef struct VspecPagedKV {
    int32_t dtype;          /* VSPEC_KV_* */
    uint32_t num_blocks;
    uint32_t block_tokens;  /* P: a multiple of 16 */
    uint32_t num_kv_heads;
    uint32_t head_dim;      /* 64 or 128 */
    void* k_data;           /* device */
    void* v_data;           /* device */
    uint16_t* k_scales;     /* device, int4 only */
    uint16_t* v_scales;     /* device, int4 only */
    uint32_t* k_flags;      /* device, int4 only, or NULL: per 16-token tile of a (block, kv
                               head) one word, bit t set when key t may reach the std clamp
                               (written on append; with NULL the decode screens every key) */
} VspecPagedKV;

/* ---- pools: hipMalloc-backed, replaces the host malloc of capi.c:2188-2219 ---- */
size_t vspec_rocm_kv_pool_bytes(int32_t dtype, uint32_t num_blocks, uint32_t block_tokens,
                                uint32_t num_kv_heads, uint32_t head_dim);
int vspec_rocm_kv_pool_create(VspecPagedKV* kv, int32_t dtype, uint32_t num_blocks,
                              uint32_t block_tokens, uint32_t num_kv_heads, uint32_t head_dim);
void vspec_rocm_kv_pool_destroy(VspecPagedKV* kv);

/* ---- append: vspec_kv_paged_append (kv_paged_cache.c:243-310) for a batch ----
 * Writes n_new tokens per sequence at logical positions start_pos[b] .. +n_new-1
 * through the block table.  k_new / v_new: device [batch][n_new][H][D] in src_dtype
 * (VSPEC_KV_F32 or VSPEC_KV_F16).  An int4 pool quantises on write (the int4 codec above).
 * block_tables: device int32 [batch][max_blocks_per_seq]; start_pos: device int32 [batch]. */
int vspec_rocm_kv_append(const VspecPagedKV* kv, uint32_t batch, const int32_t* block_tables,
                         uint32_t max_blocks_per_seq, const int32_t* start_pos, uint32_t n_new,
                         const void* k_new, const void* v_new, int32_t src_dtype, void* stream);

/* ---- rotary embedding fused with the append: runtime_inference.py:1303-1313 (q, k
 * rotated by the cached cos/sin of the token position, :1186-1192) then the append ----
 * As vspec_rocm_kv_append, with K rotated before it is stored: pairs (i, i + rope_dim/2)
 * of the first rope_dim elements become (x1*c - x2*s, x1*s + x2*c) with c, s from row
 * `position` of the device fp32 tables rope_cos / rope_sin [max_pos][rope_dim/2]; every
 * product and sum is rounded separately (fp32), as numpy's float32 arithmetic does.
 * When q_in is given ([batch][n_new][num_q_heads][D] fp32, device) its rows are rotated
 * into q_out the same way.  A token whose position has no table row is not written. */
int vspec_rocm_kv_append_rope(const VspecPagedKV* kv, uint32_t batch, const int32_t* block_tables,
                              uint32_t max_blocks_per_seq, const int32_t* start_pos, uint32_t n_new,
                              const void* k_new, const void* v_new, int32_t src_dtype,
                              const float* rope_cos, const float* rope_sin, uint32_t rope_dim,
                              uint32_t max_pos, const float* q_in, float* q_out,
                              uint32_t num_q_heads, void* stream);

/* ---- gather: vspec_py_kv_cache_read (capi.c:2263-2299) for a batch ----
 * Sequence b's tokens 0..ctx_lens[b]-1 go to output tokens out_token_offset[b]+t in
 * [T][H][D] order.  out_mode VSPEC_GATHER_RAW copies the pool format (f32, f16, or
 * int4 codes [T][H][D/2] plus scales [T][H][D/32]); VSPEC_GATHER_F32 dequantises.
 * max_ctx_len (host) bounds ctx_lens and sizes the grid. */
int vspec_rocm_kv_gather(const VspecPagedKV* kv, uint32_t batch, const int32_t* block_tables,
                         uint32_t max_blocks_per_seq, const int32_t* ctx_lens,
                         uint32_t max_ctx_len, const int64_t* out_token_offset, int32_t out_mode,
                         void* out_k, void* out_v, uint16_t* out_k_scales,
                         uint16_t* out_v_scales, void* stream);

/* ---- compaction: copy whole physical blocks (all heads, data and scales) ----
 * dst_blocks[i] <- src_blocks[i]; device int32 arrays.  The destination set must
 * not intersect the source set (moves run in parallel). */
int vspec_rocm_kv_compact(const VspecPagedKV* kv, uint32_t n, const int32_t* src_blocks,
                          const int32_t* dst_blocks, void* stream);

/* ---- single-query GQA decode attention over the paged cache ---- */
typedef struct VspecPagedAttnDesc {
    VspecPagedKV kv;
    uint32_t batch;
    uint32_t num_q_heads;            /* multiple of kv.num_kv_heads */
    const int32_t* block_tables;     /* device [batch][max_blocks_per_seq] */
    uint32_t max_blocks_per_seq;
    const int32_t* ctx_lens;         /* device [batch] */
    uint32_t max_ctx_len;            /* host upper bound of ctx_lens (sizes the workspace);
                                        0: max_blocks_per_seq * block_tokens */
    const float* q;                  /* device [batch][Hq][D] f32 */
    float* out;                      /* device [batch][Hq][D] f32 (ctx 0 -> zeros) */
    float scale;                     /* <= 0: 1/sqrtf(D) */
    int32_t numerics;                /* VSPEC_NUMERICS_PLAIN or VSPEC_NUMERICS_3BIT */
    float clamp_alpha;               /* <= 0: 4.5 */
    uint32_t partition_tokens;       /* tokens per workgroup range (multiple of 16); 0: even split */
    void* workspace;                 /* device scratch (no init needed) or NULL: library's */
    size_t workspace_bytes;
    void* stream;                    /* hipStream_t or NULL */
    /* Optional, device int32 [batch][max_blocks_per_seq], or NULL: tokens held by the
     * block of each table entry, slots 0 .. used-1 (reference page_meta.used_tokens,
     * kv_paged_cache.c:335-347).  Prefix reuse leaves partly filled blocks in the middle
     * of a session (kv_paged_cache.c:223-234, 276); with block_used set, ctx_lens[b] is
     * the sequence's span in table-slot space -- entry i covers positions [i*P, (i+1)*P),
     * span = (last entry) * P + its used count -- and positions at or above their block's
     * used count are skipped.  The decode step appends at span - 1.  NULL: every block is
     * full except the last, and ctx_lens[b] is the token count. */
    const int32_t* block_used;
    /* Optional host lower bound of ctx_lens (0: none).  When it equals max_ctx_len (every
     * context the same) the host knows the work split exactly: it skips the merge launch
     * if no work item spans two workgroups (e.g. 64 x 4097 tokens on 256 CUs), and f16
     * batches whose work items about fill the CUs run one whole item per 8-wave workgroup.
     * A context below a non-zero bound is a caller error (its output may be left
     * unwritten). */
    uint32_t min_ctx_len;
} VspecPagedAttnDesc;

size_t vspec_rocm_paged_decode_workspace_bytes(const VspecPagedAttnDesc* desc);
int vspec_rocm_paged_decode_attention(const VspecPagedAttnDesc* desc);

/* One decode step in one call, the reference step's append + attention pair
 * (capi.c:2247-2253 -> kv_paged_cache.c:243-310, then cpu_backend.c:40-51 over the
 * gathered rows): appends one new token per sequence at position ctx_lens[b] - 1 (the
 * context includes it; a context of 0 appends nothing), exactly as vspec_rocm_kv_append
 * with start_pos = ctx_lens - 1 and n_new = 1, then attends as
 * vspec_rocm_paged_decode_attention.  k_new, v_new: device [batch][num_kv_heads][head_dim]
 * in src_dtype (VSPEC_KV_F32 or VSPEC_KV_F16).  f16 and int4 pools do both in one kernel
 * launch; f32 pools launch the append first.  A batch of 0 is a no-op returning 1 (k_new
 * and v_new may then be NULL), as with every entry point here. */
int vspec_rocm_paged_decode_step(const VspecPagedAttnDesc* desc, const void* k_new, const void* v_new,
                                 int32_t src_dtype);

/* No counterpart in the reference: for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * vspec_rocm_paged_decode_step with its scratch (the partial states of work items split
 * over several workgroups) in a fixed 6 MiB device array that the library holds per GPU
 * for the life of the process; desc->workspace is ignored and nothing is allocated or
 * freed.  A plan whose partial states need more (vspec_rocm_paged_decode_workspace_bytes
 * above 6 MiB: chunked partitions of long batches, f32 pools split into many
 * partitions) is rejected with an error before any launch.  Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (other streams, other host threads)
 * race and must be serialised by the caller. */
int vspec_rocm_paged_decode_step_noalloc(const VspecPagedAttnDesc* desc, const void* k_new, const void* v_new,
                                         int32_t src_dtype);

/* Free the library workspaces that later, larger decodes replaced on the current device.
 * They are kept until this call because a captured HIP graph may still use them; call it
 * only when no such graph will be replayed again. */
int vspec_rocm_release_retired_workspaces(void);

/* ---- misc ---- */
int vspec_rocm_sync(void* stream);
const char* vspec_rocm_last_error(void);
int vspec_rocm_device_count(void);

/* The legacy contiguous-cache path (launch_attention with a host VspecKVCache*) keeps a
 * device mirror per cache.  By default every call uploads all current_tokens rows, as the
 * reference's per-call copies do (cuda_attention_f32.cu:108-110), so any in-place edit of
 * the caller's rows is seen.  A caller whose caches only grow by appends (kv_cache.c:160-226)
 * may switch to uploading only the rows appended since the previous call; the mirror then
 * still resyncs when current_tokens shrinks or the first or last synced row changes, but
 * other in-place rewrites of earlier rows go unseen.  enable: 1 appends only, 0 every row,
 * -1 back to the environment (VSPEC_ROCM_MIRROR_APPEND_ONLY, off when unset).  Process-wide;
 * returns the previous setting (1/0).  No counterpart in the reference. */
int vspec_rocm_cache_mirror_append_only(int enable);

/* Free the device mirror of a cache (call when the cache is destroyed); NULL releases
 * every mirror.  Returns 1. */
int vspec_rocm_release_cache_mirror(const VspecKVCache* cache);

/* ---- backend registry entry: replaces rocm_backend_stub.c:3-21 ----
 * launch_attention accepts either the reference context (ctx->input host q [H][D],
 * ctx->weight const VspecKVCache*, ctx->output host out [H][D]; cpu_backend.c:40-51)
 * or, with VSPEC_KCTX_FLAG_PAGED in ctx->config.flags, a VspecPagedAttnDesc* in
 * ctx->weight (device pointers).  launch_linear is out of scope and is a no-op that
 * records an error, like the stub it replaces.  Bad arguments are silent no-ops,
 * as in the reference, with the reason in vspec_rocm_last_error(). */
int vspec_rocm_backend_available(void);
VspecBackend vspec_make_rocm_backend(void);

#ifdef __cplusplus
}
#endif

#endif
