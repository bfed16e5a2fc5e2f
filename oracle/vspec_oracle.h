/*
 * vspec_oracle.h -- CPU restatement of the Vspec paged-KV decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP path is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  No product code links it.
 *
 * Every function names the reference file:line it restates (paths relative to
 * the reference repository root).  The restatement is written from scratch in
 * plain C11 + libm and follows the reference's operation order so that it is
 * bit-identical to the reference C path where the reference defines the
 * behaviour (pinned by tests/test_oracle_pin.py against oracle/_ref, the
 * reference's own sources compiled by oracle/Makefile).
 *
 * Formats the reference does not define (fp16 KV, int4 KV) are defined here
 * and in the product header include/vspec_rocm.h identically:
 *   fp16:  IEEE binary16, float->half by round-to-nearest-even, half->float exact.
 *   int4:  per (token, kv-head) groups of 32 elements; rep = 2nd-largest |x|
 *          (kv_cache.c:32-59 percentile 99.5 at n=32); scale = rep/8 (1.0 if
 *          rep==0), floored at 1e-6, rounded to fp16 (RNE, saturating at
 *          65504); code = clip(rint(x / float(scale16)), -8, 7), saturating
 *          (NaN -> -8); nibble-packed, even element in the low nibble
 *          (int4.c:31-37).
 */
#ifndef VSPEC_ORACLE_H
#define VSPEC_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------- fp16 ---------------- */
float vo_half_to_float(uint16_t h);          /* q4_k.c:6-34 */
uint16_t vo_float_to_half(float f);          /* IEEE RNE */
void vo_f16_to_f32(const uint16_t* src, float* dst, size_t n);
void vo_f32_to_f16(const float* src, uint16_t* dst, size_t n);

/* ---------------- deterministic host RNG ---------------- */
void vo_fill_normal(uint64_t seed, float* out, size_t n);
void vo_permutation(uint64_t seed, int32_t* out, size_t n);
void vo_uniform_int(uint64_t seed, int32_t lo, int32_t hi, int32_t* out, size_t n);

/* ---------------- bit packing (pack.c, int4.c) ---------------- */
size_t vo_quant_packed_bytes(size_t elements, uint8_t bits);
int8_t vo_quant_clip_signed(int8_t value, uint8_t bits);
void vo_quant_pack_signed(const int8_t* src, size_t elements, uint8_t bits, uint8_t* dst);
int8_t vo_quant_get_signed(const uint8_t* packed, size_t index, uint8_t bits);
void vo_quant_unpack_signed(const uint8_t* packed, size_t elements, uint8_t bits, int8_t* dst);
size_t vo_int4_packed_bytes(size_t elements);
void vo_int4_pack(const int8_t* src, size_t elements, uint8_t* dst);
int8_t vo_int4_get(const uint8_t* packed, size_t index);

/* ---------------- KV codecs ---------------- */
float vo_percentile_abs_block(const float* data, size_t n, float percentile);
/* int3 head codec of kv_cache.c:61-107 (fp32 scales, group 16|32). */
void vo_int3_quantize_head(const float* src, size_t head_dim, size_t block_size,
                           uint8_t* packed_out, float* scales_out);
void vo_int3_dequantize_head(const uint8_t* packed, const float* scales, size_t head_dim,
                             size_t block_size, float* out);
/* int4 head codec: groups of 32, fp16 scales.  head_dim % 32 == 0. */
void vo_int4_quantize_head(const float* src, size_t head_dim, uint8_t* codes_out,
                           uint16_t* scales_out);
void vo_int4_dequantize_head(const uint8_t* codes, const uint16_t* scales, size_t head_dim,
                             float* out);

/* ---------------- 3-bit runtime numerics (three_bit_runtime_modules.c) ----------------
 * The reference reads its mode from the environment on every call; here it is an
 * explicit argument:  mode 0 = "P" (VSPEC_3BIT_RUNTIME_MODULE unset),
 * mode 1 = "R" (set, as after vspec_runtime_init_default with the default config).
 * dot_block is VSPEC_3BIT_BLOCK_SIZE (32 or 64; anything else -> 64). */
void vo_dynamic_clamp_std(const float* input, size_t n, float alpha, float* output);
void vo_noise_reduce_vector(int mode, const float* input, size_t n, float* output);
float vo_accum_dot_f32(int mode, size_t dot_block, const float* a, const float* b, size_t n);
float vo_qk_score(int mode, size_t dot_block, const float* q, const float* k, size_t d,
                  float inv_sqrt_d);
void vo_softmax_apply(int mode, const float* logits, size_t n, float* probs);

/* ---------------- attention_ref.c ---------------- */
/* One head: q[D]; key row t at k + t*k_stride, value row t at v + t*v_stride. */
void vo_attention_head(int mode, size_t dot_block, const float* q, const float* k, size_t k_stride,
                       const float* v, size_t v_stride, size_t tokens, size_t head_dim, float* out);
/* attention_ref.c:7-88 over a contiguous [T][H][D] cache (MHA). */
void vo_attention_ref_single_query(int mode, size_t dot_block, const float* query,
                                   const float* key, const float* value, size_t tokens,
                                   size_t num_heads, size_t head_dim, float* out);

/* ---------------- paged block-table layout (the build's HBM format) ----------------
 * dtype: 0 = f32, 1 = f16, 2 = int4.
 * Element (block b, kv-head h, slot s, dim d):
 *   f32/f16 data index  ((b*H + h)*P + s)*D + d           (k_data / v_data)
 *   except f16 V        (b*H + h)*D*P + (s/4)*4*D + 4*d + s%4  (groups of 4 tokens)
 *   int4 K code byte    ((b*H + h)*P + s)*(D/2) + d/2     (nibble d&1)
 *   int4 V scale index  ((b*H + h)*P + s)*(D/32) + d/32   (v_scales, fp16 bits)
 *   int4 K scales and V codes: vo_int4_ks_index, vo_int4_v_byte (below)
 */
typedef struct VoPagedKV {
    int dtype;
    uint32_t num_blocks;
    uint32_t block_tokens;
    uint32_t num_kv_heads;
    uint32_t head_dim;
    void* k_data;
    void* v_data;
    uint16_t* k_scales;
    uint16_t* v_scales;
} VoPagedKV;

/* int4 pool addressing (block_tokens a multiple of 16): index of the K scale of
 * (block b, head h, slot, group) in k_scales, and byte offset of V element (slot, d)
 * in v_data (*high: 1 when it is the byte's high nibble).  K codes and V scales are
 * token-major rows. */
size_t vo_int4_ks_index(const VoPagedKV* kv, size_t b, size_t h, size_t slot, size_t group);
size_t vo_int4_v_byte(const VoPagedKV* kv, size_t b, size_t h, size_t slot, size_t d, int* high);

/* f16 pool addressing (block_tokens a multiple of 16): index (in halves) of V element
 * (slot, d) of block b, head h in v_data: groups of 4 tokens, d-major inside a group.
 * K is token-major. */
size_t vo_f16_v_index(const VoPagedKV* kv, size_t b, size_t h, size_t slot, size_t d);

/* Append n_new tokens per sequence at logical positions start_pos[b] .. +n_new-1.
 * k_new/v_new: [B][n_new][H][D] in src_dtype (0 f32, 1 f16).  Returns 1/0. */
int vo_paged_append(const VoPagedKV* kv, uint32_t batch, const int32_t* block_tables,
                    uint32_t max_blocks_per_seq, const int32_t* start_pos, uint32_t n_new,
                    const void* k_new, const void* v_new, int src_dtype);

/* Rotary embedding of one row (runtime_inference.py:1307-1311): pairs (i, i + rope_dim/2)
 * of the first rope_dim elements rotate by (cos_row[i], sin_row[i]) with separately
 * rounded fp32 products and sums; the rest pass through. */
void vo_rope_row(const float* x, float* out, size_t d, size_t rope_dim, const float* cos_row,
                 const float* sin_row);

/* vo_paged_append with K rotated first: token position t uses row t of the
 * [max_pos][rope_dim/2] cos/sin tables (V is stored as given). */
int vo_paged_append_rope(const VoPagedKV* kv, uint32_t batch, const int32_t* block_tables,
                         uint32_t max_blocks_per_seq, const int32_t* start_pos, uint32_t n_new,
                         const void* k_new, const void* v_new, int src_dtype, const float* rope_cos,
                         const float* rope_sin, size_t rope_dim, size_t max_pos);

/* Gather through the block table into per-sequence [T][H][D] (capi.c:2263-2299 order).
 * Sequences are concatenated; sequence b starts at token out_token_offset[b].
 * out_mode 0: raw pool format (f32/f16 elements; int4 codes [T][H][D/2] + scales
 * [T][H][D/32]); out_mode 1: dequantised f32. */
int vo_paged_gather(const VoPagedKV* kv, uint32_t batch, const int32_t* block_tables,
                    uint32_t max_blocks_per_seq, const int32_t* ctx_lens,
                    const int64_t* out_token_offset, int out_mode, void* out_k, void* out_v,
                    uint16_t* out_k_scales, uint16_t* out_v_scales);

/* Copy whole physical blocks (all heads, data and scales): dst[i] <- src[i]. */
int vo_paged_compact(const VoPagedKV* kv, uint32_t n, const int32_t* src_blocks,
                     const int32_t* dst_blocks);

/* GQA single-query decode attention over the paged cache: for each sequence b and
 * query head hq, kv head = hq / (Hq/Hkv); the head's tokens are gathered to fp32 and
 * fed to vo_attention_head.  q, out: [B][Hq][D] f32. */
int vo_paged_decode_attention(int mode, size_t dot_block, const VoPagedKV* kv, uint32_t batch,
                              uint32_t num_q_heads, const int32_t* block_tables,
                              uint32_t max_blocks_per_seq, const int32_t* ctx_lens,
                              const float* q, float* out);

/* Scale-free textbook attention in double (no clamp): used only by tests to pin
 * the oracle through the identity "clamp never fires". */
void vo_attention_textbook_f64(const float* q, const float* k, size_t k_stride, const float* v,
                               size_t v_stride, size_t tokens, size_t head_dim, double* out);

#ifdef __cplusplus
}
#endif

#endif
