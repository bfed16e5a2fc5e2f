/*
 * vspec_oracle.c -- CPU restatement of the Vspec paged-KV decode path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the thing measured or shipped).
 * See vspec_oracle.h for the contract and the formats defined here.
 * Reference citations are file:line in the reference repository.
 */
#include "vspec_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ======================================================================== */
/* fp16                                                                      */
/* ======================================================================== */

/* Exact binary16 -> binary32.  Same case split as q4_k.c:6-34
 * (zero / subnormal renormalised / inf-nan / normal). */
float vo_half_to_float(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
    const uint32_t f = (uint32_t)h & 0x3ffu;
    uint32_t bits;
    if (e == 0u) {
        if (f == 0u) {
            bits = sign;
        } else {
            /* value = f * 2^-24; normalise the mantissa */
            uint32_t m = f;
            uint32_t exp32 = 127u - 14u; /* exponent of 2^-14 */
            while ((m & 0x400u) == 0u) {
                m <<= 1;
                exp32 -= 1u;
            }
            bits = sign | (exp32 << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (e == 31u) {
        bits = sign | 0x7f800000u | (f << 13);
    } else {
        bits = sign | ((e - 15u + 127u) << 23) | (f << 13);
    }
    float out;
    memcpy(&out, &bits, sizeof(out));
    return out;
}

/* binary32 -> binary16, round to nearest, ties to even; overflow -> inf;
 * NaN -> quiet NaN keeping the top payload bits. */
uint16_t vo_float_to_half(float value) {
    uint32_t x;
    memcpy(&x, &value, sizeof(x));
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {
        if (ax > 0x7f800000u) {
            return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
        }
        return (uint16_t)(sign | 0x7c00u);
    }
    const int e = (int)(ax >> 23) - 127;
    const uint32_t m = ax & 0x7fffffu;
    if (e >= -14) {
        uint32_t hm = m >> 13;
        const uint32_t rem = m & 0x1fffu;
        uint32_t h = ((uint32_t)(e + 15) << 10) + hm;
        if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) {
            h += 1u; /* carries into the exponent correctly */
        }
        if (h >= 0x7c00u) {
            h = 0x7c00u;
        }
        return (uint16_t)(sign | h);
    }
    /* subnormal half: value = M * 2^(e-23), in units of 2^-24 -> M >> (-e-1) */
    const int s = -e - 1;
    if (s > 24) {
        return (uint16_t)sign;
    }
    const uint32_t full = m | 0x800000u;
    const uint32_t q = full >> s;
    const uint32_t rem = full & ((1u << s) - 1u);
    const uint32_t half = 1u << (s - 1);
    uint32_t h = q;
    if (rem > half || (rem == half && (q & 1u))) {
        h += 1u;
    }
    return (uint16_t)(sign | h);
}

void vo_f16_to_f32(const uint16_t* src, float* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        dst[i] = vo_half_to_float(src[i]);
    }
}

void vo_f32_to_f16(const float* src, uint16_t* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        dst[i] = vo_float_to_half(src[i]);
    }
}

/* ======================================================================== */
/* RNG: splitmix64 stream, Box-Muller in double                              */
/* ======================================================================== */

static uint64_t vo_splitmix64(uint64_t* state) {
    uint64_t z = (*state += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

void vo_fill_normal(uint64_t seed, float* out, size_t n) {
    uint64_t st = seed;
    const double two_pi = 6.283185307179586476925286766559;
    size_t i = 0;
    while (i < n) {
        const double u1 = ((double)(vo_splitmix64(&st) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
        const double u2 = (double)(vo_splitmix64(&st) >> 11) * (1.0 / 9007199254740992.0);
        const double r = sqrt(-2.0 * log(u1));
        out[i++] = (float)(r * cos(two_pi * u2));
        if (i < n) {
            out[i++] = (float)(r * sin(two_pi * u2));
        }
    }
}

void vo_permutation(uint64_t seed, int32_t* out, size_t n) {
    uint64_t st = seed;
    for (size_t i = 0; i < n; ++i) {
        out[i] = (int32_t)i;
    }
    for (size_t i = n; i > 1; --i) {
        const size_t j = (size_t)(vo_splitmix64(&st) % (uint64_t)i);
        const int32_t t = out[i - 1];
        out[i - 1] = out[j];
        out[j] = t;
    }
}

void vo_uniform_int(uint64_t seed, int32_t lo, int32_t hi, int32_t* out, size_t n) {
    uint64_t st = seed;
    const uint64_t span = (uint64_t)((int64_t)hi - (int64_t)lo + 1);
    for (size_t i = 0; i < n; ++i) {
        out[i] = (int32_t)((int64_t)lo + (int64_t)(vo_splitmix64(&st) % span));
    }
}

/* ======================================================================== */
/* bit packing                                                               */
/* ======================================================================== */

static int vo_valid_bits(uint8_t bits) { return bits >= 2u && bits <= 4u; }

/* pack.c:11-16 */
size_t vo_quant_packed_bytes(size_t elements, uint8_t bits) {
    if (!vo_valid_bits(bits) || elements == 0u) {
        return 0u;
    }
    return (elements * (size_t)bits + 7u) / 8u;
}

/* pack.c:18-28 */
int8_t vo_quant_clip_signed(int8_t value, uint8_t bits) {
    if (!vo_valid_bits(bits)) {
        return 0;
    }
    const int lo = -(1 << (bits - 1u));
    const int hi = (1 << (bits - 1u)) - 1;
    if (value < lo) return (int8_t)lo;
    if (value > hi) return (int8_t)hi;
    return value;
}

/* pack.c:30-51: element i occupies bits [i*b, i*b+b) of a little-endian stream. */
void vo_quant_pack_signed(const int8_t* src, size_t elements, uint8_t bits, uint8_t* dst) {
    if (!src || !dst || !vo_valid_bits(bits)) {
        return;
    }
    memset(dst, 0, vo_quant_packed_bytes(elements, bits));
    const uint32_t mask = (1u << bits) - 1u;
    for (size_t i = 0; i < elements; ++i) {
        const uint32_t code = (uint32_t)(uint8_t)vo_quant_clip_signed(src[i], bits) & mask;
        const size_t pos = i * bits;
        const uint32_t sh = (uint32_t)(pos & 7u);
        dst[pos >> 3] |= (uint8_t)(code << sh);
        if (sh + bits > 8u) {
            dst[(pos >> 3) + 1u] |= (uint8_t)(code >> (8u - sh));
        }
    }
}

/* pack.c:53-74 (sign-extending read) */
int8_t vo_quant_get_signed(const uint8_t* packed, size_t index, uint8_t bits) {
    if (!packed || !vo_valid_bits(bits)) {
        return 0;
    }
    const size_t pos = index * bits;
    const uint32_t sh = (uint32_t)(pos & 7u);
    uint32_t code = (uint32_t)packed[pos >> 3] >> sh;
    if (sh + bits > 8u) {
        code |= (uint32_t)packed[(pos >> 3) + 1u] << (8u - sh);
    }
    code &= (1u << bits) - 1u;
    if (code & (1u << (bits - 1u))) {
        return (int8_t)((int)code - (1 << bits));
    }
    return (int8_t)code;
}

void vo_quant_unpack_signed(const uint8_t* packed, size_t elements, uint8_t bits, int8_t* dst) {
    if (!packed || !dst || !vo_valid_bits(bits)) {
        return;
    }
    for (size_t i = 0; i < elements; ++i) {
        dst[i] = vo_quant_get_signed(packed, i, bits);
    }
}

/* int4.c:7-9 */
size_t vo_int4_packed_bytes(size_t elements) { return (elements + 1u) / 2u; }

/* int4.c:11-37: even index -> low nibble, odd -> high nibble, clip to [-8,7] */
void vo_int4_pack(const int8_t* src, size_t elements, uint8_t* dst) {
    if (!src || !dst) {
        return;
    }
    for (size_t i = 0; i < elements; i += 2u) {
        int lo = src[i] < -8 ? -8 : (src[i] > 7 ? 7 : src[i]);
        int hi = 0;
        if (i + 1u < elements) {
            hi = src[i + 1u] < -8 ? -8 : (src[i + 1u] > 7 ? 7 : src[i + 1u]);
            hi = (hi & 0xf) << 4;
        }
        dst[i / 2u] = (uint8_t)((lo & 0xf) | hi);
    }
}

/* int4.c:39-45 */
int8_t vo_int4_get(const uint8_t* packed, size_t index) {
    const uint32_t b = packed[index / 2u];
    const uint32_t nib = (index & 1u) ? ((b >> 4) & 0xfu) : (b & 0xfu);
    return (int8_t)((nib & 8u) ? (int)nib - 16 : (int)nib);
}

/* ======================================================================== */
/* KV codecs                                                                 */
/* ======================================================================== */

/* kv_cache.c:32-59: |x| of at most 32 values, ascending order statistic at
 * floor((n-1) * pct/100).  Selection by insertion sort gives the same element
 * as qsort for finite inputs. */
float vo_percentile_abs_block(const float* data, size_t n, float percentile) {
    if (!data || n == 0u) {
        return 0.0f;
    }
    if (percentile < 50.0f) percentile = 50.0f;
    if (percentile > 100.0f) percentile = 100.0f;
    if (n > 32u) n = 32u;
    float t[32];
    for (size_t i = 0; i < n; ++i) {
        const float a = fabsf(data[i]);
        size_t j = i;
        while (j > 0 && t[j - 1] > a) {
            t[j] = t[j - 1];
            --j;
        }
        t[j] = a;
    }
    size_t idx = (size_t)((double)(n - 1u) * ((double)percentile / 100.0));
    if (idx >= n) idx = n - 1u;
    return t[idx];
}

/* kv_cache.c:61-107.  Note the reference narrows lrintf's result to int8_t
 * before clipping (:100-101); this restatement keeps that behaviour. */
void vo_int3_quantize_head(const float* src, size_t head_dim, size_t block_size,
                           uint8_t* packed_out, float* scales_out) {
    if (!src || !packed_out || !scales_out || head_dim == 0u) {
        return;
    }
    const size_t blocks = (head_dim + block_size - 1u) / block_size;
    int8_t q[1024] = {0};
    int8_t* qt = head_dim <= 1024u ? q : (int8_t*)malloc(head_dim);
    if (!qt) {
        return;
    }
    for (size_t b = 0; b < blocks; ++b) {
        const size_t base = b * block_size;
        size_t len = block_size;
        if (base + len > head_dim) len = head_dim - base;
        const float rep = vo_percentile_abs_block(src + base, len, 99.5f);
        float scale = (rep > 0.0f) ? (rep / 4.0f) : 1.0f;
        if (scale < 1e-6f) scale = 1e-6f;
        scales_out[b] = scale;
        for (size_t i = 0; i < len; ++i) {
            const float v = src[base + i] / scale;
            const int qi = (int)lrintf(v);
            qt[base + i] = vo_quant_clip_signed((int8_t)qi, 3u);
        }
    }
    vo_quant_pack_signed(qt, head_dim, 3u, packed_out);
    if (qt != q) free(qt);
}

/* kv_cache.c:109-126 */
void vo_int3_dequantize_head(const uint8_t* packed, const float* scales, size_t head_dim,
                             size_t block_size, float* out) {
    for (size_t i = 0; i < head_dim; ++i) {
        out[i] = (float)vo_quant_get_signed(packed, i, 3u) * scales[i / block_size];
    }
}

/* int4 KV codec, the b=4 generalisation of kv_cache.c:61-107 with fp16 scales
 * and a saturating clip. */
void vo_int4_quantize_head(const float* src, size_t head_dim, uint8_t* codes_out,
                           uint16_t* scales_out) {
    const size_t groups = head_dim / 32u;
    for (size_t g = 0; g < groups; ++g) {
        const float* x = src + g * 32u;
        const float rep = vo_percentile_abs_block(x, 32u, 99.5f);
        float scale = (rep > 0.0f) ? (rep / 8.0f) : 1.0f;
        if (scale < 1e-6f) scale = 1e-6f;
        uint16_t s16 = vo_float_to_half(scale);
        if ((s16 & 0x7fffu) >= 0x7c00u) s16 = 0x7bffu; /* saturate at 65504 */
        scales_out[g] = s16;
        const float sc = vo_half_to_float(s16);
        for (size_t i = 0; i < 32u; i += 2u) {
            int code[2];
            for (int k = 0; k < 2; ++k) {
                const float r = rintf(x[i + (size_t)k] / sc);
                code[k] = (r > 7.0f) ? 7 : ((r >= -8.0f) ? (int)r : -8);
            }
            codes_out[(g * 32u + i) / 2u] = (uint8_t)((code[0] & 0xf) | ((code[1] & 0xf) << 4));
        }
    }
}

void vo_int4_dequantize_head(const uint8_t* codes, const uint16_t* scales, size_t head_dim,
                             float* out) {
    for (size_t i = 0; i < head_dim; ++i) {
        out[i] = (float)vo_int4_get(codes, i) * vo_half_to_float(scales[i / 32u]);
    }
}

/* ======================================================================== */
/* 3-bit runtime numerics                                                    */
/* ======================================================================== */

static float vo_clipf(float x, float lo, float hi) {
    if (x < lo) return lo;
    if (x > hi) return hi;
    return x;
}

typedef struct VoAccum {
    double sum;
    double comp;
} VoAccum;

/* three_bit_runtime_modules.c:260-282 (compensation limit 1e7, :104) */
static void vo_accum_add(int mode, VoAccum* s, float value) {
    if (!mode) {
        s->sum += (double)value;
        return;
    }
    const double y = (double)value - s->comp;
    const double t = s->sum + y;
    s->comp = (t - s->sum) - y;
    s->sum = t;
    if (fabs(s->sum) > (double)1e7f) {
        s->sum = vo_clipf((float)s->sum, -1e7f, 1e7f);
        s->comp = 0.0;
    }
}

/* three_bit_runtime_modules.c:175-203: mean and population variance in double,
 * threshold max(1e-6, |alpha| * float(sqrt(var))), clip to [-th, th]. */
void vo_dynamic_clamp_std(const float* input, size_t n, float alpha, float* output) {
    if (!input || !output || n == 0u) {
        return;
    }
    double mean = 0.0;
    for (size_t i = 0; i < n; ++i) mean += (double)input[i];
    mean /= (double)n;
    double var = 0.0;
    for (size_t i = 0; i < n; ++i) {
        const double d = (double)input[i] - mean;
        var += d * d;
    }
    var /= (double)n;
    const float sd = (float)sqrt(var);
    const float th = fmaxf(1e-6f, fabsf(alpha) * sd);
    for (size_t i = 0; i < n; ++i) output[i] = vo_clipf(input[i], -th, th);
}

/* three_bit_runtime_modules.c:138-173 with the defaults of :108-117
 * (input_clip 16, smooth_alpha 0, outlier_threshold 32). */
void vo_noise_reduce_vector(int mode, const float* input, size_t n, float* output) {
    if (!input || !output || n == 0u) {
        return;
    }
    if (!mode) {
        for (size_t i = 0; i < n; ++i) output[i] = input[i];
        return;
    }
    const float clip = 16.0f;
    const float outlier = 32.0f;
    float prev = vo_clipf(input[0], -clip, clip);
    output[0] = prev;
    for (size_t i = 1; i < n; ++i) {
        float v = vo_clipf(input[i], -clip, clip);
        const float delta = v - prev;
        if (fabsf(delta) > outlier) v = prev + ((delta > 0.0f) ? outlier : -outlier);
        output[i] = v;
        prev = v;
    }
}

/* three_bit_runtime_modules.c:41-46 */
static size_t vo_resolve_block(size_t b) { return (b == 32u || b == 64u) ? b : 64u; }

/* three_bit_runtime_modules.c:291-342 */
float vo_accum_dot_f32(int mode, size_t dot_block, const float* a, const float* b, size_t n) {
    if (!a || !b || n == 0u) {
        return 0.0f;
    }
    if (!mode) {
        float out = 0.0f;
        for (size_t i = 0; i < n; ++i) out += a[i] * b[i];
        return out;
    }
    const size_t blk = vo_resolve_block(dot_block == 0u ? 64u : dot_block);
    VoAccum total = {0.0, 0.0};
    for (size_t base = 0; base < n; base += blk) {
        const size_t end = base + blk > n ? n : base + blk;
        float babs = 0.0f;
        for (size_t i = base; i < end; ++i) {
            const float av = fabsf(a[i]);
            const float bv = fabsf(b[i]);
            if (av > babs) babs = av;
            if (bv > babs) babs = bv;
        }
        const float bs = fmaxf(babs, 1e-6f);
        VoAccum local = {0.0, 0.0};
        for (size_t i = base; i < end; ++i) {
            const float an = a[i] / bs;
            const float bn = b[i] / bs;
            vo_accum_add(mode, &local, an * bn);
        }
        vo_accum_add(mode, &total, (float)local.sum * bs * bs);
    }
    return (float)total.sum;
}

/* three_bit_runtime_modules.c:344-361 (qk scale clip [1e-4, 32], :127-128) */
float vo_qk_score(int mode, size_t dot_block, const float* q, const float* k, size_t d,
                  float inv_sqrt_d) {
    if (!q || !k || d == 0u) {
        return 0.0f;
    }
    const float score = vo_accum_dot_f32(mode, dot_block, q, k, d);
    float scale = inv_sqrt_d;
    if (mode) scale = vo_clipf(scale, 1e-4f, 32.0f);
    return score * scale;
}

/* three_bit_runtime_modules.c:205-250 (logit clip 24, temperature floor 0.85,
 * min_denom 1e-12; :89-97) */
void vo_softmax_apply(int mode, const float* logits, size_t n, float* probs) {
    if (!logits || !probs || n == 0u) {
        return;
    }
    const float temp = mode ? vo_clipf(1.0f, 0.85f, 1.0f) : 1.0f;
    const float inv_temp = 1.0f / fmaxf(1e-6f, temp);
    float max_v = -FLT_MAX;
    for (size_t i = 0; i < n; ++i) {
        float v = logits[i] * inv_temp;
        if (mode) v = vo_clipf(v, -24.0f, 24.0f);
        probs[i] = v;
        if (v > max_v) max_v = v;
    }
    double denom = 0.0;
    for (size_t i = 0; i < n; ++i) {
        const float ex = expf(probs[i] - max_v);
        probs[i] = ex;
        denom += (double)ex;
    }
    if (denom < (double)fmaxf(1e-12f, 1e-30f)) {
        const float u = 1.0f / (float)n;
        for (size_t i = 0; i < n; ++i) probs[i] = u;
        return;
    }
    const float inv = 1.0f / (float)denom;
    for (size_t i = 0; i < n; ++i) probs[i] *= inv;
}

/* ======================================================================== */
/* attention_ref.c                                                           */
/* ======================================================================== */

/* attention_ref.c:23-87 for one head. */
void vo_attention_head(int mode, size_t dot_block, const float* q, const float* k, size_t k_stride,
                       const float* v, size_t v_stride, size_t tokens, size_t head_dim,
                       float* out) {
    if (!q || !k || !v || !out || tokens == 0u) {
        return;
    }
    const size_t d = head_dim;
    const float inv_sqrt_d = 1.0f / sqrtf((float)d);
    float* scores = (float*)malloc(tokens * sizeof(float));
    float* qc = (float*)malloc(d * sizeof(float));
    float* qd = (float*)malloc(d * sizeof(float));
    float* kc = (float*)malloc(d * sizeof(float));
    float* kd = (float*)malloc(d * sizeof(float));
    VoAccum* acc = (VoAccum*)calloc(d, sizeof(VoAccum));
    if (!scores || !qc || !qd || !kc || !kd || !acc) {
        free(scores); free(qc); free(qd); free(kc); free(kd); free(acc);
        return;
    }
    for (size_t x = 0; x < d; ++x) out[x] = 0.0f;
    vo_dynamic_clamp_std(q, d, 4.5f, qc);
    vo_noise_reduce_vector(mode, qc, d, qd);
    for (size_t t = 0; t < tokens; ++t) {
        vo_dynamic_clamp_std(k + t * k_stride, d, 4.5f, kc);
        vo_noise_reduce_vector(mode, kc, d, kd);
        scores[t] = vo_qk_score(mode, dot_block, qd, kd, d, inv_sqrt_d);
    }
    vo_softmax_apply(mode, scores, tokens, scores);
    for (size_t t = 0; t < tokens; ++t) {
        const float w = scores[t];
        const float* vr = v + t * v_stride;
        for (size_t x = 0; x < d; ++x) vo_accum_add(mode, &acc[x], w * vr[x]);
    }
    for (size_t x = 0; x < d; ++x) out[x] = (float)acc[x].sum;
    free(scores); free(qc); free(qd); free(kc); free(kd); free(acc);
}

/* attention_ref.c:7-88: MHA over VspecKVCache [T][H][D] (key_at offset (t*H+h)*D,
 * kv_cache.c:326-328). */
void vo_attention_ref_single_query(int mode, size_t dot_block, const float* query,
                                   const float* key, const float* value, size_t tokens,
                                   size_t num_heads, size_t head_dim, float* out) {
    if (!query || !key || !value || !out || tokens == 0u) {
        return;
    }
    const size_t stride = num_heads * head_dim;
    for (size_t h = 0; h < num_heads; ++h) {
        vo_attention_head(mode, dot_block, query + h * head_dim, key + h * head_dim, stride,
                          value + h * head_dim, stride, tokens, head_dim, out + h * head_dim);
    }
}

void vo_attention_textbook_f64(const float* q, const float* k, size_t k_stride, const float* v,
                               size_t v_stride, size_t tokens, size_t head_dim, double* out) {
    double* s = (double*)malloc(tokens * sizeof(double));
    if (!s) return;
    double m = -INFINITY;
    for (size_t t = 0; t < tokens; ++t) {
        double acc = 0.0;
        for (size_t x = 0; x < head_dim; ++x) acc += (double)q[x] * (double)k[t * k_stride + x];
        s[t] = acc / sqrt((double)head_dim);
        if (s[t] > m) m = s[t];
    }
    double den = 0.0;
    for (size_t t = 0; t < tokens; ++t) {
        s[t] = exp(s[t] - m);
        den += s[t];
    }
    for (size_t x = 0; x < head_dim; ++x) {
        double acc = 0.0;
        for (size_t t = 0; t < tokens; ++t) acc += s[t] * (double)v[t * v_stride + x];
        out[x] = acc / den;
    }
    free(s);
}

/* ======================================================================== */
/* paged block-table layout                                                  */
/* ======================================================================== */

static size_t vo_row_index(const VoPagedKV* kv, size_t block, size_t head, size_t slot) {
    return (block * kv->num_kv_heads + head) * kv->block_tokens + slot;
}

static int vo_kv_valid(const VoPagedKV* kv) {
    if (!kv || !kv->k_data || !kv->v_data || kv->num_blocks == 0u || kv->block_tokens == 0u ||
        kv->num_kv_heads == 0u || kv->head_dim == 0u || kv->dtype < 0 || kv->dtype > 2) {
        return 0;
    }
    if (kv->dtype == 2 && (kv->head_dim % 32u != 0u || kv->head_dim > 1024u ||
                           kv->block_tokens % 16u != 0u || !kv->k_scales || !kv->v_scales)) {
        return 0;
    }
    if (kv->dtype == 1 && kv->block_tokens % 16u != 0u) return 0; /* f16 V in 16-token tiles */
    return 1;
}

/* Logical token (b, t) -> physical row (block, slot); -1 when out of range. */
static long vo_phys_block(const VoPagedKV* kv, const int32_t* block_tables, uint32_t max_blocks,
                          uint32_t b, size_t t) {
    const size_t lb = t / kv->block_tokens;
    if (lb >= max_blocks) return -1;
    const int32_t pb = block_tables[(size_t)b * max_blocks + lb];
    if (pb < 0 || (uint32_t)pb >= kv->num_blocks) return -1;
    return (long)pb;
}

/* f16 V: per (block b, head h), groups of 4 tokens; element (d, slot) at
 *   (b*H + h)*D*P + (slot/4)*4*D + 4*d + slot%4      (vo_f16_v_index; P a multiple of 16)
 * int4 pools (block_tokens a multiple of 16):
 *   K codes: token-major rows of D/2 bytes, element e in nibble e%2 of byte e/2;
 *   K scales: group-major, scale (group c, slot) at ((b*H + h)*G + c)*P + slot;
 *   V codes: 16-token tiles of 8*D bytes; element d of the token at tile position
 *            t = 4*g + r sits in byte (g*16 + d%16)*(D/8) + 4*(d/32) + 2*(r&1) + (r>>1)
 *            of its tile, low nibble when (d/16) is even, high nibble otherwise;
 *   V scales: token-major rows of G scales.
 * Every other array is token-major (row index (b*H + h)*P + slot). */
static int vo_v_grouped(const VoPagedKV* kv, int is_v) { return is_v && kv->dtype == 1; }

size_t vo_f16_v_index(const VoPagedKV* kv, size_t b, size_t h, size_t slot, size_t d) {
    const size_t D = kv->head_dim, P = kv->block_tokens;
    return (b * kv->num_kv_heads + h) * D * P + (slot / 4u) * 4u * D + 4u * d + slot % 4u;
}

size_t vo_int4_ks_index(const VoPagedKV* kv, size_t b, size_t h, size_t slot, size_t group) {
    const size_t G = kv->head_dim / 32u;
    return ((b * kv->num_kv_heads + h) * G + group) * kv->block_tokens + slot;
}

size_t vo_int4_v_byte(const VoPagedKV* kv, size_t b, size_t h, size_t slot, size_t d, int* high) {
    const size_t D = kv->head_dim, P = kv->block_tokens;
    const size_t t = slot % 16u, g = t / 4u, r = t % 4u;
    *high = (int)((d / 16u) & 1u);
    return (b * kv->num_kv_heads + h) * (P * D / 2u) + (slot / 16u) * (8u * D) +
           (g * 16u + d % 16u) * (D / 8u) + 4u * (d / 32u) + 2u * (r & 1u) + (r >> 1);
}

/* Canonical packed row (D/2 bytes, element e in nibble e%2 of byte e/2) <-> pool. */
static void vo_int4_put_row(const VoPagedKV* kv, int is_v, size_t b, size_t h, size_t slot,
                            const uint8_t* codes, const uint16_t* sc) {
    const size_t D = kv->head_dim, G = D / 32u;
    const size_t row = vo_row_index(kv, b, h, slot);
    if (!is_v) {
        memcpy((uint8_t*)kv->k_data + row * (D / 2u), codes, D / 2u);
        for (size_t c = 0; c < G; ++c) kv->k_scales[vo_int4_ks_index(kv, b, h, slot, c)] = sc[c];
        return;
    }
    uint8_t* v = (uint8_t*)kv->v_data;
    for (size_t d = 0; d < D; ++d) {
        int high = 0;
        const size_t at = vo_int4_v_byte(kv, b, h, slot, d, &high);
        const uint8_t nib = (uint8_t)((codes[d / 2u] >> (4u * (d % 2u))) & 0xfu);
        v[at] = high ? (uint8_t)((v[at] & 0x0fu) | (nib << 4)) : (uint8_t)((v[at] & 0xf0u) | nib);
    }
    memcpy(kv->v_scales + row * G, sc, G * 2u);
}

static void vo_int4_get_row(const VoPagedKV* kv, int is_v, size_t b, size_t h, size_t slot,
                            uint8_t* codes, uint16_t* sc) {
    const size_t D = kv->head_dim, G = D / 32u;
    const size_t row = vo_row_index(kv, b, h, slot);
    if (!is_v) {
        memcpy(codes, (const uint8_t*)kv->k_data + row * (D / 2u), D / 2u);
        for (size_t c = 0; c < G; ++c) sc[c] = kv->k_scales[vo_int4_ks_index(kv, b, h, slot, c)];
        return;
    }
    const uint8_t* v = (const uint8_t*)kv->v_data;
    memset(codes, 0, D / 2u);
    for (size_t d = 0; d < D; ++d) {
        int high = 0;
        const size_t at = vo_int4_v_byte(kv, b, h, slot, d, &high);
        const uint8_t nib = (uint8_t)(high ? (v[at] >> 4) : (v[at] & 0xfu));
        codes[d / 2u] |= (uint8_t)(nib << (4u * (d % 2u)));
    }
    memcpy(sc, kv->v_scales + row * G, G * 2u);
}

/* Write one token-head row (D elements) from fp32 values into the pool. */
static void vo_store_row(const VoPagedKV* kv, int is_v, size_t b, size_t h, size_t slot,
                         const float* src) {
    const size_t D = kv->head_dim;
    void* data = is_v ? kv->v_data : kv->k_data;
    uint16_t* scales = is_v ? kv->v_scales : kv->k_scales;
    const size_t row = vo_row_index(kv, b, h, slot);
    if (vo_v_grouped(kv, is_v)) {
        uint16_t* t = (uint16_t*)data;
        for (size_t d = 0; d < D; ++d) t[vo_f16_v_index(kv, b, h, slot, d)] = vo_float_to_half(src[d]);
    } else if (kv->dtype == 0) {
        memcpy((float*)data + row * D, src, D * sizeof(float));
    } else if (kv->dtype == 1) {
        vo_f32_to_f16(src, (uint16_t*)data + row * D, D);
    } else {
        uint8_t codes[512];
        uint16_t sc[32];
        (void)data;
        (void)scales;
        vo_int4_quantize_head(src, D, codes, sc);
        vo_int4_put_row(kv, is_v, b, h, slot, codes, sc);
    }
}

/* Read one token-head row from the pool as fp32 (exact for all three formats). */
static void vo_load_row(const VoPagedKV* kv, int is_v, size_t b, size_t h, size_t slot,
                        float* dst) {
    const size_t D = kv->head_dim;
    const void* data = is_v ? kv->v_data : kv->k_data;
    const uint16_t* scales = is_v ? kv->v_scales : kv->k_scales;
    const size_t row = vo_row_index(kv, b, h, slot);
    if (vo_v_grouped(kv, is_v)) {
        const uint16_t* t = (const uint16_t*)data;
        for (size_t d = 0; d < D; ++d) dst[d] = vo_half_to_float(t[vo_f16_v_index(kv, b, h, slot, d)]);
    } else if (kv->dtype == 0) {
        memcpy(dst, (const float*)data + row * D, D * sizeof(float));
    } else if (kv->dtype == 1) {
        vo_f16_to_f32((const uint16_t*)data + row * D, dst, D);
    } else {
        uint8_t codes[512];
        uint16_t sc[32];
        (void)data;
        (void)scales;
        vo_int4_get_row(kv, is_v, b, h, slot, codes, sc);
        vo_int4_dequantize_head(codes, sc, D, dst);
    }
}

/* Raw (pool-format) copy of one token-head row into a token-major output row. */
static void vo_copy_row_raw(const VoPagedKV* kv, int is_v, size_t b, size_t h, size_t slot,
                            void* out_row, uint16_t* out_scales) {
    const size_t D = kv->head_dim, G = D / 32u;
    const void* data = is_v ? kv->v_data : kv->k_data;
    const uint16_t* scales = is_v ? kv->v_scales : kv->k_scales;
    const size_t row = vo_row_index(kv, b, h, slot);
    if (vo_v_grouped(kv, is_v)) {
        const uint16_t* t = (const uint16_t*)data;
        for (size_t d = 0; d < D; ++d) ((uint16_t*)out_row)[d] = t[vo_f16_v_index(kv, b, h, slot, d)];
    } else if (kv->dtype == 0) {
        memcpy(out_row, (const float*)data + row * D, D * 4u);
    } else if (kv->dtype == 1) {
        memcpy(out_row, (const uint16_t*)data + row * D, D * 2u);
    } else {
        (void)data;
        (void)scales;
        (void)G;
        vo_int4_get_row(kv, is_v, b, h, slot, (uint8_t*)out_row, out_scales);
    }
}

/* Rotary embedding of one row, runtime_inference.py:1307-1311 (and _apply_rotary,
 * :621-636; _apply_partial_rotary, :1096-1106): pairs (i, i + half) of the first
 * rope_dim elements, half = rope_dim / 2, become (x1*c - x2*s, x1*s + x2*c) with
 * c = cos_row[i], s = sin_row[i], each product and sum rounded to fp32 as numpy's
 * elementwise float32 arithmetic does; elements past rope_dim pass through. */
void vo_rope_row(const float* x, float* out, size_t d, size_t rope_dim, const float* cos_row,
                 const float* sin_row) {
    const size_t half = rope_dim / 2u;
    for (size_t i = 0; i < d; ++i) out[i] = x[i];
    /* built with -ffp-contract=off: every product and sum is rounded separately */
    for (size_t i = 0; i < half; ++i) {
        out[i] = x[i] * cos_row[i] - x[i + half] * sin_row[i];
        out[i + half] = x[i] * sin_row[i] + x[i + half] * cos_row[i];
    }
}

static int vo_paged_append_impl(const VoPagedKV* kv, uint32_t batch, const int32_t* block_tables,
                                uint32_t max_blocks_per_seq, const int32_t* start_pos, uint32_t n_new,
                                const void* k_new, const void* v_new, int src_dtype,
                                const float* rope_cos, const float* rope_sin, size_t rope_dim,
                                size_t max_pos);

int vo_paged_append(const VoPagedKV* kv, uint32_t batch, const int32_t* block_tables,
                    uint32_t max_blocks_per_seq, const int32_t* start_pos, uint32_t n_new,
                    const void* k_new, const void* v_new, int src_dtype) {
    return vo_paged_append_impl(kv, batch, block_tables, max_blocks_per_seq, start_pos, n_new, k_new,
                                v_new, src_dtype, NULL, NULL, 0, 0);
}

int vo_paged_append_rope(const VoPagedKV* kv, uint32_t batch, const int32_t* block_tables,
                         uint32_t max_blocks_per_seq, const int32_t* start_pos, uint32_t n_new,
                         const void* k_new, const void* v_new, int src_dtype, const float* rope_cos,
                         const float* rope_sin, size_t rope_dim, size_t max_pos) {
    if (!rope_cos || !rope_sin || rope_dim == 0 || rope_dim % 2u || rope_dim > kv->head_dim) return 0;
    return vo_paged_append_impl(kv, batch, block_tables, max_blocks_per_seq, start_pos, n_new, k_new,
                                v_new, src_dtype, rope_cos, rope_sin, rope_dim, max_pos);
}

static int vo_paged_append_impl(const VoPagedKV* kv, uint32_t batch, const int32_t* block_tables,
                                uint32_t max_blocks_per_seq, const int32_t* start_pos, uint32_t n_new,
                                const void* k_new, const void* v_new, int src_dtype,
                                const float* rope_cos, const float* rope_sin, size_t rope_dim,
                                size_t max_pos) {
    if (!vo_kv_valid(kv) || !block_tables || !start_pos || !k_new || !v_new ||
        (src_dtype != 0 && src_dtype != 1)) {
        return 0;
    }
    const size_t H = kv->num_kv_heads, D = kv->head_dim;
    float* kr = (float*)malloc(D * sizeof(float));
    float* vr = (float*)malloc(D * sizeof(float));
    if (!kr || !vr) { free(kr); free(vr); return 0; }
    int ok = 1;
    for (uint32_t b = 0; b < batch && ok; ++b) {
        for (uint32_t i = 0; i < n_new && ok; ++i) {
            if (start_pos[b] < 0) { ok = 0; break; }
            const size_t t = (size_t)start_pos[b] + i;
            const long pb = vo_phys_block(kv, block_tables, max_blocks_per_seq, b, t);
            if (pb < 0) { ok = 0; break; }
            const size_t slot = t % kv->block_tokens;
            for (size_t h = 0; h < H; ++h) {
                const size_t src_off = (((size_t)b * n_new + i) * H + h) * D;
                if (src_dtype == 0) {
                    memcpy(kr, (const float*)k_new + src_off, D * sizeof(float));
                    memcpy(vr, (const float*)v_new + src_off, D * sizeof(float));
                } else {
                    vo_f16_to_f32((const uint16_t*)k_new + src_off, kr, D);
                    vo_f16_to_f32((const uint16_t*)v_new + src_off, vr, D);
                }
                if (rope_cos) {
                    if (t >= max_pos) { ok = 0; break; }
                    float rot[1024];
                    vo_rope_row(kr, rot, D, rope_dim, rope_cos + t * (rope_dim / 2u),
                                rope_sin + t * (rope_dim / 2u));
                    memcpy(kr, rot, D * sizeof(float));
                }
                vo_store_row(kv, 0, (size_t)pb, h, slot, kr);
                vo_store_row(kv, 1, (size_t)pb, h, slot, vr);
            }
        }
    }
    free(kr);
    free(vr);
    return ok;
}

int vo_paged_gather(const VoPagedKV* kv, uint32_t batch, const int32_t* block_tables,
                    uint32_t max_blocks_per_seq, const int32_t* ctx_lens,
                    const int64_t* out_token_offset, int out_mode, void* out_k, void* out_v,
                    uint16_t* out_k_scales, uint16_t* out_v_scales) {
    if (!vo_kv_valid(kv) || !block_tables || !ctx_lens || !out_token_offset || !out_k || !out_v) {
        return 0;
    }
    const size_t H = kv->num_kv_heads, D = kv->head_dim, G = D / 32u;
    if (out_mode == 0 && kv->dtype == 2 && (!out_k_scales || !out_v_scales)) {
        return 0;
    }
    for (uint32_t b = 0; b < batch; ++b) {
        if (ctx_lens[b] < 0) return 0;
        for (size_t t = 0; t < (size_t)ctx_lens[b]; ++t) {
            const long pb = vo_phys_block(kv, block_tables, max_blocks_per_seq, b, t);
            if (pb < 0) return 0;
            const size_t slot = t % kv->block_tokens;
            const size_t ot = (size_t)out_token_offset[b] + t;
            for (size_t h = 0; h < H; ++h) {
                const size_t orow = ot * H + h;
                if (out_mode == 1) {
                    vo_load_row(kv, 0, (size_t)pb, h, slot, (float*)out_k + orow * D);
                    vo_load_row(kv, 1, (size_t)pb, h, slot, (float*)out_v + orow * D);
                } else {
                    const size_t rb = kv->dtype == 0 ? D * 4u : (kv->dtype == 1 ? D * 2u : D / 2u);
                    vo_copy_row_raw(kv, 0, (size_t)pb, h, slot, (uint8_t*)out_k + orow * rb,
                                    out_k_scales ? out_k_scales + orow * G : NULL);
                    vo_copy_row_raw(kv, 1, (size_t)pb, h, slot, (uint8_t*)out_v + orow * rb,
                                    out_v_scales ? out_v_scales + orow * G : NULL);
                }
            }
        }
    }
    return 1;
}

int vo_paged_compact(const VoPagedKV* kv, uint32_t n, const int32_t* src_blocks,
                     const int32_t* dst_blocks) {
    if (!vo_kv_valid(kv) || (n > 0u && (!src_blocks || !dst_blocks))) {
        return 0;
    }
    const size_t rows = (size_t)kv->num_kv_heads * kv->block_tokens;
    const size_t D = kv->head_dim;
    const size_t row_bytes = kv->dtype == 0 ? D * 4u : (kv->dtype == 1 ? D * 2u : D / 2u);
    const size_t blk_bytes = rows * row_bytes;
    const size_t blk_scales = rows * (D / 32u);
    for (uint32_t i = 0; i < n; ++i) {
        if (src_blocks[i] < 0 || (uint32_t)src_blocks[i] >= kv->num_blocks || dst_blocks[i] < 0 ||
            (uint32_t)dst_blocks[i] >= kv->num_blocks) {
            return 0;
        }
    }
    for (uint32_t i = 0; i < n; ++i) {
        const size_t s = (size_t)src_blocks[i], d = (size_t)dst_blocks[i];
        memmove((uint8_t*)kv->k_data + d * blk_bytes, (const uint8_t*)kv->k_data + s * blk_bytes, blk_bytes);
        memmove((uint8_t*)kv->v_data + d * blk_bytes, (const uint8_t*)kv->v_data + s * blk_bytes, blk_bytes);
        if (kv->dtype == 2) {
            memmove(kv->k_scales + d * blk_scales, kv->k_scales + s * blk_scales, blk_scales * 2u);
            memmove(kv->v_scales + d * blk_scales, kv->v_scales + s * blk_scales, blk_scales * 2u);
        }
    }
    return 1;
}

int vo_paged_decode_attention(int mode, size_t dot_block, const VoPagedKV* kv, uint32_t batch,
                              uint32_t num_q_heads, const int32_t* block_tables,
                              uint32_t max_blocks_per_seq, const int32_t* ctx_lens,
                              const float* q, float* out) {
    if (!vo_kv_valid(kv) || !block_tables || !ctx_lens || !q || !out || num_q_heads == 0u ||
        num_q_heads % kv->num_kv_heads != 0u) {
        return 0;
    }
    const size_t Hq = num_q_heads, D = kv->head_dim;
    const size_t group = Hq / kv->num_kv_heads;
    size_t tmax = 0;
    for (uint32_t b = 0; b < batch; ++b) {
        if (ctx_lens[b] < 0) return 0;
        if ((size_t)ctx_lens[b] > tmax) tmax = (size_t)ctx_lens[b];
    }
    float* kh = (float*)malloc((tmax ? tmax : 1u) * D * sizeof(float));
    float* vh = (float*)malloc((tmax ? tmax : 1u) * D * sizeof(float));
    if (!kh || !vh) { free(kh); free(vh); return 0; }
    int ok = 1;
    for (uint32_t b = 0; b < batch && ok; ++b) {
        const size_t T = (size_t)ctx_lens[b];
        for (size_t hk = 0; hk < kv->num_kv_heads && ok; ++hk) {
            for (size_t t = 0; t < T; ++t) {
                const long pb = vo_phys_block(kv, block_tables, max_blocks_per_seq, b, t);
                if (pb < 0) { ok = 0; break; }
                vo_load_row(kv, 0, (size_t)pb, hk, t % kv->block_tokens, kh + t * D);
                vo_load_row(kv, 1, (size_t)pb, hk, t % kv->block_tokens, vh + t * D);
            }
            for (size_t g = 0; g < group && ok; ++g) {
                const size_t hq = hk * group + g;
                float* o = out + ((size_t)b * Hq + hq) * D;
                if (T == 0u) {
                    /* attention_ref.c:12-14 returns without writing; define zeros */
                    for (size_t x = 0; x < D; ++x) o[x] = 0.0f;
                    continue;
                }
                vo_attention_head(mode, dot_block, q + ((size_t)b * Hq + hq) * D, kh, D, vh, D, T, D, o);
            }
        }
    }
    free(kh);
    free(vh);
    return ok;
}
