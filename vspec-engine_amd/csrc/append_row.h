// append_row.h -- block-table append of one chunk of a token-head row of K or V
// (kv_paged_cache.c:292-303 in the reference, with quantise-on-write for int4 pools),
// shared by the append kernels (paged_kv.hip) and the decode kernels' fused decode-step
// append (decode_mfma.hip, decode_mfma_int4.hip).
#pragma once
#include "kv_common.h"

namespace vkv {

struct AppendParams {
    uint8_t* k;
    uint8_t* v;
    uint16_t* ks;
    uint16_t* vs;
    uint32_t* kf;  // int4 clamp flags or null
    const int32_t* block_tables;
    const int32_t* start_pos;
    // packed-token mode (token_item != null): source token b (n_new == 1) goes to
    // position token_pos[b] of block-table row token_item[b]
    const int32_t* token_item;
    const int32_t* token_pos;
    uint32_t n_items;  // block-table rows in packed-token mode
    // rotary embedding of K (rope_cos != null): rows [max_pos][rope_dim / 2]
    const float* rope_cos;
    const float* rope_sin;
    uint32_t rope_dim;
    uint32_t max_pos;
    // with start_pos and token_item null: source token b goes to position ctx_lens[b] - 1
    // (the decode step's append; a context of 0 appends nothing)
    const int32_t* ctx_lens;
    const uint8_t* k_new;
    const uint8_t* v_new;
    uint32_t batch;
    uint32_t n_new;
    uint32_t hkv;
    uint32_t head_dim;
    uint32_t block_tokens;
    uint32_t max_blocks;
    uint32_t num_blocks;
};

// Elements per append work item: a whole 32-element quantisation group for int4 pools,
// 8 elements (16 or 32 bytes) otherwise.
constexpr int append_ept(int dt) { return dt == VSPEC_KV_INT4 ? 32 : 8; }

// Chunk c of the token-head row of K (which 0) or V (which 1) whose first source element
// is src_el, written at position pos of block-table row `seq`, kv head h.  Positions past
// the table, behind an invalid entry or (with rotary tables) past max_pos are not written.
// A clamp-flag update held back by the caller: flag word `word` gets bit `bit` set or
// cleared.
struct FlagOp {
    uint32_t* word;
    uint32_t bit;
    bool set;
};

__device__ __forceinline__ void apply_flag(const FlagOp& f) {
    if (!f.word) return;
    if (f.set) atomicOr(f.word, f.bit);
    else atomicAnd(f.word, ~f.bit);
}

// int4 codec of one 32-element group: rep = 2nd-largest |x|, scale = rep/8 (1 if rep == 0),
// floored at 1e-6, rounded to fp16 (saturating), codes rint(x/scale) in [-8,7]; element e
// in nibble e%8 of w[e/8].  c1, c2, cm: sum, sum of squares and largest magnitude of the
// codes.
struct Int4Group {
    uint32_t w[4];
    uint32_t s16;
    float sc;
    int c1, c2, cm;
};
// the largest two |x| seen (a1 >= a2; equal values count twice), updated with a
__device__ __forceinline__ void int4_top2(float a, float& a1, float& a2) {
    const bool gt1 = a > a1;
    a2 = gt1 ? a1 : (a > a2 ? a : a2);
    a1 = gt1 ? a : a1;
}
// fp16 bits of a group's scale from its 2nd-largest |x|
__device__ __forceinline__ uint32_t int4_scale_bits(float rep) {
    float scale = rep > 0.f ? rep / 8.0f : 1.0f;
    if (scale < 1e-6f) scale = 1e-6f;
    uint32_t s16 = float_to_half_bits(scale);
    if ((s16 & 0x7fffu) >= 0x7c00u) s16 = 0x7bffu;
    return s16;
}
__device__ __forceinline__ int int4_code(float x, float sc) {
    const float rr = rintf(x / sc);
    return rr > 7.0f ? 7 : (rr >= -8.0f ? (int)rr : -8);
}
__device__ __forceinline__ Int4Group int4_encode_group(const float (&x)[32]) {
    float a1 = 0.f, a2 = 0.f;
#pragma unroll
    for (int e = 0; e < 32; ++e) int4_top2(fabsf(x[e]), a1, a2);
    Int4Group q;
    q.s16 = int4_scale_bits(a2);
    q.sc = half_bits_to_float(q.s16);
    q.w[0] = q.w[1] = q.w[2] = q.w[3] = 0u;
    q.c1 = q.c2 = q.cm = 0;
#pragma unroll
    for (int e = 0; e < 32; ++e) {
        const int code = int4_code(x[e], q.sc);
        q.w[e / 8] |= ((uint32_t)code & 0xfu) << (4 * (e % 8));
        q.c1 += code;
        q.c2 += code * code;
        q.cm = max(q.cm, code < 0 ? -code : code);
    }
    return q;
}

// The clamp flag of a key from its row's sums: s1 = sum x, s2 = sum x^2 (the groups' scaled
// code sums, added pairwise (g0 + g1) + (g2 + g3)) and m = max |x|.
__device__ __forceinline__ bool int4_flag_from_sums(float s1, float s2, float m, uint32_t head_dim) {
    const float mean = s1 / (float)head_dim;
    const float ex2 = s2 / (float)head_dim;
    const float var1 = ex2 - mean * mean;
    const float th1 = fminf(fmaxf(1e-6f, 4.5f * sqrtf(fmaxf(var1, 0.f))), 16.0f);
    return m > th1 * (1.0f - 0.0009765625f) || var1 <= ex2 * 0.0009765625f;
}

// Clamp flag of a key (attention_ref.c:56 clips every key at its std threshold): set when
// some element may reach alpha * std (alpha 4.5, the reference default; threshold capped at
// 16 as in 3-bit mode) of the dequantised row.  Mean and E[x^2] come from the code sums of
// the row's groups, which sit in lanes 2c of an aligned run of 2 * head_dim / 32 lanes (the
// append work items of one row: all of these lanes call this together); the 2^-10 margins
// cover the one-pass variance (the decode kernel's screen test, run once per key here).
__device__ __forceinline__ bool int4_key_flag(const Int4Group& q, uint32_t head_dim) {
    float s1 = q.sc * (float)q.c1;
    float s2 = (q.sc * q.sc) * (float)q.c2;
    float m = q.sc * (float)q.cm;
    for (uint32_t o = 2; o < 2 * (head_dim / 32); o <<= 1) {
        s1 += __shfl_xor(s1, (int)o);
        s2 += __shfl_xor(s2, (int)o);
        m = fmaxf(m, __shfl_xor(m, (int)o));
    }
    return int4_flag_from_sums(s1, s2, m, head_dim);
}

// V code byte nn (0..15) of group c: d = 32c + nn in the low nibble, d = 32c + 16 + nn in
// the high one (int4_v_byte places it).
__device__ __forceinline__ uint32_t int4_v_group_byte(const uint32_t (&w)[4], int nn) {
    const uint32_t lo = (w[nn / 8] >> (4 * (nn % 8))) & 0xfu;
    const uint32_t hi = (w[2 + nn / 8] >> (4 * (nn % 8))) & 0xfu;
    return lo | (hi << 4);
}

// Offset of V code byte nn of group c of token `slot` within its 16-token tile.
__device__ __forceinline__ uint32_t int4_v_tile_byte(uint32_t slot, uint32_t c, uint32_t nn, uint32_t D) {
    const uint32_t tt = slot & 15u, tg = tt >> 2, tr = tt & 3u;
    return (16u * tg + nn) * (D / 8u) + 4u * c + 2u * (tr & 1u) + (tr >> 1);
}

template <int DT, int SRC>
__device__ __forceinline__ void append_chunk(const AppendParams& p, uint32_t seq, uint32_t pos, uint32_t h,
                                             uint32_t c, int which, size_t src_el, FlagOp* defer = nullptr) {
    constexpr int EPT = append_ept(DT);
    const uint32_t lb = pos / p.block_tokens;
    if (lb >= p.max_blocks) return;
    // the source elements are read before the table entry is looked at: both loads are in
    // flight together
    float x[EPT];
    const uint8_t* src = which ? p.v_new : p.k_new;
    if constexpr (SRC == VSPEC_KV_F32) {
        const float4* s4 = reinterpret_cast<const float4*>(src + src_el * 4);
#pragma unroll
        for (int j = 0; j < EPT / 4; ++j) {
            const float4 w = s4[j];
            x[4 * j] = w.x; x[4 * j + 1] = w.y; x[4 * j + 2] = w.z; x[4 * j + 3] = w.w;
        }
    } else {
        const uint4* s4 = reinterpret_cast<const uint4*>(src + src_el * 2);
#pragma unroll
        for (int j = 0; j < EPT / 8; ++j) unpack_f16x8(s4[j], x + 8 * j);
    }
    const int32_t phys = p.block_tables[(size_t)seq * p.max_blocks + lb];
    if (phys < 0 || (uint32_t)phys >= p.num_blocks) return;
    const uint32_t slot = pos % p.block_tokens;
    const size_t row = ((size_t)phys * p.hkv + h) * p.block_tokens + slot;
    const size_t e0 = (size_t)c * EPT;  // first element of this chunk within the row

    const bool rope = p.rope_cos != nullptr;
    if (rope) {
        if (pos >= p.max_pos) return;  // no table row: the token is not written
        if (!which) {
#pragma clang fp contract(off)
            // pairs (i, i + half) of the first rope_dim elements rotate by row `pos`:
            // x1*c - x2*s, x1*s + x2*c, each product and sum rounded separately (no
            // fused multiply-add: hipcc contracts by default)
            const uint32_t half = p.rope_dim / 2;
            const size_t row0 = src_el - e0;  // element 0 of this token-head row
            const float* cr = p.rope_cos + (size_t)pos * half;
            const float* sr = p.rope_sin + (size_t)pos * half;
#pragma unroll
            for (int e = 0; e < EPT; ++e) {
                const uint32_t d = (uint32_t)e0 + e;
                if (d >= p.rope_dim) continue;
                const uint32_t i = d < half ? d : d - half;
                const size_t pe = row0 + (d < half ? d + half : d - half);
                float other;
                if constexpr (SRC == VSPEC_KV_F32) {
                    other = reinterpret_cast<const float*>(src)[pe];
                } else {
                    other = half_bits_to_float(reinterpret_cast<const uint16_t*>(src)[pe]);
                }
                const float c = cr[i], sn = sr[i];
                x[e] = d < half ? x[e] * c - other * sn : other * sn + x[e] * c;
            }
        }
    }

    uint8_t* dst = which ? p.v : p.k;
    if constexpr (DT == VSPEC_KV_F32) {
        float4* d4 = reinterpret_cast<float4*>(dst + (row * p.head_dim + e0) * 4);
        d4[0] = make_float4(x[0], x[1], x[2], x[3]);
        d4[1] = make_float4(x[4], x[5], x[6], x[7]);
    } else if constexpr (DT == VSPEC_KV_F16) {
        uint32_t hb[8];
        if (SRC == VSPEC_KV_F16 && !(rope && !which)) {
            // pure copy of the source bits
            const uint4 w = *reinterpret_cast<const uint4*>(src + src_el * 2);
            const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                hb[2 * k] = ws[k] & 0xffffu;
                hb[2 * k + 1] = ws[k] >> 16;
            }
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) hb[k] = float_to_half_bits(x[k]);
        }
        if (which) {
            // V in 4-token groups: element (d, slot) at f16_v_index (stride 4 in d)
            uint16_t* vt = reinterpret_cast<uint16_t*>(dst) +
                           f16_v_index((size_t)phys * p.hkv + h, p.block_tokens, p.head_dim, slot, e0);
#pragma unroll
            for (int k = 0; k < 8; ++k) vt[4 * k] = (uint16_t)hb[k];
        } else {
            *reinterpret_cast<uint4*>(dst + (row * p.head_dim + e0) * 2) =
                make_uint4(hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16), hb[4] | (hb[5] << 16),
                           hb[6] | (hb[7] << 16));
        }
    } else {
        const Int4Group q = int4_encode_group(x);
        if (!which && p.kf) {
            const bool flag = int4_key_flag(q, p.head_dim);
            if (c == 0) {
                const FlagOp op = {p.kf + ((size_t)phys * p.hkv + h) * (p.block_tokens / 16) + slot / 16,
                                   1u << (slot % 16), flag};
                if (defer) *defer = op;
                else apply_flag(op);
            }
        }
        const size_t bh = (size_t)phys * p.hkv + h;
        if (which) {
            // V tiles: byte n of this group's 16 holds d = 32c + n (low nibble) and
            // d = 32c + 16 + n (high nibble) of this token, at lane chunk (g, n)
            uint8_t* vb = dst + bh * ((size_t)p.block_tokens * p.head_dim / 2) + (size_t)(slot >> 4) * (8u * p.head_dim);
#pragma unroll
            for (int nn = 0; nn < 16; ++nn) vb[int4_v_tile_byte(slot, c, nn, p.head_dim)] = (uint8_t)int4_v_group_byte(q.w, nn);
            p.vs[row * (p.head_dim / 32) + c] = (uint16_t)q.s16;
        } else {
            uint4* d4 = reinterpret_cast<uint4*>(dst + row * (p.head_dim / 2) + e0 / 2);
            *d4 = make_uint4(q.w[0], q.w[1], q.w[2], q.w[3]);
            p.ks[int4_ks_index(bh, p.head_dim / 32, p.block_tokens, slot, c)] = (uint16_t)q.s16;
        }
    }
}

// The append of a decode kernel's fused decode step: each sequence's new token at position
// ctx_lens[b] - 1.
__device__ __forceinline__ AppendParams decode_step_append_params(const DecodeParams& p, uint32_t head_dim) {
    AppendParams a;
    a.k = const_cast<uint8_t*>(p.k);
    a.v = const_cast<uint8_t*>(p.v);
    a.ks = const_cast<uint16_t*>(p.ks);
    a.vs = const_cast<uint16_t*>(p.vs);
    a.kf = const_cast<uint32_t*>(p.kf);
    a.block_tables = p.block_tables;
    a.start_pos = nullptr;
    a.token_item = nullptr;
    a.token_pos = nullptr;
    a.n_items = 0;
    a.rope_cos = nullptr;
    a.rope_sin = nullptr;
    a.rope_dim = 0;
    a.max_pos = 0;
    a.ctx_lens = p.ctx_lens;
    a.k_new = p.k_new;
    a.v_new = p.v_new;
    a.batch = p.batch;
    a.n_new = 1;
    a.hkv = p.hkv;
    a.head_dim = head_dim;
    a.block_tokens = p.block_tokens;
    a.max_blocks = p.max_blocks;
    a.num_blocks = p.num_blocks;
    return a;
}

// Work items of one append launch: 2 (K, V) x chunks per row x kv heads x tokens.
template <int DT>
__device__ __forceinline__ uint64_t append_items(const AppendParams& p) {
    return (uint64_t)p.batch * p.n_new * p.hkv * (p.head_dim / append_ept(DT)) * 2;
}

// One work item of the append kernel (any order; no two items write the same bytes):
// item `it` = ((token, kv head, chunk) << 1) | which.  Uniform batch (start_pos), packed
// tokens (token_item / token_pos, items not below n_items skipped) or the decode step's
// token at ctx_lens[b] - 1.
template <int DT, int SRC>
__device__ __forceinline__ void append_item(const AppendParams& p, uint64_t it) {
    constexpr int EPT = append_ept(DT);
    const uint32_t chunks = p.head_dim / EPT;
    const int which = (int)(it & 1);
    uint64_t r = it >> 1;
    const uint32_t c = (uint32_t)(r % chunks);
    r /= chunks;
    const uint32_t h = (uint32_t)(r % p.hkv);
    r /= p.hkv;
    const uint32_t i = (uint32_t)(r % p.n_new);
    const uint32_t b = (uint32_t)(r / p.n_new);

    const int32_t item = p.token_item ? p.token_item[b] : (int32_t)b;
    int32_t sp;
    if (p.token_item) {
        sp = p.token_pos[b];
    } else if (p.start_pos) {
        sp = p.start_pos[b];
    } else {
        const int32_t cl = p.ctx_lens[b];
        sp = cl > 0 ? cl - 1 : -1;
    }
    if (sp < 0 || item < 0 || (p.token_item && (uint32_t)item >= p.n_items)) return;
    const size_t src_el = (((size_t)b * p.n_new + i) * p.hkv + h) * p.head_dim + (size_t)c * EPT;
    append_chunk<DT, SRC>(p, (uint32_t)item, (uint32_t)sp + i, h, c, which, src_el);
}

// Fused decode-step append of the MFMA decode kernels (p.k_new != null).  Every work
// item whose last tile lies in this workgroup's range [ws.lo, ws.hi) -- exactly one
// workgroup per work item -- gets its sequence's new token written for its kv head at
// position ctx_lens[b] - 1, exactly as the append kernel writes it.  Threads below kItems
// (the first lanes of wave 0) write the rows: with WAIT every thread calls this (it ends in a
// barrier), without WAIT at least those, before the workgroup reads any tile the append may
// write.  WAIT: it returns with the
// stores complete and a barrier passed, so the workgroup's later loads of those tiles see
// them; without WAIT it returns with the stores issued, and the caller waits for them (every
// thread) and passes a barrier before such loads.  Other workgroups never read the rows
// written here (they belong to the item's last tile), except the owners of the other
// q-head groups of the same kv head, which write the same bytes themselves.
template <int DT, int D, bool WAIT = true>
__device__ void fused_append(const DecodeParams& p, const WorkSplit& ws, ItemCursor c, const int ips,
                             FlagOp& pending, uint32_t* pend_lds) {
    constexpr int EPT = append_ept(DT);
    constexpr int kItems = D / EPT * 2;  // append work items per token-head row (K and V)
    static_assert(kItems <= kWaves * 64, "one pass of the workgroup's threads");
    const AppendParams a = decode_step_append_params(p, D);
    const int t = (int)threadIdx.x;
    // int4 clamp flags (thread 0 of each row): the first one is handed back to the caller,
    // which applies it after the barrier below (so the barrier does not wait for it) and,
    // with pend_lds, is published there as {word index, bit, set} for the tile loop to patch
    // into the word it loads; any further ones are applied at once
    pending = {nullptr, 0u, false};
    while (true) {
        const int last = c.item0 + c.U - 1;
        if (last >= ws.lo && last < ws.hi) {
            const int ctx = as_const(p.ctx_lens)[c.b];
            if (ctx > 0 && t < kItems) {
                const uint32_t hk = (uint32_t)c.y / p.gsplit;
                const uint32_t ch = (uint32_t)t >> 1;
                const size_t src_el = ((size_t)c.b * p.hkv + hk) * D + (size_t)ch * EPT;
                FlagOp op = {nullptr, 0u, false};
                if (p.append_src == VSPEC_KV_F32) {
                    append_chunk<DT, VSPEC_KV_F32>(a, (uint32_t)c.b, (uint32_t)ctx - 1u, hk, ch, t & 1, src_el, &op);
                } else {
                    append_chunk<DT, VSPEC_KV_F16>(a, (uint32_t)c.b, (uint32_t)ctx - 1u, hk, ch, t & 1, src_el, &op);
                }
                if (op.word) {
                    if (!pending.word) pending = op;
                    else apply_flag(op);
                }
            }
        }
        if (c.item0 + c.U >= ws.hi) break;
        cursor_next(p, ips, c);
    }
    if (pend_lds && t == 0) {
        pend_lds[0] = pending.word ? (uint32_t)(pending.word - p.kf) : 0xffffffffu;
        pend_lds[1] = pending.bit;
        pend_lds[2] = pending.set ? pending.bit : 0u;
    }
    if constexpr (WAIT) {
        __builtin_amdgcn_s_waitcnt(0);  // this thread's stores are done
        __syncthreads();
    }
}

}  // namespace vkv
