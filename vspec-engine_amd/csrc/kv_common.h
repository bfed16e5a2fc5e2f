// kv_common.h -- device helpers and kernel parameter blocks shared by the
// paged-KV kernels (paged_kv.hip, decode_mfma.hip).
#pragma once
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include "vspec_rocm.h"

namespace vkv {


constexpr int kTile = 16;   // tokens per attention tile
constexpr int kWaves = 4;   // waves per attention workgroup
constexpr float kLog2e = 1.4426950408889634f;

// Streaming loads of K/V tiles: every tile is read once per decode, so they go out with
// the non-temporal cache policy (measured on random 4 KB tiles: 6.5-6.8 TB/s against
// 5.8-6.0 TB/s for ordinary loads).
typedef uint32_t nt_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t nt_u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 load_stream4(const void* p) {
    const nt_u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const nt_u32x4*>(p));
    return make_uint4(w[0], w[1], w[2], w[3]);
}
__device__ __forceinline__ uint2 load_stream2(const void* p) {
    const nt_u32x2 w = __builtin_nontemporal_load(reinterpret_cast<const nt_u32x2*>(p));
    return make_uint2(w[0], w[1]);
}
__device__ __forceinline__ uint32_t load_stream1(const uint32_t* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ uint16_t load_stream_u16(const uint16_t* p) { return __builtin_nontemporal_load(p); }

__device__ __forceinline__ float half_bits_to_float(uint32_t bits) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
}

__device__ __forceinline__ uint32_t float_to_half_bits(float x) {
    // v_cvt_f16_f32 under the default round-to-nearest-even mode
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(x)));
}

__device__ __forceinline__ void unpack_f16x8(const uint4 w, float* out) {
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        out[2 * i] = half_bits_to_float(ws[i] & 0xffffu);
        out[2 * i + 1] = half_bits_to_float(ws[i] >> 16);
    }
}

// signed nibble i (0..7) of a 32-bit word, even element in the low nibble
__device__ __forceinline__ float nibble(uint32_t w, int i) {
    return static_cast<float>(static_cast<int32_t>(w << (28 - 4 * i)) >> 28);
}

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}

// DPP controls
constexpr int kQuadXor1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kRowHalfMirror = 0x141;
constexpr int kRowMirror = 0x140;
// rotations inside each row of 16: lane i takes lane i - n (mod 16) of its row
constexpr int kRowRor4 = 0x124;
constexpr int kRowRor8 = 0x128;
constexpr int kRowRor12 = 0x12C;    // lane i takes lane i + 4 of its row

// x(lane) combined with x(lane ^ 16) / x(lane ^ 32) through the gfx950 permlane swaps
// (VALU, no LDS).  v_permlane16_swap exchanges the odd 16-lane rows of its first
// operand with the even rows of its second, v_permlane32_swap the upper half of the
// first with the lower half of the second; with both operands = x, the two results
// hold x and its partner.  They are issued as inline asm: hipcc 7.2 merges the two
// results of the corresponding builtins into one value.  The s_nop covers the
// VALU-write -> permlane-read hazard.
__device__ __forceinline__ void swap16(float x, float& a, float& b) {
    a = x;
    b = x;
    asm("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap32(float x, float& a, float& b) {
    a = x;
    b = x;
    asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ float add_xor16(float x) {
    float a, b;
    swap16(x, a, b);
    return a + b;
}
__device__ __forceinline__ float add_xor32(float x) {
    float a, b;
    swap32(x, a, b);
    return a + b;
}
__device__ __forceinline__ float max_xor16(float x) {
    float a, b;
    swap16(x, a, b);
    return fmaxf(a, b);
}
__device__ __forceinline__ float max_xor32(float x) {
    float a, b;
    swap32(x, a, b);
    return fmaxf(a, b);
}
// sum / max over the four rows of 16 lanes
__device__ __forceinline__ float add_rows(float x) { return add_xor32(add_xor16(x)); }
__device__ __forceinline__ float max_rows(float x) { return max_xor32(max_xor16(x)); }

// x of the lane `CTRL` names inside its row of 16 (row rotations: every source exists)
template <int CTRL>
__device__ __forceinline__ float row_dpp(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xf, 0xf, true));
}

// ---------------------------------------------------------------------------
// f16 pool layout (block_tokens a multiple of 16; bh = physical block * Hkv + head)
//   K: token-major rows of D halves
//   V: per (block, head), groups of 4 tokens: element (d, slot) at
//      bh*D*P + (slot/4)*4*D + 4*d + slot%4.  A decode tile (16 tokens) is 4 KB in one
//      piece; the MFMA operand of lane (g, n), 4 tokens of one d, is 8 contiguous bytes;
//      and one token's row spans 1 KB (32 rows of 32 bytes), so a single token's
//      append writes 4x fewer memory rows than in a d-major tile (128).
// ---------------------------------------------------------------------------
__host__ __device__ __forceinline__ size_t f16_v_index(size_t bh, uint32_t P, uint32_t D, uint32_t slot, uint32_t d) {
    return bh * D * P + (size_t)(slot >> 2) * (4u * D) + 4u * d + (slot & 3u);
}

// ---------------------------------------------------------------------------
// int4 pool layout (block_tokens a multiple of 16; bh = physical block * Hkv + head)
//   K codes : token-major rows of D/2 bytes, element e in nibble e%2 of byte e/2
//   K scales: group-major, (group c, slot) at (bh*G + c)*P + slot
//   V codes : 16-token tiles of 8*D bytes; lane chunk (g, n) of a tile (D/8 bytes at
//             (16*g + n)*(D/8)) holds tokens 4g..4g+3 of d = 16*j + n; element d of
//             token 4g+r is in byte 4*(d/32) + 2*(r&1) + (r>>1) of the chunk, low
//             nibble for even j, high nibble for odd j
//   V scales: token-major rows of G scales
// ---------------------------------------------------------------------------
__device__ __forceinline__ size_t int4_ks_index(size_t bh, uint32_t groups, uint32_t P, uint32_t slot,
                                                uint32_t c) {
    return (bh * groups + c) * P + slot;
}

__device__ __forceinline__ size_t int4_v_byte(size_t bh, uint32_t P, uint32_t D, uint32_t slot, uint32_t d,
                                              uint32_t* high) {
    const uint32_t t = slot & 15u, g = t >> 2, r = t & 3u;
    *high = (d >> 4) & 1u;
    return bh * ((size_t)P * D / 2) + (size_t)(slot >> 4) * (8u * D) + (size_t)(16u * g + (d & 15u)) * (D / 8u) +
           4u * (d >> 5) + 2u * (r & 1u) + (r >> 1);
}

// Canonical code dword c (elements 8c..8c+7, element e in nibble e) of V row `slot`.
__device__ __forceinline__ uint32_t int4_v_canonical_dword(const uint8_t* v, size_t bh, uint32_t P, uint32_t D,
                                                           uint32_t slot, uint32_t c) {
    uint32_t w = 0;
#pragma unroll
    for (uint32_t e = 0; e < 8; ++e) {
        uint32_t high = 0;
        const uint32_t byte = v[int4_v_byte(bh, P, D, slot, 8u * c + e, &high)];
        w |= ((high ? byte >> 4 : byte) & 0xfu) << (4u * e);
    }
    return w;
}

// Sum over aligned groups of N lanes (N = 4, 8, 16); every lane gets the total.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
    static_assert(N == 4 || N == 8 || N == 16, "group size");
    x += dpp<kQuadXor1>(x);
    x += dpp<kQuadXor2>(x);
    if constexpr (N >= 8) x += dpp<kRowHalfMirror>(x);
    if constexpr (N >= 16) x += dpp<kRowMirror>(x);
    return x;
}

// full-wave sum (every lane gets it)
__device__ __forceinline__ float wave_sum(float x) { return add_rows(group_sum<16>(x)); }

// full-wave max (every lane gets it)
__device__ __forceinline__ float wave_max(float x) {
    x = fmaxf(x, dpp<kQuadXor1>(x));
    x = fmaxf(x, dpp<kQuadXor2>(x));
    x = fmaxf(x, dpp<kRowHalfMirror>(x));
    x = fmaxf(x, dpp<kRowMirror>(x));
    return max_rows(x);
}

// Power-of-two shift e of a score operand row (q' of one query head) before its fp16 hi + lo
// split: the MFMAs read q' * 2^e and the scores are multiplied by 2^-e, both exact.  amax is
// max |q'| of the row.  Rows with amax in [2^-4, 2^15) keep e = 0: hi stays below 65504, and
// lo's fp16 rounding (absolute 2^-25 where lo is subnormal) stays within 2^-21 of amax.  Other
// rows move to amax * 2^e in [2^14, 2^15); e is clamped to +-100 so that 2^e and 2^-e are
// normal floats.  amax = 0, inf or NaN keeps e = 0.
__device__ __forceinline__ int qnorm_shift(float amax) {
    if (!(amax > 0.f) || !(amax < INFINITY) || (amax >= 0.0625f && amax < 32768.0f)) return 0;
    // amax in [2^(x-1), 2^x)
    int x;
    (void)frexpf(amax, &x);
    return min(max(15 - x, -100), 100);
}
// 2^e for e in [-126, 127]
__device__ __forceinline__ float pow2i(int e) { return __builtin_bit_cast(float, (e + 127) << 23); }

// Max over the 64/N groups of a wave when x is uniform inside each aligned group of N.
template <int N>
__device__ __forceinline__ float max_across_groups(float x) {
    if constexpr (N <= 4) x = fmaxf(x, dpp<kRowHalfMirror>(x));
    if constexpr (N <= 8) x = fmaxf(x, dpp<kRowMirror>(x));
    x = fmaxf(x, __shfl_xor(x, 16));
    x = fmaxf(x, __shfl_xor(x, 32));
    return x;
}

// ---------------------------------------------------------------------------
// decode attention
// ---------------------------------------------------------------------------
struct DecodeParams {
    const uint8_t* k;
    const uint8_t* v;
    const uint16_t* ks;
    const uint16_t* vs;
    const uint32_t* kf;  // int4 clamp flags [num_blocks][hkv][P/16] or null (a fused append keeps them)
    bool read_flags;     // the decode takes the flags instead of screening every tile
    const int32_t* block_tables;
    const int32_t* ctx_lens;
    const int32_t* block_used;  // [B][max_blocks] tokens per table entry's block, or null (full)
    const float* q;
    float* out;
    float* part_ml;    // [B][Hq][max_parts][2] (max in log2 units, sum)
    float* part_acc;   // [B][Hq][max_parts][D]
    uint32_t hq;
    uint32_t hkv;
    uint32_t block_tokens;
    uint32_t max_blocks;
    uint32_t num_blocks;
    uint32_t tiles_per_part;
    uint32_t max_parts;
    uint32_t gsplit;   // work items per kv head (Hq/Hkv/GW)
    float qscale;      // softmax scale * log2(e)
    float alpha;       // std-clamp alpha
    float logit_clip;  // +-24*log2(e) in 3-bit mode, +inf otherwise
    float input_clip;  // 16 in 3-bit mode, +inf otherwise
    // split of the MFMA kernels (see WorkSplit): part_ml / part_acc then hold two
    // partial slots per workgroup, [grid][2][GW][2] and [grid][2][GW][D]
    uint32_t split_grid;   // workgroups of the split kernel's grid (the merge launch redoes the split)
    bool merge;            // the host could not rule out work items spanning two workgroups
    uint32_t batch;
    uint32_t max_tiles;    // tiles of the host's context bound (max_ctx_len)
    uint32_t chunk_tiles;  // tiles per workgroup, or 0: split evenly over gridDim.x
    // fused decode-step append of the MFMA kernels (k_new != null): each sequence's new
    // token, [batch][hkv][D] in append_src (VSPEC_KV_F32 / VSPEC_KV_F16), is written at
    // position ctx_lens[b] - 1 before any tile is read
    const uint8_t* k_new;
    const uint8_t* v_new;
    int32_t append_src;
    // balanced split with a grid of two workgroups per CU: share of the first-half
    // workgroup of each (g, g + G/2) pair in 1/1000 (500: equal shares)
    uint32_t split_old_permille;
    // least tiles per workgroup of the balanced split (>= 1), applied to the actual total
    // so that the split does not depend on the host's bound
    uint32_t min_tiles;
    // tiles per work item when the host knows every context to be the same (min_ctx_len ==
    // max_ctx_len), else 0: the split then needs no pass over ctx_lens
    uint32_t uniform_tiles;
    // f16 pools: workgroups of 8 waves, each taking whole work items (chunk_tiles is a
    // multiple of the uniform tiles per item), for batches with few, short items
    bool wide;
    // balanced split of a ragged batch: each work item also costs this many tiles (its
    // set-up and merge in every workgroup that starts it), 0: tiles only
    uint32_t seg_cost;
};

// Launch the MFMA decode kernels for f16 pools (decode_mfma.hip) and int4 pools
// (decode_mfma_int4.hip), each followed by its merge launch (decode_merge_split); they
// return 0 when no instantiation matches (head_dim, heads per work item).
int launch_decode_mfma_f16(const DecodeParams& p, uint32_t head_dim, uint32_t gw, dim3 grid,
                           hipStream_t stream);
int launch_decode_mfma_int4(const DecodeParams& p, uint32_t head_dim, uint32_t gw, dim3 grid,
                            hipStream_t stream);

// Merge the kWaves per-wave softmax states of a workgroup (comb[w][h] = {max, sum,
// acc[D]}) and write the output row (one partition) or the split-K partial.
template <int D, int GW>
__device__ __forceinline__ void merge_waves(const DecodeParams& p, const float (*comb)[GW][D + 2], int b,
                                            int hq0, int part, int nparts) {
    for (int idx = threadIdx.x; idx < GW * D; idx += kWaves * 64) {
        const int h = idx / D;
        const int d = idx % D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) M = fmaxf(M, comb[w][h][0]);
        float a = 0.f, l = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float mw = comb[w][h][0];
            if (mw != -INFINITY) {
                const float f = exp2f(mw - M);
                a = fmaf(comb[w][h][2 + d], f, a);
                l = fmaf(comb[w][h][1], f, l);
            }
        }
        const size_t hq = (size_t)b * p.hq + hq0 + h;
        if (nparts == 1) {
            p.out[hq * D + d] = l > 0.f ? a / l : 0.f;
        } else {
            const size_t slot = hq * p.max_parts + part;
            p.part_acc[slot * D + d] = a;
            if (d == 0) {
                p.part_ml[2 * slot] = M;
                p.part_ml[2 * slot + 1] = l;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Work split of the MFMA decode kernels.
//
// A work item is (sequence b, kv head, group of GW query heads); it has
// U_b = max(1, min(ceil(ctx_b / 16), max_tiles)) tiles.  The tiles of all work items
// are laid end to end, sequence-major in ctx_lens order with the hkv * gsplit items of
// a sequence adjacent, T tiles in all.  Workgroup g takes the tiles [lo_g, lo_{g+1}):
//   balanced  lo_g = floor(g * T / G), G = min(split_grid, T)
//   chunked   lo_g = g * chunk_tiles
// so every workgroup streams the same number of tiles whatever the context lengths.  In
// a ragged batch each work item can also cost alpha tiles (DecodeParams.seg_cost): the
// split then runs over a cost axis on which item i occupies [c_i, c_i + alpha + U_i)
// (c_i = its first tile + alpha * i), alpha units of set-up followed by its tiles, and a
// workgroup's cost range maps back to the tiles it covers (a boundary inside an item's
// set-up units falls on its first tile).
// A work item that lies inside one workgroup's range goes straight to the output; one
// that spans several leaves one partial (max, sum, acc) per workgroup, in slot 0 when
// it is that workgroup's first segment and slot 1 when its last.  A second launch on the
// same stream (decode_merge_split) merges them: it redoes the split from ctx_lens and
// merges every item whose tiles meet more than one workgroup's range.  The kernel
// boundary orders the partial stores before the merge's loads, so no workgroup waits
// for or signals another, and no device state outlives a launch.
// ---------------------------------------------------------------------------
// Block tables and context lengths do not change while a decode kernel runs.  Read
// through the constant address space, their wave-uniform reads stay scalar loads even
// in loops that also store to global memory (the compiler cannot otherwise prove that
// those stores leave them untouched).
typedef const __attribute__((address_space(4))) int32_t const_i32;
__device__ __forceinline__ const const_i32* as_const(const int32_t* ptr) { return (const const_i32*)ptr; }

constexpr int kSplitEqual = 0;
constexpr int kSplitRagged = 1;
constexpr int kSplitAlways = 2;

struct WorkSplit {
    int total;   // T (balanced split with a segment cost: tiles plus alpha per work item)
    int tiles;   // tiles of all work items
    int alpha;   // cost of a work item in tiles on top of its own (0: none)
    int groups;  // G (balanced split), 0 for the chunked split
    int half;    // G / 2 when the two halves of the grid get different shares, else 0
    int wa;      // share of a first-half workgroup in a (first, second) pair, in 1/1000
    int ragged;  // the sequences' contexts differ in tiles
    int lo, hi;  // this workgroup's tiles
    int b;       // sequence holding tile lo
    int seq0;    // index of that sequence's first tile
};

template <int NW>
struct SplitSharedN {
    int wsum[NW];
    int umin[NW];  // per wave: least and greatest tiles per work item (U_b)
    int umax[NW];
    int wpre[NW];  // merge launch: per wave, tiles of the sequences before the item's
    int b;
    int seq0;
    int lo_t, hi_t;  // balanced split with a segment cost: the range in tiles
};
using SplitShared = SplitSharedN<kWaves>;

__device__ __forceinline__ int item_tiles(const DecodeParams& p, int b) {
    if (p.uniform_tiles) return (int)p.uniform_tiles;
    const int ctx = min(max(as_const(p.ctx_lens)[b], 0), (int)(p.max_blocks * p.block_tokens));
    return max(1, min((ctx + kTile - 1) / kTile, (int)p.max_tiles));
}

// Valid tokens of a 16-token tile whose block holds `used` tokens (slots 0 .. used-1) and
// whose first slot in that block is slot0.
__device__ __forceinline__ int used_cap(int used, int slot0) { return min(kTile, max(0, used - slot0)); }

// First tile of workgroup g.  The balanced split gives workgroup g the tiles
// [C(g) T / W, C(g+1) T / W) with C the cumulative share: equal shares, or, with a grid
// of two workgroups per CU (`half` set), wa/1000 of each pair's tiles to the first-half
// workgroup and the rest to the second-half one.  Workgroups g and g + G/2 share a CU,
// g dispatched first; the CU's wave arbiter favours the older waves, so with equal
// shares the first-half workgroup finishes well before its partner.
// UNEVEN: the pair-share policy of the kernel: kSplitEqual (the weighted arithmetic is
// compiled out), kSplitRagged (unequal shares for ragged batches: the f16 kernel) or
// kSplitAlways (unequal shares for any batch: the int4 kernel).
template <int UNEVEN>
__device__ __forceinline__ int split_lo(const DecodeParams& p, const WorkSplit& w, int g) {
    if (!w.groups) return g * (int)p.chunk_tiles;
    if (!UNEVEN || !w.half) return (int)((long long)g * w.total / w.groups);
    const long long c = (long long)w.wa * min(g, w.half) + (long long)(1000 - w.wa) * max(0, g - w.half);
    return (int)(c * w.total / (1000LL * w.half));
}

// The workgroup whose range holds tile t (the inverse of split_lo).
template <int UNEVEN>
__device__ __forceinline__ int split_group_of(const DecodeParams& p, const WorkSplit& w, int t) {
    if (!w.groups) return t / (int)p.chunk_tiles;
    if (!UNEVEN || !w.half) return (int)(((long long)(t + 1) * w.groups - 1) / w.total);
    // largest g with split_lo(g) <= t: first half while C(g) T < (t + 1) W
    const long long n = (long long)(t + 1) * 1000LL * w.half;
    const long long a = (long long)w.wa * w.total;
    const long long g = (n - 1) / a;
    if (g < w.half) return (int)g;
    return w.half + (int)((n - a * w.half - 1) / ((long long)(1000 - w.wa) * w.total));
}

// Tile position of cost position xc inside sequence b, whose tiles start at tile ex_t and
// cost unit ex_c, with u tiles per work item (the cost axis of work_split).
__device__ __forceinline__ int cost_to_tile(int xc, int ex_t, int ex_c, int u, int alpha) {
    const int d = xc - ex_c;
    const int k = d / (u + alpha);
    const int off = d - k * (u + alpha);
    return ex_t + k * u + min(max(off - alpha, 0), u);
}

// alpha of a split: the segment cost applies to ragged batches under the balanced split
__device__ __forceinline__ int split_alpha(const DecodeParams& p, int ragged) {
    return p.seg_cost && ragged && !p.chunk_tiles ? (int)p.seg_cost : 0;
}

// The split's shape once T (and whether the batch is ragged) is known: groups and pair
// shares.  The same for every workgroup of the split kernel and for the merge launch.
template <int UNEVEN>
__device__ __forceinline__ void split_shape(const DecodeParams& p, WorkSplit& r) {
    const int grid = (int)p.split_grid;
    r.half = 0;
    r.wa = 500;
    if (p.chunk_tiles) {
        r.groups = 0;
        return;
    }
    r.groups = min(grid, r.total);
    if (p.min_tiles > 1) r.groups = min(r.groups, max(1, r.total / (int)p.min_tiles));
    // Unequal shares with at least 64 tiles per workgroup, and only where every
    // second-half share is at least one tile (every workgroup of an item's span then holds
    // one of its partials).  The f16 kernel takes them for ragged batches only (measured:
    // C4 206 -> 190 us at 700; equal contexts lose, their ranges stop coinciding with
    // whole work items); the int4 kernel for every batch (its second-half workgroups
    // otherwise finish ~25 % after the first-half ones).
    if (UNEVEN && p.split_old_permille != 500 && (UNEVEN == kSplitAlways || r.ragged) && r.groups == grid &&
        (grid & 1) == 0 &&
        (long long)r.total >= 64LL * grid && (long long)(1000 - (int)p.split_old_permille) * r.total >= 500LL * grid) {
        r.half = grid / 2;
        r.wa = (int)p.split_old_permille;
    }
}

// this workgroup's tiles [lo, hi) once T is known
template <int UNEVEN>
__device__ __forceinline__ void split_range(const DecodeParams& p, WorkSplit& r) {
    const int g = blockIdx.x;
    split_shape<UNEVEN>(p, r);
    if (p.chunk_tiles) {
        r.lo = (int)min((long long)g * p.chunk_tiles, (long long)r.total);
        r.hi = (int)min((long long)r.lo + p.chunk_tiles, (long long)r.total);
    } else {
        r.lo = g < r.groups ? split_lo<UNEVEN>(p, r, g) : r.total;
        r.hi = g < r.groups ? split_lo<UNEVEN>(p, r, g + 1) : r.total;
    }
}

// Block-wide over NW waves (every thread calls it; the result is uniform).  The host keeps
// T = hkv * gsplit * sum U_b below 2^31.
template <int UNEVEN, int NW = kWaves>
__device__ __forceinline__ WorkSplit work_split(const DecodeParams& p, int ips, SplitSharedN<NW>& sh) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nb = (int)p.batch;
    WorkSplit r;
    if (p.uniform_tiles) {
        // every sequence holds uniform_tiles tiles per work item: no scan, no barrier
        const int per_seq = (int)p.uniform_tiles * ips;
        r.total = nb * per_seq;
        r.tiles = r.total;
        r.alpha = 0;
        r.ragged = 0;
        split_range<UNEVEN>(p, r);
        r.b = r.lo < r.hi ? r.lo / per_seq : 0;
        r.seq0 = r.b * per_seq;
        return r;
    }
    if (nb <= NW * 64) {
        // one sequence per thread: the total and the search come from one scan
        const int b = (int)threadIdx.x;
        const int u = b < nb ? item_tiles(p, b) : 0;
        int x = u;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(x, o);
            if (lane >= o) x += y;
        }
        int umin = b < nb ? u : 0x7fffffff, umax = u;
        if constexpr (UNEVEN != 0) {
#pragma unroll
            for (int o = 32; o; o >>= 1) {
                umin = min(umin, __shfl_xor(umin, o));
                umax = max(umax, __shfl_xor(umax, o));
            }
            if (lane == 0) {
                sh.umin[wave] = umin;
                sh.umax[wave] = umax;
            }
        }
        if (lane == 63) sh.wsum[wave] = x;
        __syncthreads();
        int before = 0, all = 0;
        umin = 0x7fffffff;
        umax = 0;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            before += w < wave ? sh.wsum[w] : 0;
            all += sh.wsum[w];
            if constexpr (UNEVEN != 0) {
                umin = min(umin, sh.umin[w]);
                umax = max(umax, sh.umax[w]);
            }
        }
        r.tiles = __builtin_amdgcn_readfirstlane(all) * ips;
        r.ragged = UNEVEN != 0 ? __builtin_amdgcn_readfirstlane(umin != umax ? 1 : 0) : 0;
        r.alpha = split_alpha(p, r.ragged);
        r.total = r.tiles + r.alpha * ips * nb;
        split_range<UNEVEN>(p, r);
        r.b = 0;
        r.seq0 = 0;
        if (r.lo >= r.hi) return r;
        const int excl = (before + x - u) * ips;
        if (r.alpha) {
            // cost range -> tiles: the sequences holding its ends map them
            const int ex_c = excl + r.alpha * ips * b;
            const int span = ips * (u + r.alpha);
            if (u > 0 && ex_c <= r.lo && r.lo < ex_c + span) {
                sh.lo_t = cost_to_tile(r.lo, excl, ex_c, u, r.alpha);
                sh.b = b;
                sh.seq0 = excl;
            }
            if (u > 0 && ex_c <= r.hi && r.hi < ex_c + span) sh.hi_t = cost_to_tile(r.hi, excl, ex_c, u, r.alpha);
            __syncthreads();
            const int lo_t = r.lo < r.total ? __builtin_amdgcn_readfirstlane(sh.lo_t) : r.tiles;
            const int hi_t = r.hi < r.total ? __builtin_amdgcn_readfirstlane(sh.hi_t) : r.tiles;
            r.b = __builtin_amdgcn_readfirstlane(sh.b);
            r.seq0 = __builtin_amdgcn_readfirstlane(sh.seq0);
            r.lo = lo_t;
            r.hi = hi_t;
            return r;
        }
        if (u > 0 && excl <= r.lo && r.lo < excl + u * ips) {
            sh.b = b;
            sh.seq0 = excl;
        }
        __syncthreads();
        r.b = __builtin_amdgcn_readfirstlane(sh.b);
        r.seq0 = __builtin_amdgcn_readfirstlane(sh.seq0);
        return r;
    }
    int s = 0, umin = 0x7fffffff, umax = 0;
    for (int b = threadIdx.x; b < nb; b += NW * 64) {
        const int u = item_tiles(p, b);
        s += u;
        if constexpr (UNEVEN != 0) {
            umin = min(umin, u);
            umax = max(umax, u);
        }
    }
#pragma unroll
    for (int o = 32; o; o >>= 1) {
        s += __shfl_xor(s, o);
        if constexpr (UNEVEN != 0) {
            umin = min(umin, __shfl_xor(umin, o));
            umax = max(umax, __shfl_xor(umax, o));
        }
    }
    if (lane == 0) {
        sh.wsum[wave] = s;
        sh.umin[wave] = umin;
        sh.umax[wave] = umax;
    }
    __syncthreads();
    int units = 0;
    umin = 0x7fffffff;
    umax = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        units += sh.wsum[w];
        umin = min(umin, sh.umin[w]);
        umax = max(umax, sh.umax[w]);
    }
    r.tiles = __builtin_amdgcn_readfirstlane(units) * ips;
    r.ragged = UNEVEN != 0 ? __builtin_amdgcn_readfirstlane(umin != umax ? 1 : 0) : 0;
    r.alpha = split_alpha(p, r.ragged);
    r.total = r.tiles + r.alpha * ips * nb;
    split_range<UNEVEN>(p, r);
    r.b = 0;
    r.seq0 = 0;
    if (r.lo >= r.hi) return r;
    // the sequence holding tile lo: exclusive prefix of U_b * ips, 256 sequences a pass
    int carry = 0;
    for (int base = 0; base < nb; base += NW * 64) {
        const int b = base + (int)threadIdx.x;
        const int u = b < nb ? item_tiles(p, b) : 0;
        int x = u;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(x, o);
            if (lane >= o) x += y;
        }
        __syncthreads();  // earlier readers of wsum are done
        if (lane == 63) sh.wsum[wave] = x;
        __syncthreads();
        int before = 0, all = 0;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            before += w < wave ? sh.wsum[w] : 0;
            all += sh.wsum[w];
        }
        const int excl = (carry + before + x - u) * ips;
        if (r.alpha) {
            const int ex_c = excl + r.alpha * ips * b;
            const int span = ips * (u + r.alpha);
            if (u > 0 && ex_c <= r.lo && r.lo < ex_c + span) {
                sh.lo_t = cost_to_tile(r.lo, excl, ex_c, u, r.alpha);
                sh.b = b;
                sh.seq0 = excl;
            }
            if (u > 0 && ex_c <= r.hi && r.hi < ex_c + span) sh.hi_t = cost_to_tile(r.hi, excl, ex_c, u, r.alpha);
        } else if (u > 0 && excl <= r.lo && r.lo < excl + u * ips) {
            sh.b = b;
            sh.seq0 = excl;
        }
        carry += all;
    }
    __syncthreads();
    r.b = __builtin_amdgcn_readfirstlane(sh.b);
    r.seq0 = __builtin_amdgcn_readfirstlane(sh.seq0);
    if (r.alpha) {
        const int lo_t = r.lo < r.total ? __builtin_amdgcn_readfirstlane(sh.lo_t) : r.tiles;
        const int hi_t = r.hi < r.total ? __builtin_amdgcn_readfirstlane(sh.hi_t) : r.tiles;
        r.lo = lo_t;
        r.hi = hi_t;
    }
    return r;
}

// Position in the sequence-major order of work items (all fields wave-uniform).  Work
// item y of sequence b covers kv head y / gsplit and query heads GW*y .. GW*y + GW - 1.
struct ItemCursor {
    int b;      // sequence
    int seq0;   // first tile of the sequence
    int U;      // tiles per work item of this sequence
    int y;      // work item within the sequence
    int item0;  // first tile of the work item
};

// the work item holding the workgroup's first tile
__device__ __forceinline__ ItemCursor cursor_at(const DecodeParams& p, const WorkSplit& w) {
    ItemCursor c;
    c.b = w.b;
    c.seq0 = w.seq0;
    c.U = item_tiles(p, w.b);
    c.y = (w.lo - w.seq0) / c.U;
    c.item0 = c.seq0 + c.y * c.U;
    return c;
}

// the next work item; callers only step onto items that hold a tile below T
__device__ __forceinline__ void cursor_next(const DecodeParams& p, int ips, ItemCursor& c) {
    if (c.y + 1 < ips) {
        ++c.y;
        c.item0 += c.U;
    } else {
        c.seq0 += c.U * ips;
        ++c.b;
        c.U = item_tiles(p, c.b);
        c.y = 0;
        c.item0 = c.seq0;
    }
}

// One wave merges the NW states of one item segment held in LDS (st[w][h] = {max, sum,
// acc[D]}, written by wave w) and writes the output rows of a whole work item, or else the
// workgroup's partial `pslot` (0: its first segment, 1: its last).
template <int D, int GW, int NW = kWaves>
__device__ __forceinline__ void merge_segment(const DecodeParams& p, const float (*st)[GW][D + 2], int lane,
                                              size_t row0, bool whole, int pslot) {
    float* pacc = p.part_acc + ((size_t)blockIdx.x * 2 + pslot) * GW * D;
    float* pml = p.part_ml + ((size_t)blockIdx.x * 2 + pslot) * GW * 2;
    for (int idx = lane; idx < GW * D; idx += 64) {
        const int h = idx / D;
        const int d = idx % D;
        float M = -INFINITY;
#pragma unroll
        for (int v = 0; v < NW; ++v) M = fmaxf(M, st[v][h][0]);
        float a = 0.f, l = 0.f;
#pragma unroll
        for (int v = 0; v < NW; ++v) {
            const float f = exp2f(st[v][h][0] - M);
            a = fmaf(st[v][h][2 + d], f, a);
            l = fmaf(st[v][h][1], f, l);
        }
        if (whole) {
            p.out[(row0 + h) * D + d] = l > 0.f ? a / l : 0.f;
        } else {
            pacc[idx] = a;
            if (d == 0) {
                pml[2 * h] = M;
                pml[2 * h + 1] = l;
            }
        }
    }
}

// Block-wide: merge the kWaves per-wave states of one segment (tiles [tile_begin,
// tile_end) of a work item of U tiles) and write the output rows when the segment is the
// whole item, else the workgroup's partial `slot` for the merge launch.
template <int D, int GW>
__device__ __forceinline__ void finish_segment(const DecodeParams& p, const float (*comb)[GW][D + 2], int b,
                                               int hq0, int U, int tile_begin, int tile_end, int slot) {
    const bool whole = tile_begin == 0 && tile_end == U;
    const size_t row0 = (size_t)b * p.hq + hq0;
    // thread index behind an opaque copy: the address arithmetic below then stays here
    // instead of being hoisted out of the caller's loops into registers that would
    // stay live through the tile loop
    int tid = (int)threadIdx.x;
    asm volatile("" : "+v"(tid));
    float* pacc = p.part_acc + ((size_t)blockIdx.x * 2 + slot) * GW * D;
    float* pml = p.part_ml + ((size_t)blockIdx.x * 2 + slot) * GW * 2;
    for (int idx = tid; idx < GW * D; idx += kWaves * 64) {
        const int h = idx / D;
        const int d = idx % D;
        float M = -INFINITY;
#pragma unroll
        for (int v = 0; v < kWaves; ++v) M = fmaxf(M, comb[v][h][0]);
        float a = 0.f, l = 0.f;
#pragma unroll
        for (int v = 0; v < kWaves; ++v) {
            const float f = exp2f(comb[v][h][0] - M);
            a = fmaf(comb[v][h][2 + d], f, a);
            l = fmaf(comb[v][h][1], f, l);
        }
        if (whole) {
            p.out[(row0 + h) * D + d] = l > 0.f ? a / l : 0.f;
        } else {
            pacc[idx] = a;
            if (d == 0) {
                pml[2 * h] = M;
                pml[2 * h + 1] = l;
            }
        }
    }
}

// Merge launch of a split decode: one workgroup per work item (grid = batch * hkv *
// gsplit, 256 threads).  It redoes the split kernel's split from ctx_lens (the same T,
// groups and pair shares), and for an item whose tiles meet the ranges of workgroups
// g0 < g1 it merges their partials in order g0..g1 and writes the item's output rows;
// items inside one range were written by the split kernel and are left alone.  Partial
// loads go out NBATCH workgroups at a time, all in flight together.  With uniform_tiles
// (every context the same) the split needs no pass over ctx_lens.
template <int D, int GW, int UNEVEN>
__global__ __launch_bounds__(kWaves * 64) void decode_merge_split(DecodeParams p) {
    constexpr int NT = kWaves * 64;
    constexpr int K = (GW * D + NT - 1) / NT;  // outputs per thread: idx = tid + NT * k
    constexpr int NBATCH = 16;
    __shared__ SplitShared sh;
    const int ips = (int)(p.hkv * p.gsplit);
    const int b = (int)blockIdx.x / ips;
    const int y = (int)blockIdx.x % ips;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nb = (int)p.batch;
    WorkSplit w;
    int pre = 0;
    if (p.uniform_tiles) {
        w.total = nb * (int)p.uniform_tiles * ips;
        w.ragged = 0;
        pre = b * (int)p.uniform_tiles;
        w.tiles = w.total;
        w.alpha = 0;
    } else {
        // T, ragged and the tiles of the sequences before b, block-wide
        int s = 0, umin = 0x7fffffff, umax = 0;
        for (int i = threadIdx.x; i < nb; i += NT) {
            const int u = item_tiles(p, i);
            s += u;
            pre += i < b ? u : 0;
            umin = min(umin, u);
            umax = max(umax, u);
        }
#pragma unroll
        for (int o = 32; o; o >>= 1) {
            s += __shfl_xor(s, o);
            pre += __shfl_xor(pre, o);
            umin = min(umin, __shfl_xor(umin, o));
            umax = max(umax, __shfl_xor(umax, o));
        }
        if (lane == 0) {
            sh.wsum[wave] = s;
            sh.wpre[wave] = pre;
            sh.umin[wave] = umin;
            sh.umax[wave] = umax;
        }
        __syncthreads();
        int all = 0;
        pre = 0;
        umin = 0x7fffffff;
        umax = 0;
#pragma unroll
        for (int v = 0; v < kWaves; ++v) {
            all += sh.wsum[v];
            pre += sh.wpre[v];
            umin = min(umin, sh.umin[v]);
            umax = max(umax, sh.umax[v]);
        }
        w.tiles = all * ips;
        w.ragged = UNEVEN != 0 && umin != umax ? 1 : 0;
        w.alpha = split_alpha(p, w.ragged);
        w.total = w.tiles + w.alpha * ips * nb;
    }
    split_shape<UNEVEN>(p, w);
    const int U = item_tiles(p, b);
    const int item0 = pre * ips + y * U;
    // the item on the split's axis: set-up units from c0, its first tile at c0 + alpha
    const int c0 = item0 + w.alpha * (b * ips + y);
    const int g0 = split_group_of<UNEVEN>(p, w, c0 + w.alpha);
    const int g1 = split_group_of<UNEVEN>(p, w, c0 + w.alpha + U - 1);
    if (g0 == g1) return;  // written by the split kernel
    // the item is g0's last segment (slot 1) when g0's range starts before it, and the
    // first segment (slot 0) of every later workgroup
    const int first_inside = split_lo<UNEVEN>(p, w, g0) < c0 ? 1 : 0;
    const int tid = (int)threadIdx.x;
    // running merge per output in log2 units; -1e30 (not -inf) keeps exp2 finite
    float M[K], A[K], Ls[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        M[k] = -1e30f;
        A[k] = 0.f;
        Ls[k] = 0.f;
    }
    for (int g = g0; g <= g1; g += NBATCH) {
        float mb[NBATCH][K], lb[NBATCH][K], ab[NBATCH][K];
#pragma unroll
        for (int i = 0; i < NBATCH; ++i) {
            const bool valid = g + i <= g1;
            const int gg = valid ? g + i : g1;
            const size_t slot = (size_t)gg * 2 + (gg == g0 ? first_inside : 0);
#pragma unroll
            for (int k = 0; k < K; ++k) {
                const int idx = min(tid + NT * k, GW * D - 1);
                const int h = idx / D;
                const int d = idx % D;
                const float m = p.part_ml[(slot * GW + h) * 2];
                const float l = p.part_ml[(slot * GW + h) * 2 + 1];
                const float a = p.part_acc[(slot * GW + h) * D + d];
                mb[i][k] = valid ? m : -1e30f;
                lb[i][k] = valid ? l : 0.f;
                ab[i][k] = valid ? a : 0.f;
            }
        }
#pragma unroll
        for (int i = 0; i < NBATCH; ++i) {
#pragma unroll
            for (int k = 0; k < K; ++k) {
                const float nm = fmaxf(M[k], mb[i][k]);
                const float fo = exp2f(M[k] - nm);
                const float fn = exp2f(mb[i][k] - nm);
                A[k] = fmaf(ab[i][k], fn, A[k] * fo);
                Ls[k] = fmaf(lb[i][k], fn, Ls[k] * fo);
                M[k] = nm;
            }
        }
    }
    const size_t row0 = (size_t)b * p.hq + (size_t)y * GW;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int idx = tid + NT * k;
        if (idx < GW * D) p.out[(row0 + idx / D) * D + idx % D] = Ls[k] > 0.f ? A[k] / Ls[k] : 0.f;
    }
}

}  // namespace vkv
