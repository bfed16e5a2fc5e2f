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
constexpr int kRowRor4 = 0x124;     // rotate by 4 lanes inside each row of 16
constexpr int kRowRor8 = 0x128;

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
    const int32_t* block_tables;
    const int32_t* ctx_lens;
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
};


// Launch the MFMA decode kernels for f16 pools (decode_mfma.hip) and int4 pools
// (decode_mfma_int4.hip); they return 0 when no instantiation matches (head_dim,
// heads per work item).
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

}  // namespace vkv
