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


// Launch the MFMA decode kernel for f16 pools (decode_mfma.hip); returns 0 when no
// instantiation matches (head_dim, heads per work item).
int launch_decode_mfma_f16(const DecodeParams& p, uint32_t head_dim, uint32_t gw, dim3 grid,
                           hipStream_t stream);

}  // namespace vkv
