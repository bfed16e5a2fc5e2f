// decode_mfma_int4.hip -- single-query GQA decode attention over int4 paged KV
// (32-element groups, one fp16 scale each) with both contractions on the matrix
// cores and the reference numerics (per-key std clamp, attention_ref.c:50-62) on
// the vector ALUs.
//
// Codes are exact small integers in fp16, so the MFMAs run on raw codes and the
// scales are applied around them:
//
//   scores  S^T[16 tok][16 col] = K codes x Q'^T   v_mfma_f32_16x16x32_f16
//     Lane (g, n) feeds token n's code dwords g*NQ .. g*NQ+NQ-1 (one quantisation
//     group, one 16-byte load).  Column n of the product collects group n/4 of query
//     head n%4: the B operand is zero wherever a k-slot's group differs from its
//     column's group.  Scaling column n by the K scale of (token, group n/4) and
//     summing the four columns of each head (DPP row rotations) gives the scores.
//   output  O^T[d][16 col] += V codes^T x P'^T     v_mfma_f32_16x16x32_f16
//     over two tiles (32 tokens) per step.  P' = p * (V scale of the token's group of
//     d), rounded once to fp16: column n carries head n%4 with the V scales of group
//     n/4, so one P' serves every group and output column 4q + h is read for group q's
//     d.  The V pool is stored in 16-token tiles whose lane chunks are half of these A
//     operands.
//
// Operand ranges: q' of a head whose max |q'| lies outside [2^-4, 2^15) enters the score
// MFMAs shifted by a power of two (qnorm_shift), taken back out of the scores; P' = p * scale
// stays below 65504 because p <= 2^thr and a tile pair holding a V scale at or above
// 2^(16 - thr) first lowers thr (and moves the softmax reference point up by the same amount).
//
// A nibble t (two's complement code c = (t ^ 8) - 8) becomes an exact fp16 through a
// magic exponent, two codes per 32-bit operation, plus a bias that the MFMAs cancel
// (biased_codes_to_f16).
//
// Each wave streams its tile pairs through an LDS ring (buffer loads straight into LDS)
// two pairs ahead of the one it works on.
//
// The std clamp is screened per key from v_dot8 sums of the codes (sum c, sum c^2)
// and the bound |x| <= 8 * scale; keys it may affect get exact fp32 scores.
#include "append_row.h"
#include "kv_common.h"

namespace vkv {
namespace {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

template <bool B>
struct BoolTag {
    static constexpr bool value = B;
};

// fp16 bits of 2^(16 - thr) minus one, in both halves: a V scale s reaches that bound exactly
// when the saturating difference s - (bits - 1) is nonzero
__device__ __forceinline__ u16x2 vscale_bound_bits(int thr) {
    const unsigned short b = (unsigned short)(((31 - thr) << 10) - 1);
    return u16x2{b, b};
}

// Four fp16 pairs from one code dword: pair k = (nibble k, nibble k + 4).  A nibble t
// sits in an fp16 mantissa under a magic exponent (1024 + u for bits 0..3, 64 + u for
// bits 4..7, u = t ^ 8 = code + 8), so one shift and four three-input bit operations
// give eight codes exactly, each plus a bias: code + 1032 in pairs 0 and 2 (nibbles 0-3),
// code + 72 in pairs 1 and 3 (nibbles 4-7).
__device__ __forceinline__ void biased_codes_to_f16(uint32_t w, uint32_t out[4]) {
    const uint32_t w8 = w >> 8;
    out[0] = ((w ^ 0x00080008u) & 0x000F000Fu) | 0x64006400u;
    out[1] = ((w ^ 0x00800080u) & 0x00F000F0u) | 0x54005400u;
    out[2] = ((w8 ^ 0x00080008u) & 0x000F000Fu) | 0x64006400u;
    out[3] = ((w8 ^ 0x00800080u) & 0x00F000F0u) | 0x54005400u;
}

// K codes for the score MFMAs: pairs 0 and 2 lose their bias (a packed subtraction each);
// pairs 1 and 3 keep code + 72, and the score MFMAs start from minus that bias' share of
// every column (72 times the column's B operands on those k-slots), which cancels it.
// V codes for the P.V MFMAs keep both biases: a second MFMA per d-tile whose A operand is
// the constant -1032 or -72 takes each pair's share back right away (it rounds once in
// fp32 at up to 1040 times the pair's P' sum: below 2^-24 * 1040 / 8 of max |v| over the
// whole context).
__device__ __forceinline__ void k_codes_to_f16(uint32_t w, uint32_t out[4]) {
    biased_codes_to_f16(w, out);
    const h2_t b0 = {(_Float16)1032.0f, (_Float16)1032.0f};
    out[0] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, out[0]) - b0);
    out[2] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, out[2]) - b0);
}

template <int D>
struct I4Frags {
    static constexpr int NQ = D / 32;
    uint32_t k[NQ];       // token n: canonical code dwords g*NQ .. g*NQ+NQ-1
    uint32_t v[NQ];       // V tile lane chunk (g, n)
    uint32_t ks_own;      // K scale of (token n, this lane's group), low 16 bits
    uint2 ks_col;         // K scales of tokens 4g..4g+3 for column group (n/4) % G
    _Float16 vs[4];       // V scales of tokens 4g..4g+3 for column group (n/4) % G
    uint32_t flags;       // clamp flags of the tile's 16 keys (the same in every lane)
    uint32_t fword;       // index of that flag word (wave-uniform)
};

// ---- tile loads straight into LDS (buffer_load ... lds) ----
//
// A wave's next tile pairs stream into an LDS ring while it works on the current pair
// from registers, so the loads in flight take no VGPRs.  Each load goes through a buffer
// descriptor bounded to the tile's bytes (out-of-range lanes and descriptors of size 0
// write zeros and read nothing), built on the scalar unit per tile; the per-lane offsets
// are loop invariants.  Lane i of a load writes its bytes at M0 + size * i.
//
// The loads are issued from inline asm (a compiler-visible LDS DMA makes every later LDS
// read wait for all of them), so their waits are explicit: vector memory operations
// complete in issue order, and s_waitcnt vmcnt(n) returns once at most n are in flight,
// so waiting for (pairs in flight - 1) x 8 loads lands the oldest pair.  Loads the
// compiler issues itself in between could only make such a wait longer.
typedef int32_t rsrc_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ rsrc_t tile_rsrc(const void* base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    // word 1: base bits 32..47, stride 0 (the host admits pool addresses below 2^47, so
    // bits 48..63 are zero); word 3: 32-bit data format (raw buffer access)
    return rsrc_t{(int32_t)(uint32_t)a, (int32_t)(uint32_t)(a >> 32), (int32_t)bytes, 0x00020000};
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)reinterpret_cast<uintptr_t>(p); }
// 16 (4) bytes per lane from the descriptor's base + voff into LDS at lds + 16 (4) * lane
__device__ __forceinline__ void lds_load16(uint32_t lds, rsrc_t r, uint32_t voff) {
    asm volatile("buffer_load_dwordx4 %0, %1, 0 offen nt lds" ::"v"(voff), "s"(r), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void lds_load4(uint32_t lds, rsrc_t r, uint32_t voff) {
    asm volatile("buffer_load_dword %0, %1, 0 offen nt lds" ::"v"(voff), "s"(r), "{m0}"(lds) : "memory");
}

template <int N>
__device__ __forceinline__ void wait_loads() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// LDS reads done (before a load overwrites what they read)
__device__ __forceinline__ void wait_lds_reads() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// One tile pair of a wave in LDS: codes and scales of tiles a and b.  K and V codes are
// stored so that lane (g, n) finds its operand chunk at 16 * lane (D = 128) or at the
// chunk's offset in the tile (D = 64); the scales as in the pools, K [group][16 tokens]
// then V [16 tokens][group] (fp16), loaded by lanes 0..31 only (at most 128 bytes each).
struct I4Stage {
    uint4 k[2][64];
    uint4 v[2][64];
    uint32_t sc[2][64];  // [0, 32): K scales, [32, 64): V scales
};
constexpr int kLoadsPerPair = 8;  // LDS loads per tile pair (K, V, K scales, V scales per tile)

// A decode step's new token as its pool writes will hold it: the K row's codes, the V code
// bytes of each group c (byte n at 16c + n, as int4_v_tile_byte places them in the tile),
// the K and V scales and the key's clamp flag.
template <int D>
struct I4NewToken {
    uint4 k[D / 32];
    uint32_t vb[D / 8];
    uint16_t ks[D / 32];
    uint16_t vs[D / 32];
    uint32_t flag;
};

#ifndef VSPEC_I4_MIN_WG_PER_CU
#define VSPEC_I4_MIN_WG_PER_CU 2
#endif

// ST: tile pairs in flight per wave (LDS stages); FL: the tile loop takes the pool's clamp
// flags (and screens only what they cannot say); without FL it screens every tile, a
// lighter loop for short per-workgroup shares.  USED: per-block used counts cap each tile
// (block_used).
template <int D, int GW, int PB, int ST, bool FL, bool USED>
__global__ __launch_bounds__(256, VSPEC_I4_MIN_WG_PER_CU) void decode_mfma_i4(DecodeParams p) {
    constexpr int NQ = D / 32;   // code dwords per lane = QK MFMAs per tile = groups
    constexpr int NG = D / 32;
    constexpr int NDT = D / 16;  // PV d-tiles
    __shared__ I4Stage stg[ST][kWaves];
    // the waves' softmax states at the end of a work item, in the ring's memory (between
    // the barrier after the tile loops and the one before the next item's loads)
    static_assert(sizeof(float) * kWaves * GW * (D + 2) <= sizeof(stg), "wave states fit the ring");
    float(*comb)[GW][D + 2] = reinterpret_cast<float(*)[GW][D + 2]>(&stg[0][0]);
    __shared__ float qs[GW][D];
    __shared__ uint4 qb_lds[NQ][2][64];  // QK B operands (hi, lo) per lane
    __shared__ float kbias_lds[NQ][16];   // per score MFMA and column: the K bias' share (k_codes_to_f16)
    __shared__ int qexp_lds[4];           // per head: the q' operand shift (qnorm_shift)
    __shared__ float patch_val[kWaves][kTile][4];
    __shared__ int patch_flag[kWaves][kTile];
    __shared__ SplitShared split_sh;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4;
    const int n = lane & 15;

    const int ips = (int)(p.hkv * p.gsplit);  // work items per sequence
    const WorkSplit ws = work_split<kSplitAlways>(p, ips, split_sh);
    // q rows of a work item (wave w < GW: head w), loaded ahead of the item's set-up
    constexpr int E = D / 64;
    float q_rows[E];
    auto load_q = [&](const int bb, const int yy) {
        if (wave < GW) {
            const int hq = (yy / (int)p.gsplit) * ((int)p.gsplit * GW) + (yy % (int)p.gsplit) * GW + wave;
            const float* qrow = p.q + ((size_t)bb * p.hq + hq) * D;
#pragma unroll
            for (int e = 0; e < E; ++e) q_rows[e] = qrow[lane * E + e];
        }
    };
    ItemCursor c0 = {0, 0, 1, 0, 0};
    if (ws.lo < ws.hi) {
        c0 = cursor_at(p, ws);
        load_q(c0.b, c0.y);
    }
    const bool appending = p.k_new != nullptr && ws.lo < ws.hi;
    // The fused decode step's new token of the range's first work item, when the range holds
    // that item's last tile (exactly one workgroup appends each item) and the token's
    // position lies in the table.  Lanes below kNtLanes of wave 0 (4 elements of the K or
    // V row each) quantise it from the source rows alone into `nt` before the workgroup's
    // first barrier; the tile loop copies it into the stage of the item's last tile once
    // that tile has landed, and its clamp flag into the tile's flag word, so the launch never
    // waits for its own pool writes, which lanes below kAppendLanes (one group of K, even
    // lanes, or V, odd lanes) issue after the item's tile loop.
    constexpr int kNtLanes = 16 * NG;
    constexpr int kAppendLanes = 2 * NG;
    static_assert(kNtLanes <= 64, "the new token's lanes fit one wave");
    __shared__ I4NewToken<D> nt;
    const int ctx0 = appending ? as_const(p.ctx_lens)[c0.b] : 0;
    const bool nt_in = appending && c0.item0 + c0.U <= ws.hi && ctx0 > 0 &&
                       ctx0 <= (int)(p.max_blocks * p.block_tokens);
    const uint32_t nt_pos = nt_in ? (uint32_t)ctx0 - 1u : 0u;
    const uint32_t nt_slot = nt_pos % kTile;  // in its tile
    const uint32_t nt_bit = 1u << nt_slot;
    int nt_phys = -1;  // (appending lanes) table entry of the token's block
    // Lane (row, c, k) of a token's encoding holds elements 4k..4k+3 of group c of the K
    // (row 0) or V row (lanes below kNtLanes).
    const int e_row = lane / (8 * NG), e_c = (lane >> 3) % NG, e_k = lane & 7;
    auto load_token = [&](const int bb, const uint32_t hk, float (&x)[4]) {
        const size_t src_el = ((size_t)bb * p.hkv + hk) * D + 32 * e_c + 4 * e_k;
        const uint8_t* src = e_row ? p.v_new : p.k_new;
        if (p.append_src == VSPEC_KV_F32) {
            const float4 w = *reinterpret_cast<const float4*>(src + src_el * 4);
            x[0] = w.x; x[1] = w.y; x[2] = w.z; x[3] = w.w;
        } else {
            const uint2 w = *reinterpret_cast<const uint2*>(src + src_el * 2);
            x[0] = half_bits_to_float(w.x & 0xffffu); x[1] = half_bits_to_float(w.x >> 16);
            x[2] = half_bits_to_float(w.y & 0xffffu); x[3] = half_bits_to_float(w.y >> 16);
        }
    };
    // One token quantised by the lanes below kNtLanes of a wave: the group's 2nd-largest |x|,
    // code sums and V bytes come from its 8 lanes, so every value equals the one-lane encoding
    // of the append kernel (int4_encode_group).  The lane's 4 codes (element 4k + e in nibble
    // e, at bytes 16c + 2k of a K row), for V lanes with k < 4 the V code bytes n = 4k..4k+3
    // of group c, the group's scale bits and (lane 0) the key's clamp flag.
    struct TokenLane {
        uint32_t chunk, vword, s16;
        bool flag;
    };
    auto encode_token = [&](const float (&x)[4]) -> TokenLane {
        TokenLane r = {0u, 0u, 0u, false};
        // the top two |x| of the lane, merged over the group's lanes by DPP moves (its
        // quad partners, then the other quad: exact, comparisons only)
        float a1 = 0.f, a2 = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) int4_top2(fabsf(x[e]), a1, a2);
        auto merge_top2 = [&](const float b1, const float b2) {
            a2 = fmaxf(fminf(a1, b1), fmaxf(a2, b2));
            a1 = fmaxf(a1, b1);
        };
        merge_top2(dpp<kQuadXor1>(a1), dpp<kQuadXor1>(a2));
        merge_top2(dpp<kQuadXor2>(a1), dpp<kQuadXor2>(a2));
        merge_top2(dpp<kRowHalfMirror>(a1), dpp<kRowHalfMirror>(a2));
        r.s16 = int4_scale_bits(a2);
        const float sc = half_bits_to_float(r.s16);
        int c1 = 0, c2 = 0, cm = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int code = int4_code(x[e], sc);
            r.chunk |= ((uint32_t)code & 0xfu) << (4 * e);
            c1 += code;
            c2 += code * code;
            cm = max(cm, code < 0 ? -code : code);
        }
        if (e_row == 0) {
            // the key's clamp flag from the row's sums, the groups added pairwise as
            // int4_key_flag adds them (integer code sums: exact in fp32 in any order)
            const float gc1 = group_sum<8>((float)c1), gc2 = group_sum<8>((float)c2);
            float gcm = (float)cm;
            gcm = fmaxf(gcm, dpp<kQuadXor1>(gcm));
            gcm = fmaxf(gcm, dpp<kQuadXor2>(gcm));
            gcm = fmaxf(gcm, dpp<kRowHalfMirror>(gcm));
            float s1 = sc * gc1, s2 = (sc * sc) * gc2, m = sc * gcm;
            // group g0 + g1 (lane ^ 8: the row's other half), then (g0 + g1) + (g2 + g3)
            s1 += row_dpp<kRowRor8>(s1);
            s2 += row_dpp<kRowRor8>(s2);
            m = fmaxf(m, row_dpp<kRowRor8>(m));
            if constexpr (NG == 4) {
                s1 = add_xor16(s1);
                s2 = add_xor16(s2);
                m = max_xor16(m);
            }
            r.flag = p.kf && int4_flag_from_sums(s1, s2, m, D);
        } else {
            // V: byte n of group c holds d = 32c + n (low nibble, lane n/4) and d = 32c + 16 + n
            // (high nibble, lane 4 + n/4)
            const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)r.chunk, kRowRor12, 0xf, 0xf, true);  // lane + 4
#pragma unroll
            for (int e = 0; e < 4; ++e) r.vword |= (((r.chunk >> (4 * e)) & 0xfu) | (((hi >> (4 * e)) & 0xfu) << 4)) << (8 * e);
        }
        return r;
    };
    if (appending && wave == 0 && nt_in && lane < kNtLanes) {
        float x[4];
        load_token(c0.b, (uint32_t)c0.y / p.gsplit, x);
        // a vector load (the barriers wait for scalar ones), used after the tile loop
        const __amdgpu_buffer_rsrc_t trow = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<int32_t*>(p.block_tables + (size_t)c0.b * p.max_blocks), (short)0,
            (int)(4u * p.max_blocks), 0x00020000);
        nt_phys = __builtin_amdgcn_raw_buffer_load_b32(trow, (int)(4u * (nt_pos / p.block_tokens)), 0, 0);
        const TokenLane tl = encode_token(x);
        if (e_row == 0) {
            reinterpret_cast<uint16_t*>(nt.k)[8 * e_c + e_k] = (uint16_t)tl.chunk;
            if (e_k == 0) nt.ks[e_c] = (uint16_t)tl.s16;
            if (lane == 0) nt.flag = tl.flag ? 1u : 0u;
        } else {
            if (e_k < 4) nt.vb[4 * e_c + e_k] = tl.vword;
            if (e_k == 0) nt.vs[e_c] = (uint16_t)tl.s16;
        }
    }
    // The range's further appended items (short ones), the j-th of them by wave j % kWaves,
    // are written to the pool at once (the same bytes as the append kernel's), and their
    // tiles are read after the first barrier: these waves wait for their stores.
    if (appending) {
        const uint32_t P0 = PB ? (uint32_t)PB : p.block_tokens;
        ItemCursor c = c0;
        bool direct = false;
        int j = 0;
        while (c.item0 + c.U < ws.hi) {
            cursor_next(p, ips, c);
            const int ctx = as_const(p.ctx_lens)[c.b];
            if (c.item0 + c.U > ws.hi || ctx <= 0) continue;
            if (j++ % kWaves != wave || ctx > (int)(p.max_blocks * P0)) continue;
            direct = true;
            const uint32_t pos = (uint32_t)ctx - 1u, hk = (uint32_t)c.y / p.gsplit;
            const int phys = as_const(p.block_tables)[(size_t)c.b * p.max_blocks + pos / P0];
            if (lane < kNtLanes) {
                float x[4];
                load_token(c.b, hk, x);
                const TokenLane tl = encode_token(x);
                if (phys >= 0 && (uint32_t)phys < p.num_blocks) {
                    const uint32_t slot = pos % P0;
                    const size_t bh = (size_t)phys * p.hkv + hk;
                    if (e_row == 0) {
                        *reinterpret_cast<uint16_t*>(const_cast<uint8_t*>(p.k) + (bh * P0 + slot) * (D / 2) + 16 * e_c + 2 * e_k) =
                            (uint16_t)tl.chunk;
                        if (e_k == 0) const_cast<uint16_t*>(p.ks)[int4_ks_index(bh, NG, P0, slot, e_c)] = (uint16_t)tl.s16;
                        if (lane == 0 && p.kf) {
                            apply_flag({const_cast<uint32_t*>(p.kf) + bh * (P0 / kTile) + slot / kTile,
                                        1u << (slot % kTile), tl.flag});
                        }
                    } else if (e_k < 4) {
                        uint8_t* vt = const_cast<uint8_t*>(p.v) + bh * ((size_t)P0 * D / 2) + (size_t)(slot / kTile) * (8 * D);
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            vt[int4_v_tile_byte(slot, e_c, 4 * e_k + e, D)] = (uint8_t)(tl.vword >> (8 * e));
                        }
                        if (e_k == 0) const_cast<uint16_t*>(p.vs)[(bh * P0 + slot) * NG + e_c] = (uint16_t)tl.s16;
                    }
                }
            }
        }
        if (direct) __builtin_amdgcn_s_waitcnt(0);
    }
    int b = ws.b;
    int seq0 = ws.seq0;
    for (int pos = ws.lo; pos < ws.hi;) {
        const int U = item_tiles(p, b);
        if (pos >= seq0 + U * ips) {
            seq0 += U * ips;
            ++b;
            continue;
        }
        const int y = (pos - seq0) / U;
        const int item0 = seq0 + y * U;
        const int tile_begin = pos - item0;
        const int tile_end = min(ws.hi, item0 + U) - item0;
        const int hk = y / (int)p.gsplit;
        const int hq0 = hk * ((int)p.gsplit * GW) + (y % (int)p.gsplit) * GW;
        const int ctx = min(max(as_const(p.ctx_lens)[b], 0), (int)(p.max_blocks * p.block_tokens));

        const int P = PB ? PB : (int)p.block_tokens;
        const int tiles_per_block = P / kTile;
        const const_i32* table = as_const(p.block_tables) + (size_t)b * p.max_blocks;
        const const_i32* used_row = USED ? as_const(p.block_used) + (size_t)b * p.max_blocks : nullptr;
        const int own_group = (g * NQ) >> 2;
        const int col_group = (n >> 2) % NG;

        // clamp flags from the pool (see screen below); `fused`: this launch appended each
        // work item's last token
        const bool flags_on = FL && p.alpha >= 4.5f;
        const bool fused = p.k_new != nullptr;
        // nvalid is at most kTile (16): the shift stays below 32
        auto valid_mask = [](int nvalid) -> uint32_t { return (1u << nvalid) - 1u; };

        // ---- tile pairs into this wave's LDS ring ----
        // Per-lane byte offsets of the loads: K lane (g, n) takes token n's code dwords
        // g*NQ.. (D = 128: 16 bytes, stored lane-major; D = 64: the tile's 512 bytes copied
        // by lanes 0-31); V tiles are lane-major chunks already; the K scales' NG rows of 16
        // tokens (row stride P) and the V scales' 16 x NG go one dword per lane.
        const uint32_t off_k = NQ == 4 ? (uint32_t)(n * (D / 2) + 16 * g) : 16u * (uint32_t)lane;
        const uint32_t off_v = 16u * (uint32_t)lane;
        const uint32_t off_ks = lane < 8 * NG ? (uint32_t)((lane >> 3) * P * 2 + 4 * (lane & 7)) : 0x40000000u;
        static_assert(8 * NG <= 32, "the scales of a tile fit lanes 0..31");
        const uint32_t off_vs = 4u * (uint32_t)lane;
        // per stage: how many of each tile's tokens its block holds (16, or block_used's
        // cap; 0: none), its clamp flag word and that word's index (all wave-uniform)
        int cap_s[ST][2];
        uint32_t flag_s[ST][2], fword_s[ST][2];
        // Table entries (and used counts) of a pair's tiles, read one pair ahead of its loads
        // so that the scalar reads are not waited for on the way to the loads.  The tile
        // index is wave-uniform, so the table, used-count and flag reads stay on the scalar
        // unit.
        struct Look {
            int entry[2];
            int used[2];
        };
        auto lookup = [&](int tile_a) -> Look {
            Look l;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int tile = __builtin_amdgcn_readfirstlane(tile_a + h);
                const int entry_idx = (tile < tile_end ? tile : tile_end - 1) / tiles_per_block;
                l.entry[h] = table[entry_idx];
                l.used[h] = USED ? used_row[entry_idx] : kTile;
            }
            return l;
        };
        // The loads of one tile.  A tile past the range or behind an invalid table entry gets
        // descriptors of size 0 (zeros, no memory traffic) and cap 0.
        auto issue_tile = [&](int tile, const int entry, const int used, I4Stage& st, const int h, int& cap,
                              uint32_t& flag, uint32_t& fword) {
            tile = __builtin_amdgcn_readfirstlane(tile);
            // 1 when the tile is in the range and its entry a valid block (the host bounds
            // num_blocks by INT32_MAX, so a negative entry fails the unsigned compare); kept
            // as an integer, which stays on the scalar unit without lane-mask conversions
            const uint32_t ok = (uint32_t)(tile < tile_end) & (uint32_t)((uint32_t)entry < p.num_blocks);
            const int slot0 = (tile % tiles_per_block) * kTile;
            // block x head index in 32 bits (check_kv bounds num_blocks * hkv)
            const size_t bh = ((uint32_t)entry & (0u - ok)) * p.hkv + (uint32_t)hk;
            const uint32_t code_bytes = ok * (8u * D);
            lds_load16(lds_addr(&st.k[h][0]), tile_rsrc(p.k + (bh * P + slot0) * (D / 2), code_bytes), off_k);
            lds_load16(lds_addr(&st.v[h][0]),
                       tile_rsrc(p.v + bh * ((size_t)P * D / 2) + (size_t)(slot0 / kTile) * (8 * D), code_bytes), off_v);
            if (lane < 8 * NG) {
                lds_load4(lds_addr(&st.sc[h][0]),
                          tile_rsrc(p.ks + bh * NG * P + slot0, ok * (uint32_t)(((NG - 1) * P + kTile) * 2)), off_ks);
                lds_load4(lds_addr(&st.sc[h][32]), tile_rsrc(p.vs + (bh * P + slot0) * NG, ok * (32u * NG)), off_vs);
            }
            fword = (uint32_t)(bh * (P / kTile) + slot0 / kTile);
            flag = flags_on ? (uint32_t)as_const(reinterpret_cast<const int32_t*>(p.kf))[fword] : 0u;
            if constexpr (USED) cap = ok ? used_cap(used, slot0) : 0;
            else cap = (int)ok * kTile;
        };
        auto issue = [&](int tile_a, int u, const Look& l) {
            issue_tile(tile_a, l.entry[0], l.used[0], stg[u][wave], 0, cap_s[u][0], flag_s[u][0], fword_s[u][0]);
            issue_tile(tile_a + 1, l.entry[1], l.used[1], stg[u][wave], 1, cap_s[u][1], flag_s[u][1], fword_s[u][1]);
        };
        // a stage's tile h into registers: the K half (codes, K scales) and the V half
        auto fetch_k = [&](const I4Stage& st, const int h, I4Frags<D>& f) {
            if constexpr (NQ == 4) {
                const uint4 a = st.k[h][lane];
                f.k[0] = a.x; f.k[1] = a.y; f.k[2] = a.z; f.k[3] = a.w;
            } else {
                const uint2 a = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint8_t*>(&st.k[h][0]) + n * (D / 2) + 8 * g);
                f.k[0] = a.x; f.k[1] = a.y;
            }
            const uint8_t* ks = reinterpret_cast<const uint8_t*>(&st.sc[h][0]);
            f.ks_own = *reinterpret_cast<const uint16_t*>(ks + own_group * 32 + 2 * n);
            f.ks_col = *reinterpret_cast<const uint2*>(ks + col_group * 32 + 8 * g);
        };
        auto fetch_v = [&](const I4Stage& st, const int h, I4Frags<D>& f) {
            if constexpr (NQ == 4) {
                const uint4 c = st.v[h][lane];
                f.v[0] = c.x; f.v[1] = c.y; f.v[2] = c.z; f.v[3] = c.w;
            } else {
                const uint2 c = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint8_t*>(&st.v[h][0]) + 8 * lane);
                f.v[0] = c.x; f.v[1] = c.y;
            }
            const _Float16* vs = reinterpret_cast<const _Float16*>(&st.sc[h][32]) + 4 * NG * g + col_group;
#pragma unroll
            for (int r = 0; r < 4; ++r) f.vs[r] = vs[r * NG];
        };
        // nt over whatever the load of its tile (stage tile h, landed) read at its slot:
        // the K row's 16-byte chunks where the K load put them, the K scales (group-major
        // rows of 16) and V scales (token-major) of the slot, and the V code bytes
        auto patch_new_token = [&](I4Stage& st, const int h) {
            if (lane < D / 32) st.k[h][NQ == 4 ? 16 * lane + (int)nt_slot : 2 * (int)nt_slot + lane] = nt.k[lane];
            uint16_t* sc16 = reinterpret_cast<uint16_t*>(&st.sc[h][0]);
            if (lane < NG) {
                sc16[16 * lane + nt_slot] = nt.ks[lane];
                sc16[64 + NG * nt_slot + lane] = nt.vs[lane];
            }
            if (lane < 16 * NG) {
                reinterpret_cast<uint8_t*>(&st.v[h][0])[int4_v_tile_byte(nt_slot, (uint32_t)lane >> 4, (uint32_t)lane & 15u, D)] =
                    reinterpret_cast<const uint8_t*>(nt.vb)[lane];
            }
        };

        const int step = 2 * kWaves;
        const int t0 = tile_begin + 2 * wave;

        // ---- q' = clip(q) * scale * log2(e): wave w prepares head w ----
        if (wave < GW) {
            float x[E];
            float s = 0.f;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                x[e] = q_rows[e];
                s += x[e];
            }
            s = wave_sum(s);
            const float mean = s * (1.0f / D);
            float v = 0.f;
#pragma unroll
            for (int e = 0; e < E; ++e) v = fmaf(x[e] - mean, x[e] - mean, v);
            v = wave_sum(v);
            const float th = fminf(fmaxf(1e-6f, p.alpha * sqrtf(v * (1.0f / D))), p.input_clip);
            float am = 0.f;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const float y = fminf(fmaxf(x[e], -th), th) * p.qscale;
                qs[wave][lane * E + e] = y;
                am = fmaxf(am, fabsf(y));
            }
            am = wave_max(am);
            if (lane == 0) qexp_lds[wave] = qnorm_shift(am);
        }
        // The first ST pairs are on their way while the q operands are prepared (after the
        // q rows are in registers: a wait for those would also wait for these).
        // the ring's first table reads go out together
        Look first_look[ST];
#pragma unroll
        for (int u = 0; u < ST; ++u) first_look[u] = lookup(t0 + u * step);
#pragma unroll
        for (int u = 0; u < ST; ++u) issue(t0 + u * step, u, first_look[u]);
        Look next = lookup(t0 + ST * step);
        __syncthreads();
        // this item takes its new token from nt (written before the barrier): the token's
        // slot in the item's last tile, and its clamp flag bit in that tile's flag word
        const bool nt_item = nt_in && pos == ws.lo;
        const uint32_t nt_val = nt_item && __builtin_amdgcn_readfirstlane(nt.flag) ? nt_bit : 0u;
        // the tile this launch appended into without taking nt: its flags come from the screen
        const int scr_tile = fused && !nt_item ? U - 1 : -2;

        // ---- QK B operands: k-slots 8g..8g+7 of MFMA m carry code dword dw = g*NQ + m in
        // the order e = 0,4,1,5,2,6,3,7; column n takes group n/4 of head n%4 ----
        // head h's operands carry q' * 2^e_h (qnorm_shift), taken back out of the scores by
        // qfac = 2^-e_h; the tile loop is instantiated twice, and only the one run for items
        // where some head has e != 0 (qnorm, wave-uniform) multiplies
        // wave m builds the operands of score MFMA m (NQ <= kWaves)
        if (wave < NQ) {
            const int m = wave;
            const int hh = n & 3;
            const int hs = hh < GW ? hh : 0;
            const float qin = pow2i(qexp_lds[hs]);
            float odd = 0.f;  // this lane's B operands on the k-slots of odd elements
            const int dw = g * NQ + m;
            const bool on = (dw >> 2) == (n >> 2) && hh < GW;
            h8_t hi8, lo8;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int e = (j >> 1) + 4 * (j & 1);
                const float qv = qs[hs][8 * dw + e] * (on ? qin : 0.0f);
                const _Float16 hi = (_Float16)qv;
                hi8[j] = hi;
                lo8[j] = (_Float16)(qv - (float)hi);
                if (e & 1) odd += (float)hi8[j] + (float)lo8[j];
            }
            qb_lds[m][0][lane] = __builtin_bit_cast(uint4, hi8);
            qb_lds[m][1][lane] = __builtin_bit_cast(uint4, lo8);
            odd = add_rows(odd);
            if (g == 0) kbias_lds[m][n] = odd;
        }
        __syncthreads();
        float kb = 0.f;
#pragma unroll
        for (int m = 0; m < NQ; ++m) kb += kbias_lds[m][n];
        const float kbias = 72.0f * kb;
        int qe_any = 0;
#pragma unroll
        for (int h = 0; h < GW; ++h) qe_any |= qexp_lds[h];
        const bool qnorm = __builtin_amdgcn_readfirstlane(qe_any) != 0;
        const float qfac = (n & 3) < GW ? pow2i(-qexp_lds[(n & 3) < GW ? (n & 3) : 0]) : 1.0f;
        // the B operands stay in registers for the whole item (32 VGPRs): read from LDS per
        // pair they cost 8 reads and a wait before each score MFMA
        h8_t qreg[NQ][2];
#pragma unroll
        for (int m = 0; m < NQ; ++m) {
            qreg[m][0] = __builtin_bit_cast(h8_t, qb_lds[m][0][lane]);
            qreg[m][1] = __builtin_bit_cast(h8_t, qb_lds[m][1][lane]);
        }

        f4_t acc[NDT];
#pragma unroll
        for (int j = 0; j < NDT; ++j) acc[j] = f4_t{0.f, 0.f, 0.f, 0.f};
        // Online softmax state.  Scores are formed relative to the running max m_run
        // (the K-scale FMA subtracts it), so the score clip moves with it: clip_lo/hi hold
        // the clip bounds minus m_run; columns that hold no head clip to -inf (3-bit mode:
        // +-24*log2e).  The wave's first scored pair of a work item sets m_run outright.
        // Columns n, n+4, n+8 and n+12 hold head n%4's scores (the same values), so each
        // keeps the head's whole state.
        float m_run = 0.f;
        float l_run = 0.f;
        const bool head_col = (n & 3) < GW;
        float clip_hi = head_col ? p.logit_clip : -INFINITY;
        float clip_lo = head_col ? -p.logit_clip : -INFINITY;
        bool first = true;
        // p = exp2(s) stays at or below 2^thr (the lazy max below), so P' = p * (V scale) stays
        // below 65504 while every V scale is below 2^(16 - thr); vtb holds that bound's fp16
        // bits minus one, twice (see pv)
        int thr = 8;
        u16x2 vtb = vscale_bound_bits(thr);
        // every column holds a head and the logits are not clipped: the clip is the identity
        const bool clip_on = GW < 4 || p.logit_clip < INFINITY;

        // Clamp screen of key n of a tile (this lane: one group's codes): mean and E[x^2]
        // from integer code sums; this group's |x| <= 8 * scale.  `flag` is set in a lane
        // whose group may reach the clamp threshold; key n is flagged when any of its four
        // lanes is (tokens() folds the wave's ballot).  The flag kernel (FL) skips it: the
        // append ran the same test once per key (alpha 4.5; a larger alpha only clamps
        // less).  Only tiles this launch's fused append wrote into are screened there,
        // except the one whose new flag the append published in LDS.
        struct Screen {
            float mean;
            bool flag;
        };
        auto screen = [&](const I4Frags<D>& f, const int nvalid) -> Screen {
            int c1 = 0, c2 = 0;
#pragma unroll
            for (int m = 0; m < NQ; ++m) {
                c1 = __builtin_amdgcn_sdot8((int)f.k[m], 0x11111111, c1, false);
                c2 = __builtin_amdgcn_sdot8((int)f.k[m], (int)f.k[m], c2, false);
            }
            const float s_own = (float)__builtin_bit_cast(_Float16, (uint16_t)f.ks_own);
            const float s1 = add_rows(s_own * (float)c1);
            const float s2 = add_rows((s_own * s_own) * (float)c2);
            const float mean = s1 * (1.0f / D);
            const float ex2 = s2 * (1.0f / D);
            const float var1 = ex2 - mean * mean;
            // hardware square root (1 ulp): the 2^-10 margin below absorbs it
            const float th1 = fminf(fmaxf(1e-6f, p.alpha * __builtin_amdgcn_sqrtf(fmaxf(var1, 0.f))), p.input_clip);
            return {mean, (n < nvalid) && (8.0f * s_own > th1 * (1.0f - 0.0009765625f) || var1 <= ex2 * 0.0009765625f)};
        };
        // keys (bit n) with a flagged lane, from a wave ballot
        auto tokens = [](uint64_t m) -> uint32_t { return (uint32_t)((m | (m >> 16) | (m >> 32) | (m >> 48)) & 0xffffu); };

        // Scores of a tile on the matrix cores, minus m_run: lane (g, n) gets tokens
        // 4g..4g+3 for head n%4.  The hi and lo products accumulate in one chain (the lo
        // part is 2^-11 of the hi part: one fp32 accumulator keeps both), from minus the K
        // bias' share of the column (its magnitude, 72 |sum q'|, costs 2^-24 of it); each of the four
        // group columns of a head is scaled by its fp16 K scale and takes a quarter of
        // m_run in the same mixed-precision FMA, so the column sum is score - m_run.
        auto qk = [&](const I4Frags<D>& f, auto qn) -> f4_t {
            f4_t sacc = {-kbias, -kbias, -kbias, -kbias};
#pragma unroll
            for (int m = 0; m < NQ; ++m) {
                uint32_t pr4[4];
                k_codes_to_f16(f.k[m], pr4);
                const h8_t a = __builtin_bit_cast(h8_t, make_uint4(pr4[0], pr4[1], pr4[2], pr4[3]));
                sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qreg[m][0], sacc, 0, 0, 0);
                sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qreg[m][1], sacc, 0, 0, 0);
            }
            if constexpr (decltype(qn)::value) sacc *= qfac;
            const h2_t kc[2] = {__builtin_bit_cast(h2_t, f.ks_col.x), __builtin_bit_cast(h2_t, f.ks_col.y)};
            const float mq = -0.25f * m_run;
            f4_t sc;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float v = __builtin_fmaf(sacc[r], (float)kc[r >> 1][r & 1], mq);
                v += row_dpp<kRowRor8>(v);
                v += row_dpp<kRowRor4>(v);
                sc[r] = v;
            }
            return sc;
        };

        // Exact fp32 scores for the flagged keys of a tile (reference clamp, two-pass variance).
        auto exact = [&](const I4Frags<D>& f, const uint32_t flagged, f4_t& sc) {
            const float s_own = (float)__builtin_bit_cast(_Float16, (uint16_t)f.ks_own);
            float x[8 * NQ];
#pragma unroll
            for (int m = 0; m < NQ; ++m) {
#pragma unroll
                for (int e = 0; e < 8; ++e) x[8 * m + e] = nibble(f.k[m], e) * s_own;
            }
            float s1 = 0.f;
#pragma unroll
            for (int i = 0; i < 8 * NQ; ++i) s1 += x[i];
            const float mean = add_rows(s1) * (1.0f / D);
            float v2 = 0.f;
#pragma unroll
            for (int i = 0; i < 8 * NQ; ++i) v2 = fmaf(x[i] - mean, x[i] - mean, v2);
            v2 = add_rows(v2);
            const float th = fminf(fmaxf(1e-6f, p.alpha * sqrtf(v2 * (1.0f / D))), p.input_clip);
            float part[GW];
#pragma unroll
            for (int h = 0; h < GW; ++h) {
                float a = 0.f;
#pragma unroll
                for (int i = 0; i < 8 * NQ; ++i) a = fmaf(qs[h][8 * g * NQ + i], fminf(fmaxf(x[i], -th), th), a);
                part[h] = add_rows(a);
            }
            // Exchange through this wave's LDS slots: a wave's LDS accesses complete in
            // program order and the compiler keeps these possibly-aliasing accesses in
            // order, so no fence is needed.  (A fence or wave barrier here would count as
            // a memory clobber and push the block-table reads off the scalar unit.)
            if (g == 0) {
                patch_flag[wave][n] = (int)((flagged >> n) & 1u);
#pragma unroll
                for (int h = 0; h < GW; ++h) patch_val[wave][n][h] = part[h];
            }
            if (head_col) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int t = 4 * g + r;
                    if (patch_flag[wave][t]) sc[r] = patch_val[wave][t][n & 3] - m_run;
                }
            }
        };

        // Slots past the context (or a whole missing tile) may hold any scale bits (NaN):
        // their V scales become 0 so that p' = p * scale = 0.
        auto clear_masked_scales = [&](I4Frags<D>& f, const int nvalid) {
            if (nvalid < kTile) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (4 * g + r >= nvalid) f.vs[r] = (_Float16)0.0f;
                }
            }
        };

        // Two tiles per step: k-slot 8g + i of the PV MFMA is token 4g + i of tile A (i < 4)
        // or token 4g + i - 4 of tile B.
        // Scores and softmax weights of a pair (the V half of the fragments is not read yet).
        auto scores = [&](auto qn, I4Frags<D>& fa, I4Frags<D>& fb, const int nva, const int nvb, const int tile_a,
                          float (&pr)[8]) {
            // clamp flags: from the pool, or from the screen (both tiles in one basic block:
            // their chains interleave)
            // the tile this launch appended into: its word with nt's flag bit in (the item
            // that takes nt: patched in the tile loop), or (another appended item of this
            // range) the screen
            const bool scr_a = !flags_on || tile_a == scr_tile;
            const bool scr_b = !flags_on || tile_a + 1 == scr_tile;
            auto word_of = [&](const I4Frags<D>& f) -> uint32_t { return __builtin_amdgcn_readfirstlane(f.flags); };
            uint32_t fla, flb;
            f4_t sa, sb;
            if (scr_a || scr_b) {
                const Screen sna = screen(fa, nva);
                const Screen snb = screen(fb, nvb);
                sa = qk(fa, qn);
                sb = qk(fb, qn);
                fla = scr_a ? tokens(__builtin_amdgcn_ballot_w64(sna.flag)) : word_of(fa) & valid_mask(nva);
                flb = scr_b ? tokens(__builtin_amdgcn_ballot_w64(snb.flag)) : word_of(fb) & valid_mask(nvb);
            } else {
                sa = qk(fa, qn);
                sb = qk(fb, qn);
                fla = word_of(fa) & valid_mask(nva);
                flb = word_of(fb) & valid_mask(nvb);
            }
            if ((fla | flb) != 0u) {
                if (fla != 0u) exact(fa, fla, sa);
                if (flb != 0u) exact(fb, flb, sb);
            }

            // ---- online softmax for head n over this lane's 8 tokens (scores relative to
            // m_run).  The running max moves only when a score exceeds it by more than 8
            // (p stays <= 2^8), so the cross-lane max is taken only then, and on the first
            // scored pair. ----
            float s[8];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                s[r] = sa[r];
                s[4 + r] = sb[r];
            }
            if (clip_on) {
#pragma unroll
                for (int i = 0; i < 8; ++i) s[i] = __builtin_amdgcn_fmed3f(s[i], clip_lo, clip_hi);
            }
            if (nva < kTile || nvb < kTile) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    s[r] = 4 * g + r < nva ? s[r] : -INFINITY;
                    s[4 + r] = 4 * g + r < nvb ? s[4 + r] : -INFINITY;
                }
            }
            float smax = s[0];
#pragma unroll
            for (int i = 1; i < 8; ++i) smax = fmaxf(smax, s[i]);
            if (first || __builtin_amdgcn_ballot_w64(smax > (float)thr) != 0) {
                const float mt = max_rows(smax);
                // columns without a head (all -inf) do not move; the four columns of a head
                // (each subtracts a quarter of its own m_run in qk) take the same move
                const bool need = first ? mt > -INFINITY : mt > (float)thr;
                const float dm = need ? mt : 0.0f;
                const float fct = first ? 1.0f : __builtin_amdgcn_exp2f(-dm);
                m_run += dm;
                clip_lo -= dm;
                clip_hi -= dm;
#pragma unroll
                for (int i = 0; i < 8; ++i) s[i] -= dm;
                l_run *= fct;
#pragma unroll
                for (int j = 0; j < NDT; ++j) acc[j] *= fct;
            }
            if (nva > 0 || nvb > 0) first = false;
            // v_exp_f32 of -inf is +0: masked tokens and unused columns drop out
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                pr[i] = __builtin_amdgcn_exp2f(s[i]);
                l_run += pr[i];
            }
        };

        // O^T += V^T P'^T for a pair whose V half of the fragments is in registers
        const h8_t bias_lo = {(_Float16)-1032.0f, (_Float16)-1032.0f, (_Float16)-1032.0f, (_Float16)-1032.0f,
                              (_Float16)-1032.0f, (_Float16)-1032.0f, (_Float16)-1032.0f, (_Float16)-1032.0f};
        const h8_t bias_hi = {(_Float16)-72.0f, (_Float16)-72.0f, (_Float16)-72.0f, (_Float16)-72.0f,
                              (_Float16)-72.0f, (_Float16)-72.0f, (_Float16)-72.0f, (_Float16)-72.0f};
        auto pv = [&](I4Frags<D>& fa, I4Frags<D>& fb, const int nva, const int nvb, float (&pr)[8], const uint32_t vsw) {
            clear_masked_scales(fa, nva);
            clear_masked_scales(fb, nvb);

            // A V scale of the pair at or above 2^(16 - thr) (checked on the stage's raw scale
            // bits: garbage past a context only costs the exact check) may overflow P'.  Then
            // thr drops to 15 - X, X = floor(log2) of the largest valid scale of the pair, and
            // the reference point m_run moves up by the difference: acc, l_run and this pair's
            // p scale by the same power of two, so acc / l_run is unchanged.
            const u16x2 over = __builtin_elementwise_sub_sat(__builtin_bit_cast(u16x2, vsw), vtb);
            if (__builtin_amdgcn_ballot_w64(__builtin_bit_cast(uint32_t, over) != 0u) != 0) {
                float vm = 0.f;
#pragma unroll
                for (int r = 0; r < 4; ++r) vm = fmaxf(vm, fmaxf((float)fa.vs[r], (float)fb.vs[r]));
                vm = wave_max(vm);
                // vm in [2^X, 2^(X + 1)); vm = 0 gives X = -1
                int X;
                (void)frexpf(vm, &X);
                X -= 1;
                const int tnew = __builtin_amdgcn_readfirstlane(min(thr, 15 - X));
                if (tnew < thr) {
                    const int dl = thr - tnew;
                    const float f = pow2i(-dl);
#pragma unroll
                    for (int i = 0; i < 8; ++i) pr[i] *= f;
                    l_run *= f;
#pragma unroll
                    for (int j = 0; j < NDT; ++j) acc[j] *= f;
                    m_run += (float)dl;
                    clip_lo -= (float)dl;
                    clip_hi -= (float)dl;
                    thr = tnew;
                    vtb = vscale_bound_bits(thr);
                }
            }

            // P' = p * scale rounded once to fp16 (v_fma_mix, relative error <= 2^-12): the
            // output error stays below 2.4e-4 * max|v|.  Column n carries the V scales of
            // group (n/4) % G, so one B operand serves every group: output column 4q + h is
            // head h's for the d-tiles of group q, the other columns are not read.
            h8_t pq;
#pragma unroll
            for (int i = 0; i < 8; ++i) pq[i] = (_Float16)__builtin_fmaf(pr[i], (float)(i < 4 ? fa.vs[i] : fb.vs[i - 4]), 0.0f);
            // ---- O^T += V^T P'^T over 32 tokens, one V scale group (two d-tiles) at a time ----
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
                uint32_t ka[4], kb[4];
                biased_codes_to_f16(fa.v[q], ka);
                biased_codes_to_f16(fb.v[q], kb);
                const h8_t a0 = __builtin_bit_cast(h8_t, make_uint4(ka[0], ka[2], kb[0], kb[2]));  // code + 1032
                const h8_t a1 = __builtin_bit_cast(h8_t, make_uint4(ka[1], ka[3], kb[1], kb[3]));  // code + 72
                acc[2 * q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, pq, acc[2 * q], 0, 0, 0);
                acc[2 * q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bias_lo, pq, acc[2 * q], 0, 0, 0);
                acc[2 * q + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, pq, acc[2 * q + 1], 0, 0, 0);
                acc[2 * q + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bias_hi, pq, acc[2 * q + 1], 0, 0, 0);
            }
        };

        auto tile_loop = [&](auto qn) {
            for (int tile = t0; tile < tile_end; tile += ST * step) {
#pragma unroll
                for (int u = 0; u < ST; ++u) {
                    const int t = tile + u * step;
                    if (t >= tile_end) break;
                    // the oldest pair in flight is this one
                    wait_loads<kLoadsPerPair * (ST - 1)>();
                    I4Frags<D> fa, fb;
                    fa.flags = flag_s[u][0];
                    fa.fword = fword_s[u][0];
                    fb.flags = flag_s[u][1];
                    fb.fword = fword_s[u][1];
                    const int capa = cap_s[u][0], capb = cap_s[u][1];
                    const int nva = max(0, min(capa, ctx - t * kTile));
                    const int nvb = max(0, min(capb, ctx - (t + 1) * kTile));
                    const bool live = capa > 0 || capb > 0;
                    float pr[8];
                    uint32_t vsw = 0u;
                    if (nt_item && (t == U - 1 || t + 1 == U - 1)) {
                        patch_new_token(stg[u][wave], t == U - 1 ? 0 : 1);
                        // nt's clamp flag bit in its tile's flag word
                        if (t == U - 1) fa.flags = (fa.flags & ~nt_bit) | nt_val;
                        else fb.flags = (fb.flags & ~nt_bit) | nt_val;
                    }
                    if (live) {
                        fetch_k(stg[u][wave], 0, fa);
                        fetch_k(stg[u][wave], 1, fb);
                        // raw V scale bits of the pair: lanes 0-31 tile a, 32-63 tile b (read
                        // ahead of the scores, which hide its latency)
                        vsw = (lane & 31) < 8 * NG ? stg[u][wave].sc[lane >> 5][32 + (lane & 31)] : 0u;
                        scores(qn, fa, fb, nva, nvb, t, pr);
                        fetch_v(stg[u][wave], 0, fa);
                        fetch_v(stg[u][wave], 1, fb);
                    }
                    // the stage is read: reload it with the pair ST steps ahead
                    wait_lds_reads();
                    issue(t + ST * step, u, next);
                    next = lookup(t + (ST + 1) * step);
                    if (live) pv(fa, fb, nva, nvb, pr, vsw);
                }
            }
        };
        if (qnorm) tile_loop(BoolTag<true>{});
        else tile_loop(BoolTag<false>{});
        // every load has landed before the ring is reused (the wave results below share
        // its memory) or the wave ends
        wait_loads<0>();
        // nt into the pool (and its flag into the pool's flag word), after the item's tiles:
        // nothing in this launch reads it back
        if (nt_item && wave == 0 && lane < kAppendLanes && nt_phys >= 0 && (uint32_t)nt_phys < p.num_blocks) {
            const uint32_t slot = nt_pos % (uint32_t)P;
            const size_t bh = (size_t)nt_phys * p.hkv + hk;
            const int ch = lane >> 1;
            if (!(lane & 1)) {
                *reinterpret_cast<uint4*>(const_cast<uint8_t*>(p.k) + (bh * P + slot) * (D / 2) + 16 * ch) = nt.k[ch];
                const_cast<uint16_t*>(p.ks)[int4_ks_index(bh, NG, P, slot, ch)] = nt.ks[ch];
                if (ch == 0 && p.kf) {
                    apply_flag({const_cast<uint32_t*>(p.kf) + bh * (P / kTile) + slot / kTile, 1u << (slot % kTile),
                                nt.flag != 0u});
                }
            } else {
                uint8_t* vt = const_cast<uint8_t*>(p.v) + bh * ((size_t)P * D / 2) + (size_t)(slot / kTile) * (8 * D);
                const uint8_t* vb = reinterpret_cast<const uint8_t*>(nt.vb) + 16 * ch;
#pragma unroll
                for (int nn = 0; nn < 16; ++nn) vt[int4_v_tile_byte(slot, ch, nn, D)] = vb[nn];
                const_cast<uint16_t*>(p.vs)[(bh * P + slot) * NG + ch] = nt.vs[ch];
            }
        }
        // the next item's q rows load while this one's states are merged
        if (item0 + tile_end < ws.hi) {
            const int npos = item0 + tile_end;
            const bool next_seq = npos >= seq0 + U * ips;
            const int nb = next_seq ? b + 1 : b;
            const int nU = next_seq ? item_tiles(p, nb) : U;
            load_q(nb, (npos - (next_seq ? seq0 + U * ips : seq0)) / nU);
        }
        __syncthreads();

        // ---- wave result: column 4q + h holds head h for the d-tiles 2q, 2q + 1 of V scale
        // group q; lane (g, n) has d = 16j + 4g + r ----
        l_run = add_rows(l_run);
        if (head_col) {
#pragma unroll
            for (int j = 0; j < NDT; ++j) {
                if ((n >> 2) == j / 2) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) comb[wave][n & 3][2 + 16 * j + 4 * g + r] = acc[j][r];
                }
            }
        }
        if (n < GW && g == 0) {
            // a wave that scored no token: exp2 of its state's max is 0 in the merge
            comb[wave][n][0] = first ? -1e30f : m_run;
            comb[wave][n][1] = l_run;
        }
        __syncthreads();
        finish_segment<D, GW>(p, comb, b, hq0, U, tile_begin, tile_end, pos == ws.lo ? 0 : 1);
        __syncthreads();  // the wave states are read before the next item's loads refill the ring
        pos = item0 + tile_end;
    }
}

#ifndef VSPEC_I4_STAGES
#define VSPEC_I4_STAGES 2
#endif

template <int D, int GW, bool USED>
void launch_used(const DecodeParams& p, dim3 grid, hipStream_t s) {
    constexpr int ST = VSPEC_I4_STAGES;
    if (p.read_flags) {
        if (p.block_tokens == 16)
            hipLaunchKernelGGL((decode_mfma_i4<D, GW, 16, ST, true, USED>), grid, dim3(256), 0, s, p);
        else
            hipLaunchKernelGGL((decode_mfma_i4<D, GW, 0, ST, true, USED>), grid, dim3(256), 0, s, p);
    } else {
        if (p.block_tokens == 16)
            hipLaunchKernelGGL((decode_mfma_i4<D, GW, 16, ST, false, USED>), grid, dim3(256), 0, s, p);
        else
            hipLaunchKernelGGL((decode_mfma_i4<D, GW, 0, ST, false, USED>), grid, dim3(256), 0, s, p);
    }
}

template <int D, int GW>
void launch(const DecodeParams& p, dim3 grid, hipStream_t s) {
    if (p.block_used) launch_used<D, GW, true>(p, grid, s);
    else launch_used<D, GW, false>(p, grid, s);
    // items split over several workgroups (same split: equal shares)
    if (p.merge) {
        const dim3 merge_grid(p.batch * p.hkv * p.gsplit);
        hipLaunchKernelGGL((decode_merge_split<D, GW, kSplitAlways>), merge_grid, dim3(kWaves * 64), 0, s, p);
    }
}

template <int D>
int launch_gw(uint32_t gw, const DecodeParams& p, dim3 grid, hipStream_t s) {
    switch (gw) {
        case 1: launch<D, 1>(p, grid, s); return 1;
        case 2: launch<D, 2>(p, grid, s); return 1;
        case 3: launch<D, 3>(p, grid, s); return 1;
        case 4: launch<D, 4>(p, grid, s); return 1;
        default: return 0;
    }
}

}  // namespace

int launch_decode_mfma_int4(const DecodeParams& p, uint32_t head_dim, uint32_t gw, dim3 grid,
                            hipStream_t stream) {
    if (head_dim == 64) return launch_gw<64>(gw, p, grid, stream);
    if (head_dim == 128) return launch_gw<128>(gw, p, grid, stream);
    return 0;
}

}  // namespace vkv
