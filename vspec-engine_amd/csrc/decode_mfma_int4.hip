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
//     d), rounded once to fp16.  The V pool is stored in 16-token tiles whose lane
//     chunks are half of these A operands.
//
// A nibble t (two's complement code c = (t ^ 8) - 8) becomes an exact fp16 through a
// magic exponent, two codes per 32-bit operation (codes_to_f16).
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

// Four fp16 pairs from one code dword: pair k = (nibble k, nibble k + 4).  A nibble t
// sits in an fp16 mantissa under a magic exponent (1024 + u for bits 0..3, 64 + u for
// bits 4..7, u = t ^ 8 = code + 8), so one shift, four three-input bit operations and
// four packed subtractions convert eight codes exactly.
__device__ __forceinline__ void codes_to_f16(uint32_t w, uint32_t out[4]) {
    const uint32_t w8 = w >> 8;
    const uint32_t p0 = ((w ^ 0x00080008u) & 0x000F000Fu) | 0x64006400u;   // 1024 + u
    const uint32_t p1 = ((w ^ 0x00800080u) & 0x00F000F0u) | 0x54005400u;   // 64 + u
    const uint32_t p2 = ((w8 ^ 0x00080008u) & 0x000F000Fu) | 0x64006400u;
    const uint32_t p3 = ((w8 ^ 0x00800080u) & 0x00F000F0u) | 0x54005400u;
    const h2_t b0 = {(_Float16)1032.0f, (_Float16)1032.0f};
    const h2_t b1 = {(_Float16)72.0f, (_Float16)72.0f};
    out[0] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, p0) - b0);
    out[1] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, p1) - b1);
    out[2] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, p2) - b0);
    out[3] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, p3) - b1);
}

template <int D>
struct I4Frags {
    static constexpr int NQ = D / 32;
    uint32_t k[NQ];       // token n: canonical code dwords g*NQ .. g*NQ+NQ-1
    uint32_t v[NQ];       // V tile lane chunk (g, n)
    uint32_t ks_own;      // K scale of (token n, this lane's group), low 16 bits
    uint2 ks_col;         // K scales of tokens 4g..4g+3 for column group (n/4) % G
    uint32_t vs[2 * NQ];  // V scales of tokens 4g..4g+3, token-major (G per token)
    uint32_t flags;       // clamp flags of the tile's 16 keys (the same in every lane)
    uint32_t fword;       // index of that flag word (wave-uniform)
};

// fp16 number i of a packed array, as the f16 operand of a mixed-precision FMA
__device__ __forceinline__ _Float16 half_at(const uint32_t* w, int i) {
    return __builtin_bit_cast(h2_t, w[i >> 1])[i & 1];
}

#ifndef VSPEC_I4_MIN_WG_PER_CU
#define VSPEC_I4_MIN_WG_PER_CU 2
#endif

// FL: the tile loop takes the pool's clamp flags (and screens only what they cannot say);
// without FL it screens every tile, a lighter loop for short per-workgroup shares.
// USED: per-block used counts cap each tile (block_used).
template <int D, int GW, int PB, int NB, bool FL, bool USED>
__global__ __launch_bounds__(256, VSPEC_I4_MIN_WG_PER_CU) void decode_mfma_i4(DecodeParams p) {
    constexpr int NQ = D / 32;   // code dwords per lane = QK MFMAs per tile = groups
    constexpr int NG = D / 32;
    constexpr int NDT = D / 16;  // PV d-tiles
    __shared__ float qs[GW][D];
    __shared__ uint4 qb_lds[NQ][2][64];  // QK B operands (hi, lo) per lane
    __shared__ float comb[kWaves][GW][D + 2];
    __shared__ float patch_val[kWaves][kTile][4];
    __shared__ int patch_flag[kWaves][kTile];
    __shared__ SplitShared split_sh;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4;
    const int n = lane & 15;

    const int ips = (int)(p.hkv * p.gsplit);  // work items per sequence
    const WorkSplit ws = work_split<false>(p, ips, split_sh);
    FlagOp pending = {nullptr, 0u, false};
    __shared__ uint32_t pend_lds[3];  // the fused append's first clamp flag: {word, bit, value}
    if (FL && threadIdx.x == 0) pend_lds[0] = 0xffffffffu;
    if (p.k_new && ws.lo < ws.hi)
        fused_append<VSPEC_KV_INT4, D>(p, ws, cursor_at(p, ws), ips, pending, FL ? pend_lds : nullptr);
    uint32_t pend_word = 0xffffffffu, pend_bit = 0u, pend_val = 0u;
    if (FL) {
        __syncthreads();
        pend_word = __builtin_amdgcn_readfirstlane(pend_lds[0]);
        pend_bit = __builtin_amdgcn_readfirstlane(pend_lds[1]);
        pend_val = __builtin_amdgcn_readfirstlane(pend_lds[2]);
    }
    // the append's first flag update, after the barrier: it overlaps the first tile loads
    // instead of holding up the barrier (a tile read of its word takes the patched value)
    apply_flag(pending);
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

        // ---- q' = clip(q) * scale * log2(e): wave w prepares head w ----
        if (wave < GW) {
            const float* qrow = p.q + ((size_t)b * p.hq + hq0 + wave) * D;
            constexpr int E = D / 64;
            float x[E];
            float s = 0.f;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                x[e] = qrow[lane * E + e];
                s += x[e];
            }
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) s += __shfl_xor(s, o);
            const float mean = s * (1.0f / D);
            float v = 0.f;
#pragma unroll
            for (int e = 0; e < E; ++e) v = fmaf(x[e] - mean, x[e] - mean, v);
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o);
            const float th = fminf(fmaxf(1e-6f, p.alpha * sqrtf(v * (1.0f / D))), p.input_clip);
#pragma unroll
            for (int e = 0; e < E; ++e) qs[wave][lane * E + e] = fminf(fmaxf(x[e], -th), th) * p.qscale;
        }
        __syncthreads();

        // ---- QK B operands: k-slots 8g..8g+7 of MFMA m carry code dword dw = g*NQ + m in
        // the order e = 0,4,1,5,2,6,3,7; column n takes group n/4 of head n%4 ----
        if (wave == 0) {
            const int hh = n & 3;
#pragma unroll
            for (int m = 0; m < NQ; ++m) {
                const int dw = g * NQ + m;
                const bool on = (dw >> 2) == (n >> 2) && hh < GW;
                h8_t hi8, lo8;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int e = (j >> 1) + 4 * (j & 1);
                    const float qv = on ? qs[hh < GW ? hh : 0][8 * dw + e] : 0.f;
                    const _Float16 hi = (_Float16)qv;
                    hi8[j] = hi;
                    lo8[j] = (_Float16)(qv - (float)hi);
                }
                qb_lds[m][0][lane] = __builtin_bit_cast(uint4, hi8);
                qb_lds[m][1][lane] = __builtin_bit_cast(uint4, lo8);
            }
        }
        __syncthreads();

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
        auto valid_mask = [](int nvalid) -> uint32_t { return nvalid >= kTile ? 0xffffu : (1u << nvalid) - 1u; };

        // Loads are issued unconditionally (a tile past the range or behind an invalid
        // table entry reads block 0 and holds no valid token): with no branches around
        // them the compiler counts outstanding loads exactly and waits only for the tile
        // it needs.  The tile index is wave-uniform, so the table read stays on the scalar
        // unit.  Returns how many of the tile's tokens its block holds (16, or
        // block_used's cap; 0: none).
        auto load = [&](int tile, I4Frags<D>& f) -> int {
            tile = __builtin_amdgcn_readfirstlane(tile);
            const bool in_range = tile < tile_end;
            const int entry_idx = (in_range ? tile : tile_end - 1) / tiles_per_block;
            const int entry = table[entry_idx];
            const bool ok = in_range && entry >= 0 && (uint32_t)entry < p.num_blocks;
            const int phys = ok ? entry : 0;
            const size_t bh = (size_t)phys * p.hkv + hk;
            const int slot0 = (tile % tiles_per_block) * kTile;
            const uint8_t* kr = p.k + (bh * P + slot0 + n) * (D / 2) + 4 * g * NQ;
            const uint8_t* vc = p.v + bh * ((size_t)P * D / 2) + (size_t)(slot0 / kTile) * (8 * D) + (16 * g + n) * (D / 8);
            if constexpr (NQ == 4) {
                const uint4 a = load_stream4(kr);
                const uint4 c = load_stream4(vc);
                f.k[0] = a.x; f.k[1] = a.y; f.k[2] = a.z; f.k[3] = a.w;
                f.v[0] = c.x; f.v[1] = c.y; f.v[2] = c.z; f.v[3] = c.w;
            } else {
                const uint2 a = load_stream2(kr);
                const uint2 c = load_stream2(vc);
                f.k[0] = a.x; f.k[1] = a.y;
                f.v[0] = c.x; f.v[1] = c.y;
            }
            f.ks_own = load_stream_u16(p.ks + (bh * NG + own_group) * P + slot0 + n);
            f.ks_col = load_stream2(p.ks + (bh * NG + col_group) * P + slot0 + 4 * g);
            // a vector load, waited for with the tile's other loads (a scalar load would be
            // waited for by every LDS wait of the loop: the two share a counter)
            f.fword = (uint32_t)(bh * (P / kTile) + slot0 / kTile);
            f.flags = flags_on ? __hip_atomic_load(p.kf + f.fword, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) : 0u;
            const uint4* vs = reinterpret_cast<const uint4*>(p.vs + (bh * P + slot0 + 4 * g) * NG);
#pragma unroll
            for (int i = 0; i < NQ / 2; ++i) {
                const uint4 w = load_stream4(vs + i);
                f.vs[4 * i] = w.x; f.vs[4 * i + 1] = w.y; f.vs[4 * i + 2] = w.z; f.vs[4 * i + 3] = w.w;
            }
            if constexpr (USED) return ok ? used_cap(used_row[entry_idx], slot0) : 0;
            return ok ? kTile : 0;
        };

        // score clip per lane: columns that hold no head clip to -inf (3-bit mode: +-24*log2e)
        const float clip_hi = n < GW ? p.logit_clip : -INFINITY;
        const float clip_lo = n < GW ? -p.logit_clip : -INFINITY;

        f4_t acc[NDT];
#pragma unroll
        for (int j = 0; j < NDT; ++j) acc[j] = f4_t{0.f, 0.f, 0.f, 0.f};
        // running max starts finite so exp2(s - m_run) is 0, never NaN, in the columns
        // that hold no head (their scores stay -inf)
        float m_run = -1e30f;
        float l_run = 0.f;

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

        // Scores of a tile on the matrix cores: lane (g, n) gets tokens 4g..4g+3 for head
        // n%4 (hi and lo products accumulate in separate chains).
        auto qk = [&](const I4Frags<D>& f) -> f4_t {
            f4_t sh = {0.f, 0.f, 0.f, 0.f}, sl = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int m = 0; m < NQ; ++m) {
                uint32_t pr4[4];
                codes_to_f16(f.k[m], pr4);
                const h8_t a = __builtin_bit_cast(h8_t, make_uint4(pr4[0], pr4[1], pr4[2], pr4[3]));
                sh = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(h8_t, qb_lds[m][0][lane]), sh, 0, 0, 0);
                sl = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(h8_t, qb_lds[m][1][lane]), sl, 0, 0, 0);
            }
            const uint32_t kc[2] = {f.ks_col.x, f.ks_col.y};
            f4_t sc;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float ks = (float)half_at(kc, r);
                float v = __builtin_fmaf(sh[r], ks, sl[r] * ks);
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
            if (n < GW) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int t = 4 * g + r;
                    if (patch_flag[wave][t]) sc[r] = patch_val[wave][t][n];
                }
            }
        };

        // Slots past the context (or a whole missing tile) may hold any scale bits (NaN):
        // their V scales become 0 so that p' = p * scale = 0.
        auto clear_masked_scales = [&](I4Frags<D>& f, const int nvalid) {
            if (nvalid < kTile) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (4 * g + r >= nvalid) {
#pragma unroll
                        for (int i = 0; i < NG / 2; ++i) f.vs[r * (NG / 2) + i] = 0u;
                    }
                }
            }
        };

        // Two tiles per step: k-slot 8g + i of the PV MFMA is token 4g + i of tile A (i < 4)
        // or token 4g + i - 4 of tile B.
        auto process = [&](I4Frags<D>& fa, I4Frags<D>& fb, const int capa, const int capb, const int tile_a) {
            const int nva = max(0, min(capa, ctx - tile_a * kTile));
            const int nvb = max(0, min(capb, ctx - (tile_a + 1) * kTile));
            // clamp flags: from the pool, or from the screen (both tiles in one basic block:
            // their chains interleave)
            // the tile this launch appended into: its word with the appended key's flag
            // patched in, or (another appended item of this range) the screen
            const bool scr_a = !flags_on || (fused && tile_a == U - 1 && fa.fword != pend_word);
            const bool scr_b = !flags_on || (fused && tile_a + 1 == U - 1 && fb.fword != pend_word);
            auto word_of = [&](const I4Frags<D>& f) -> uint32_t {
                const uint32_t w = __builtin_amdgcn_readfirstlane(f.flags);
                return f.fword == pend_word ? (w & ~pend_bit) | pend_val : w;
            };
            uint32_t fla, flb;
            f4_t sa, sb;
            if (scr_a || scr_b) {
                const Screen sna = screen(fa, nva);
                const Screen snb = screen(fb, nvb);
                sa = qk(fa);
                sb = qk(fb);
                fla = scr_a ? tokens(__builtin_amdgcn_ballot_w64(sna.flag)) : word_of(fa) & valid_mask(nva);
                flb = scr_b ? tokens(__builtin_amdgcn_ballot_w64(snb.flag)) : word_of(fb) & valid_mask(nvb);
            } else {
                sa = qk(fa);
                sb = qk(fb);
                fla = word_of(fa) & valid_mask(nva);
                flb = word_of(fb) & valid_mask(nvb);
            }
            if ((fla | flb) != 0u) {
                if (fla != 0u) exact(fa, fla, sa);
                if (flb != 0u) exact(fb, flb, sb);
            }

            // ---- online softmax for head n over this lane's 8 tokens.  The running max
            // moves only when a score exceeds it by more than 8 (p stays <= 2^8), so the
            // cross-lane max is taken only then. ----
            float s[8];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                s[r] = __builtin_amdgcn_fmed3f(sa[r], clip_lo, clip_hi);
                s[4 + r] = __builtin_amdgcn_fmed3f(sb[r], clip_lo, clip_hi);
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
            const bool over = smax > m_run + 8.0f;
            if (__builtin_amdgcn_ballot_w64(over) != 0) {
                const float mt = max_rows(smax);
                const bool need = mt > m_run + 8.0f;
                const float fct = need ? __builtin_amdgcn_exp2f(m_run - mt) : 1.0f;
                m_run = need ? mt : m_run;
                l_run *= fct;
#pragma unroll
                for (int j = 0; j < NDT; ++j) acc[j] *= fct;
            }
            // v_exp_f32 of -inf is +0: masked tokens and unused columns drop out
            float pr[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                pr[i] = __builtin_amdgcn_exp2f(s[i] - m_run);
                l_run += pr[i];
            }
            clear_masked_scales(fa, nva);
            clear_masked_scales(fb, nvb);

            // ---- O^T += V^T P'^T over 32 tokens, one V scale group (two d-tiles) at a time ----
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
                // P' = p * scale rounded once to fp16 (v_fma_mix, relative error <= 2^-12):
                // the output error stays below 2.4e-4 * max|v|
                h8_t pq;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const _Float16 sv = i < 4 ? half_at(fa.vs, (i & 3) * NG + q) : half_at(fb.vs, (i & 3) * NG + q);
                    pq[i] = (_Float16)__builtin_fmaf(pr[i], (float)sv, 0.0f);
                }
                uint32_t ka[4], kb[4];
                codes_to_f16(fa.v[q], ka);
                codes_to_f16(fb.v[q], kb);
                const h8_t a0 = __builtin_bit_cast(h8_t, make_uint4(ka[0], ka[2], kb[0], kb[2]));
                const h8_t a1 = __builtin_bit_cast(h8_t, make_uint4(ka[1], ka[3], kb[1], kb[3]));
                acc[2 * q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, pq, acc[2 * q], 0, 0, 0);
                acc[2 * q + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, pq, acc[2 * q + 1], 0, 0, 0);
            }
        };

        // Pairs of consecutive tiles; NB pairs in flight per wave.  Pair i (from the
        // partition start) is tiles tile_begin + 2i, +1; wave w takes i = w, w + kWaves, ...
        I4Frags<D> fa[NB], fb[NB];
        int oka[NB], okb[NB];
        const int step = 2 * kWaves;
        const int t0 = tile_begin + 2 * wave;
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int t = t0 + u * step;
            oka[u] = load(t, fa[u]);
            okb[u] = load(t + 1, fb[u]);
        }
        for (int tile = t0; tile < tile_end; tile += NB * step) {
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                const int t = tile + u * step;
                if (t >= tile_end) break;
                if (oka[u] > 0 || okb[u] > 0) process(fa[u], fb[u], oka[u], okb[u], t);
                const int nt = t + NB * step;
                oka[u] = load(nt, fa[u]);
                okb[u] = load(nt + 1, fb[u]);
            }
        }

        // ---- wave result: column n < GW holds head n; lane (g, n) has d = 16j + 4g + r ----
        l_run = add_rows(l_run);
        if (n < GW) {
#pragma unroll
            for (int j = 0; j < NDT; ++j) {
#pragma unroll
                for (int r = 0; r < 4; ++r) comb[wave][n][2 + 16 * j + 4 * g + r] = acc[j][r];
            }
            if (g == 0) {
                comb[wave][n][0] = m_run;
                comb[wave][n][1] = l_run;
            }
        }
        __syncthreads();
        finish_segment<D, GW>(p, comb, b, hq0, U, tile_begin, tile_end, pos == ws.lo ? 0 : 1);
        pos = item0 + tile_end;
    }
}

#ifndef VSPEC_I4_PAIRS_IN_FLIGHT
#define VSPEC_I4_PAIRS_IN_FLIGHT 1
#endif

template <int D, int GW, bool USED>
void launch_used(const DecodeParams& p, dim3 grid, hipStream_t s) {
    constexpr int NB = VSPEC_I4_PAIRS_IN_FLIGHT;
    if (p.read_flags) {
        if (p.block_tokens == 16)
            hipLaunchKernelGGL((decode_mfma_i4<D, GW, 16, NB, true, USED>), grid, dim3(256), 0, s, p);
        else
            hipLaunchKernelGGL((decode_mfma_i4<D, GW, 0, NB, true, USED>), grid, dim3(256), 0, s, p);
    } else {
        if (p.block_tokens == 16)
            hipLaunchKernelGGL((decode_mfma_i4<D, GW, 16, NB, false, USED>), grid, dim3(256), 0, s, p);
        else
            hipLaunchKernelGGL((decode_mfma_i4<D, GW, 0, NB, false, USED>), grid, dim3(256), 0, s, p);
    }
}

template <int D, int GW>
void launch(const DecodeParams& p, dim3 grid, hipStream_t s) {
    if (p.block_used) launch_used<D, GW, true>(p, grid, s);
    else launch_used<D, GW, false>(p, grid, s);
    // items split over several workgroups (same split: equal shares)
    if (p.merge) {
        const dim3 merge_grid(p.batch * p.hkv * p.gsplit);
        hipLaunchKernelGGL((decode_merge_split<D, GW, false>), merge_grid, dim3(kWaves * 64), 0, s, p);
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
