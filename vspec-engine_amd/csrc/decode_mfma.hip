// decode_mfma.hip -- single-query GQA decode attention over f16 paged KV, with the
// two contractions on the matrix cores (gfx950 MFMA) and the reference numerics
// (per-key std clamp, attention_ref.c:50-62) on the vector ALUs.
//
// Per wave and 16-token tile of one kv head:
//   S^T[16 tok][16 col] = K[16 tok][D] x Q'^T      v_mfma_f32_16x16x32_f16, A = K rows as
//                                                   loaded, B = q' split in fp16 hi + lo
//                                                   (separate accumulator chains)
//   O^T[d][16 col]     += V^T[d][16 tok] x P^T     v_mfma_f32_16x16x16f16, A = V^T rows
//                                                   (V is stored in groups of 4 tokens,
//                                                   f16_v_index), B = p
//                                                   hi + lo taken straight from the S^T
//                                                   accumulator registers
// Columns 0..GW-1 are the GQA query heads that share the tile; the rest stay zero.
// q' of a head whose max |q'| lies outside [2^-4, 2^15) enters the MFMAs shifted by a power
// of two (qnorm_shift), so that neither fp16 part overflows or loses its relative precision
// in the subnormal range; the lane then keeps its scores in the shifted unit and takes the
// factor back inside the exp2 argument.  p is at most 2^8 (lazy running max), so the P^T
// operands stay in range whatever the data.
//
// The std clamp is screened per key from v_dot2 sums (sum x, sum x^2) and a packed
// max|x|; keys it may affect (about 0.1% for N(0,1) data) get their scores recomputed
// exactly in fp32 from the clipped row, replacing the MFMA value.
#include "kv_common.h"

namespace vkv {
namespace {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ h8_t as_h8(uint4 w) { return __builtin_bit_cast(h8_t, w); }
__device__ __forceinline__ h2_t as_h2(uint32_t w) { return __builtin_bit_cast(h2_t, w); }

template <int D>
struct Frags {
    uint4 k[D / 32];  // K row of token n, d = 32i + 8g .. +7
    uint2 v[D / 16];  // V^T row d = 16j + n, slots 4g .. 4g+3 of the tile
};

// PB: block_tokens known at compile time (16), or 0 for any multiple of 16;
// NB: tiles in flight per wave; USED: per-block used counts cap each tile (block_used)
//
// Schedule: the workgroup takes the tile range [lo, hi) of the work split (it may start
// and end inside work items and span several); wave w streams the range's tiles
// lo + w, lo + w + 4, ... through its ring of NB tile buffers without stopping at work
// item boundaries: the ring's loads run NB tiles ahead on their own cursor, and where
// the processed tiles enter a new work item the wave hands its softmax state for the
// old one to an LDS merge slot, resets it and prepares the new item's q operands from
// q rows staged in LDS up front.  The last of the waves to hand in an item's state
// merges them all; no barrier stops the ring.
template <int D, int GW, int PB, int NB, bool USED, int NW>
__global__ __launch_bounds__(NW * 64, 8 / NW) void decode_mfma_f16(DecodeParams p) {
    constexpr int NQK = D / 32;   // QK MFMAs per tile (each on 32 d)
    constexpr int NDT = D / 16;   // PV d-tiles
    constexpr int kQStage = 4;    // item segments whose q rows are staged up front
    constexpr int kSlots = 2;     // item segments being merged at once
    __shared__ float qraw[kQStage][GW][D];
    __shared__ float qs[NW][GW][D];  // per wave: q' of its current item
    // per wave: QK B operands (hi, lo for each 32-wide d chunk), read back every tile
    __shared__ float comb[kSlots][NW][GW][D + 2];
    __shared__ float patch_val[NW][kTile][4];
    __shared__ int patch_flag[NW][kTile];
    __shared__ int slot_cnt[kSlots];
    __shared__ int slot_seg[kSlots];
    // fused decode step: the new token's K and V rows (f16 bits, two per word) of segment s
    // in row s < kQStage (staged up front), of a later segment in row kQStage + wave (staged
    // by the wave itself); the wave that processes the tile holding the token patches them
    // into its fragments and stores them to the pool, so no wave waits for those stores
    __shared__ uint32_t newtok[kQStage + NW][2][D / 2];
    __shared__ SplitSharedN<NW> split_sh;

    const int lane = threadIdx.x & 63;
    // wave index as a scalar: tile loop control and block-table reads stay on the
    // scalar unit (s_load), so they never wait behind the vector K/V loads
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4;   // row group
    const int n = lane & 15;   // column / token within the tile

    const int ips = (int)(p.hkv * p.gsplit);  // work items per sequence
    const WorkSplit ws = work_split<kSplitRagged, NW>(p, ips, split_sh);
    if (ws.lo >= ws.hi) return;
    const ItemCursor first = cursor_at(p, ws);


    // ---- q' = clip(q) * scale * log2(e) of work item c (segment s) for this wave, and
    // the B operands of the QK MFMAs: column n < GW holds head n, split hi + lo ----
    // score MFMA B operands (q' hi and lo) of the wave's current item, in registers
    h8_t qreg[NQK][2];
    // Head n's operands carry q' * 2^e_n (qnorm_shift), so the MFMAs return scores times
    // 2^e_n.  The lane keeps them in that unit (raw) and so do its running max (m_raw), lazy
    // threshold and clip bounds; qfac = 2^-e_n turns a raw difference into log2 units inside
    // the exp2 argument, fma(s, qfac, -mf) with mf = m_raw * qfac, which costs no more than
    // the subtraction it replaces and is exact in the power of two.
    float qfac = 1.0f, qinv = 1.0f, thr_raw = 8.0f, clo_raw = -INFINITY, chi_raw = -INFINITY;
    // score clip per lane: columns that hold no head clip to -inf (3-bit mode: +-24*log2e)
    const float clip_hi = n < GW ? p.logit_clip : -INFINITY;
    const float clip_lo = n < GW ? -p.logit_clip : -INFINITY;
    // The new token rows of item c into newtok[row] (one wave; lane l takes elements 2l,
    // 2l + 1 of K and of V).  The bits are those the pool append writes (f16 source bits, or
    // the round-to-nearest-even conversion of f32 ones).  load() issues the loads, store()
    // writes LDS once they have landed.
    struct NewRow {
        uint32_t kw, vw;
        float2 kf, vf;
    };
    auto newrow_load = [&](const ItemCursor& c) -> NewRow {
        NewRow r = {0u, 0u, make_float2(0.f, 0.f), make_float2(0.f, 0.f)};
        const size_t el = ((size_t)c.b * p.hkv + c.y / (int)p.gsplit) * D + 2 * lane;
        if (p.append_src == VSPEC_KV_F32) {
            r.kf = *reinterpret_cast<const float2*>(p.k_new + el * 4);
            r.vf = *reinterpret_cast<const float2*>(p.v_new + el * 4);
        } else {
            r.kw = *reinterpret_cast<const uint32_t*>(p.k_new + el * 2);
            r.vw = *reinterpret_cast<const uint32_t*>(p.v_new + el * 2);
        }
        return r;
    };
    auto newrow_store = [&](const NewRow& r, const int row) {
        uint32_t kw = r.kw, vw = r.vw;
        if (p.append_src == VSPEC_KV_F32) {
            kw = float_to_half_bits(r.kf.x) | (float_to_half_bits(r.kf.y) << 16);
            vw = float_to_half_bits(r.vf.x) | (float_to_half_bits(r.vf.y) << 16);
        }
        newtok[row][0][lane] = kw;
        newtok[row][1][lane] = vw;
    };

    auto qprep = [&](const int s, const ItemCursor& c) {
        constexpr int E = D / 64;
        if (s >= kQStage) {
            // rows past the staged ones go through this wave's qs first, so that only this
            // rare branch waits for a global load (the other path keeps the ring's loads
            // in flight)
#pragma unroll
            for (int h = 0; h < GW; ++h) {
                const float* qrow = p.q + ((size_t)c.b * p.hq + (size_t)c.y * GW + h) * D;
#pragma unroll
                for (int e = 0; e < E; ++e) qs[wave][h][lane * E + e] = qrow[lane * E + e];
            }
            if (p.k_new) newrow_store(newrow_load(c), kQStage + wave);
        }
        float (*src)[D] = s < kQStage ? qraw[s] : qs[wave];
        int eh[GW];
#pragma unroll
        for (int h = 0; h < GW; ++h) {
            float x[E];
#pragma unroll
            for (int e = 0; e < E; ++e) x[e] = src[h][lane * E + e];
            float sm = 0.f;
#pragma unroll
            for (int e = 0; e < E; ++e) sm += x[e];
            const float mean = wave_sum(sm) * (1.0f / D);
            float v = 0.f;
#pragma unroll
            for (int e = 0; e < E; ++e) v = fmaf(x[e] - mean, x[e] - mean, v);
            v = wave_sum(v);
            const float th = fminf(fmaxf(1e-6f, p.alpha * sqrtf(v * (1.0f / D))), p.input_clip);
            float am = 0.f;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const float y = fminf(fmaxf(x[e], -th), th) * p.qscale;
                qs[wave][h][lane * E + e] = y;
                am = fmaxf(am, fabsf(y));
            }
            eh[h] = __builtin_amdgcn_readfirstlane(qnorm_shift(wave_max(am)));
        }
        int en = 0;
#pragma unroll
        for (int h = 0; h < GW; ++h) en = n == h ? eh[h] : en;
        qfac = pow2i(-en);
        qinv = pow2i(en);
        thr_raw = 8.0f * qinv;
        clo_raw = clip_lo * qinv;
        chi_raw = clip_hi * qinv;
        // columns without a head get zero operands (the LDS read stays unconditional)
        const int hn = n < GW ? n : 0;
        const float qin = n < GW ? qinv : 0.0f;
        // this wave's own LDS writes are read back below: a wave's LDS accesses complete
        // in program order
#pragma unroll
        for (int i = 0; i < NQK; ++i) {
            h8_t hi8, lo8;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float qv = qs[wave][hn][32 * i + 8 * g + j] * qin;
                const _Float16 hi = (_Float16)qv;
                hi8[j] = hi;
                lo8[j] = (_Float16)(qv - (float)hi);
            }
            qreg[i][0] = hi8;
            qreg[i][1] = lo8;
        }
    };

    const int P = PB ? PB : (int)p.block_tokens;
    const int tiles_per_block = P / kTile;
    const _Float16* kbase = reinterpret_cast<const _Float16*>(p.k);
    const _Float16* vbase = reinterpret_cast<const _Float16*>(p.v);
    const int ctx_cap = (int)(p.max_blocks * p.block_tokens);

    // Loads are issued unconditionally (a tile past the range or behind an invalid
    // table entry reads block 0 and holds no valid token): with no branches around them
    // the compiler counts outstanding loads exactly and waits only for the tile it needs.
    // `lc` is the work item of the tiles being loaded (it runs NB tiles ahead).  Returns
    // how many of the tile's tokens its block holds (16, or block_used's cap; 0: none).
    ItemCursor lc = first;
    auto load = [&](int t, Frags<D>& f) -> int {
        t = __builtin_amdgcn_readfirstlane(t);
        const bool in_range = t < ws.hi;
        if (in_range) {
            while (t >= lc.item0 + lc.U) cursor_next(p, ips, lc);
        }
        const int tile = in_range ? t - lc.item0 : 0;
        const size_t row = (size_t)lc.b * p.max_blocks + tile / tiles_per_block;
        const int entry = as_const(p.block_tables)[row];
        const bool ok = in_range && entry >= 0 && (uint32_t)entry < p.num_blocks;
        const size_t tidx = (size_t)(ok ? entry : 0) * p.hkv + lc.y / (int)p.gsplit;
        const int slot0 = (tile % tiles_per_block) * kTile;
        const uint4* kr = reinterpret_cast<const uint4*>(kbase + (tidx * P + slot0 + n) * D + 8 * g);
#pragma unroll
        for (int i = 0; i < NQK; ++i) f.k[i] = load_stream4(kr + 4 * i);
        // tokens slot0 + 4g .. + 3 of d = 16j + n: 8 bytes at f16_v_index (one 512-byte span per j)
        const _Float16* vt = vbase + f16_v_index(tidx, P, D, slot0 + 4 * g, n);
#pragma unroll
        for (int j = 0; j < NDT; ++j) f.v[j] = load_stream2(vt + 64 * j);
        if constexpr (USED) return ok ? used_cap(as_const(p.block_used)[row], slot0) : 0;
        return ok ? kTile : 0;
    };

    f4_t acc[NDT];
    // Running max: m_raw in the lane's raw score unit starts at -inf, so the first valid
    // score always moves it; mf = m_raw * qfac in log2 units starts finite, so that exp2 of
    // a -inf score minus it is 0, never NaN, in columns that hold no head or no token yet.
    float m_raw, mf;
    float l_run;  // sum of p for head n over this lane's tokens
    auto reset = [&]() {
#pragma unroll
        for (int j = 0; j < NDT; ++j) acc[j] = f4_t{0.f, 0.f, 0.f, 0.f};
        m_raw = -INFINITY;
        mf = -1e30f;
        l_run = 0.f;
    };
    const h2_t ones = {(_Float16)1.0f, (_Float16)1.0f};

    // Clamp screen of key n (this lane holds 8*NQK of its elements): mean and E[x^2]
    // from v_dot2 sums over the whole key, max|x| over this lane's part.  `flag` is set
    // in a lane whose part may reach the clamp threshold; key n is flagged when any of
    // its four lanes is (tokens() folds the wave's ballot).
    struct Screen {
        float mean;
        bool flag;
    };
    auto screen = [&](const Frags<D>& f, const int nvalid) -> Screen {
        float s1 = 0.f, s2 = 0.f;
        h2_t mx2 = {(_Float16)0.f, (_Float16)0.f};
#pragma unroll
        for (int i = 0; i < NQK; ++i) {
            const uint32_t w4[4] = {f.k[i].x, f.k[i].y, f.k[i].z, f.k[i].w};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const h2_t kv2 = as_h2(w4[c]);
                s1 = __builtin_amdgcn_fdot2(kv2, ones, s1, false);
                s2 = __builtin_amdgcn_fdot2(kv2, kv2, s2, false);
                mx2 = __builtin_elementwise_max(mx2, __builtin_elementwise_abs(kv2));
            }
        }
        const float mx = fmaxf((float)mx2[0], (float)mx2[1]);
        s1 = add_rows(s1);
        s2 = add_rows(s2);
        const float mean = s1 * (1.0f / D);
        const float ex2 = s2 * (1.0f / D);
        const float var1 = ex2 - mean * mean;
        const float th1 = fminf(fmaxf(1e-6f, p.alpha * __builtin_amdgcn_sqrtf(fmaxf(var1, 0.f))), p.input_clip);
        // a margin of 2^-10 covers the one-pass variance error and the 1-ulp square root;
        // ill-conditioned rows (variance tiny against the mean square) always take the
        // exact path
        return {mean, (n < nvalid) && (mx > th1 * (1.0f - 0.0009765625f) || var1 <= ex2 * 0.0009765625f)};
    };
    auto tokens = [](uint64_t m) -> uint32_t { return (uint32_t)((m | (m >> 16) | (m >> 32) | (m >> 48)) & 0xffffu); };

    // scores S^T = K Q'^T of a tile: lane (g, n) gets tokens 4g..4g+3 of head n
    auto qk = [&](const Frags<D>& f) -> f4_t {
        f4_t sh = {0.f, 0.f, 0.f, 0.f}, sl = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < NQK; ++i) {
            sh = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(f.k[i]), qreg[i][0], sh, 0, 0, 0);
            sl = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(f.k[i]), qreg[i][1], sl, 0, 0, 0);
        }
        return sh + sl;
    };

    // exact fp32 scores for the flagged keys of a tile (reference clamp, two-pass variance)
    auto exact = [&](const Frags<D>& f, const Screen& sn, const uint32_t flagged, f4_t& sc) {
        float v2 = 0.f;
#pragma unroll
        for (int i = 0; i < NQK; ++i) {
            const uint32_t w4[4] = {f.k[i].x, f.k[i].y, f.k[i].z, f.k[i].w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float x = half_bits_to_float((w4[e / 2] >> (16 * (e % 2))) & 0xffffu);
                v2 = fmaf(x - sn.mean, x - sn.mean, v2);
            }
        }
        v2 = add_rows(v2);
        const float th = fminf(fmaxf(1e-6f, p.alpha * sqrtf(v2 * (1.0f / D))), p.input_clip);
        float part[GW];
#pragma unroll
        for (int h = 0; h < GW; ++h) {
            float a = 0.f;
#pragma unroll
            for (int i = 0; i < NQK; ++i) {
                const uint32_t w4[4] = {f.k[i].x, f.k[i].y, f.k[i].z, f.k[i].w};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float x = half_bits_to_float((w4[e / 2] >> (16 * (e % 2))) & 0xffffu);
                    a = fmaf(qs[wave][h][32 * i + 8 * g + e], fminf(fmaxf(x, -th), th), a);
                }
            }
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
                if (patch_flag[wave][t]) sc[r] = patch_val[wave][t][n] * qinv;
            }
        }
    };

    // slots past the context (or a whole missing tile) may hold any bits (NaN): zero them
    auto clear_masked_v = [&](Frags<D>& f, const int nvalid) {
        if (nvalid < kTile) {
#pragma unroll
            for (int j = 0; j < NDT; ++j) {
                h4_t vv = __builtin_bit_cast(h4_t, f.v[j]);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (4 * g + r >= nvalid) vv[r] = (_Float16)0.f;
                }
                f.v[j] = __builtin_bit_cast(uint2, vv);
            }
        }
    };

    // one tile holding `cap` valid tokens (slots 0 .. cap-1 of its block; 0 for a tile
    // out of range or behind an invalid table entry, which contributes nothing)
    auto process = [&](Frags<D>& f, const int cap, const int tile, const int ctx) {
        const int nvalid = max(0, min(cap, ctx - tile * kTile));
        const Screen sn = screen(f, nvalid);
        f4_t sc = qk(f);
        const uint32_t flagged = tokens(__builtin_amdgcn_ballot_w64(sn.flag));
        if (flagged != 0u) exact(f, sn, flagged, sc);

        // ---- online softmax for head n over tokens 4g..4g+3.  The running max moves
        // only when a score exceeds it by more than 8 (p stays <= 2^8), so the
        // cross-lane max is taken only then. ----
        float s[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) s[r] = __builtin_amdgcn_fmed3f(sc[r], clo_raw, chi_raw);
        if (nvalid < kTile) {
#pragma unroll
            for (int r = 0; r < 4; ++r) s[r] = 4 * g + r < nvalid ? s[r] : -INFINITY;
            clear_masked_v(f, nvalid);
        }
        const float smax = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
        if (__builtin_amdgcn_ballot_w64(smax > m_raw + thr_raw) != 0) {
            const float mt = max_rows(smax);
            const bool need = mt > m_raw + thr_raw;
            const float fct = need ? __builtin_amdgcn_exp2f((m_raw - mt) * qfac) : 1.0f;
            m_raw = need ? mt : m_raw;
            mf = need ? mt * qfac : mf;
            l_run *= fct;
#pragma unroll
            for (int j = 0; j < NDT; ++j) acc[j] *= fct;
        }
        // v_exp_f32 of -inf is +0: masked tokens and unused columns drop out
        h4_t phi, plo;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], qfac, -mf));
            l_run += pv;
            const _Float16 hi = (_Float16)pv;
            phi[r] = hi;
            plo[r] = (_Float16)(pv - (float)hi);
        }

        // ---- O^T += V^T P^T ----
#pragma unroll
        for (int j = 0; j < NDT; ++j) {
            const h4_t a = __builtin_bit_cast(h4_t, f.v[j]);
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, phi, acc[j], 0, 0, 0);
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, plo, acc[j], 0, 0, 0);
        }
    };

    // Hand this wave's state for segment s (work item c) to merge slot s % kSlots; the
    // last of the NW waves to hand in merges their states.  A slot serves segment
    // s once segment s - kSlots is merged; waves hand in segments in order, so the wave
    // furthest behind never waits here and every wait ends.
    auto arrive = [&](const int s, const ItemCursor& c) {
        const int slot = s % kSlots;
        while (__hip_atomic_load(&slot_seg[slot], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != s)
            __builtin_amdgcn_s_sleep(1);
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        const float l = add_rows(l_run);
        if (n < GW) {
#pragma unroll
            for (int j = 0; j < NDT; ++j) {
#pragma unroll
                for (int r = 0; r < 4; ++r) comb[slot][wave][n][2 + 16 * j + 4 * g + r] = acc[j][r];
            }
            if (g == 0) {
                comb[slot][wave][n][0] = mf;
                comb[slot][wave][n][1] = l;
            }
        }
        // LDS-only fences: the merge order needs no wait for the ring's global loads
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        int before = 0;
        if (lane == 0) before = __hip_atomic_fetch_add(&slot_cnt[slot], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        before = __builtin_amdgcn_readfirstlane(before);
        if (before == NW - 1) {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
            const bool whole = c.item0 >= ws.lo && c.item0 + c.U <= ws.hi;
            merge_segment<D, GW, NW>(p, comb[slot], lane, (size_t)c.b * p.hq + (size_t)c.y * GW, whole, s == 0 ? 0 : 1);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            if (lane == 0) {
                slot_cnt[slot] = 0;
                __hip_atomic_store(&slot_seg[slot], s + kSlots, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
        }
    };

    // The staged new token (segment s, slot ts of the tile) into a tile's fragments: lanes
    // n == ts hold its K row, lanes g == ts / 4 its V column (element ts % 4 of each pack).
    auto patch_new = [&](Frags<D>& f, const int s, const int ts) {
        const int row = s < kQStage ? s : kQStage + wave;
        if (n == ts) {
#pragma unroll
            for (int i = 0; i < NQK; ++i) {
                const uint32_t* kw = &newtok[row][0][16 * i + 4 * g];
                f.k[i] = make_uint4(kw[0], kw[1], kw[2], kw[3]);
            }
        }
        if (g == ts / 4) {
#pragma unroll
            for (int j = 0; j < NDT; ++j) {
                const int d = 16 * j + n;
                const uint16_t h = (uint16_t)(newtok[row][1][d / 2] >> (16 * (d & 1)));
                uint16_t e[4];
                e[0] = (uint16_t)f.v[j].x;
                e[1] = (uint16_t)(f.v[j].x >> 16);
                e[2] = (uint16_t)f.v[j].y;
                e[3] = (uint16_t)(f.v[j].y >> 16);
#pragma unroll
                for (int r = 0; r < 4; ++r) e[r] = r == ts % 4 ? h : e[r];
                f.v[j] = make_uint2(e[0] | ((uint32_t)e[1] << 16), e[2] | ((uint32_t)e[3] << 16));
            }
        }
    };

    // The staged new token of item c (segment s, position pos) into the pool, by the wave
    // that processes the item's tile holding it (or, for a token past the decoded tiles,
    // the item's last decoded tile): the lanes that hold its K row store it, and every lane
    // stores D / 64 elements of its V row, from LDS, with no wait.  Nothing in this launch reads these bytes back from the pool:
    // every reader of the tile patches the token in from LDS.  The bytes are those of
    // append_chunk<VSPEC_KV_F16>; a position past the table or an invalid block writes
    // nothing.
    auto store_new = [&](const ItemCursor& c, const int s, const int pos) {
        const int row = s < kQStage ? s : kQStage + wave;
        const uint32_t lb = (uint32_t)pos / p.block_tokens;
        if (lb >= p.max_blocks) return;
        const int entry = as_const(p.block_tables)[(size_t)c.b * p.max_blocks + lb];
        if (entry < 0 || (uint32_t)entry >= p.num_blocks) return;
        const uint32_t slot = (uint32_t)pos % p.block_tokens;
        const size_t bh = (size_t)entry * p.hkv + c.y / (int)p.gsplit;
        const int ts = pos % kTile;
        if (n == ts) {
            uint4* kd = reinterpret_cast<uint4*>(const_cast<uint8_t*>(p.k) + ((bh * p.block_tokens + slot) * D) * 2);
#pragma unroll
            for (int i = 0; i < NQK; ++i) {
                const uint32_t* kw = &newtok[row][0][16 * i + 4 * g];
                kd[4 * i + g] = make_uint4(kw[0], kw[1], kw[2], kw[3]);
            }
        }
        {
            // the V row (stride 4 in its group of 4 tokens): every lane, D / 64 elements each, so
            // that each store instruction covers whole 32-byte rows of the group
            uint16_t* vd = reinterpret_cast<uint16_t*>(const_cast<uint8_t*>(p.v)) + f16_v_index(bh, p.block_tokens, D, slot, 0);
#pragma unroll
            for (int h = 0; h < D / 64; ++h) {
                const int d = lane + 64 * h;
                vd[4 * d] = (uint16_t)(newtok[row][1][d / 2] >> (16 * (d & 1)));
            }
        }
    };

    // NB tiles in flight per wave: buffer u holds the wave's tile k + u and is reloaded
    // with the tile NB steps ahead right after it is processed.  The trip count is
    // uniform per wave (rounded up to NB; the extra tiles are out of range and fully
    // masked) and every step loads and processes unconditionally, so the compiler's
    // wait counts stay exact.
    ItemCursor pc = first;  // work item of the tiles being processed
    int seg = 0;            // its segment index in this workgroup
    // position of the item's new token (fused decode step), -1: none or outside the table
    auto new_pos = [&](const int b) -> int {
        const int c = as_const(p.ctx_lens)[b];
        return p.k_new && c >= 1 && c <= ctx_cap ? c - 1 : -1;
    };
    int pctx = min(max(as_const(p.ctx_lens)[pc.b], 0), ctx_cap);
    int papp = new_pos(pc.b);
    const int len = ws.hi - ws.lo;
    const int t0 = ws.lo + wave;
    const int nt = wave < len ? (len - wave + NW - 1) / NW : 0;
    Frags<D> f[NB];
    int ok[NB];
    // Set-up.  Wave 0 loads the q rows of the range's first kQStage segments (rows GW*y ..
    // GW*y + GW - 1 of sequence b are contiguous; merge slot s serves segment s first) and,
    // for a fused decode step, their new token rows, waits for these loads only, stages
    // both in LDS, then issues its first NB tiles.  Waves 1.. issue their first NB tiles at
    // once.  The barrier (an LDS-only wait: the other waves' tile loads stay in flight)
    // publishes the staged rows, and every wave prepares its q operands while its tiles are
    // on the way.  The tile holding an item's new token may be read from the pool before
    // the token is stored there: the wave that processes it patches the token's K row and V
    // column in from LDS and then issues the token's pool stores.
    constexpr int QPL = (GW * D + 63) / 64;  // q floats per lane of wave 0 and segment
    if (wave == 0) {
        int nseg = 1;
        {
            ItemCursor c = first;
            while (nseg < kQStage && c.item0 + c.U < ws.hi) {
                cursor_next(p, ips, c);
                ++nseg;
            }
        }
        float qreg[kQStage][QPL];
        NewRow nrow[kQStage];
        {
            ItemCursor c = first;
#pragma unroll
            for (int s = 0; s < kQStage; ++s) {
                if (s < nseg) {
                    const float* qrow = p.q + ((size_t)c.b * p.hq + (size_t)c.y * GW) * D;
#pragma unroll
                    for (int j = 0; j < QPL; ++j) {
                        const int i = lane + 64 * j;
                        qreg[s][j] = i < GW * D ? qrow[i] : 0.f;
                    }
                    if (p.k_new) nrow[s] = newrow_load(c);
                    if (s + 1 < nseg) cursor_next(p, ips, c);
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(0);  // q rows and new token rows loaded
#pragma unroll
        for (int s = 0; s < kQStage; ++s) {
            if (s < nseg) {
#pragma unroll
                for (int j = 0; j < QPL; ++j) {
                    const int i = lane + 64 * j;
                    if (i < GW * D) qraw[s][i / D][i % D] = qreg[s][j];
                }
                if (p.k_new) newrow_store(nrow[s], s);
            }
        }
        if (lane < kSlots) {
            slot_cnt[lane] = 0;
            slot_seg[lane] = lane;
        }
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) ok[u] = load(t0 + u * NW, f[u]);
    __syncthreads();
    reset();
    qprep(0, pc);
    for (int k = 0; k < nt; k += NB) {
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int t = t0 + (k + u) * NW;
            if (t < ws.hi && t >= pc.item0 + pc.U) {
                do {
                    arrive(seg, pc);
                    ++seg;
                    cursor_next(p, ips, pc);
                    reset();
                } while (t >= pc.item0 + pc.U);
                pctx = min(max(as_const(p.ctx_lens)[pc.b], 0), ctx_cap);
                papp = new_pos(pc.b);
                qprep(seg, pc);
            }
            // (a tile past the range belongs to another workgroup, which stores the token)
            if (papp >= 0 && t < ws.hi && t - pc.item0 == min(papp / kTile, pc.U - 1)) {
                if (t - pc.item0 == papp / kTile) patch_new(f[u], seg, papp % kTile);
                store_new(pc, seg, papp);
            }
            process(f[u], ok[u], t - pc.item0, pctx);
            ok[u] = load(t + NB * NW, f[u]);
        }
    }
    // hand in the current segment and every later one of the workgroup (empty states)
    while (true) {
        arrive(seg, pc);
        if (pc.item0 + pc.U >= ws.hi) break;
        ++seg;
        cursor_next(p, ips, pc);
        reset();
    }
}

#ifndef VSPEC_F16_TILES_IN_FLIGHT
#define VSPEC_F16_TILES_IN_FLIGHT 2
#endif

template <int D, int GW, bool USED>
void launch_used(const DecodeParams& p, dim3 grid, hipStream_t s) {
    constexpr int NB = VSPEC_F16_TILES_IN_FLIGHT;
    if (p.wide) {
        // one work item per workgroup of 8 waves (no item spans two workgroups)
        if (p.block_tokens == 16) {
            hipLaunchKernelGGL((decode_mfma_f16<D, GW, 16, NB, USED, 8>), grid, dim3(512), 0, s, p);
        } else {
            hipLaunchKernelGGL((decode_mfma_f16<D, GW, 0, NB, USED, 8>), grid, dim3(512), 0, s, p);
        }
    } else if (p.block_tokens == 16) {
        hipLaunchKernelGGL((decode_mfma_f16<D, GW, 16, NB, USED, kWaves>), grid, dim3(256), 0, s, p);
    } else {
        hipLaunchKernelGGL((decode_mfma_f16<D, GW, 0, NB, USED, kWaves>), grid, dim3(256), 0, s, p);
    }
}

template <int D, int GW>
void launch(const DecodeParams& p, dim3 grid, hipStream_t s) {
    if (p.block_used) launch_used<D, GW, true>(p, grid, s);
    else launch_used<D, GW, false>(p, grid, s);
    // items split over several workgroups (same split: the f16 kernel's pair shares)
    if (p.merge) {
        const dim3 merge_grid(p.batch * p.hkv * p.gsplit);
        hipLaunchKernelGGL((decode_merge_split<D, GW, kSplitRagged>), merge_grid, dim3(kWaves * 64), 0, s, p);
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

int launch_decode_mfma_f16(const DecodeParams& p, uint32_t head_dim, uint32_t gw, dim3 grid,
                           hipStream_t stream) {
    if (head_dim == 64) return launch_gw<64>(gw, p, grid, stream);
    if (head_dim == 128) return launch_gw<128>(gw, p, grid, stream);
    return 0;
}

}  // namespace vkv
