// paged_kv.hip -- gfx950 kernels and C-ABI for the Vspec paged KV-cache decode path.
//
// Kernels (all wave64):
//   kv_append      block-table append of new K/V; int4 pools quantise on write
//   kv_gather      block-table gather into [T][H][D] (raw bytes or dequantised f32)
//   kv_compact     whole-block moves (compaction after eviction)
//   decode_partial single-query GQA attention, split-K over 16-token tiles
//   decode_combine log-sum-exp merge of the split-K partials
//
// The C-ABI is declared in include/vspec_rocm.h.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>
#include <vector>

#include "vspec_rocm_paged.h"

// ---------------------------------------------------------------------------
// error reporting
// ---------------------------------------------------------------------------
namespace {
thread_local char g_err[512] = "";

void set_err(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}
}  // namespace

extern "C" void vspec_rocm_set_error_(const char* msg) { set_err("%s", msg ? msg : ""); }

#define HIP_CHECK(call, what)                                              \
    do {                                                                   \
        hipError_t e_ = (call);                                            \
        if (e_ != hipSuccess) {                                            \
            set_err("%s: %s", (what), hipGetErrorString(e_));              \
            return 0;                                                      \
        }                                                                  \
    } while (0)

#include "kv_common.h"
#include "append_row.h"

namespace {
using namespace vkv;

// Per-dtype geometry of one row (one token of one kv head).
template <int DT, int D>
struct Row {
    static constexpr int kBytes = DT == VSPEC_KV_F32 ? D * 4 : (DT == VSPEC_KV_F16 ? D * 2 : D / 2);
    static constexpr int kScales = DT == VSPEC_KV_INT4 ? D / 32 : 0;
};

// K-side layout of the VALU decode kernel (f32 and f16 pools): LPK lanes hold one
// key, 16 elements per lane.
//   f16:  chunks of 8 elements (16 B), lane chunks sub, sub+LPK
//   f32:  chunks of 4 elements (16 B), lane chunks sub + j*LPK, j < 4
template <int DT, int D>
__device__ __forceinline__ int k_elem(int sub, int e) {
    static_assert(DT != VSPEC_KV_INT4, "int4 pools decode on the matrix cores");
    constexpr int LPK = D / 16;
    if constexpr (DT == VSPEC_KV_F16) {
        return 8 * (sub + (e / 8) * LPK) + (e % 8);
    } else {
        return 4 * (sub + (e / 4) * LPK) + (e % 4);
    }
}

template <int DT, int D>
__device__ __forceinline__ void load_k16(const DecodeParams& p, size_t row, int sub, float* x) {
    constexpr int LPK = D / 16;
    if constexpr (DT == VSPEC_KV_F16) {
        const uint4* src = reinterpret_cast<const uint4*>(p.k + row * (size_t)(D * 2));
        unpack_f16x8(src[sub], x);
        unpack_f16x8(src[sub + LPK], x + 8);
    } else {
        const float4* src = reinterpret_cast<const float4*>(p.k + row * (size_t)(D * 4));
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float4 w = src[sub + j * LPK];
            x[4 * j] = w.x;
            x[4 * j + 1] = w.y;
            x[4 * j + 2] = w.z;
            x[4 * j + 3] = w.w;
        }
    }
}

// V-side layout of the VALU decode kernel (f32 pools: token-major rows): D/8 lanes per
// token, lane chunk c holds elements 8c..8c+7.
template <int DT, int D>
__device__ __forceinline__ void load_v8(const DecodeParams& p, size_t row, int c, float* x) {
    static_assert(DT == VSPEC_KV_F32, "the VALU decode kernel serves f32 pools");
    const float4* src = reinterpret_cast<const float4*>(p.v + row * (size_t)(D * 4));
    const float4 a = src[2 * c];
    const float4 b = src[2 * c + 1];
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}

// Clip a row held by LPK lanes (16 elements each) to +-max(1e-6, alpha*std),
// then to +-input_clip (three_bit_runtime_modules.c:175-203, :138-173).
template <int LPK, int D>
__device__ __forceinline__ void clamp_row(float* x, float alpha, float input_clip) {
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) s += x[e];
    const float mean = group_sum<LPK>(s) * (1.0f / D);
    float v = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const float d = x[e] - mean;
        v = fmaf(d, d, v);
    }
    const float var = group_sum<LPK>(v) * (1.0f / D);
    const float th = fminf(fmaxf(1e-6f, alpha * sqrtf(var)), input_clip);
#pragma unroll
    for (int e = 0; e < 16; ++e) x[e] = fminf(fmaxf(x[e], -th), th);
}

template <int DT, int D, int GW>
__global__ __launch_bounds__(256, 2) void decode_partial(DecodeParams p) {
    constexpr int LPK = D / 16;           // lanes per key
    constexpr int KPP = 64 / LPK;         // keys per K pass
    constexpr int KPASS = kTile / KPP;    // K passes per tile
    constexpr int VLPT = D / 8;           // lanes per token on the V side
    constexpr int VTPP = 64 / VLPT;       // tokens per V pass
    constexpr int VPASS = kTile / VTPP;   // V passes per tile
    static_assert(KPASS >= 1 && VPASS >= 1, "tile geometry");

    __shared__ float p_lds[kWaves][2][kTile][GW];
    __shared__ float comb[kWaves][GW][D + 2];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int part = blockIdx.x;
    const int b = blockIdx.z;
    const int hk = blockIdx.y / p.gsplit;
    const int hq0 = hk * (p.gsplit * GW) + (blockIdx.y % p.gsplit) * GW;

    // tiles beyond the block table or the planned partitions are never read
    const int tiles_per_block = (int)p.block_tokens / kTile;
    const int ctx = min(max(p.ctx_lens[b], 0), (int)(p.max_blocks * p.block_tokens));
    const int ntiles = min((ctx + kTile - 1) / kTile, (int)(p.max_parts * p.tiles_per_part));
    const int nparts = max(1, (ntiles + (int)p.tiles_per_part - 1) / (int)p.tiles_per_part);
    if (part >= nparts) return;
    const int tile_begin = part * (int)p.tiles_per_part;
    const int tile_end = min(ntiles, tile_begin + (int)p.tiles_per_part);

    const int kk = lane / LPK;      // key within a K pass
    const int sub = lane % LPK;     // lane within the key
    const int vc = lane % VLPT;     // V chunk
    const int vt = lane / VLPT;     // token within a V pass

    // q' = clip(q) * scale * log2(e), in the K-side lane layout
    float qv[GW][16];
#pragma unroll
    for (int h = 0; h < GW; ++h) {
        const float* qrow = p.q + ((size_t)b * p.hq + hq0 + h) * D;
        float x[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) x[e] = qrow[k_elem<DT, D>(sub, e)];
        clamp_row<LPK, D>(x, p.alpha, p.input_clip);
#pragma unroll
        for (int e = 0; e < 16; ++e) qv[h][e] = x[e] * p.qscale;
    }

    float m_run[GW], l_run[GW], acc[GW][8];
#pragma unroll
    for (int h = 0; h < GW; ++h) {
        m_run[h] = -INFINITY;
        l_run[h] = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
    }

    const int32_t* table = p.block_tables + (size_t)b * p.max_blocks;
    int buf = 0;
    for (int tile = tile_begin + wave; tile < tile_end; tile += kWaves) {
        const int lblock = tile / tiles_per_block;
        const int phys = table[lblock];
        if (phys < 0 || (uint32_t)phys >= p.num_blocks) continue;  // invalid entry: tile skipped
        const size_t row0 = ((size_t)phys * p.hkv + hk) * p.block_tokens +
                            (size_t)(tile % tiles_per_block) * kTile;
        const int tok0 = tile * kTile;
        // valid slots of this tile: below the context and, with block_used, below its
        // block's used count (a prefix of the block's slots)
        const int lim = p.block_used ? min(ctx - tok0, used_cap(p.block_used[(size_t)b * p.max_blocks + lblock],
                                                                (tile % tiles_per_block) * kTile))
                                     : ctx - tok0;

        // ---- scores ----
        float s[KPASS][GW];
#pragma unroll
        for (int kp = 0; kp < KPASS; ++kp) {
            const int slot = kp * KPP + kk;
            float x[16];
            load_k16<DT, D>(p, row0 + slot, sub, x);
            clamp_row<LPK, D>(x, p.alpha, p.input_clip);
            const bool valid = slot < lim;
#pragma unroll
            for (int h = 0; h < GW; ++h) {
                float d = 0.f;
#pragma unroll
                for (int e = 0; e < 16; ++e) d = fmaf(qv[h][e], x[e], d);
                d = group_sum<LPK>(d);
                d = fminf(fmaxf(d, -p.logit_clip), p.logit_clip);
                s[kp][h] = valid ? d : -INFINITY;
            }
        }

        // ---- online softmax (rescale only when the max grows by > 2^8) ----
#pragma unroll
        for (int h = 0; h < GW; ++h) {
            float mt = s[0][h];
#pragma unroll
            for (int kp = 1; kp < KPASS; ++kp) mt = fmaxf(mt, s[kp][h]);
            mt = max_across_groups<LPK>(mt);
            // uniform across the wave after the reduction: keep it in an SGPR
            mt = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, mt)));
            if (mt > m_run[h] + 8.0f) {
                const float f = exp2f(m_run[h] - mt);
                l_run[h] *= f;
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[h][e] *= f;
                m_run[h] = mt;
            }
        }
#pragma unroll
        for (int kp = 0; kp < KPASS; ++kp) {
            if (sub < GW) {
                float sv = s[kp][0], mv = m_run[0];
#pragma unroll
                for (int h = 1; h < GW; ++h) {
                    if (sub == h) {
                        sv = s[kp][h];
                        mv = m_run[h];
                    }
                }
                p_lds[wave][buf][kp * KPP + kk][sub] = exp2f(sv - mv);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        // ---- P.V ----
        const bool tail = lim < kTile;
#pragma unroll
        for (int vp = 0; vp < VPASS; ++vp) {
            const int slot = vp * VTPP + vt;
            float x[8];
            load_v8<DT, D>(p, row0 + slot, vc, x);
            if (tail && slot >= lim) {
#pragma unroll
                for (int e = 0; e < 8; ++e) x[e] = 0.f;
            }
            float pv[GW];
#pragma unroll
            for (int h = 0; h < GW; ++h) pv[h] = p_lds[wave][buf][slot][h];
#pragma unroll
            for (int h = 0; h < GW; ++h) {
                l_run[h] += pv[h];
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[h][e] = fmaf(pv[h], x[e], acc[h][e]);
            }
        }
        buf ^= 1;
    }

    // ---- reduce the token groups of the V layout (lanes with equal chunk) ----
#pragma unroll
    for (int h = 0; h < GW; ++h) {
#pragma unroll
        for (int off = VLPT; off < 64; off <<= 1) {
            l_run[h] += __shfl_xor(l_run[h], off);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[h][e] += __shfl_xor(acc[h][e], off);
        }
    }
    if (lane < VLPT) {
#pragma unroll
        for (int h = 0; h < GW; ++h) {
#pragma unroll
            for (int e = 0; e < 8; ++e) comb[wave][h][2 + 8 * vc + e] = acc[h][e];
            if (vc == 0) {
                comb[wave][h][0] = m_run[h];
                comb[wave][h][1] = l_run[h];
            }
        }
    }
    __syncthreads();

    // ---- merge the waves of this workgroup ----
    for (int idx = threadIdx.x; idx < GW * D; idx += 256) {
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

template <int D>
__global__ __launch_bounds__(D) void decode_combine(DecodeParams p) {
    const int b = blockIdx.y;
    const int hq = blockIdx.x;
    const int d = threadIdx.x;
    const int ctx = min(max(p.ctx_lens[b], 0), (int)(p.max_blocks * p.block_tokens));
    const int ntiles = min((ctx + kTile - 1) / kTile, (int)(p.max_parts * p.tiles_per_part));
    const int nparts = max(1, (ntiles + (int)p.tiles_per_part - 1) / (int)p.tiles_per_part);
    if (nparts == 1) return;
    const size_t base = ((size_t)b * p.hq + hq) * p.max_parts;
    float M = -INFINITY;
    for (int i = 0; i < nparts; ++i) M = fmaxf(M, p.part_ml[2 * (base + i)]);
    float a = 0.f, l = 0.f;
    for (int i = 0; i < nparts; ++i) {
        const float mi = p.part_ml[2 * (base + i)];
        if (mi != -INFINITY) {
            const float f = exp2f(mi - M);
            a = fmaf(p.part_acc[(base + i) * D + d], f, a);
            l = fmaf(p.part_ml[2 * (base + i) + 1], f, l);
        }
    }
    p.out[((size_t)b * p.hq + hq) * D + d] = l > 0.f ? a / l : 0.f;
}

// ---------------------------------------------------------------------------
// append (quantise-on-write for int4)
// ---------------------------------------------------------------------------
// One work item = EPT consecutive elements of one token-head row of K or V: a whole
// 32-element quantisation group for int4 pools, 8 elements (16 or 32 bytes) otherwise.
template <int DT, int SRC>
__global__ __launch_bounds__(256) void kv_append(AppendParams p) {
    const uint64_t total = append_items<DT>(p);
    for (uint64_t it = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; it < total;
         it += (uint64_t)gridDim.x * blockDim.x) {
        append_item<DT, SRC>(p, it);
    }
}

// Rotary embedding of the query rows of the appended tokens: q [B][n_new][Hq][D] fp32,
// token (b, i) at position start_pos[b] + i; tokens without a table row are not written.
struct RopeQParams {
    const float* q_in;
    float* q_out;
    const int32_t* start_pos;
    const float* rope_cos;
    const float* rope_sin;
    uint32_t batch, n_new, hq, head_dim, rope_dim, max_pos;
};

__global__ __launch_bounds__(256) void rope_q(RopeQParams p) {
    const uint64_t total = (uint64_t)p.batch * p.n_new * p.hq * p.head_dim;
    for (uint64_t it = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; it < total;
         it += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t d = (uint32_t)(it % p.head_dim);
        const uint64_t row = it / p.head_dim;  // ((b * n_new + i) * hq + h)
        const uint32_t i = (uint32_t)((row / p.hq) % p.n_new);
        const uint32_t b = (uint32_t)(row / ((uint64_t)p.hq * p.n_new));
        const int32_t sp = p.start_pos[b];
        if (sp < 0) continue;
        const uint32_t pos = (uint32_t)sp + i;
        if (pos >= p.max_pos) continue;
        const float* x = p.q_in + row * p.head_dim;
        float y = x[d];
        if (d < p.rope_dim) {
#pragma clang fp contract(off)
            const uint32_t half = p.rope_dim / 2;
            const uint32_t k = d < half ? d : d - half;
            const float c = p.rope_cos[(size_t)pos * half + k], sn = p.rope_sin[(size_t)pos * half + k];
            y = d < half ? x[d] * c - x[d + half] * sn : x[d - half] * sn + x[d] * c;
        }
        p.q_out[row * p.head_dim + d] = y;
    }
}

// ---------------------------------------------------------------------------
// gather / compaction
// ---------------------------------------------------------------------------
struct GatherParams {
    const uint8_t* k;
    const uint8_t* v;
    const uint16_t* ks;
    const uint16_t* vs;
    const int32_t* block_tables;
    const int32_t* ctx_lens;
    const int64_t* out_off;
    uint8_t* ok;
    uint8_t* ov;
    uint16_t* oks;
    uint16_t* ovs;
    uint32_t hkv;
    uint32_t head_dim;
    uint32_t block_tokens;
    uint32_t max_blocks;
    uint32_t num_blocks;
    uint32_t max_ctx;
};

// Raw gather: one thread per 16-byte chunk of a row (int4: 4-byte chunks plus
// the row's scales).  Dequantising gather (OUTF32): one thread per 8 elements.
template <int DT, int OUTF32>
__global__ __launch_bounds__(256) void kv_gather(GatherParams p) {
    const int b = blockIdx.y;
    const int ctx = p.ctx_lens[b];
    const uint32_t D = p.head_dim;
    const uint32_t row_bytes = DT == VSPEC_KV_F32 ? D * 4 : (DT == VSPEC_KV_F16 ? D * 2 : D / 2);
    const uint32_t cpr = OUTF32 ? D / 8 : (DT == VSPEC_KV_INT4 ? row_bytes / 4 : row_bytes / 16);
    const uint64_t total = (uint64_t)p.max_ctx * p.hkv * cpr * 2;
    for (uint64_t it = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; it < total;
         it += (uint64_t)gridDim.x * blockDim.x) {
        const int which = (int)(it & 1);
        uint64_t r = it >> 1;
        const uint32_t c = (uint32_t)(r % cpr);
        r /= cpr;
        const uint32_t h = (uint32_t)(r % p.hkv);
        const uint32_t t = (uint32_t)(r / p.hkv);
        if ((int)t >= ctx) continue;
        const uint32_t lb = t / p.block_tokens;
        if (lb >= p.max_blocks) continue;
        const int32_t phys = p.block_tables[(size_t)b * p.max_blocks + lb];
        if (phys < 0 || (uint32_t)phys >= p.num_blocks) continue;
        const size_t row = ((size_t)phys * p.hkv + h) * p.block_tokens + t % p.block_tokens;
        const size_t orow = ((size_t)p.out_off[b] + t) * p.hkv + h;
        const uint8_t* src = which ? p.v : p.k;
        uint8_t* dst = which ? p.ov : p.ok;
        if (DT == VSPEC_KV_F16 && which) {
            // V in 4-token groups: 8 elements of row `slot`, stride 4
            const uint16_t* vt = reinterpret_cast<const uint16_t*>(src) +
                                 f16_v_index((size_t)phys * p.hkv + h, p.block_tokens, D, t % p.block_tokens, 8 * c);
            uint16_t e16[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) e16[i] = vt[4 * i];
            if (OUTF32) {
                float4* d = reinterpret_cast<float4*>(dst + orow * (size_t)D * 4) + 2 * c;
                d[0] = make_float4(half_bits_to_float(e16[0]), half_bits_to_float(e16[1]),
                                   half_bits_to_float(e16[2]), half_bits_to_float(e16[3]));
                d[1] = make_float4(half_bits_to_float(e16[4]), half_bits_to_float(e16[5]),
                                   half_bits_to_float(e16[6]), half_bits_to_float(e16[7]));
            } else {
                reinterpret_cast<uint4*>(dst + orow * row_bytes)[c] =
                    make_uint4(e16[0] | ((uint32_t)e16[1] << 16), e16[2] | ((uint32_t)e16[3] << 16),
                               e16[4] | ((uint32_t)e16[5] << 16), e16[6] | ((uint32_t)e16[7] << 16));
            }
            continue;
        }
        if constexpr (OUTF32) {
            float x[8];
            if constexpr (DT == VSPEC_KV_F32) {
                const float4* s = reinterpret_cast<const float4*>(src + row * row_bytes) + 2 * c;
                const float4 a = s[0], bb = s[1];
                x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
                x[4] = bb.x; x[5] = bb.y; x[6] = bb.z; x[7] = bb.w;
            } else if constexpr (DT == VSPEC_KV_F16) {
                unpack_f16x8(reinterpret_cast<const uint4*>(src + row * row_bytes)[c], x);
            } else {
                const size_t bh = (size_t)phys * p.hkv + h;
                const uint32_t slot = t % p.block_tokens;
                const uint32_t w = which ? int4_v_canonical_dword(src, bh, p.block_tokens, D, slot, c)
                                         : reinterpret_cast<const uint32_t*>(src + row * row_bytes)[c];
                const float s = half_bits_to_float(
                    which ? p.vs[row * (D / 32) + c / 4] : p.ks[int4_ks_index(bh, D / 32, p.block_tokens, slot, c / 4)]);
#pragma unroll
                for (int i = 0; i < 8; ++i) x[i] = nibble(w, i) * s;
            }
            float4* d = reinterpret_cast<float4*>(dst + orow * (size_t)D * 4) + 2 * c;
            d[0] = make_float4(x[0], x[1], x[2], x[3]);
            d[1] = make_float4(x[4], x[5], x[6], x[7]);
        } else if constexpr (DT == VSPEC_KV_INT4) {
            // output rows are canonical packed codes whatever the pool layout
            const size_t bh = (size_t)phys * p.hkv + h;
            const uint32_t slot = t % p.block_tokens;
            reinterpret_cast<uint32_t*>(dst + orow * row_bytes)[c] =
                which ? int4_v_canonical_dword(src, bh, p.block_tokens, D, slot, c)
                      : reinterpret_cast<const uint32_t*>(src + row * row_bytes)[c];
            if (c < D / 32) {
                uint16_t* od = which ? p.ovs : p.oks;
                od[orow * (D / 32) + c] =
                    which ? p.vs[row * (D / 32) + c] : p.ks[int4_ks_index(bh, D / 32, p.block_tokens, slot, c)];
            }
        } else {
            reinterpret_cast<uint4*>(dst + orow * row_bytes)[c] =
                reinterpret_cast<const uint4*>(src + row * row_bytes)[c];
        }
    }
}

struct GatherRowsParams {
    const uint8_t* k;
    const uint8_t* v;
    const uint16_t* ks;
    const uint16_t* vs;
    const int32_t* pages;
    const int32_t* slots;
    float* ok;
    float* ov;
    uint32_t n;
    uint32_t hkv;
    uint32_t head_dim;
    uint32_t block_tokens;
    uint32_t num_blocks;
};

// Row-list gather to f32: output token i is (pages[i], slots[i]) of every head, [n][H][D].
// One thread per 8 elements of one row of K or V.
template <int DT>
__global__ __launch_bounds__(256) void kv_gather_rows(GatherRowsParams p) {
    const uint32_t D = p.head_dim, P = p.block_tokens;
    const uint32_t cpr = D / 8;
    const uint64_t total = (uint64_t)p.n * p.hkv * cpr * 2;
    for (uint64_t it = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; it < total;
         it += (uint64_t)gridDim.x * blockDim.x) {
        const int which = (int)(it & 1);
        uint64_t r = it >> 1;
        const uint32_t c = (uint32_t)(r % cpr);
        r /= cpr;
        const uint32_t h = (uint32_t)(r % p.hkv);
        const uint32_t i = (uint32_t)(r / p.hkv);
        const int32_t page = p.pages[i], slot = p.slots[i];
        if (page < 0 || (uint32_t)page >= p.num_blocks || slot < 0 || (uint32_t)slot >= P) continue;
        const size_t tile = (size_t)page * p.hkv + h;
        const size_t row = tile * P + slot;
        const uint8_t* src = which ? p.v : p.k;
        float x[8];
        if constexpr (DT == VSPEC_KV_F32) {
            const float4* s4 = reinterpret_cast<const float4*>(src + row * D * 4) + 2 * c;
            const float4 a = s4[0], bb = s4[1];
            x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
            x[4] = bb.x; x[5] = bb.y; x[6] = bb.z; x[7] = bb.w;
        } else if constexpr (DT == VSPEC_KV_F16) {
            if (which) {
                const uint16_t* vt = reinterpret_cast<const uint16_t*>(src) + f16_v_index(tile, P, D, slot, 8 * c);
#pragma unroll
                for (int e = 0; e < 8; ++e) x[e] = half_bits_to_float(vt[4 * e]);
            } else {
                unpack_f16x8(reinterpret_cast<const uint4*>(src + row * D * 2)[c], x);
            }
        } else {
            const uint32_t w = which ? int4_v_canonical_dword(src, tile, P, D, slot, c)
                                     : reinterpret_cast<const uint32_t*>(src + row * (D / 2))[c];
            const float sc = half_bits_to_float(which ? p.vs[row * (D / 32) + c / 4]
                                                      : p.ks[int4_ks_index(tile, D / 32, P, slot, c / 4)]);
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = nibble(w, e) * sc;
        }
        float4* d = reinterpret_cast<float4*>((which ? p.ov : p.ok) + ((size_t)i * p.hkv + h) * D) + 2 * c;
        d[0] = make_float4(x[0], x[1], x[2], x[3]);
        d[1] = make_float4(x[4], x[5], x[6], x[7]);
    }
}

struct CompactParams {
    uint8_t* k;
    uint8_t* v;
    uint16_t* ks;
    uint16_t* vs;
    uint32_t* kf;            // int4 clamp flags or null
    uint32_t block_flags;    // flag words per physical block
    const int32_t* src;
    const int32_t* dst;
    uint32_t n;
    uint32_t num_blocks;
    uint64_t block_bytes;    // data bytes per physical block (all heads), multiple of 16
    uint64_t block_scales;   // scale entries per physical block (int4)
};

__global__ __launch_bounds__(256) void kv_compact(CompactParams p) {
    const uint32_t i = blockIdx.y;
    const int32_t s = p.src[i], d = p.dst[i];
    if (s < 0 || d < 0 || (uint32_t)s >= p.num_blocks || (uint32_t)d >= p.num_blocks) return;
    const uint64_t n16 = p.block_bytes / 16;
    for (uint64_t j = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; j < 2 * n16;
         j += (uint64_t)gridDim.x * blockDim.x) {
        uint8_t* base = j < n16 ? p.k : p.v;
        const uint64_t jj = j < n16 ? j : j - n16;
        // each byte moves once: streaming (non-temporal) load and store
        const uint4 w = load_stream4(reinterpret_cast<const uint4*>(base + (uint64_t)s * p.block_bytes) + jj);
        nt_u32x4 wv = {w.x, w.y, w.z, w.w};
        __builtin_nontemporal_store(wv, reinterpret_cast<nt_u32x4*>(base + (uint64_t)d * p.block_bytes) + jj);
    }
    if (p.block_scales) {
        for (uint64_t j = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; j < 2 * p.block_scales;
             j += (uint64_t)gridDim.x * blockDim.x) {
            uint16_t* base = j < p.block_scales ? p.ks : p.vs;
            const uint64_t jj = j < p.block_scales ? j : j - p.block_scales;
            base[(uint64_t)d * p.block_scales + jj] = base[(uint64_t)s * p.block_scales + jj];
        }
    }
    if (p.kf) {
        for (uint32_t j = blockIdx.x * blockDim.x + threadIdx.x; j < p.block_flags; j += gridDim.x * blockDim.x)
            p.kf[(uint64_t)d * p.block_flags + j] = p.kf[(uint64_t)s * p.block_flags + j];
    }
}

// ---------------------------------------------------------------------------
// host helpers
// ---------------------------------------------------------------------------
int g_num_cus = 0;

int num_cus() {
    if (g_num_cus > 0) return g_num_cus;
    int dev = 0;
    hipDeviceProp_t prop;
    if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess &&
        prop.multiProcessorCount > 0) {
        g_num_cus = prop.multiProcessorCount;
    } else {
        g_num_cus = 256;
    }
    return g_num_cus;
}

size_t row_bytes_of(int32_t dtype, uint32_t d) {
    return dtype == VSPEC_KV_F32 ? (size_t)d * 4 : (dtype == VSPEC_KV_F16 ? (size_t)d * 2 : d / 2);
}

// Geometry every kernel accepts; `decode` adds the attention kernels' limits
// (head_dim 64 or 128, block_tokens a multiple of the 16-token tile).
int check_kv(const VspecPagedKV* kv, const char* who, bool decode = false) {
    if (!kv) {
        set_err("%s: null pool", who);
        return 0;
    }
    if (kv->dtype < VSPEC_KV_F32 || kv->dtype > VSPEC_KV_INT4) {
        set_err("%s: bad dtype %d", who, (int)kv->dtype);
        return 0;
    }
    if (kv->num_blocks == 0 || kv->num_kv_heads == 0 || kv->block_tokens == 0 || kv->head_dim == 0) {
        set_err("%s: empty pool geometry", who);
        return 0;
    }
    // block-table entries are int32, and the kernels index (block, kv head) pairs in 32 bits
    if (kv->num_blocks > 0x7fffffffu || (uint64_t)kv->num_blocks * kv->num_kv_heads > 0xffffffffull) {
        set_err("%s: num_blocks must fit int32 and num_blocks x num_kv_heads 32 bits", who);
        return 0;
    }
    const uint32_t quantum = kv->dtype == VSPEC_KV_INT4 ? 32u : 8u;
    if (kv->head_dim % quantum != 0) {
        set_err("%s: head_dim must be a multiple of %u", who, quantum);
        return 0;
    }
    // int4 and f16 pools keep tiles of 16 tokens (f16 V: groups of 4 tokens, f16_v_index)
    if (kv->dtype != VSPEC_KV_F32 && kv->block_tokens % kTile != 0) {
        set_err("%s: %s pools need block_tokens a multiple of %d", who, kv->dtype == VSPEC_KV_INT4 ? "int4" : "f16",
                kTile);
        return 0;
    }
    if (decode && kv->block_tokens % kTile != 0) {
        set_err("%s: block_tokens must be a positive multiple of %d", who, kTile);
        return 0;
    }
    if (decode && kv->head_dim != 64 && kv->head_dim != 128) {
        set_err("%s: head_dim must be 64 or 128", who);
        return 0;
    }
    if (!kv->k_data || !kv->v_data) {
        set_err("%s: null pool data", who);
        return 0;
    }
    if (kv->dtype == VSPEC_KV_INT4 && (!kv->k_scales || !kv->v_scales)) {
        set_err("%s: int4 pool without scales", who);
        return 0;
    }
    // the int4 decode builds buffer descriptors whose base field holds address bits 0..47
    // (device addresses of user allocations lie below 2^47)
    const uintptr_t hi = ((uintptr_t)kv->k_data | (uintptr_t)kv->v_data | (uintptr_t)kv->k_scales |
                          (uintptr_t)kv->v_scales | (uintptr_t)kv->k_flags) >> 47;
    if (hi != 0) {
        set_err("%s: pool address at or above 2^47", who);
        return 0;
    }
    return 1;
}

// Grow-only library workspace per device (used when the caller passes none); the mutex
// keeps host threads that decode on one device from growing it at the same time (its
// contents are shared: concurrent decodes need workspaces of their own).  A buffer that
// is outgrown is retired, not freed: a HIP graph captured from an earlier decode still
// holds its address, and replays must find it allocated.  Retired buffers are freed by
// vspec_rocm_release_retired_workspaces() or at process exit.
struct Workspace {
    void* ptr = nullptr;
    size_t bytes = 0;
};
Workspace g_ws[64];
std::vector<void*> g_retired[64];
std::mutex g_ws_mu;

void* library_workspace(size_t bytes) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::lock_guard<std::mutex> lock(g_ws_mu);
    Workspace& w = g_ws[dev];
    if (w.bytes >= bytes) return w.ptr;
    void* fresh = nullptr;
    if (hipMalloc(&fresh, bytes) != hipSuccess) return nullptr;
    if (w.ptr) g_retired[dev].push_back(w.ptr);
    w.ptr = fresh;
    w.bytes = bytes;
    return w.ptr;
}

// ---- the no-allocation decode step's device scratch ----
// Partial states of vspec_rocm_paged_decode_step_noalloc live in this file-scope array,
// one copy per device for the life of the process.  Host code never uses its name as an
// address: the per-device address comes from hipGetSymbolAddress on the entry point's
// first call on that device.
constexpr size_t kScratchBytes = (size_t)6 << 20;  // partial (max, sum, acc) slots
static __device__ __align__(256) uint8_t scratch[kScratchBytes];
void* g_scratch_ptr[64];
bool g_scratch_ready[64];

uint8_t* scratch_address(int dev) {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    if (!g_scratch_ready[dev]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            set_err("paged_decode_step_noalloc: hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
            return nullptr;
        }
        g_scratch_ptr[dev] = ptr;
        g_scratch_ready[dev] = true;
    }
    return (uint8_t*)g_scratch_ptr[dev];
}

constexpr uint32_t kDefaultOldPermille = 700;
constexpr uint32_t kDefaultOldPermilleInt4 = 500;

// workgroups per CU of the balanced MFMA split: VSPEC_ROCM_DECODE_WGS_PER_CU (1..8) when
// set, else 0 (the plan decides)
uint32_t decode_wgs_per_cu_env() {
    static const uint32_t v = [] {
        const char* e = getenv("VSPEC_ROCM_DECODE_WGS_PER_CU");
        const long x = e ? strtol(e, nullptr, 10) : 0;
        return x >= 1 && x <= 8 ? (uint32_t)x : 0u;
    }();
    return v;
}

// Share of the first-half workgroup of each pair sharing a CU under the balanced split,
// in 1/1000 (VSPEC_ROCM_DECODE_OLD_PERMILLE for f16 pools, ..._INT4 for int4 pools,
// 500..900).  Read on every call.  int4 keeps equal shares by default: measured per
// workgroup at the north-star shape, the first-half workgroups end at ~65 us and their
// partners at ~86 us (the CU's wave arbiter favours the older waves), yet unequal shares
// are slower there (80.6 us at 500, 88.3 at 600, 98.7 at 700: work items then span two
// workgroups, and each extra item costs its set-up and a merge launch; with the current
// kernel 74.8 us at 500, 84.1 / 83.0 / 81.9 at 530 / 560 / 600, and equal at 16k tokens).
uint32_t decode_old_permille(uint32_t dtype) {
    const bool i4 = dtype == VSPEC_KV_INT4;
    const char* e = getenv(i4 ? "VSPEC_ROCM_DECODE_OLD_PERMILLE_INT4" : "VSPEC_ROCM_DECODE_OLD_PERMILLE");
    const long x = e ? strtol(e, nullptr, 10) : 0;
    return x >= 500 && x <= 900 ? (uint32_t)x : i4 ? kDefaultOldPermilleInt4 : kDefaultOldPermille;
}

// Least tiles per workgroup of the balanced split: VSPEC_ROCM_DECODE_MIN_TILES_PER_WG
// (1..256) when set, else 16 for batches of at most 8 work items and 1 otherwise.  With
// 8 work items (one sequence, 8 kv heads) and a grid of 2 workgroups per CU, a 1k-4k
// context leaves 1-4 tiles per workgroup and 64 partials per work item for its last
// workgroup to merge (eight rounds of loads); 16 tiles per workgroup cut the int4 step at
// B=1 from 30 to 21 us and the f16 one from 23 to 21 us.  At 16 work items the same floor
// loses (f16 at 1k: 21 -> 26 us), and from 16k tokens on it makes no difference.  Read
// on every call.
uint32_t decode_min_tiles_per_wg(uint64_t items) {
    const char* e = getenv("VSPEC_ROCM_DECODE_MIN_TILES_PER_WG");
    const long x = e ? strtol(e, nullptr, 10) : 0;
    if (x >= 1 && x <= 256) return (uint32_t)x;
    return items <= 8 ? 16u : 1u;
}

// f16 batches whose contexts the host knows to be the same, whose work items about fill the
// CUs (between 15/16 of them and all of them) and hold at least 96 tiles each run one whole
// item per workgroup of 8 waves instead of splitting items over workgroups and merging
// their partial states in a second launch.  VSPEC_ROCM_DECODE_WIDE (read on every call): 0
// never, 2 whenever the items fit the CUs, else (default, 1) the rule above.  Measured at
// B = 32 (256 items), whole against split: 1025 tokens 33.6 / 32.3 us, 2049 53.9 / 57.4,
// 4097 94.0 / 97.6, 8193 174.1 / 177.4, 32769 665 / 669; B = 30 at 4097: 90.4 / 97.1.
// With fewer items the split over all CUs wins (C2, 128 items: 36.0 split, 44.0 whole).
bool decode_wide(uint64_t items, uint64_t cus, uint64_t tiles) {
    const char* e = getenv("VSPEC_ROCM_DECODE_WIDE");
    const long x = e ? strtol(e, nullptr, 10) : 1;
    if (x == 0 || items > cus) return false;
    return x == 2 || (items * 16 >= cus * 15 && tiles >= 96);
}

// Balanced split of ragged f16 batches: every work item also costs this many tiles
// (VSPEC_ROCM_DECODE_SEGMENT_COST, 0..64; 0: tiles only), the set-up of its q operands and
// the merge of its waves' states in each workgroup that holds part of it.  Measured on C4
// (64 sequences, contexts U[128, 8192]): workgroups ran ~2 us longer per work item they
// started, so those holding many short items ended the launch; decode step with a cost of
// 0 / 2 / 4 / 8 / 12 / 16 / 24 / 32 tiles: 183.1 / 179.1 / 177.6 / 175.3 / 172.6 / 174.1 /
// 176.6 / 180.0 us (another seed of the same distribution: 226.1 at 0, 197.0 at 16).  Read on
// every call.
constexpr uint32_t kDefaultSegmentCost = 12;
uint32_t decode_segment_cost() {
    const char* e = getenv("VSPEC_ROCM_DECODE_SEGMENT_COST");
    const long x = e ? strtol(e, nullptr, 10) : -1;
    return x >= 0 && x <= 64 ? (uint32_t)x : kDefaultSegmentCost;
}

// The same for int4 pools (VSPEC_ROCM_DECODE_SEGMENT_COST_INT4, 0..64), whose work items
// cost more set-up against their tiles (q operands, three barriers, the merge of the waves'
// states): decode step at the C4 shape with int4 KV (64 sequences, contexts U[128, 8192])
// with a cost of 0 / 8 / 16 / 24 / 32 / 40 / 48 / 64 tiles: 128.8 / 105.4 / 86.7 / 81.4 /
// 79.2 / 78.6 / 78.0 / 81.6 us; two other seeds 124.6 -> 86.3 (40) and 104.7 -> 86.8 (32,
// 48); C5 decode 53.8 -> 50.8 (32) / 51.2 (48).  Read on every call.
constexpr uint32_t kDefaultSegmentCostInt4 = 40;
uint32_t decode_segment_cost_int4() {
    const char* e = getenv("VSPEC_ROCM_DECODE_SEGMENT_COST_INT4");
    const long x = e ? strtol(e, nullptr, 10) : -1;
    return x >= 0 && x <= 64 ? (uint32_t)x : kDefaultSegmentCostInt4;
}

// int4 clamp flags are read by the decode only when the balanced split gives each workgroup
// at least this many tiles (VSPEC_ROCM_DECODE_FLAG_MIN_TILES, 0..4096); shorter shares read
// no flags and screen every tile.  Measured (fused step, µs): C3 (32 tiles per workgroup)
// 23.1 with flags against 23.9 screening; B = 8 at 4k 23.2 against 24.0; B = 1-4 equal;
// B = 16 at 6k 38.6 against 40.7.  Read on every call.
constexpr uint32_t kDefaultFlagMinTiles = 16;
uint32_t decode_flag_min_tiles() {
    const char* e = getenv("VSPEC_ROCM_DECODE_FLAG_MIN_TILES");
    const long x = e ? strtol(e, nullptr, 10) : -1;
    return x >= 0 && x <= 4096 ? (uint32_t)x : kDefaultFlagMinTiles;
}

struct DecodePlan {
    bool merge;  // split MFMA kernels: some work item may span two workgroups (merge launch)
    bool wide;   // f16: one whole work item per workgroup of 8 waves (no merge launch)
    uint32_t gw;
    uint32_t gsplit;
    uint32_t tiles_per_part;
    uint32_t max_parts;
    size_t ws_bytes;
    // MFMA kernels (f16 / int4 pools): tiles of all work items split over grid_x workgroups
    bool split;
    uint32_t grid_x;
    uint32_t chunk_tiles;
    uint64_t split_tiles;  // tiles the balanced split spreads over grid_x (upper bound)
    uint32_t min_tiles;    // least tiles per workgroup of the balanced split
    uint32_t max_tiles;
    uint32_t old_permille;  // pair share of the first-half workgroups (500: equal shares)
    uint32_t uniform_tiles; // tiles per work item when every context is known to be the same
};

// With every context known to be the same (min_ctx_len == the context bound), the split
// of the MFMA kernels (kv_common.h work_split with equal shares, as for any batch whose
// contexts are equal) is known on the host: returns whether some range boundary falls
// strictly inside a work item.  Without that knowledge a merge launch is always needed.
// Tiles per work item when every context is known to be the same (min_ctx_len at least
// the bound), as the kernels' item_tiles computes them; 0 otherwise.
uint32_t uniform_item_tiles(const VspecPagedAttnDesc* d, const DecodePlan* pl, uint64_t ctx_bound) {
    if (!d->min_ctx_len || d->min_ctx_len < ctx_bound) return 0;
    const uint64_t ctx = ctx_bound < (uint64_t)d->max_blocks_per_seq * d->kv.block_tokens
                             ? ctx_bound : (uint64_t)d->max_blocks_per_seq * d->kv.block_tokens;
    uint64_t U = (ctx + kTile - 1) / kTile;
    if (U > pl->max_tiles) U = pl->max_tiles;
    if (U < 1) U = 1;
    return (uint32_t)U;
}

bool uniform_split_has_partials(const VspecPagedAttnDesc* d, const DecodePlan* pl, uint64_t ctx_bound) {
    const uint64_t U = uniform_item_tiles(d, pl, ctx_bound);
    if (!U) return true;
    const uint64_t items = (uint64_t)d->batch * d->kv.num_kv_heads * pl->gsplit;
    const uint64_t T = items * U;
    if (pl->chunk_tiles) return pl->chunk_tiles % U != 0 && T > pl->chunk_tiles;
    uint64_t G = pl->grid_x < T ? pl->grid_x : T;
    if (pl->min_tiles > 1) {
        const uint64_t cap = T / pl->min_tiles > 1 ? T / pl->min_tiles : 1;
        if (cap < G) G = cap;
    }
    // the int4 kernel's unequal pair shares (the kernels' split_shape: contexts are equal
    // here, so the f16 kernel keeps equal shares)
    const uint64_t wa = pl->old_permille;
    if (d->kv.dtype == VSPEC_KV_INT4 && wa != 500 && G == pl->grid_x && G % 2 == 0 && T >= 64 * G &&
        (1000 - wa) * T >= 500 * G) {
        const uint64_t half = G / 2;
        for (uint64_t g = 1; g < G; ++g) {
            const uint64_t c = wa * (g < half ? g : half) + (1000 - wa) * (g > half ? g - half : 0);
            if ((c * T / (1000 * half)) % U != 0) return true;
        }
        return false;
    }
    for (uint64_t g = 1; g < G; ++g) {
        if ((g * T / G) % U != 0) return true;
    }
    return false;
}

int plan_decode(const VspecPagedAttnDesc* d, DecodePlan* pl) {
    pl->merge = true;
    const uint32_t hkv = d->kv.num_kv_heads;
    if (d->num_q_heads == 0 || d->num_q_heads % hkv != 0) {
        set_err("paged_decode: num_q_heads must be a positive multiple of num_kv_heads");
        return 0;
    }
    const uint32_t g = d->num_q_heads / hkv;
    if (g <= 4) {
        pl->gw = g;
        pl->gsplit = 1;
    } else if (g % 4 == 0) {
        pl->gw = 4;
        pl->gsplit = g / 4;
    } else {
        set_err("paged_decode: GQA group %u unsupported (need <= 4 or a multiple of 4)", g);
        return 0;
    }
    // the host's bound on ctx_lens; 0 stands for the block table's capacity
    const uint64_t ctx_bound = d->max_ctx_len ? (uint64_t)d->max_ctx_len
                                              : (uint64_t)d->max_blocks_per_seq * d->kv.block_tokens;
    if (ctx_bound > (uint64_t)INT32_MAX) {
        set_err("paged_decode: context bound beyond 2^31 tokens");
        return 0;
    }
    const uint32_t max_tiles = (uint32_t)((ctx_bound + kTile - 1) / kTile);
    pl->split = d->kv.dtype != VSPEC_KV_F32;
    pl->wide = false;
    pl->min_tiles = decode_min_tiles_per_wg((uint64_t)d->batch * hkv * pl->gsplit);
    if (pl->split) {
        // every workgroup streams an equal share of all work items' tiles
        const uint64_t bound = (uint64_t)d->batch * hkv * pl->gsplit * (max_tiles ? max_tiles : 1);
        if (bound > (uint64_t)INT32_MAX) {
            set_err("paged_decode: batch * work items * tiles exceeds 2^31");
            return 0;
        }
        uint64_t grid;
        if (d->partition_tokens) {
            if (d->partition_tokens % kTile) {
                set_err("paged_decode: partition_tokens must be a multiple of %d", kTile);
                return 0;
            }
            pl->chunk_tiles = d->partition_tokens / kTile;
            grid = (bound + pl->chunk_tiles - 1) / pl->chunk_tiles;
        } else if (d->kv.dtype == VSPEC_KV_F16 && d->min_ctx_len && d->min_ctx_len >= ctx_bound &&
                   decode_wide((uint64_t)d->batch * hkv * pl->gsplit, (uint64_t)num_cus(), max_tiles)) {
            // whole items on 8-wave workgroups: every context is the same (the host says so),
            // so chunks of one item's tiles are exactly the items
            pl->wide = true;
            pl->chunk_tiles = 0;  // set below from the items' tiles
            grid = (uint64_t)d->batch * hkv * pl->gsplit;
        } else {
            pl->chunk_tiles = 0;
            // two workgroups per CU; small f16 batches (under 64 tiles per workgroup at two
            // per CU) take one, which halves the cross-workgroup merges per work item
            // (C2: 41.6 -> 38.9 us; the int4 kernel, bound by vector ALU work, needs both)
            uint32_t wpc = decode_wgs_per_cu_env();
            if (!wpc) wpc = d->kv.dtype == VSPEC_KV_F16 && bound < 128ull * (uint64_t)num_cus() ? 1u : 2u;
            grid = (uint64_t)wpc * (uint64_t)num_cus();
            // the kernel caps its groups at total / min_tiles of the actual split total (tiles,
            // plus the segment cost of every work item of a ragged batch); the grid, from a
            // bound of that total, only trims idle workgroups, so the split does not depend on
            // the host's context bound
            const uint64_t seg = d->kv.dtype == VSPEC_KV_F16    ? decode_segment_cost()
                                 : d->kv.dtype == VSPEC_KV_INT4 ? decode_segment_cost_int4()
                                                                : 0u;
            const uint64_t cost_bound = bound + seg * (uint64_t)d->batch * hkv * pl->gsplit;
            const uint64_t min_tiles = pl->min_tiles;
            if (grid * min_tiles > cost_bound) grid = cost_bound / min_tiles;
        }
        pl->grid_x = (uint32_t)(grid ? grid : 1);
        pl->split_tiles = bound;
        pl->max_tiles = max_tiles;
        pl->tiles_per_part = 0;
        pl->max_parts = 1;
        // unequal pair shares need the grid of two workgroups per CU (g and g + G/2 share one)
        pl->old_permille = !pl->chunk_tiles && pl->grid_x == 2u * (uint32_t)num_cus()
                               ? decode_old_permille(d->kv.dtype) : 500u;
        if (pl->wide) pl->chunk_tiles = uniform_item_tiles(d, pl, ctx_bound);
        pl->merge = uniform_split_has_partials(d, pl, ctx_bound);
        pl->uniform_tiles = uniform_item_tiles(d, pl, ctx_bound);
        // the workspace stays even without a merge launch: a context below min_ctx_len (a
        // caller error) then leaves its partial states in valid memory, not its output
        pl->ws_bytes = (size_t)pl->grid_x * 2 * pl->gw * (2 + d->kv.head_dim) * sizeof(float);
        return 1;
    }
    uint32_t tpp;
    if (d->partition_tokens) {
        if (d->partition_tokens % kTile) {
            set_err("paged_decode: partition_tokens must be a multiple of %d", kTile);
            return 0;
        }
        tpp = d->partition_tokens / kTile;
    } else {
        // split each (sequence, kv head) only as far as needed to occupy every resident
        // workgroup slot once (two 4-wave workgroups per CU at the kernels' register
        // use); extra partitions only add combine traffic and per-workgroup setup
        const uint64_t items = (uint64_t)d->batch * hkv * pl->gsplit;
        const uint64_t target = 2ull * (uint64_t)num_cus();
        uint64_t parts = items ? (target + items - 1) / items : 1;
        if (parts < 1) parts = 1;
        tpp = (uint32_t)((max_tiles + parts - 1) / parts);
        if (tpp < 16) tpp = 16;
        tpp = (tpp + kWaves - 1) / kWaves * kWaves;
    }
    if (tpp == 0) tpp = 1;
    pl->tiles_per_part = tpp;
    pl->max_parts = max_tiles ? (max_tiles + tpp - 1) / tpp : 1;
    if (pl->max_parts == 0) pl->max_parts = 1;
    pl->ws_bytes = pl->max_parts > 1
                       ? (size_t)d->batch * d->num_q_heads * pl->max_parts * (2 + d->kv.head_dim) * sizeof(float)
                       : 0;
    return 1;
}

template <int DT, int D, int GW>
void launch_partial(const DecodeParams& p, dim3 grid, hipStream_t s) {
    hipLaunchKernelGGL((decode_partial<DT, D, GW>), grid, dim3(256), 0, s, p);
}

template <int DT, int D>
int dispatch_gw(uint32_t gw, const DecodeParams& p, dim3 grid, hipStream_t s) {
    switch (gw) {
        case 1: launch_partial<DT, D, 1>(p, grid, s); return 1;
        case 2: launch_partial<DT, D, 2>(p, grid, s); return 1;
        case 3: launch_partial<DT, D, 3>(p, grid, s); return 1;
        case 4: launch_partial<DT, D, 4>(p, grid, s); return 1;
        default: return 0;
    }
}

template <int DT>
int dispatch_d(uint32_t d, uint32_t gw, const DecodeParams& p, dim3 grid, hipStream_t s) {
    if (d == 64) return dispatch_gw<DT, 64>(gw, p, grid, s);
    if (d == 128) return dispatch_gw<DT, 128>(gw, p, grid, s);
    return 0;
}

}  // namespace

// ---------------------------------------------------------------------------
// C-ABI
// ---------------------------------------------------------------------------
extern "C" {

const char* vspec_rocm_last_error(void) { return g_err; }

int vspec_rocm_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

int vspec_rocm_sync(void* stream) {
    HIP_CHECK(hipStreamSynchronize((hipStream_t)stream), "sync");
    return 1;
}

size_t vspec_rocm_kv_pool_bytes(int32_t dtype, uint32_t num_blocks, uint32_t block_tokens,
                                uint32_t num_kv_heads, uint32_t head_dim) {
    const size_t rows = (size_t)num_blocks * num_kv_heads * block_tokens;
    size_t bytes = 2 * rows * row_bytes_of(dtype, head_dim);
    if (dtype == VSPEC_KV_INT4) {
        bytes += 2 * rows * (head_dim / 32) * sizeof(uint16_t);
        bytes += (rows / 16) * sizeof(uint32_t);  // clamp flags
    }
    return bytes;
}

int vspec_rocm_kv_pool_create(VspecPagedKV* kv, int32_t dtype, uint32_t num_blocks,
                              uint32_t block_tokens, uint32_t num_kv_heads, uint32_t head_dim) {
    if (!kv) {
        set_err("kv_pool_create: null descriptor");
        return 0;
    }
    memset(kv, 0, sizeof(*kv));
    kv->dtype = dtype;
    kv->num_blocks = num_blocks;
    kv->block_tokens = block_tokens;
    kv->num_kv_heads = num_kv_heads;
    kv->head_dim = head_dim;
    kv->k_data = kv->v_data = (void*)1;  // placeholders for validation
    kv->k_scales = kv->v_scales = (uint16_t*)1;
    if (!check_kv(kv, "kv_pool_create")) {
        memset(kv, 0, sizeof(*kv));
        return 0;
    }
    kv->k_data = kv->v_data = nullptr;
    kv->k_scales = kv->v_scales = nullptr;
    const size_t rows = (size_t)num_blocks * num_kv_heads * block_tokens;
    const size_t data = rows * row_bytes_of(dtype, head_dim);
    if (hipMalloc(&kv->k_data, data) != hipSuccess || hipMalloc(&kv->v_data, data) != hipSuccess) {
        set_err("kv_pool_create: hipMalloc of %zu bytes failed", 2 * data);
        vspec_rocm_kv_pool_destroy(kv);
        return 0;
    }
    if (dtype == VSPEC_KV_INT4) {
        const size_t sb = rows * (head_dim / 32) * sizeof(uint16_t);
        const size_t fb = (rows / 16) * sizeof(uint32_t);
        if (hipMalloc((void**)&kv->k_scales, sb) != hipSuccess ||
            hipMalloc((void**)&kv->v_scales, sb) != hipSuccess ||
            hipMalloc((void**)&kv->k_flags, fb) != hipSuccess ||
            hipMemset(kv->k_flags, 0, fb) != hipSuccess) {
            set_err("kv_pool_create: hipMalloc of scales or flags failed");
            vspec_rocm_kv_pool_destroy(kv);
            return 0;
        }
    }
    return 1;
}

void vspec_rocm_kv_pool_destroy(VspecPagedKV* kv) {
    if (!kv) return;
    if (kv->k_data) (void)hipFree(kv->k_data);
    if (kv->v_data) (void)hipFree(kv->v_data);
    if (kv->k_scales) (void)hipFree(kv->k_scales);
    if (kv->v_scales) (void)hipFree(kv->v_scales);
    if (kv->k_flags) (void)hipFree(kv->k_flags);
    memset(kv, 0, sizeof(*kv));
}

static int append_launch(const char* who, const VspecPagedKV* kv, AppendParams& p, int32_t src_dtype,
                         void* stream) {
    p.k = (uint8_t*)kv->k_data;
    p.v = (uint8_t*)kv->v_data;
    p.ks = kv->k_scales;
    p.vs = kv->v_scales;
    p.kf = kv->dtype == VSPEC_KV_INT4 ? kv->k_flags : nullptr;
    p.hkv = kv->num_kv_heads;
    p.head_dim = kv->head_dim;
    p.block_tokens = kv->block_tokens;
    p.num_blocks = kv->num_blocks;
    const uint32_t ept = kv->dtype == VSPEC_KV_INT4 ? 32 : 8;
    const uint64_t items = (uint64_t)p.batch * p.n_new * kv->num_kv_heads * (kv->head_dim / ept) * 2;
    uint64_t blocks = (items + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    const dim3 grid((unsigned)blocks);
    hipStream_t s = (hipStream_t)stream;
#define VSPEC_APPEND(DT, SRC) hipLaunchKernelGGL((kv_append<DT, SRC>), grid, dim3(256), 0, s, p)
    if (src_dtype == VSPEC_KV_F32) {
        if (kv->dtype == VSPEC_KV_F32) VSPEC_APPEND(VSPEC_KV_F32, VSPEC_KV_F32);
        else if (kv->dtype == VSPEC_KV_F16) VSPEC_APPEND(VSPEC_KV_F16, VSPEC_KV_F32);
        else VSPEC_APPEND(VSPEC_KV_INT4, VSPEC_KV_F32);
    } else {
        if (kv->dtype == VSPEC_KV_F32) VSPEC_APPEND(VSPEC_KV_F32, VSPEC_KV_F16);
        else if (kv->dtype == VSPEC_KV_F16) VSPEC_APPEND(VSPEC_KV_F16, VSPEC_KV_F16);
        else VSPEC_APPEND(VSPEC_KV_INT4, VSPEC_KV_F16);
    }
#undef VSPEC_APPEND
    HIP_CHECK(hipGetLastError(), who);
    return 1;
}

int vspec_rocm_kv_append(const VspecPagedKV* kv, uint32_t batch, const int32_t* block_tables,
                         uint32_t max_blocks_per_seq, const int32_t* start_pos, uint32_t n_new,
                         const void* k_new, const void* v_new, int32_t src_dtype, void* stream) {
    if (!check_kv(kv, "kv_append")) return 0;
    if (src_dtype != VSPEC_KV_F32 && src_dtype != VSPEC_KV_F16) {
        set_err("kv_append: src_dtype must be f32 or f16");
        return 0;
    }
    if (batch == 0 || n_new == 0) return 1;
    if (!block_tables || !start_pos || !k_new || !v_new || max_blocks_per_seq == 0) {
        set_err("kv_append: null argument");
        return 0;
    }
    AppendParams p = {};
    p.block_tables = block_tables;
    p.start_pos = start_pos;
    p.k_new = (const uint8_t*)k_new;
    p.v_new = (const uint8_t*)v_new;
    p.batch = batch;
    p.n_new = n_new;
    p.max_blocks = max_blocks_per_seq;
    return append_launch("kv_append launch", kv, p, src_dtype, stream);
}

int vspec_rocm_kv_append_rope(const VspecPagedKV* kv, uint32_t batch, const int32_t* block_tables,
                              uint32_t max_blocks_per_seq, const int32_t* start_pos, uint32_t n_new,
                              const void* k_new, const void* v_new, int32_t src_dtype, const float* rope_cos,
                              const float* rope_sin, uint32_t rope_dim, uint32_t max_pos, const float* q_in,
                              float* q_out, uint32_t num_q_heads, void* stream) {
    if (!check_kv(kv, "kv_append_rope")) return 0;
    if (src_dtype != VSPEC_KV_F32 && src_dtype != VSPEC_KV_F16) {
        set_err("kv_append_rope: src_dtype must be f32 or f16");
        return 0;
    }
    if (!rope_cos || !rope_sin || rope_dim == 0 || rope_dim % 2 != 0 || rope_dim > kv->head_dim || max_pos == 0) {
        set_err("kv_append_rope: need cos/sin tables and an even rope_dim <= head_dim");
        return 0;
    }
    if ((q_in == nullptr) != (q_out == nullptr) || (q_in && num_q_heads == 0)) {
        set_err("kv_append_rope: q_in and q_out go together, with num_q_heads > 0");
        return 0;
    }
    if (batch == 0 || n_new == 0) return 1;
    if (!block_tables || !start_pos || !k_new || !v_new || max_blocks_per_seq == 0) {
        set_err("kv_append_rope: null argument");
        return 0;
    }
    AppendParams p = {};
    p.block_tables = block_tables;
    p.start_pos = start_pos;
    p.k_new = (const uint8_t*)k_new;
    p.v_new = (const uint8_t*)v_new;
    p.batch = batch;
    p.n_new = n_new;
    p.max_blocks = max_blocks_per_seq;
    p.rope_cos = rope_cos;
    p.rope_sin = rope_sin;
    p.rope_dim = rope_dim;
    p.max_pos = max_pos;
    if (!append_launch("kv_append_rope launch", kv, p, src_dtype, stream)) return 0;
    if (q_in) {
        RopeQParams rq = {q_in, q_out, start_pos, rope_cos, rope_sin, batch, n_new, num_q_heads,
                          kv->head_dim, rope_dim, max_pos};
        const uint64_t total = (uint64_t)batch * n_new * num_q_heads * kv->head_dim;
        uint64_t blocks = (total + 255) / 256;
        if (blocks > 65536) blocks = 65536;
        hipLaunchKernelGGL(rope_q, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, rq);
        HIP_CHECK(hipGetLastError(), "rope_q launch");
    }
    return 1;
}

int vspec_rocm_kv_append_tokens(const VspecPagedKV* kv, uint32_t n_tokens, const int32_t* token_item,
                                const int32_t* token_pos, const int32_t* block_tables, uint32_t n_items,
                                uint32_t max_blocks_per_seq, const void* k_new, const void* v_new,
                                int32_t src_dtype, void* stream) {
    if (!check_kv(kv, "kv_append_tokens")) return 0;
    if (src_dtype != VSPEC_KV_F32 && src_dtype != VSPEC_KV_F16) {
        set_err("kv_append_tokens: src_dtype must be f32 or f16");
        return 0;
    }
    if (n_tokens == 0) return 1;
    if (!token_item || !token_pos || !block_tables || !k_new || !v_new || max_blocks_per_seq == 0 || n_items == 0) {
        set_err("kv_append_tokens: null argument or no block-table rows");
        return 0;
    }
    AppendParams p = {};
    p.block_tables = block_tables;
    p.token_item = token_item;
    p.token_pos = token_pos;
    p.n_items = n_items;
    p.k_new = (const uint8_t*)k_new;
    p.v_new = (const uint8_t*)v_new;
    p.batch = n_tokens;
    p.n_new = 1;
    p.max_blocks = max_blocks_per_seq;
    return append_launch("kv_append_tokens launch", kv, p, src_dtype, stream);
}

int vspec_rocm_kv_gather(const VspecPagedKV* kv, uint32_t batch, const int32_t* block_tables,
                         uint32_t max_blocks_per_seq, const int32_t* ctx_lens,
                         uint32_t max_ctx_len, const int64_t* out_token_offset, int32_t out_mode,
                         void* out_k, void* out_v, uint16_t* out_k_scales,
                         uint16_t* out_v_scales, void* stream) {
    if (!check_kv(kv, "kv_gather")) return 0;
    if (out_mode != VSPEC_GATHER_RAW && out_mode != VSPEC_GATHER_F32) {
        set_err("kv_gather: bad out_mode");
        return 0;
    }
    if (batch == 0 || max_ctx_len == 0) return 1;
    if (!block_tables || !ctx_lens || !out_token_offset || !out_k || !out_v || max_blocks_per_seq == 0) {
        set_err("kv_gather: null argument");
        return 0;
    }
    if (out_mode == VSPEC_GATHER_RAW && kv->dtype == VSPEC_KV_INT4 && (!out_k_scales || !out_v_scales)) {
        set_err("kv_gather: int4 raw gather needs scale outputs");
        return 0;
    }
    GatherParams p = {};
    p.k = (const uint8_t*)kv->k_data;
    p.v = (const uint8_t*)kv->v_data;
    p.ks = kv->k_scales;
    p.vs = kv->v_scales;
    p.block_tables = block_tables;
    p.ctx_lens = ctx_lens;
    p.out_off = out_token_offset;
    p.ok = (uint8_t*)out_k;
    p.ov = (uint8_t*)out_v;
    p.oks = out_k_scales;
    p.ovs = out_v_scales;
    p.hkv = kv->num_kv_heads;
    p.head_dim = kv->head_dim;
    p.block_tokens = kv->block_tokens;
    p.max_blocks = max_blocks_per_seq;
    p.num_blocks = kv->num_blocks;
    p.max_ctx = max_ctx_len;
    const uint32_t D = kv->head_dim;
    const size_t rb = row_bytes_of(kv->dtype, D);
    const uint32_t cpr = out_mode == VSPEC_GATHER_F32 ? D / 8 : (kv->dtype == VSPEC_KV_INT4 ? rb / 4 : rb / 16);
    const uint64_t items = (uint64_t)max_ctx_len * kv->num_kv_heads * cpr * 2;
    uint64_t gx = (items + 255) / 256;
    if (gx > 16384) gx = 16384;
    const dim3 grid((unsigned)gx, batch);
    hipStream_t s = (hipStream_t)stream;
#define VSPEC_GATHER(DT, OF) hipLaunchKernelGGL((kv_gather<DT, OF>), grid, dim3(256), 0, s, p)
    if (out_mode == VSPEC_GATHER_F32) {
        if (kv->dtype == VSPEC_KV_F32) VSPEC_GATHER(VSPEC_KV_F32, 1);
        else if (kv->dtype == VSPEC_KV_F16) VSPEC_GATHER(VSPEC_KV_F16, 1);
        else VSPEC_GATHER(VSPEC_KV_INT4, 1);
    } else {
        if (kv->dtype == VSPEC_KV_F32) VSPEC_GATHER(VSPEC_KV_F32, 0);
        else if (kv->dtype == VSPEC_KV_F16) VSPEC_GATHER(VSPEC_KV_F16, 0);
        else VSPEC_GATHER(VSPEC_KV_INT4, 0);
    }
#undef VSPEC_GATHER
    HIP_CHECK(hipGetLastError(), "kv_gather launch");
    return 1;
}

int vspec_rocm_kv_compact(const VspecPagedKV* kv, uint32_t n, const int32_t* src_blocks,
                          const int32_t* dst_blocks, void* stream) {
    if (!check_kv(kv, "kv_compact")) return 0;
    if (n == 0) return 1;
    if (!src_blocks || !dst_blocks) {
        set_err("kv_compact: null block list");
        return 0;
    }
    CompactParams p = {};
    p.k = (uint8_t*)kv->k_data;
    p.v = (uint8_t*)kv->v_data;
    p.ks = kv->k_scales;
    p.vs = kv->v_scales;
    p.src = src_blocks;
    p.dst = dst_blocks;
    p.n = n;
    p.num_blocks = kv->num_blocks;
    const uint64_t rows = (uint64_t)kv->num_kv_heads * kv->block_tokens;
    p.block_bytes = rows * row_bytes_of(kv->dtype, kv->head_dim);
    p.block_scales = kv->dtype == VSPEC_KV_INT4 ? rows * (kv->head_dim / 32) : 0;
    p.kf = kv->dtype == VSPEC_KV_INT4 ? kv->k_flags : nullptr;
    p.block_flags = (uint32_t)(rows / 16);
    uint64_t gx = (2 * (p.block_bytes / 16) + 255) / 256;
    if (gx > 64) gx = 64;
    if (gx == 0) gx = 1;
    hipLaunchKernelGGL(kv_compact, dim3((unsigned)gx, n), dim3(256), 0, (hipStream_t)stream, p);
    HIP_CHECK(hipGetLastError(), "kv_compact launch");
    return 1;
}

int vspec_rocm_kv_gather_rows(const VspecPagedKV* kv, uint32_t n, const int32_t* pages,
                              const int32_t* slots, float* out_k, float* out_v, void* stream) {
    if (!check_kv(kv, "kv_gather_rows")) return 0;
    if (n == 0) return 1;
    if (!pages || !slots || !out_k || !out_v) {
        set_err("kv_gather_rows: null argument");
        return 0;
    }
    GatherRowsParams p = {};
    p.k = (const uint8_t*)kv->k_data;
    p.v = (const uint8_t*)kv->v_data;
    p.ks = kv->k_scales;
    p.vs = kv->v_scales;
    p.pages = pages;
    p.slots = slots;
    p.ok = out_k;
    p.ov = out_v;
    p.n = n;
    p.hkv = kv->num_kv_heads;
    p.head_dim = kv->head_dim;
    p.block_tokens = kv->block_tokens;
    p.num_blocks = kv->num_blocks;
    const uint64_t items = (uint64_t)n * kv->num_kv_heads * (kv->head_dim / 8) * 2;
    uint64_t gx = (items + 255) / 256;
    if (gx > 16384) gx = 16384;
    hipStream_t s = (hipStream_t)stream;
    if (kv->dtype == VSPEC_KV_F32) hipLaunchKernelGGL(kv_gather_rows<VSPEC_KV_F32>, dim3((unsigned)gx), dim3(256), 0, s, p);
    else if (kv->dtype == VSPEC_KV_F16) hipLaunchKernelGGL(kv_gather_rows<VSPEC_KV_F16>, dim3((unsigned)gx), dim3(256), 0, s, p);
    else hipLaunchKernelGGL(kv_gather_rows<VSPEC_KV_INT4>, dim3((unsigned)gx), dim3(256), 0, s, p);
    HIP_CHECK(hipGetLastError(), "kv_gather_rows launch");
    return 1;
}

size_t vspec_rocm_paged_decode_workspace_bytes(const VspecPagedAttnDesc* desc) {
    DecodePlan pl;
    if (!desc) {
        set_err("paged_decode_workspace_bytes: null descriptor");
        return 0;
    }
    if (!check_kv(&desc->kv, "paged_decode_workspace_bytes", true) || !plan_decode(desc, &pl)) return 0;
    return pl.ws_bytes;
}

}  // extern "C"

namespace {

// Decode attention, with the decode step's append of k_new / v_new first when they are
// given (one launch for the f16 and int4 kernels, an append launch before the f32 one).
// noalloc: the partial states come from the file-scope scratch array
// (no allocation, no library state beyond it); the descriptor's workspace is ignored.
int paged_decode(const VspecPagedAttnDesc* desc, const void* k_new, const void* v_new, int32_t src_dtype,
                 bool noalloc) {
    if (!desc) {
        set_err("paged_decode: null descriptor");
        return 0;
    }
    if (!check_kv(&desc->kv, "paged_decode", true)) return 0;
    if (desc->batch == 0) return 1;
    if (!desc->block_tables || !desc->ctx_lens || !desc->q || !desc->out || desc->max_blocks_per_seq == 0) {
        set_err("paged_decode: null argument");
        return 0;
    }
    if (desc->numerics != VSPEC_NUMERICS_PLAIN && desc->numerics != VSPEC_NUMERICS_3BIT) {
        set_err("paged_decode: bad numerics mode");
        return 0;
    }
    if ((uint64_t)desc->max_ctx_len > (uint64_t)desc->max_blocks_per_seq * desc->kv.block_tokens) {
        set_err("paged_decode: max_ctx_len exceeds the block table");
        return 0;
    }
    DecodePlan pl;
    if (!plan_decode(desc, &pl)) return 0;
    void* ws = nullptr;
    if (noalloc) {
        if (pl.ws_bytes > kScratchBytes) {
            set_err("paged_decode_step_noalloc: the plan needs %zu bytes of partial states, more than the "
                    "%zu-byte scratch (use vspec_rocm_paged_decode_step with a workspace)",
                    pl.ws_bytes, kScratchBytes);
            return 0;
        }
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
            set_err("paged_decode_step_noalloc: no current device");
            return 0;
        }
        uint8_t* base = scratch_address(dev);
        if (!base) return 0;
        ws = pl.ws_bytes ? base : nullptr;
    } else if (pl.ws_bytes) {
        if (desc->workspace) {
            if (desc->workspace_bytes < pl.ws_bytes) {
                set_err("paged_decode: workspace too small (%zu < %zu)", desc->workspace_bytes, pl.ws_bytes);
                return 0;
            }
            ws = desc->workspace;
        } else {
            ws = library_workspace(pl.ws_bytes);
            if (!ws) {
                set_err("paged_decode: cannot allocate %zu workspace bytes", pl.ws_bytes);
                return 0;
            }
        }
    }
    const uint32_t D = desc->kv.head_dim;
    float scale = desc->scale > 0.f ? desc->scale : 1.0f / sqrtf((float)D);
    const bool three = desc->numerics == VSPEC_NUMERICS_3BIT;
    if (three) scale = fminf(fmaxf(scale, 1e-4f), 32.0f);

    DecodeParams p = {};
    p.k = (const uint8_t*)desc->kv.k_data;
    p.v = (const uint8_t*)desc->kv.v_data;
    p.ks = desc->kv.k_scales;
    p.vs = desc->kv.v_scales;
    p.kf = desc->kv.dtype == VSPEC_KV_INT4 ? desc->kv.k_flags : nullptr;
    p.read_flags = p.kf && pl.split && pl.split_tiles >= (uint64_t)decode_flag_min_tiles() * pl.grid_x;
    p.block_tables = desc->block_tables;
    p.ctx_lens = desc->ctx_lens;
    p.block_used = desc->block_used;
    p.q = desc->q;
    p.out = desc->out;
    p.part_ml = (float*)ws;
    p.part_acc = ws ? (float*)ws + (size_t)desc->batch * desc->num_q_heads * pl.max_parts * 2 : nullptr;
    p.hq = desc->num_q_heads;
    p.hkv = desc->kv.num_kv_heads;
    p.block_tokens = desc->kv.block_tokens;
    p.max_blocks = desc->max_blocks_per_seq;
    p.num_blocks = desc->kv.num_blocks;
    p.tiles_per_part = pl.tiles_per_part;
    p.max_parts = pl.max_parts;
    p.gsplit = pl.gsplit;
    p.qscale = scale * kLog2e;
    p.alpha = desc->clamp_alpha > 0.f ? desc->clamp_alpha : 4.5f;
    p.logit_clip = three ? 24.0f * kLog2e : INFINITY;
    p.input_clip = three ? 16.0f : INFINITY;
    p.split_grid = pl.split ? pl.grid_x : 0u;
    p.merge = pl.split && pl.merge;
    p.batch = desc->batch;
    p.max_tiles = pl.max_tiles;
    p.chunk_tiles = pl.chunk_tiles;
    p.k_new = nullptr;
    p.v_new = nullptr;
    p.append_src = src_dtype;
    p.split_old_permille = pl.split ? pl.old_permille : 500u;
    p.uniform_tiles = pl.split ? pl.uniform_tiles : 0u;
    p.min_tiles = pl.split && !pl.chunk_tiles ? pl.min_tiles : 1u;
    p.wide = pl.wide;
    p.seg_cost = !pl.split || pl.chunk_tiles ? 0u
                 : desc->kv.dtype == VSPEC_KV_F16 ? decode_segment_cost()
                 : desc->kv.dtype == VSPEC_KV_INT4 ? decode_segment_cost_int4() : 0u;

    hipStream_t s = (hipStream_t)desc->stream;
    if (k_new) {
        if (pl.split) {
            p.k_new = (const uint8_t*)k_new;
            p.v_new = (const uint8_t*)v_new;
        } else {
            AppendParams a = {};
            a.k = (uint8_t*)desc->kv.k_data;
            a.v = (uint8_t*)desc->kv.v_data;
            a.ks = desc->kv.k_scales;
            a.vs = desc->kv.v_scales;
            a.block_tables = desc->block_tables;
            a.ctx_lens = desc->ctx_lens;
            a.k_new = (const uint8_t*)k_new;
            a.v_new = (const uint8_t*)v_new;
            a.batch = desc->batch;
            a.n_new = 1;
            a.hkv = desc->kv.num_kv_heads;
            a.head_dim = desc->kv.head_dim;
            a.block_tokens = desc->kv.block_tokens;
            a.max_blocks = desc->max_blocks_per_seq;
            a.num_blocks = desc->kv.num_blocks;
            if (!append_launch("paged_decode_step append launch", &desc->kv, a, src_dtype, s)) return 0;
        }
    }
    if (pl.split) {
        // partial slots [grid][2][GW] of (max, sum) then of acc[D]
        p.part_acc = (float*)ws + (size_t)pl.grid_x * 2 * pl.gw * 2;
    }
    const dim3 grid = pl.split ? dim3(pl.grid_x) : dim3(pl.max_parts, desc->kv.num_kv_heads * pl.gsplit, desc->batch);
    int ok = 0;
    switch (desc->kv.dtype) {
        case VSPEC_KV_F32: ok = dispatch_d<VSPEC_KV_F32>(D, pl.gw, p, grid, s); break;
        case VSPEC_KV_F16: ok = launch_decode_mfma_f16(p, D, pl.gw, grid, s); break;
        default: ok = launch_decode_mfma_int4(p, D, pl.gw, grid, s); break;
    }
    if (!ok) {
        set_err("paged_decode: no kernel for head_dim %u, group %u", D, pl.gw);
        return 0;
    }
    HIP_CHECK(hipGetLastError(), "decode launch");
    if (!pl.split && pl.max_parts > 1) {
        const dim3 cg(desc->num_q_heads, desc->batch);
        if (D == 64) hipLaunchKernelGGL(decode_combine<64>, cg, dim3(64), 0, s, p);
        else hipLaunchKernelGGL(decode_combine<128>, cg, dim3(128), 0, s, p);
        HIP_CHECK(hipGetLastError(), "decode_combine launch");
    }
    return 1;
}

}  // namespace

extern "C" {

int vspec_rocm_paged_decode_attention(const VspecPagedAttnDesc* desc) {
    return paged_decode(desc, nullptr, nullptr, VSPEC_KV_F32, false);
}

static int decode_step(const char* who, const VspecPagedAttnDesc* desc, const void* k_new, const void* v_new,
                       int32_t src_dtype, bool noalloc) {
    const bool empty = desc && desc->batch == 0;  // a no-op, like every other entry point
    if (!empty && (!k_new || !v_new)) {
        set_err("%s: null k_new or v_new", who);
        return 0;
    }
    if (src_dtype != VSPEC_KV_F32 && src_dtype != VSPEC_KV_F16) {
        set_err("%s: src_dtype must be f32 or f16", who);
        return 0;
    }
    return paged_decode(desc, k_new, v_new, src_dtype, noalloc);
}

int vspec_rocm_paged_decode_step(const VspecPagedAttnDesc* desc, const void* k_new, const void* v_new,
                                 int32_t src_dtype) {
    return decode_step("paged_decode_step", desc, k_new, v_new, src_dtype, false);
}

int vspec_rocm_paged_decode_step_noalloc(const VspecPagedAttnDesc* desc, const void* k_new, const void* v_new,
                                         int32_t src_dtype) {
    return decode_step("paged_decode_step_noalloc", desc, k_new, v_new, src_dtype, true);
}

int vspec_rocm_release_retired_workspaces(void) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        set_err("release_retired_workspaces: no current device");
        return 0;
    }
    std::lock_guard<std::mutex> lock(g_ws_mu);
    int ok = 1;
    for (void* ptr : g_retired[dev]) {
        if (hipFree(ptr) != hipSuccess) ok = 0;
    }
    g_retired[dev].clear();
    if (!ok) set_err("release_retired_workspaces: hipFree failed");
    return ok;
}

}  // extern "C"
