// decode_mfma.hip -- single-query GQA decode attention over f16 paged KV, with the
// two contractions on the matrix cores (gfx950 MFMA) and the reference numerics
// (per-key std clamp, attention_ref.c:50-62) on the vector ALUs.
//
// Per wave and 16-token tile of one kv head:
//   S^T[16 tok][16 col] = K[16 tok][D] x Q'^T      v_mfma_f32_16x16x32_f16, A = K rows as
//                                                   loaded, B = q' split in fp16 hi + lo
//                                                   (two MFMAs per 32-wide d chunk)
//   O^T[d][16 col]     += V^T[d][16 tok] x P^T     v_mfma_f32_16x16x16f16, A = V^T rows
//                                                   (V is stored d-major per tile), B = p
//                                                   hi + lo taken straight from the S^T
//                                                   accumulator registers
// Columns 0..GW-1 are the GQA query heads that share the tile; the rest stay zero.
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
__device__ __forceinline__ h4_t as_h4(uint2 w) { return __builtin_bit_cast(h4_t, w); }
__device__ __forceinline__ h2_t as_h2(uint32_t w) { return __builtin_bit_cast(h2_t, w); }

template <int D>
struct Frags {
    uint4 k[D / 32];  // K row of token n, d = 32i + 8g .. +7
    uint2 v[D / 16];  // V^T row d = 16j + n, slots 4g .. 4g+3 of the tile
};

// PB: block_tokens known at compile time (16), or 0 for any multiple of 16
template <int D, int GW, int PB>
__global__ __launch_bounds__(256, 2) void decode_mfma_f16(DecodeParams p) {
    constexpr int NQK = D / 32;  // QK MFMAs per tile (each on 32 d)
    constexpr int NDT = D / 16;  // PV d-tiles
    __shared__ float qs[GW][D];
    // QK B operands per lane (hi, lo for each 32-wide d chunk), read back every tile
    __shared__ uint4 qb_lds[NQK][2][64];
    __shared__ float comb[kWaves][GW][D + 2];
    __shared__ float patch_val[kWaves][kTile][4];
    __shared__ int patch_flag[kWaves][kTile];

    const int lane = threadIdx.x & 63;
    // wave index as a scalar: tile loop control and block-table reads stay on the
    // scalar unit (s_load), so they never wait behind the vector K/V loads
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4;   // row group
    const int n = lane & 15;   // column / token within the tile
    const int part = blockIdx.x;
    const int b = blockIdx.z;
    const int hk = blockIdx.y / p.gsplit;
    const int hq0 = hk * (p.gsplit * GW) + (blockIdx.y % p.gsplit) * GW;

    const int ctx = min(max(p.ctx_lens[b], 0), (int)(p.max_blocks * p.block_tokens));
    const int ntiles = min((ctx + kTile - 1) / kTile, (int)(p.max_parts * p.tiles_per_part));
    const int nparts = max(1, (ntiles + (int)p.tiles_per_part - 1) / (int)p.tiles_per_part);
    if (part >= nparts) return;
    const int tile_begin = part * (int)p.tiles_per_part;
    const int tile_end = min(ntiles, tile_begin + (int)p.tiles_per_part);

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

    // B operands of the QK MFMAs: column n < GW holds head n, split hi + lo
    if (wave == 0) {
#pragma unroll
        for (int i = 0; i < NQK; ++i) {
            h8_t hi8, lo8;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float qv = n < GW ? qs[n < GW ? n : 0][32 * i + 8 * g + j] : 0.f;
                const _Float16 hi = (_Float16)qv;
                hi8[j] = hi;
                lo8[j] = (_Float16)(qv - (float)hi);
            }
            qb_lds[i][0][lane] = __builtin_bit_cast(uint4, hi8);
            qb_lds[i][1][lane] = __builtin_bit_cast(uint4, lo8);
        }
    }
    __syncthreads();

    const int P = PB ? PB : (int)p.block_tokens;
    const int tiles_per_block = P / kTile;
    const int32_t* table = p.block_tables + (size_t)b * p.max_blocks;
    const _Float16* kbase = reinterpret_cast<const _Float16*>(p.k);
    const _Float16* vbase = reinterpret_cast<const _Float16*>(p.v);

    auto load = [&](int tile, Frags<D>& f) -> bool {
        const int phys = table[tile / tiles_per_block];
        if (phys < 0 || (uint32_t)phys >= p.num_blocks) return false;
        const size_t tidx = (size_t)phys * p.hkv + hk;
        const int slot0 = (tile % tiles_per_block) * kTile;
        const uint4* kr = reinterpret_cast<const uint4*>(kbase + (tidx * P + slot0 + n) * D + 8 * g);
#pragma unroll
        for (int i = 0; i < NQK; ++i) f.k[i] = kr[4 * i];
        const _Float16* vt = vbase + tidx * (size_t)D * P + slot0 + 4 * g;
#pragma unroll
        for (int j = 0; j < NDT; ++j) f.v[j] = *reinterpret_cast<const uint2*>(vt + (size_t)(16 * j + n) * P);
        return true;
    };

    f4_t acc[NDT];
#pragma unroll
    for (int j = 0; j < NDT; ++j) acc[j] = f4_t{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY;  // running max of head n (log2 units), per lane
    float l_run = 0.f;        // running sum of p for head n over this lane's tokens
    const h2_t ones = {(_Float16)1.0f, (_Float16)1.0f};

    // one 16-token tile: clamp screen, scores, online softmax, P.V
    auto process = [&](Frags<D>& f, const int tile) {
        const int tok0 = tile * kTile;
        const int nvalid = min(kTile, ctx - tok0);

        // ---- clamp screen for key n (this lane holds 8*NQK of its elements) ----
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
        float mx = fmaxf((float)mx2[0], (float)mx2[1]);
        s1 += __shfl_xor(s1, 16);
        s1 += __shfl_xor(s1, 32);
        s2 += __shfl_xor(s2, 16);
        s2 += __shfl_xor(s2, 32);
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mean = s1 * (1.0f / D);
        const float ex2 = s2 * (1.0f / D);
        const float var1 = ex2 - mean * mean;
        const float th1 = fminf(fmaxf(1e-6f, p.alpha * sqrtf(fmaxf(var1, 0.f))), p.input_clip);
        // a margin of 2^-10 covers the one-pass variance error; ill-conditioned rows
        // (variance tiny against the mean square) always take the exact path
        const bool flag = (n < nvalid) && (mx > th1 * (1.0f - 0.0009765625f) || var1 <= ex2 * 0.0009765625f);

        // ---- scores: S^T = K Q'^T (hi and lo accumulate into one column) ----
        f4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < NQK; ++i) {
            sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(f.k[i]), as_h8(qb_lds[i][0][lane]), sc, 0, 0, 0);
            sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(f.k[i]), as_h8(qb_lds[i][1][lane]), sc, 0, 0, 0);
        }

        // ---- exact scores for keys the clamp may change ----
        if (__builtin_amdgcn_ballot_w64(flag) != 0) {
            float part[GW];
            float v2 = 0.f;
#pragma unroll
            for (int i = 0; i < NQK; ++i) {
                const uint32_t w4[4] = {f.k[i].x, f.k[i].y, f.k[i].z, f.k[i].w};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float x = half_bits_to_float((w4[e / 2] >> (16 * (e % 2))) & 0xffffu);
                    v2 = fmaf(x - mean, x - mean, v2);
                }
            }
            v2 += __shfl_xor(v2, 16);
            v2 += __shfl_xor(v2, 32);
            const float th = fminf(fmaxf(1e-6f, p.alpha * sqrtf(v2 * (1.0f / D))), p.input_clip);
#pragma unroll
            for (int h = 0; h < GW; ++h) {
                float a = 0.f;
#pragma unroll
                for (int i = 0; i < NQK; ++i) {
                    const uint32_t w4[4] = {f.k[i].x, f.k[i].y, f.k[i].z, f.k[i].w};
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float x = half_bits_to_float((w4[e / 2] >> (16 * (e % 2))) & 0xffffu);
                        a = fmaf(qs[h][32 * i + 8 * g + e], fminf(fmaxf(x, -th), th), a);
                    }
                }
                a += __shfl_xor(a, 16);
                a += __shfl_xor(a, 32);
                part[h] = a;
            }
            if (g == 0) {
                patch_flag[wave][n] = flag ? 1 : 0;
#pragma unroll
                for (int h = 0; h < GW; ++h) patch_val[wave][n][h] = part[h];
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            if (n < GW) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int t = 4 * g + r;
                    if (patch_flag[wave][t]) sc[r] = patch_val[wave][t][n];
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
        }

        // ---- online softmax for head n over tokens 4g..4g+3 ----
        float s[4];
        float mt = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float v = fminf(fmaxf(sc[r], -p.logit_clip), p.logit_clip);
            s[r] = (n < GW && 4 * g + r < nvalid) ? v : -INFINITY;
            mt = fmaxf(mt, s[r]);
        }
        mt = fmaxf(mt, __shfl_xor(mt, 16));
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const bool need = mt > m_run + 8.0f;
        if (__builtin_amdgcn_ballot_w64(need) != 0) {
            const float f = need ? exp2f(m_run - mt) : 1.0f;
            m_run = need ? mt : m_run;
            l_run *= f;
#pragma unroll
            for (int j = 0; j < NDT; ++j) acc[j] *= f;
        }
        float pr[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            pr[r] = s[r] == -INFINITY ? 0.f : exp2f(s[r] - m_run);  // masked / unused -> 0
            l_run += pr[r];
        }
        h4_t phi, plo;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const _Float16 hi = (_Float16)pr[r];
            phi[r] = hi;
            plo[r] = (_Float16)(pr[r] - (float)hi);
        }

        // ---- O^T += V^T P^T ----
        if (nvalid < kTile) {
            // slots past the context may hold any bits (NaN): zero them
#pragma unroll
            for (int j = 0; j < NDT; ++j) {
                h4_t vv = as_h4(f.v[j]);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (4 * g + r >= nvalid) vv[r] = (_Float16)0.f;
                }
                f.v[j] = __builtin_bit_cast(uint2, vv);
            }
        }
#pragma unroll
        for (int j = 0; j < NDT; ++j) {
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(as_h4(f.v[j]), phi, acc[j], 0, 0, 0);
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(as_h4(f.v[j]), plo, acc[j], 0, 0, 0);
        }
    };

    // two tiles in flight per wave: buffers A and B alternate, so a tile's loads are
    // issued two tiles before it is processed and no registers are copied
    Frags<D> fa, fb;
    int tile = tile_begin + wave;
    bool oka = tile < tile_end ? load(tile, fa) : false;
    bool okb = tile + kWaves < tile_end ? load(tile + kWaves, fb) : false;
    for (; tile < tile_end; tile += 2 * kWaves) {
        if (oka) process(fa, tile);
        oka = tile + 2 * kWaves < tile_end ? load(tile + 2 * kWaves, fa) : false;
        if (tile + kWaves >= tile_end) break;
        if (okb) process(fb, tile + kWaves);
        okb = tile + 3 * kWaves < tile_end ? load(tile + 3 * kWaves, fb) : false;
    }

    // ---- wave result: column n < GW holds head n; lane (g, n) has d = 16j + 4g + r ----
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);
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

template <int D, int GW>
void launch(const DecodeParams& p, dim3 grid, hipStream_t s) {
    if (p.block_tokens == 16) {
        hipLaunchKernelGGL((decode_mfma_f16<D, GW, 16>), grid, dim3(256), 0, s, p);
    } else {
        hipLaunchKernelGGL((decode_mfma_f16<D, GW, 0>), grid, dim3(256), 0, s, p);
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
