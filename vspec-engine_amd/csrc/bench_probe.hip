// bench_probe.hip -- HBM bandwidth probes for bench.py (lib/libvspec_probe.so).
//
// Not part of the paged-KV C-ABI: these kernels give the measured ceilings that the decode
// kernels' bandwidth is reported against, next to the 8 TB/s datasheet peak.
//   vspec_probe_copy        streaming copy, 16 B per lane, non-temporal loads and stores
//                           (bytes moved = 2 x size)
//   vspec_probe_read_tiles  read-only: whole tiles of tile_bytes at the indices of a
//                           device table (a random permutation gives the decode kernels'
//                           access pattern: 4 KB (block, kv head) tiles in random order),
//                           ordinary or non-temporal loads; each thread folds what it read
//                           into one word of `sink` so that no load is dead
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void probe_copy(const u32x4* __restrict__ src, u32x4* __restrict__ dst, size_t n16) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const u32x4 a = __builtin_nontemporal_load(src + i);
        const u32x4 b = __builtin_nontemporal_load(src + i + stride);
        const u32x4 c = __builtin_nontemporal_load(src + i + 2 * stride);
        const u32x4 d = __builtin_nontemporal_load(src + i + 3 * stride);
        __builtin_nontemporal_store(a, dst + i);
        __builtin_nontemporal_store(b, dst + i + stride);
        __builtin_nontemporal_store(c, dst + i + 2 * stride);
        __builtin_nontemporal_store(d, dst + i + 3 * stride);
    }
    for (; i < n16; i += stride) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

// One workgroup reads a whole tile per step (tile_bytes / 16 lanes' worth of 16-byte
// loads, looping over the 256 lanes), UNROLL tiles in flight.
template <bool NT, int UNROLL>
__global__ __launch_bounds__(256) void probe_read_tiles(const uint8_t* __restrict__ base, const int32_t* __restrict__ tiles,
                                                        uint32_t n_tiles, uint32_t tile_bytes, uint32_t* __restrict__ sink) {
    const uint32_t per_tile = tile_bytes / 16u;  // 16-byte chunks
    uint32_t acc = 0;
    for (uint32_t t0 = blockIdx.x * UNROLL; t0 < n_tiles; t0 += gridDim.x * UNROLL) {
        u32x4 w[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) w[u] = u32x4{0u, 0u, 0u, 0u};
        for (uint32_t c = threadIdx.x; c < per_tile; c += blockDim.x) {
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                const uint32_t t = t0 + u;
                if (t < n_tiles) {
                    const u32x4* p = reinterpret_cast<const u32x4*>(base + (size_t)tiles[t] * tile_bytes) + c;
                    const u32x4 x = NT ? __builtin_nontemporal_load(p) : *p;
                    w[u] ^= x;
                }
            }
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) acc ^= w[u][0] ^ w[u][1] ^ w[u][2] ^ w[u][3];
    }
    sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

}  // namespace

extern "C" {

// Copy `bytes` (a multiple of 16) from src to dst on `stream`; returns 1 on launch.
int vspec_probe_copy(const void* src, void* dst, size_t bytes, void* stream) {
    if (!src || !dst || bytes % 16) return 0;
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    hipLaunchKernelGGL(probe_copy, dim3(8 * cus), dim3(256), 0, (hipStream_t)stream, (const u32x4*)src, (u32x4*)dst,
                       bytes / 16);
    return hipGetLastError() == hipSuccess;
}

// Read n_tiles tiles of tile_bytes (a multiple of 16) at base + tiles[i] * tile_bytes.
// sink: device, at least sink_words() = grid * 256 words.  nontemporal: 0 or 1.
uint32_t vspec_probe_read_tiles_grid(void) {
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    return 8u * (uint32_t)cus;
}

int vspec_probe_read_tiles(const void* base, const int32_t* tiles, uint32_t n_tiles, uint32_t tile_bytes,
                           uint32_t* sink, int nontemporal, void* stream) {
    if (!base || !tiles || !sink || tile_bytes == 0 || tile_bytes % 16) return 0;
    const dim3 grid(vspec_probe_read_tiles_grid());
    if (nontemporal)
        hipLaunchKernelGGL((probe_read_tiles<true, 4>), grid, dim3(256), 0, (hipStream_t)stream, (const uint8_t*)base,
                           tiles, n_tiles, tile_bytes, sink);
    else
        hipLaunchKernelGGL((probe_read_tiles<false, 4>), grid, dim3(256), 0, (hipStream_t)stream, (const uint8_t*)base,
                           tiles, n_tiles, tile_bytes, sink);
    return hipGetLastError() == hipSuccess;
}

}  // extern "C"
