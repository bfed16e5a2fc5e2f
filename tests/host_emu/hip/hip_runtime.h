// Host stand-in for <hip/hip_runtime.h>, used only by the CPU emulation of the append
// kernel's per-item code (tests/host_emu/append_emu.cpp): the HIP keywords and vector
// types become plain C++ so that vspec-engine_amd/csrc/append_row.h compiles for the
// host.  Cross-lane operations, barriers and atomics with ordering have no serial
// meaning; the append path of f32/f16 pools (and int4 pools without clamp flags) never
// calls them, and the stand-ins abort if it does.
#pragma once
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#define __device__
#define __host__
#define __global__
#define __shared__ static
#define __forceinline__ inline __attribute__((always_inline))
#define __launch_bounds__(...)

typedef void* hipStream_t;
struct dim3 {
    unsigned x, y, z;
    dim3(unsigned a = 1, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};
struct EmuIdx {
    unsigned x = 0, y = 0, z = 0;
};
inline EmuIdx threadIdx, blockIdx, blockDim, gridDim;

struct uint2 { uint32_t x, y; };
struct uint4 { uint32_t x, y, z, w; };
struct float4 { float x, y, z, w; };
inline uint2 make_uint2(uint32_t a, uint32_t b) { return {a, b}; }
inline uint4 make_uint4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) { return {a, b, c, d}; }
inline float4 make_float4(float a, float b, float c, float d) { return {a, b, c, d}; }

[[noreturn]] inline void emu_unsupported(const char* what) {
    fprintf(stderr, "host emulation: %s has no serial meaning\n", what);
    abort();
}
inline void __syncthreads() { emu_unsupported("__syncthreads"); }
template <class T> T __shfl_xor(T, int, int = 64) { emu_unsupported("__shfl_xor"); }
template <class T> T __shfl_up(T, int, int = 64) { emu_unsupported("__shfl_up"); }
inline uint32_t atomicOr(uint32_t*, uint32_t) { emu_unsupported("atomicOr (int4 clamp flags)"); }
inline uint32_t atomicAnd(uint32_t*, uint32_t) { emu_unsupported("atomicAnd (int4 clamp flags)"); }
// integer min/max of the HIP device library
inline int min(int a, int b) { return a < b ? a : b; }
inline int max(int a, int b) { return a > b ? a : b; }
inline unsigned min(unsigned a, unsigned b) { return a < b ? a : b; }
inline unsigned max(unsigned a, unsigned b) { return a > b ? a : b; }
inline long long min(long long a, long long b) { return a < b ? a : b; }
inline long long max(long long a, long long b) { return a > b ? a : b; }
inline unsigned long long min(unsigned long long a, unsigned long long b) { return a < b ? a : b; }
inline unsigned long long max(unsigned long long a, unsigned long long b) { return a > b ? a : b; }
inline unsigned long min(unsigned long a, unsigned long b) { return a < b ? a : b; }
inline unsigned long max(unsigned long a, unsigned long b) { return a > b ? a : b; }
// lane-exchange builtins named by kv_common.h's reduction helpers (not on the append path)
inline int __builtin_amdgcn_update_dpp(int, int, int, int, int, bool) { emu_unsupported("dpp"); }
inline int __builtin_amdgcn_mov_dpp(int, int, int, int, bool) { emu_unsupported("dpp"); }
inline int __builtin_amdgcn_readfirstlane(int) { emu_unsupported("readfirstlane"); }
inline void __builtin_amdgcn_s_waitcnt(int) { emu_unsupported("s_waitcnt"); }
#define __HIP_MEMORY_SCOPE_WAVEFRONT 1
#define __HIP_MEMORY_SCOPE_WORKGROUP 2
#define __HIP_MEMORY_SCOPE_AGENT 3
#define __HIP_MEMORY_SCOPE_SYSTEM 4
#define __hip_atomic_load(p, order, scope) (*(p))
#define __hip_atomic_store(p, v, order, scope) (*(p) = (v))
