// Shared device helpers for the gfx950 tree-growing kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace yabt {

constexpr int NB = 256;          // histogram width: bins are uint8 (grow_c.py:417)
constexpr int WAVE = 64;         // CDNA wavefront
constexpr int LEAF = -1;         // grow.c:28

// Fixed-point contract shared with oracle/grow_oracle.c (or_quant_shift):
// q = rint(x * 2^s), s = 61 - k - e with max|x| < 2^e, n <= 2^k, so every
// partial sum of <= n quantised values stays below 2^62 in magnitude.
__host__ __device__ inline int quant_shift(float maxabs, int64_t n) {
    if (!(maxabs > 0.0f)) return 0;
    int e = 0;
    (void)frexpf(maxabs, &e);
    int k = 0;
    while (k < 62 && ((int64_t)1 << k) < n) ++k;
    return 61 - k - e;
}

__device__ __forceinline__ int64_t quantise(float x, double scale) {
    return (int64_t)rint((double)x * scale);
}

// Wave-wide exclusive prefix sum of a 64-bit value.
__device__ __forceinline__ int64_t wave_excl_scan(int64_t v, int lane) {
    int64_t incl = v;
#pragma unroll
    for (int d = 1; d < WAVE; d <<= 1) {
        int64_t o = __shfl_up(incl, d, WAVE);
        if (lane >= d) incl += o;
    }
    return incl - v;
}

__device__ __forceinline__ uint32_t wave_excl_scan_u32(uint32_t v, int lane) {
    uint32_t incl = v;
#pragma unroll
    for (int d = 1; d < WAVE; d <<= 1) {
        uint32_t o = __shfl_up(incl, d, WAVE);
        if (lane >= d) incl += o;
    }
    return incl - v;
}

}  // namespace yabt
