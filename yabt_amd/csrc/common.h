// Shared device helpers for the gfx950 tree-growing kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <climits>
#include <type_traits>

namespace yabt {

constexpr int NB = 256;   // histogram width: bins are uint8 (grow_c.py:417)
constexpr int WAVE = 64;  // CDNA wavefront
constexpr int LEAF = -1;  // grow.c:28

// ---------------------------------------------------------------------------
// fixed-point quantisation, shared with oracle/grow_oracle.c (or_quant_shift):
// q = rint(x * 2^s), s = 61 - k - e with max|x| < 2^e and n <= 2^k, so every
// partial sum of <= n quantised values stays below 2^62 in magnitude (the
// K-slot histogram and the leaf-model sums).
// ---------------------------------------------------------------------------

__host__ __device__ inline int quant_shift(float maxabs, int64_t n) {
    if (!(maxabs > 0.0f)) return 0;
    int e = 0;
    (void)frexpf(maxabs, &e);
    int k = 0;
    while (k < 62 && ((int64_t)1 << k) < n) ++k;
    return 61 - k - e;
}

// Node histograms use one of two contracts, chosen per call from the data
// (quant_resid, quant_finish):
//   narrow: s = 30 - min(k, 11) - e, so |q| <= 2^(30 - min(k, 11)) and any
//     min(n, 2048) values sum within 2^30 < 2^31: the streaming root kernel
//     adds the word (q(g) << 32) + q(h) into one 64-bit LDS cell per update
//     and unpacks the two 32-bit halves after every epoch.  q keeps 19 bits
//     of the largest |x| for n > 2048 (more below), and every partial sum of
//     <= n values stays below 2^51;
//   wide: s = 61 - max(k, 21) - e, so |q| <= 2^(61 - max(k, 21)) (37 bits of
//     the largest |x| at 10M rows, 40 at <= 2M) and every partial sum of
//     <= n values stays below 2^61; g and h take a 64-bit LDS cell each.
// The narrow contract is used only when its quantisation residual is small
// against the data: per channel, R = sum rint(|x 2^s - rint(x 2^s)| 2^21)
// and M = sum rint(|x| 2^(s + 1)) at the narrow shift s (exact integers,
// so the decision does not depend on any order), narrow iff R <= 8 M for
// both g and h, i.e. sum |x - q 2^-s| <= 2^-17 sum |x| up to the rounding of
// the two integer sums (M counts half quanta, so it errs towards wide).  One large value among small ones (an outlier,
// heavy-tailed targets) makes q coarse against most rows and selects wide.
// Shared with oracle/grow_oracle.c (or_hist_shift, or_wide_shift,
// or_hist_contract).
__host__ __device__ inline int ceil_log2_rows(int64_t n, int cap) {
    int k = 0;
    while (k < cap && ((int64_t)1 << k) < n) ++k;
    return k;
}

__host__ __device__ inline int hist_shift(float maxabs, int64_t n) {
    if (!(maxabs > 0.0f)) return 0;
    int e = 0;
    (void)frexpf(maxabs, &e);
    return 30 - ceil_log2_rows(n, 11) - e;
}

constexpr int WIDE_MIN_K = 21;   // the wide shift counts n as at least 2^21 rows

__host__ __device__ inline int wide_shift(float maxabs, int64_t n) {
    if (!(maxabs > 0.0f)) return 0;
    int e = 0;
    (void)frexpf(maxabs, &e);
    const int k = ceil_log2_rows(n, 62);
    return 61 - (k > WIDE_MIN_K ? k : WIDE_MIN_K) - e;
}

// log2 of the packing window of the gathered histograms (see
// hist_gather_rows: the count rides in the low cb = w + 1 bits of a 64-bit
// word, (q << cb) + 1 per row, unpacked every 2^w rows).  Narrow: |q| <= 2^19
// (2^30 for tiny n, whose windows never fill), w = 16: a window's sum stays
// below 2^35 << cb < 2^63.  Wide: |q| <= 2^(61 - K), K = max(k, 21),
// w = K / 2: a window's sum times 2^cb is at most 2^(62 - K + 2w) <= 2^62.
// Both are at least 10 (one block step of 1024 rows).
constexpr int NARROW_WINDOW_LOG2 = 16;
__host__ __device__ inline int wide_window_log2(int64_t n) {
    const int k = ceil_log2_rows(n, 62);
    return (k > WIDE_MIN_K ? k : WIDE_MIN_K) / 2;
}
__host__ __device__ inline int window_log2(int64_t n, bool wide) {
    return wide ? wide_window_log2(n) : NARROW_WINDOW_LOG2;
}

__device__ __forceinline__ int64_t quantise(float x, double scale) {
    return (int64_t)rint((double)x * scale);
}

// quantise for the node histograms, whose shift keeps |x * 2^s| <= 2^30
// (hist_shift): evaluated in fp32 -- the scaling by a power of two is exact
// while the result is a normal float, anything smaller rounds to 0 either
// way, and rounding to an integer is exact -- so it equals quantise, in
// three VALU operations instead of eight.  `scale` is 2^s.
__device__ __forceinline__ int64_t quantise_node(float x, double scale) {
    return (int64_t)(int32_t)rintf(ldexpf(x, ilogb(scale)));
}

// quantise for either contract: the same fp32 steps, converted to 64 bits
// (the wide shift's |x * 2^s| reaches 2^40); equal to quantise_node wherever
// that one applies.
__device__ __forceinline__ int64_t quantise_wide(float x, double scale) {
    return (int64_t)rintf(ldexpf(x, ilogb(scale)));
}

// Per-call quantisation record, filled on the device.
struct Quant {
    int32_t sg, sh;            // shifts
    double scg, sch;           // 2^sg, 2^sh
    double ig, ih;             // 2^-sg, 2^-sh
    uint32_t maxg_bits;        // max |g| (float bits; non-negative floats order like uints)
    uint32_t maxh_bits;        // max |h|
    uint32_t hmin_key;         // order-preserving key of min h
    uint32_t hmax_key;         // order-preserving key of max h
    int32_t nonfinite;         // any g or h is inf/nan
    int32_t const_h;           // every h equal and nonzero: sum q(h) = count * hq_const
    int64_t hq_const;
    int64_t tot_g, tot_h;      // sum of q(g), q(h) over all rows (root totals)
    uint32_t ticket;
    int32_t wide;              // 1: the wide contract (hist_shift's notes)
    int32_t wlog;              // the gathers' packing window, window_log2(n, wide)
    int32_t pad2;
    uint64_t res_g, res_h;     // quantisation residuals at the narrow shift (quant_resid)
    uint64_t mass_g, mass_h;   // and the masses they are measured against
};

__device__ __forceinline__ uint32_t float_key(float x) {
    const uint32_t b = __float_as_uint(x);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// ---------------------------------------------------------------------------
// cross-lane helpers
// ---------------------------------------------------------------------------

// Broadcast lane J of every 16-lane row to the whole row (DPP row_newbcast;
// every lane has a source, so no old value is needed).
template <int J>
__device__ __forceinline__ uint32_t row_bcast32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x150 + J, 0xf, 0xf, false);
}

// 64-bit form: one v_mov_b64_dpp (row_newbcast is a 64-bit DPP control on
// this target).
template <int J>
__device__ __forceinline__ uint64_t row_bcast64(uint64_t v) {
    return (uint64_t)__builtin_amdgcn_mov_dpp((long)v, 0x150 + J, 0xf, 0xf, false);
}

// DPP move within 16-lane rows; lanes whose source is outside the row read 0.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, true);
}

template <int CTRL>
__device__ __forceinline__ uint64_t dpp64(uint64_t v) {
    return ((uint64_t)dpp32<CTRL>((uint32_t)(v >> 32)) << 32) | dpp32<CTRL>((uint32_t)v);
}

template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
    return __longlong_as_double((long long)dpp64<CTRL>((uint64_t)__double_as_longlong(v)));
}

// Buffer resource over `bytes` bytes at p (raw, untyped): a load at an offset
// past the end returns zeros instead of faulting.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// Number of set bits of mask in the lanes below this one.
__device__ __forceinline__ uint32_t lane_prefix(uint64_t mask) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

constexpr int DPP_ROW_SHR = 0x110;    // row_shr:n   = 0x110 + n
constexpr int DPP_ROW_ROR = 0x120;    // row_ror:n   = 0x120 + n (rotate inside the row)

__device__ __forceinline__ int64_t readlane64(int64_t v, int lane) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), lane);
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ double readlane_f64(double v, int lane) {
    return __longlong_as_double(readlane64(__double_as_longlong(v), lane));
}

// Inclusive prefix sum over the 64 lanes: DPP shifts inside each 16-lane row,
// then the three lower row totals (read into scalars) are added per row.
__device__ __forceinline__ int64_t wave_incl_scan_i64(int64_t v, int lane) {
    uint64_t u = (uint64_t)v;
    u += dpp64<DPP_ROW_SHR + 1>(u);
    u += dpp64<DPP_ROW_SHR + 2>(u);
    u += dpp64<DPP_ROW_SHR + 4>(u);
    u += dpp64<DPP_ROW_SHR + 8>(u);
    const int64_t t0 = readlane64((int64_t)u, 15), t1 = readlane64((int64_t)u, 31), t2 = readlane64((int64_t)u, 47);
    const int64_t off = (lane >= 16 ? t0 : 0) + (lane >= 32 ? t1 : 0) + (lane >= 48 ? t2 : 0);
    return (int64_t)u + off;
}

// Sum over the 64 lanes, returned in every lane (row rotations 8, 4, 2, 1
// leave each row's total in all of its lanes).
__device__ __forceinline__ int64_t wave_sum_i64(int64_t v) {
    uint64_t u = (uint64_t)v;
    u += dpp64<DPP_ROW_ROR + 8>(u);
    u += dpp64<DPP_ROW_ROR + 4>(u);
    u += dpp64<DPP_ROW_ROR + 2>(u);
    u += dpp64<DPP_ROW_ROR + 1>(u);
    return readlane64((int64_t)u, 0) + readlane64((int64_t)u, 16) + readlane64((int64_t)u, 32) +
           readlane64((int64_t)u, 48);
}

__device__ __forceinline__ int32_t wave_sum_i32(int32_t v) {
    v += (int32_t)dpp32<DPP_ROW_ROR + 8>((uint32_t)v);
    v += (int32_t)dpp32<DPP_ROW_ROR + 4>((uint32_t)v);
    v += (int32_t)dpp32<DPP_ROW_ROR + 2>((uint32_t)v);
    v += (int32_t)dpp32<DPP_ROW_ROR + 1>((uint32_t)v);
    return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) + __builtin_amdgcn_readlane(v, 32) +
           __builtin_amdgcn_readlane(v, 48);
}

// Inclusive prefix sum over the 64 lanes of a 32-bit integer (as the 64-bit
// one above).
__device__ __forceinline__ int32_t wave_incl_scan_i32(int32_t v, int lane) {
    uint32_t u = (uint32_t)v;
    u += dpp32<DPP_ROW_SHR + 1>(u);
    u += dpp32<DPP_ROW_SHR + 2>(u);
    u += dpp32<DPP_ROW_SHR + 4>(u);
    u += dpp32<DPP_ROW_SHR + 8>(u);
    const int32_t t0 = __builtin_amdgcn_readlane((int)u, 15), t1 = __builtin_amdgcn_readlane((int)u, 31),
                  t2 = __builtin_amdgcn_readlane((int)u, 47);
    return (int32_t)u + (lane >= 16 ? t0 : 0) + (lane >= 32 ? t1 : 0) + (lane >= 48 ? t2 : 0);
}

// Maximum / minimum over the 64 lanes, returned in every lane (row rotations
// leave each row's result in all of its lanes, then the four rows combine).
__device__ __forceinline__ float wave_max_f32(float v) {
    v = fmaxf(v, __uint_as_float(dpp32<DPP_ROW_ROR + 8>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(dpp32<DPP_ROW_ROR + 4>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(dpp32<DPP_ROW_ROR + 2>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(dpp32<DPP_ROW_ROR + 1>(__float_as_uint(v))));
    const int b = __float_as_int(v);
    return fmaxf(fmaxf(__int_as_float(__builtin_amdgcn_readlane(b, 0)), __int_as_float(__builtin_amdgcn_readlane(b, 16))),
                 fmaxf(__int_as_float(__builtin_amdgcn_readlane(b, 32)), __int_as_float(__builtin_amdgcn_readlane(b, 48))));
}

// Maximum of an unsigned 64-bit value over the 64 lanes, in every lane.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    uint64_t o = dpp64<DPP_ROW_ROR + 8>(v);
    v = o > v ? o : v;
    o = dpp64<DPP_ROW_ROR + 4>(v);
    v = o > v ? o : v;
    o = dpp64<DPP_ROW_ROR + 2>(v);
    v = o > v ? o : v;
    o = dpp64<DPP_ROW_ROR + 1>(v);
    v = o > v ? o : v;
    const uint64_t a = (uint64_t)readlane64((int64_t)v, 0), b = (uint64_t)readlane64((int64_t)v, 16);
    const uint64_t c = (uint64_t)readlane64((int64_t)v, 32), d = (uint64_t)readlane64((int64_t)v, 48);
    const uint64_t ab = a > b ? a : b, cd = c > d ? c : d;
    return ab > cd ? ab : cd;
}

// wave_max_u64 without scalar registers: row rotations give each 16-lane
// row its maximum, then gfx950's row and half swaps (v_permlane16_swap,
// v_permlane32_swap) put each lane's partner row, then partner half, beside
// it; whichever way a swap moves the data, a lane's two results are its own
// value and its partner's.
__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint64_t wave_max_u64_v(uint64_t v) {
    v = max_u64(v, dpp64<DPP_ROW_ROR + 8>(v));
    v = max_u64(v, dpp64<DPP_ROW_ROR + 4>(v));
    v = max_u64(v, dpp64<DPP_ROW_ROR + 2>(v));
    v = max_u64(v, dpp64<DPP_ROW_ROR + 1>(v));
    uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
    const auto l16 = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    const auto h16 = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    v = max_u64(((uint64_t)h16[0] << 32) | l16[0], ((uint64_t)h16[1] << 32) | l16[1]);
    lo = (uint32_t)v;
    hi = (uint32_t)(v >> 32);
    const auto l32 = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
    const auto h32 = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
    return max_u64(((uint64_t)h32[0] << 32) | l32[0], ((uint64_t)h32[1] << 32) | l32[1]);
}

// The same for an unsigned 32-bit value (each step one DPP-fused max).
__device__ __forceinline__ uint32_t wave_max_u32_v(uint32_t v) {
    v = max(v, dpp32<DPP_ROW_ROR + 8>(v));
    v = max(v, dpp32<DPP_ROW_ROR + 4>(v));
    v = max(v, dpp32<DPP_ROW_ROR + 2>(v));
    v = max(v, dpp32<DPP_ROW_ROR + 1>(v));
    const auto s16 = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = max((uint32_t)s16[0], (uint32_t)s16[1]);
    const auto s32 = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return max((uint32_t)s32[0], (uint32_t)s32[1]);
}

__device__ __forceinline__ int wave_min_i32(int v) {
    v = min(v, (int)dpp32<DPP_ROW_ROR + 8>((uint32_t)v));
    v = min(v, (int)dpp32<DPP_ROW_ROR + 4>((uint32_t)v));
    v = min(v, (int)dpp32<DPP_ROW_ROR + 2>((uint32_t)v));
    v = min(v, (int)dpp32<DPP_ROW_ROR + 1>((uint32_t)v));
    return min(min(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
               min(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

// Wave-wide exclusive prefix sum.
template <typename T>
__device__ __forceinline__ T wave_excl_scan(T v, int lane) {
    T incl = v;
#pragma unroll
    for (int d = 1; d < WAVE; d <<= 1) {
        T o = __shfl_up(incl, d, WAVE);
        if (lane >= d) incl += o;
    }
    return incl - v;
}

// Sum over the wave: DPP for integers (exact in any order), a butterfly of
// shuffles for floating point (its fixed order).
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
    if constexpr (std::is_integral<T>::value && sizeof(T) == 4) {
        return (T)wave_sum_i32((int32_t)v);
    } else if constexpr (std::is_integral<T>::value && sizeof(T) == 8) {
        return (T)wave_sum_i64((int64_t)v);
    } else {
#pragma unroll
        for (int d = WAVE / 2; d > 0; d >>= 1) v += __shfl_xor(v, d, WAVE);
        return v;
    }
}

// Block-wide exclusive scan of one value per thread (NT threads).
template <int NT, typename T>
__device__ __forceinline__ T block_excl_scan(T v, T* s_wave, T* total) {
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    const T ex = wave_excl_scan<T>(v, lane);
    if (lane == WAVE - 1) s_wave[w] = ex + v;
    __syncthreads();
    T off = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < NT / WAVE; ++i) {
        if (i < w) off += s_wave[i];
        tot += s_wave[i];
    }
    __syncthreads();
    *total = tot;
    return off + ex;
}

template <int NT, typename T>
__device__ __forceinline__ T block_sum(T v, T* s_red) {
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    v = wave_sum<T>(v);
    if (lane == 0) s_red[w] = v;
    __syncthreads();
    T t = 0;
#pragma unroll
    for (int i = 0; i < NT / WAVE; ++i) t += s_red[i];
    __syncthreads();
    return t;
}

// (key, idx) beats (k2, i2) iff key > k2, or equal keys and idx < i2.
__device__ __forceinline__ bool better(double k1, int i1, double k2, int i2) {
    return k1 > k2 || (k1 == k2 && i1 < i2);
}

// Block argmax (NT threads); invalid candidates carry idx = INT_MAX.
template <int NT>
__device__ void block_argmax(double& key, int& idx, double* s_key, int* s_idx) {
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
#pragma unroll
    for (int d = WAVE / 2; d > 0; d >>= 1) {
        const double ok = __shfl_xor(key, d, WAVE);
        const int oi = __shfl_xor(idx, d, WAVE);
        if (better(ok, oi, key, idx)) {
            key = ok;
            idx = oi;
        }
    }
    if (lane == 0) {
        s_key[w] = key;
        s_idx[w] = idx;
    }
    __syncthreads();
    key = s_key[0];
    idx = s_idx[0];
#pragma unroll
    for (int i = 1; i < NT / WAVE; ++i)
        if (better(s_key[i], s_idx[i], key, idx)) {
            key = s_key[i];
            idx = s_idx[i];
        }
    __syncthreads();
}

// Last-block-done: true in exactly one block, after every block of the grid
// has reached this point; that block then sees all their global writes.
__device__ inline bool last_block(uint32_t* ticket) {
    __shared__ int s_last;
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t t = atomicAdd(ticket, 1u);
        s_last = (t == gridDim.x * gridDim.y - 1);
    }
    __syncthreads();
    if (s_last) {
        __threadfence();
        if (threadIdx.x == 0) *ticket = 0;
    }
    return s_last != 0;
}

// last_block for grids in which only wave 0 of each block has written global
// memory before the call: that wave alone releases its writes (an agent-scope
// fence costs ~14 ns per fencing wave and the fences of a grid serialise, so
// fencing every wave of 256 1024-thread blocks costs ~60 us); the last block
// then acquires with every wave.
__device__ inline bool last_block_w0(uint32_t* ticket) {
    __shared__ int s_last;
    if (threadIdx.x < WAVE) {
        __threadfence();
        if (threadIdx.x == 0) {
            const uint32_t t = atomicAdd(ticket, 1u);
            s_last = (t == gridDim.x * gridDim.y - 1);
        }
    }
    __syncthreads();
    if (s_last) {
        __threadfence();
        if (threadIdx.x == 0) *ticket = 0;
    }
    return s_last != 0;
}

// ---------------------------------------------------------------------------
// quantisation passes
// ---------------------------------------------------------------------------

// Grid-stride max|g|, max|h|, min/max h and finiteness into q (NT threads);
// with gh, also the interleaved copy gh[i] = (grad[i], hess[i]).
template <int NT>
__device__ void quant_reduce(const float* grad, const float* hess, int64_t n, Quant* q, float2* gh = nullptr) {
    __shared__ float s_m[2][NT / WAVE];
    __shared__ uint32_t s_k[2][NT / WAVE];
    __shared__ int s_nf;
    if (threadIdx.x == 0) s_nf = 0;
    __syncthreads();
    float mg = 0.0f, mh = 0.0f;
    uint32_t kmin = 0xffffffffu, kmax = 0u;
    int nf = 0;
    auto take = [&](float a, float c) {
        if (!isfinite(a) || !isfinite(c)) nf = 1;
        mg = fmaxf(mg, fabsf(a));
        mh = fmaxf(mh, fabsf(c));
        const uint32_t kc = float_key(c);
        kmin = min(kmin, kc);
        kmax = max(kmax, kc);
    };
    const int64_t tid = (int64_t)blockIdx.x * NT + threadIdx.x, nth = (int64_t)gridDim.x * NT;
    int64_t head = 0;   // rows [0, head) taken by the vector loop
    if (((reinterpret_cast<uintptr_t>(grad) | reinterpret_cast<uintptr_t>(hess)) & 15) == 0) {
        // 16-byte loads, four of g and four of h in flight per thread (the
        // scalar loop kept one of each: ~1 TB/s); max, min and the finite
        // test do not depend on the order
        constexpr int U = 4;
        const int64_t n4 = n / 4;
        const float4* g4 = reinterpret_cast<const float4*>(grad);
        const float4* h4 = reinterpret_cast<const float4*>(hess);
        int64_t i = tid;
        for (; i + (U - 1) * nth < n4; i += U * nth) {
            float4 a[U], c[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                a[u] = g4[i + u * nth];
                c[u] = h4[i + u * nth];
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                take(a[u].x, c[u].x);
                take(a[u].y, c[u].y);
                take(a[u].z, c[u].z);
                take(a[u].w, c[u].w);
                if (gh) {
                    float4* o = reinterpret_cast<float4*>(gh + 4 * (i + u * nth));
                    o[0] = make_float4(a[u].x, c[u].x, a[u].y, c[u].y);
                    o[1] = make_float4(a[u].z, c[u].z, a[u].w, c[u].w);
                }
            }
        }
        for (; i < n4; i += nth) {
            const float4 a = g4[i], c = h4[i];
            take(a.x, c.x);
            take(a.y, c.y);
            take(a.z, c.z);
            take(a.w, c.w);
            if (gh) {
                float4* o = reinterpret_cast<float4*>(gh + 4 * i);
                o[0] = make_float4(a.x, c.x, a.y, c.y);
                o[1] = make_float4(a.z, c.z, a.w, c.w);
            }
        }
        head = n4 * 4;
    }
    for (int64_t i = head + tid; i < n; i += nth) {
        take(grad[i], hess[i]);
        if (gh) gh[i] = make_float2(grad[i], hess[i]);
    }
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
#pragma unroll
    for (int d = WAVE / 2; d > 0; d >>= 1) {
        mg = fmaxf(mg, __shfl_xor(mg, d, WAVE));
        mh = fmaxf(mh, __shfl_xor(mh, d, WAVE));
        kmin = min(kmin, (uint32_t)__shfl_xor(kmin, d, WAVE));
        kmax = max(kmax, (uint32_t)__shfl_xor(kmax, d, WAVE));
    }
    if (nf) atomicOr(&s_nf, 1);
    if (lane == 0) {
        s_m[0][w] = mg;
        s_m[1][w] = mh;
        s_k[0][w] = kmin;
        s_k[1][w] = kmax;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < NT / WAVE; ++i) {
            mg = fmaxf(mg, s_m[0][i]);
            mh = fmaxf(mh, s_m[1][i]);
            kmin = min(kmin, s_k[0][i]);
            kmax = max(kmax, s_k[1][i]);
        }
        // The words only move one way, so a block whose value does not beat
        // what a word already holds skips its atomic: most blocks do, and
        // the atomics of a thousand blocks on four words serialise.
        auto seen = [](uint32_t* w) { return __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
        if (__float_as_uint(mg) > seen(&q->maxg_bits)) atomicMax(&q->maxg_bits, __float_as_uint(mg));
        if (__float_as_uint(mh) > seen(&q->maxh_bits)) atomicMax(&q->maxh_bits, __float_as_uint(mh));
        if (kmin < seen(&q->hmin_key)) atomicMin(&q->hmin_key, kmin);
        if (kmax > seen(&q->hmax_key)) atomicMax(&q->hmax_key, kmax);
        if (s_nf) atomicOr(&q->nonfinite, 1);
    }
}

// Residual and mass of one value at the narrow shift s (hist_shift's notes):
// x 2^s and its distance to the nearest integer are exact in fp32, and so are
// the power-of-two scalings; rint(|d| 2^21) <= 2^20 and rint(|x| 2^(s + 1))
// <= 2^31 (|x 2^s| <= 2^30), so both convert to 32 bits exactly.  Non-finite
// values add nothing (the call reports them and stops); no branch.
__device__ __forceinline__ void resid_take(float x, int s, uint64_t& r, uint64_t& m) {
    const bool ok = isfinite(x);
    const float y = ldexpf(x, s);
    const float d = ok ? fabsf(y - rintf(y)) : 0.0f;
    const float a = ok ? fabsf(x) : 0.0f;
    r += (uint32_t)rintf(ldexpf(d, 21));
    m += (uint32_t)rintf(ldexpf(a, s + 1));
}

// Grid-stride residuals and masses of g and h at the narrow shifts, after
// quant_reduce has completed (a later launch): added into q->res_*, q->mass_*
// (exact integer sums, so the result does not depend on the grid).
template <int NT>
__device__ void quant_resid(const float* grad, const float* hess, int64_t n, Quant* q) {
    __shared__ uint64_t s_r[4][NT / WAVE];
    const int sg = hist_shift(__uint_as_float(q->maxg_bits), n), sh = hist_shift(__uint_as_float(q->maxh_bits), n);
    uint64_t rg = 0, rh = 0, mg = 0, mh = 0;
    const int64_t tid = (int64_t)blockIdx.x * NT + threadIdx.x, nth = (int64_t)gridDim.x * NT;
    int64_t head = 0;
    if (((reinterpret_cast<uintptr_t>(grad) | reinterpret_cast<uintptr_t>(hess)) & 15) == 0) {
        constexpr int U = 4;
        const int64_t n4 = n / 4;
        const float4* g4 = reinterpret_cast<const float4*>(grad);
        const float4* h4 = reinterpret_cast<const float4*>(hess);
        int64_t i = tid;
        for (; i + (U - 1) * nth < n4; i += U * nth) {
            float4 a[U], c[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                a[u] = g4[i + u * nth];
                c[u] = h4[i + u * nth];
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                resid_take(a[u].x, sg, rg, mg);
                resid_take(a[u].y, sg, rg, mg);
                resid_take(a[u].z, sg, rg, mg);
                resid_take(a[u].w, sg, rg, mg);
                resid_take(c[u].x, sh, rh, mh);
                resid_take(c[u].y, sh, rh, mh);
                resid_take(c[u].z, sh, rh, mh);
                resid_take(c[u].w, sh, rh, mh);
            }
        }
        for (; i < n4; i += nth) {
            const float4 a = g4[i], c = h4[i];
            resid_take(a.x, sg, rg, mg);
            resid_take(a.y, sg, rg, mg);
            resid_take(a.z, sg, rg, mg);
            resid_take(a.w, sg, rg, mg);
            resid_take(c.x, sh, rh, mh);
            resid_take(c.y, sh, rh, mh);
            resid_take(c.z, sh, rh, mh);
            resid_take(c.w, sh, rh, mh);
        }
        head = n4 * 4;
    }
    for (int64_t i = head + tid; i < n; i += nth) {
        resid_take(grad[i], sg, rg, mg);
        resid_take(hess[i], sh, rh, mh);
    }
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    rg = (uint64_t)wave_sum_i64((int64_t)rg);
    rh = (uint64_t)wave_sum_i64((int64_t)rh);
    mg = (uint64_t)wave_sum_i64((int64_t)mg);
    mh = (uint64_t)wave_sum_i64((int64_t)mh);
    if (lane == 0) {
        s_r[0][w] = rg;
        s_r[1][w] = rh;
        s_r[2][w] = mg;
        s_r[3][w] = mh;
    }
    __syncthreads();
    if (threadIdx.x < 4) {
        uint64_t t = 0;
        for (int i = 0; i < NT / WAVE; ++i) t += s_r[threadIdx.x][i];
        uint64_t* dst = threadIdx.x == 0 ? &q->res_g : threadIdx.x == 1 ? &q->res_h
                      : threadIdx.x == 2 ? &q->mass_g : &q->mass_h;
        if (t) atomicAdd((unsigned long long*)dst, (unsigned long long)t);
    }
}

// The contract of hist_shift's notes from the residuals: narrow iff
// R <= 8 M for both channels (M <= n 2^31 < 2^63 / 8 for n < 2^32 rows,
// so 8 M cannot wrap).
__host__ __device__ inline bool narrow_contract(uint64_t rg, uint64_t mg, uint64_t rh, uint64_t mh) {
    return rg <= 8 * mg && rh <= 8 * mh;
}

__device__ inline void quant_finish(Quant* q, int64_t n) {
    const float mg = __uint_as_float(q->maxg_bits), mh = __uint_as_float(q->maxh_bits);
    const bool wide = !narrow_contract(q->res_g, q->mass_g, q->res_h, q->mass_h);
    q->wide = wide ? 1 : 0;
    q->wlog = window_log2(n, wide);
    q->sg = wide ? wide_shift(mg, n) : hist_shift(mg, n);
    q->sh = wide ? wide_shift(mh, n) : hist_shift(mh, n);
    q->scg = ldexp(1.0, q->sg);
    q->sch = ldexp(1.0, q->sh);
    q->ig = ldexp(1.0, -q->sg);
    q->ih = ldexp(1.0, -q->sh);
    q->const_h = 0;
    q->hq_const = 0;
    if (n > 0 && q->hmin_key == q->hmax_key) {
        const uint32_t k = q->hmin_key;
        const float h = __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
        const int64_t hq = quantise_wide(h, q->sch);
        if (hq != 0) {
            q->const_h = 1;
            q->hq_const = hq;
        }
    }
}

static __global__ __attribute__((unused)) void k_quant_clear(Quant* q) {
    q->maxg_bits = 0;
    q->maxh_bits = 0;
    q->hmin_key = 0xffffffffu;
    q->hmax_key = 0u;
    q->nonfinite = 0;
    q->const_h = 0;
    q->hq_const = 0;
    q->tot_g = 0;
    q->tot_h = 0;
    q->ticket = 0;
    q->wide = 0;
    q->wlog = NARROW_WINDOW_LOG2;
    q->res_g = q->res_h = 0;
    q->mass_g = q->mass_h = 0;
}

// Second pass of the per-call quantisation: residuals for the contract
// (quant_resid), then, in the grid's last block, quant_finish.  Blocks of
// 1024 threads, at most 256 of them: every block adds its four sums into
// four words of one cache line, and those atomics serialise.
constexpr int QRB = 1024;
static __global__ __attribute__((unused)) void __launch_bounds__(QRB)
k_quant_resid(const float* grad, const float* hess, int64_t n, Quant* q) {
    quant_resid<QRB>(grad, hess, n, q);   // global writes: wave 0's four atomics
    if (last_block_w0(&q->ticket) && threadIdx.x == 0) quant_finish(q, n);
}

// Enqueue k_quant_resid after the pass that filled q's maxima.
static __attribute__((unused)) void launch_quant_resid(hipStream_t stream, const float* grad, const float* hess,
                                                       int64_t n, Quant* q) {
    const int64_t per = (int64_t)QRB * 16;   // rows per block, at least
    int64_t blocks = (n + per - 1) / per;
    blocks = blocks < 1 ? 1 : (blocks > 256 ? 256 : blocks);
    k_quant_resid<<<(unsigned)blocks, QRB, 0, stream>>>(grad, hess, n, q);
}

}  // namespace yabt
