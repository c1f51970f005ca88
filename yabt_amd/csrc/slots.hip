// K-slot histogram on gfx950: the level-wise grower's per-level build.
//
// Replaces `hist_build` (yabt/_cuda/hist.cu:101-133) behind
// `cuda_hist.build_hist(binned, slot, g, h, w, K, F, B)` (yabt/cuda_hist.py:79-89):
// out[0][s][f][b] = sum g, out[1] = sum h, out[2] = sum w over the rows i with
// slot[i] == s and binned[i, f] == b.  The reference adds fp32 with global
// atomics (order-dependent); here g, h and w are each quantised to int64
// fixed point with one shift per call (the histograms' quant_shift), summed
// exactly, and the fp32 result is the rounding of the exact fixed-point sum:
// deterministic, and within the reference test's 1e-5 normwise tolerance.
//
// Rows are counting-sorted by slot, then each block takes a tile of 16
// features and a chunk of the sorted rows and builds the histogram of every
// slot run in its chunk with the lane = feature LDS layout of hist.h.
//
// Launch sequence: k_slot_init, k_slot_count, k_slot_offsets, k_slot_scatter,
// k_slot_hist, k_slot_finish.

#include "common.h"
#include "hist.h"
#include "host.h"
#include "yabt_hip.h"

#include <string.h>

namespace yabt {

constexpr int SLB = 256;                       // threads of the row kernels
constexpr int SROWS = 4096;                    // rows per count / scatter block
constexpr int SCHUNK = 8192;                   // sorted rows per histogram block
constexpr int SLDS_SLOTS = 4096;               // slot counters kept in LDS up to this K

struct SlotStats {
    uint32_t max_bits[3];      // max |g|, |h|, |w| (float bits)
    int32_t status;            // 0 ok, -1 a non-finite input
    int32_t s[3];              // shifts
    int32_t pad;
};

struct SlotArgs {
    const uint8_t* binned;     // (n, ldb) row-major
    int64_t ldb;
    const int64_t* slot;
    const float* v[3];         // g, h, w
    int64_t n;
    int F, K;
    SlotStats* st;
    uint32_t* count;           // (K)
    int64_t* off;              // (K + 1)
    unsigned long long* cursor;   // (K)
    uint32_t* sorted;          // (n)
    int64_t* outq;             // (3, K, F, 256) fixed-point sums
};

__device__ __forceinline__ bool slot_ok(int64_t s, int K) { return s >= 0 && s < K; }

__global__ void __launch_bounds__(SLB) k_slot_init(SlotArgs A) {
    const int64_t tid = (int64_t)blockIdx.x * SLB + threadIdx.x, stride = (int64_t)gridDim.x * SLB;
    const int64_t ne = (int64_t)3 * A.K * A.F * NB;
    for (int64_t i = tid; i < ne; i += stride) A.outq[i] = 0;
    for (int64_t i = tid; i < A.K; i += stride) {
        A.count[i] = 0;
        A.cursor[i] = 0;
    }
    if (tid == 0) {
        A.st->max_bits[0] = A.st->max_bits[1] = A.st->max_bits[2] = 0;
        A.st->status = 0;
    }
}

// Rows per slot and the magnitudes of g, h, w.
template <bool LDS>
__global__ void __launch_bounds__(SLB) k_slot_count(SlotArgs A) {
    __shared__ uint32_t s_cnt[LDS ? SLDS_SLOTS : 1];
    __shared__ float s_red[3][SLB / WAVE];
    __shared__ int s_bad;
    if (threadIdx.x == 0) s_bad = 0;
    if (LDS)
        for (int i = threadIdx.x; i < A.K; i += SLB) s_cnt[i] = 0;
    __syncthreads();
    const int64_t lo = (int64_t)blockIdx.x * SROWS, hi = min(A.n, lo + SROWS);
    float m[3] = {0.0f, 0.0f, 0.0f};
    int bad = 0;
    for (int64_t i = lo + threadIdx.x; i < hi; i += SLB) {
        const int64_t s = A.slot[i];
        if (!slot_ok(s, A.K)) continue;
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            const float x = A.v[c][i];
            if (!isfinite(x)) bad = 1;
            m[c] = fmaxf(m[c], fabsf(x));
        }
        if (LDS) atomicAdd(&s_cnt[s], 1u);
        else atomicAdd(&A.count[s], 1u);
    }
    if (bad) s_bad = 1;
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
#pragma unroll
        for (int d = WAVE / 2; d > 0; d >>= 1) m[c] = fmaxf(m[c], __shfl_xor(m[c], d, WAVE));
        if (lane == 0) s_red[c][w] = m[c];
    }
    __syncthreads();
    if (threadIdx.x < 3) {
        float t = 0.0f;
        for (int i = 0; i < SLB / WAVE; ++i) t = fmaxf(t, s_red[threadIdx.x][i]);
        atomicMax(&A.st->max_bits[threadIdx.x], __float_as_uint(t));
    }
    if (threadIdx.x == 0 && s_bad) atomicMin(&A.st->status, -1);
    if (LDS)
        for (int i = threadIdx.x; i < A.K; i += SLB)
            if (s_cnt[i]) atomicAdd(&A.count[i], s_cnt[i]);
}

__global__ void __launch_bounds__(1024) k_slot_offsets(SlotArgs A) {
    __shared__ int64_t s_wave[1024 / WAVE];
    int64_t carry = 0;
    for (int base = 0; base < A.K; base += 1024) {
        const int i = base + threadIdx.x;
        const int64_t c = i < A.K ? (int64_t)A.count[i] : 0;
        int64_t tot;
        const int64_t ex = block_excl_scan<1024, int64_t>(c, s_wave, &tot);
        if (i < A.K) {
            A.off[i] = carry + ex;
            A.cursor[i] = (unsigned long long)(carry + ex);
        }
        carry += tot;
    }
    if (threadIdx.x == 0) {
        A.off[A.K] = carry;
        for (int c = 0; c < 3; ++c) A.st->s[c] = quant_shift(__uint_as_float(A.st->max_bits[c]), A.n);
    }
}

template <bool LDS>
__global__ void __launch_bounds__(SLB) k_slot_scatter(SlotArgs A) {
    __shared__ uint32_t s_cnt[LDS ? SLDS_SLOTS : 1];
    __shared__ unsigned long long s_base[LDS ? SLDS_SLOTS : 1];
    const int64_t lo = (int64_t)blockIdx.x * SROWS, hi = min(A.n, lo + SROWS);
    if (!LDS) {
        for (int64_t i = lo + threadIdx.x; i < hi; i += SLB) {
            const int64_t s = A.slot[i];
            if (slot_ok(s, A.K)) A.sorted[atomicAdd(&A.cursor[s], 1ull)] = (uint32_t)i;
        }
        return;
    }
    for (int i = threadIdx.x; i < A.K; i += SLB) s_cnt[i] = 0;
    __syncthreads();
    for (int64_t i = lo + threadIdx.x; i < hi; i += SLB) {
        const int64_t s = A.slot[i];
        if (slot_ok(s, A.K)) atomicAdd(&s_cnt[s], 1u);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < A.K; i += SLB) {
        s_base[i] = s_cnt[i] ? atomicAdd(&A.cursor[i], (unsigned long long)s_cnt[i]) : 0ull;
        s_cnt[i] = 0;
    }
    __syncthreads();
    for (int64_t i = lo + threadIdx.x; i < hi; i += SLB) {
        const int64_t s = A.slot[i];
        if (!slot_ok(s, A.K)) continue;
        const uint32_t r = atomicAdd(&s_cnt[s], 1u);
        A.sorted[s_base[s] + r] = (uint32_t)i;
    }
}

struct SlotLds {
    unsigned long long v[3][NB * HFL];        // [channel][bin][16 features]
};

// Block (tile, chunk): the sorted rows [chunk * SCHUNK, +SCHUNK), one slot run
// at a time: clear, accumulate (lane = feature layout, g/h/w of a row handed
// to its row group with DPP), add the run's histogram into outq[slot].
__global__ void __launch_bounds__(HBLOCK) k_slot_hist(SlotArgs A, int chunks) {
    __shared__ SlotLds L;
    const int tile = blockIdx.x / chunks, chunk = blockIdx.x % chunks;
    const int f0 = tile * HFL;
    const int64_t total = A.off[A.K];
    const int64_t c0 = (int64_t)chunk * SCHUNK, c1 = min(total, c0 + SCHUNK);
    if (f0 >= A.F || c0 >= c1) return;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int fl = lane & (HFL - 1), rg = lane / HFL;
    const int f = f0 + fl;
    const bool fok = f < A.F;
    const double sc[3] = {ldexp(1.0, A.st->s[0]), ldexp(1.0, A.st->s[1]), ldexp(1.0, A.st->s[2])};
    // lanes of features >= F read feature f0 and add into their own LDS
    // columns, which the flush skips
    const uint8_t* fb = A.binned + f0 + (fok ? fl : 0);
    int lo = 0, hi = A.K - 1;              // slot holding position c0: last s with off[s] <= c0
    while (lo < hi) {
        const int mid = (lo + hi + 1) / 2;
        if (A.off[mid] <= c0) lo = mid;
        else hi = mid - 1;
    }
    const size_t plane = (size_t)A.K * A.F * NB;
    for (int s = lo; s < A.K && A.off[s] < c1; ++s) {
        const int64_t a = max(c0, A.off[s]), b = min(c1, A.off[s + 1]);
        if (a >= b) continue;                          // uniform across the block
        for (int i = threadIdx.x; i < NB * HFL; i += HBLOCK) L.v[0][i] = L.v[1][i] = L.v[2][i] = 0;
        __syncthreads();
        for (int64_t i0 = a + (int64_t)wave * WAVE; i0 < b; i0 += HSTEP) {
            uint32_t r = 0;
            uint64_t q[3] = {0, 0, 0};
            if (i0 + lane < b) {
                r = A.sorted[i0 + lane];
#pragma unroll
                for (int c = 0; c < 3; ++c) q[c] = (uint64_t)quantise(A.v[c][r], sc[c]);
            }
            const int nv = (int)min((int64_t)HFL, max((int64_t)0, b - (i0 + HFL * rg)));
            uint32_t bj[HFL];
#define YABT_SLOT_LOAD(J)                                                        \
            {                                                                    \
                const uint32_t rj = row_bcast32<J>(r);                           \
                bj[J] = ((J) < nv) ? (uint32_t)fb[(size_t)rj * A.ldb] : 0u;      \
            }
            YABT_SLOT_LOAD(0) YABT_SLOT_LOAD(1) YABT_SLOT_LOAD(2) YABT_SLOT_LOAD(3)
            YABT_SLOT_LOAD(4) YABT_SLOT_LOAD(5) YABT_SLOT_LOAD(6) YABT_SLOT_LOAD(7)
            YABT_SLOT_LOAD(8) YABT_SLOT_LOAD(9) YABT_SLOT_LOAD(10) YABT_SLOT_LOAD(11)
            YABT_SLOT_LOAD(12) YABT_SLOT_LOAD(13) YABT_SLOT_LOAD(14) YABT_SLOT_LOAD(15)
#undef YABT_SLOT_LOAD
#define YABT_SLOT_ADD(J)                                                         \
            {                                                                    \
                const uint64_t q0 = row_bcast64<J>(q[0]), q1 = row_bcast64<J>(q[1]), q2 = row_bcast64<J>(q[2]); \
                if ((J) < nv) {                                                  \
                    const int at = (int)bj[J] * HFL + fl;                        \
                    atomicAdd(&L.v[0][at], (unsigned long long)q0);              \
                    atomicAdd(&L.v[1][at], (unsigned long long)q1);              \
                    atomicAdd(&L.v[2][at], (unsigned long long)q2);              \
                }                                                                \
            }
            YABT_SLOT_ADD(0) YABT_SLOT_ADD(1) YABT_SLOT_ADD(2) YABT_SLOT_ADD(3)
            YABT_SLOT_ADD(4) YABT_SLOT_ADD(5) YABT_SLOT_ADD(6) YABT_SLOT_ADD(7)
            YABT_SLOT_ADD(8) YABT_SLOT_ADD(9) YABT_SLOT_ADD(10) YABT_SLOT_ADD(11)
            YABT_SLOT_ADD(12) YABT_SLOT_ADD(13) YABT_SLOT_ADD(14) YABT_SLOT_ADD(15)
#undef YABT_SLOT_ADD
        }
        __syncthreads();
        int64_t* base = A.outq + (size_t)s * A.F * NB;
        for (int i = threadIdx.x; i < NB * HFL; i += HBLOCK) {
            const int fi = f0 + (i % HFL);
            if (fi >= A.F) continue;
            const size_t at = (size_t)fi * NB + (size_t)(i / HFL);
#pragma unroll
            for (int c = 0; c < 3; ++c)
                if (L.v[c][i]) atomicAdd((unsigned long long*)(base + c * plane + at), L.v[c][i]);
        }
        __syncthreads();
    }
}

// out = exact fixed-point sums rounded to fp32.
__global__ void __launch_bounds__(SLB) k_slot_finish(SlotArgs A, float* out) {
    const int64_t plane = (int64_t)A.K * A.F * NB;
    const double isc[3] = {ldexp(1.0, -A.st->s[0]), ldexp(1.0, -A.st->s[1]), ldexp(1.0, -A.st->s[2])};
    for (int64_t i = (int64_t)blockIdx.x * SLB + threadIdx.x; i < 3 * plane; i += (int64_t)gridDim.x * SLB)
        out[i] = (float)((double)A.outq[i] * isc[i / plane]);
}

__global__ void k_slot_status(const SlotStats* st, int32_t* out) {
    out[0] = st->status;
    out[1] = st->s[0];
    out[2] = st->s[1];
    out[3] = st->s[2];
}

size_t carve_slots(char* base, int64_t n, int F, int K, SlotArgs* A) {
    Carve c{base, 0};
    SlotArgs tmp;
    SlotArgs& a = A ? *A : tmp;
    a.st = c.take<SlotStats>(1);
    a.count = c.take<uint32_t>((size_t)K);
    a.off = c.take<int64_t>((size_t)K + 1);
    a.cursor = c.take<unsigned long long>((size_t)K);
    a.sorted = c.take<uint32_t>((size_t)(n > 0 ? n : 1));
    a.outq = c.take<int64_t>((size_t)3 * K * F * NB);
    return align_up(c.off, 256);
}

}  // namespace yabt

using namespace yabt;

extern "C" {

size_t yabt_hist_slots_workspace_bytes(int64_t n, int F, int K) {
    if (n < 0 || F < 1 || K < 1) return 0;
    return carve_slots(nullptr, n, F, K, nullptr);
}

int yabt_hist_slots(const uint8_t* binned, int64_t ldb, const int64_t* slot, const float* g, const float* h,
                    const float* w, int64_t n, int F, int K, void* workspace, size_t workspace_bytes, float* out,
                    int32_t* out_status, hipStream_t stream) {
    if (n < 0 || n > 0xFFFFFFFFll || F < 1 || K < 1 || (n > 0 && ldb < F))
        return fail(-2, "yabt_hist_slots: bad sizes (need 0 <= n < 2^32, F >= 1, K >= 1, ldb >= F)");
    if ((n > 0 && (!binned || !slot || !g || !h || !w)) || !workspace || !out || !out_status)
        return fail(-2, "yabt_hist_slots: null pointer argument");
    SlotArgs A;
    memset(&A, 0, sizeof A);
    const size_t need = carve_slots((char*)workspace, n, F, K, &A);
    if (workspace_bytes < need) return fail(-2, "yabt_hist_slots: workspace too small");
    A.binned = binned;
    A.ldb = ldb;
    A.slot = slot;
    A.v[0] = g;
    A.v[1] = h;
    A.v[2] = w;
    A.n = n;
    A.F = F;
    A.K = K;
    const bool lds = K <= SLDS_SLOTS;
    const int row_blocks = (int)((n + SROWS - 1) / SROWS);
    k_slot_init<<<launch_grid((int64_t)3 * K * F * NB, SLB, 2048), SLB, 0, stream>>>(A);
    if (row_blocks > 0) {
        if (lds) k_slot_count<true><<<row_blocks, SLB, 0, stream>>>(A);
        else k_slot_count<false><<<row_blocks, SLB, 0, stream>>>(A);
    }
    k_slot_offsets<<<1, 1024, 0, stream>>>(A);
    if (row_blocks > 0) {
        if (lds) k_slot_scatter<true><<<row_blocks, SLB, 0, stream>>>(A);
        else k_slot_scatter<false><<<row_blocks, SLB, 0, stream>>>(A);
        const int tiles = (F + HFL - 1) / HFL;
        const int chunks = (int)((n + SCHUNK - 1) / SCHUNK);
        k_slot_hist<<<tiles * chunks, HBLOCK, 0, stream>>>(A, chunks);
    }
    k_slot_finish<<<launch_grid((int64_t)3 * K * F * NB, SLB, 2048), SLB, 0, stream>>>(A, out);
    k_slot_status<<<1, 1, 0, stream>>>(A.st, out_status);
    return launch_status("yabt_hist_slots launch");
}

}  // extern "C"
