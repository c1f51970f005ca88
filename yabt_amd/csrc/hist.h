// Node-histogram kernels (exact int64 fixed point), shared by the grower and
// the stand-alone entry points.
//
// Layout: a block owns a tile of HFL = 16 features and a chunk of rows.  In a
// wave, lane = 16 * q + fl handles feature f0 + fl for row group q (4 row
// groups x 16 rows = 64 rows per wave step), so the 64 lanes of every LDS
// atomic touch 16 different features x 4 rows.  The LDS histogram is laid out
// [bin][feature] (entry bin * 16 + fl), which keeps each atomic instruction
// free of bank conflicts whatever the bin values are; a row-per-lane layout
// sends all 64 lanes of an instruction to random bins of one feature.
//
// Each row's g and h are loaded and quantised once (one row per lane) and
// handed to the 16 lanes of its row group with DPP row_newbcast.
//
// Optional skips, both exact because the sums are integers:
//   * dflt[f] (may be NULL): rows whose bin equals dflt[f] are not added; the
//     caller restores that bin as node total minus the other bins (the
//     default-bin fill of grow.c:101-106, here exact);
//   * HCH = false: no h channel (every h equal): sum q(h) = count * q(h), and
//     the h plane of the output is left untouched.
#pragma once

#include "common.h"

namespace yabt {

constexpr int HFL = 16;                       // features per tile
constexpr int HBLOCK = 1024;                  // threads per histogram block
constexpr int HWAVES = HBLOCK / WAVE;
constexpr int HSTEP = HWAVES * WAVE;          // rows per block step (64 per wave)
constexpr int GATHER_MAX_CHUNKS = 64;         // chunk slots per tile in a gather launch
constexpr int GATHER_MIN_ROWS = 8192;         // rows per gather chunk, at least

struct HistLds {
    unsigned long long g[NB * HFL];           // [bin][fl]
    unsigned long long h[NB * HFL];
    uint32_t c[NB * HFL];
};

template <bool HCH>
__device__ __forceinline__ void hist_clear(HistLds& L) {
    for (int i = threadIdx.x; i < NB * HFL; i += HBLOCK) {
        L.g[i] = 0;
        if (HCH) L.h[i] = 0;
        L.c[i] = 0;
    }
}

// Add the block's histogram into out[3][F][256] (entries that received no row
// are skipped).
template <bool HCH>
__device__ __forceinline__ void hist_flush(HistLds& L, int64_t* out, int F, int f0) {
    const size_t plane = (size_t)F * NB;
    for (int i = threadIdx.x; i < NB * HFL; i += HBLOCK) {
        const int f = f0 + (i % HFL);
        const uint32_t c = L.c[i];
        if (f >= F || c == 0) continue;
        const size_t at = (size_t)f * NB + (size_t)(i / HFL);
        atomicAdd((unsigned long long*)(out + at), L.g[i]);
        if (HCH) atomicAdd((unsigned long long*)(out + plane + at), L.h[i]);
        atomicAdd((unsigned long long*)(out + 2 * plane + at), (unsigned long long)c);
    }
}

template <bool HCH>
__device__ __forceinline__ void hist_add(HistLds& L, int b, int fl, uint64_t g, uint64_t h) {
    const int at = b * HFL + fl;
    atomicAdd(&L.g[at], (unsigned long long)g);
    if (HCH) atomicAdd(&L.h[at], (unsigned long long)h);
    atomicAdd(&L.c[at], 1u);
}

// Rows per block chunk for the streaming kernel: about two resident blocks
// per CU on 256 CUs, chunks a multiple of 8 so that all tiles of a row chunk
// run on one XCD (block id % 8) and share its L2 for the chunk's g and h.
inline int root_chunks(int64_t n, int tiles) {
    int want = 512 / tiles;
    const int64_t useful = (n + HSTEP - 1) / HSTEP;
    if (want > useful) want = (int)useful;
    want = want / 8 * 8;
    return want < 8 ? 8 : want;
}

// Streaming histogram of rows [0, n) from the feature-major bins.
// Grid: tiles * chunks blocks, block -> (tile = bid / chunks, chunk = bid % chunks).
// q_tot (may be NULL): the tile-0 blocks add sum q(g), sum q(h) of all rows
// (sum q(h) only with the h channel; without it the caller uses n * q(h)).
template <bool HCH>
__device__ __forceinline__ void hist_root_body(HistLds& L, const uint8_t* __restrict__ bins_fm, int64_t ld,
                                               const float* __restrict__ grad, const float* __restrict__ hess,
                                               int64_t n, int F, double scg, double sch,
                                               const int32_t* __restrict__ dflt, Quant* q_tot, int64_t* out,
                                               int chunks) {
    const int tile = blockIdx.x / chunks, chunk = blockIdx.x % chunks;
    const int f0 = tile * HFL;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int fl = lane & (HFL - 1), rg = lane / HFL;
    const int f = f0 + fl;
    const bool fok = f < F;
    const int64_t per = ((n + chunks - 1) / chunks + HSTEP - 1) / HSTEP * HSTEP;
    const int64_t lo = (int64_t)chunk * per, hi = min(n, lo + per);
    if (f0 >= F || lo >= hi) return;
    const int d = (fok && dflt) ? dflt[f] : -1;
    const bool totals = q_tot != nullptr && tile == 0;
    hist_clear<HCH>(L);
    __syncthreads();
    const uint8_t* col = bins_fm + (size_t)(fok ? f : f0) * ld;
    int64_t sum_g = 0, sum_h = 0;
    for (int64_t r0 = lo + (int64_t)wave * WAVE; r0 < hi; r0 += HSTEP) {
        const int64_t rl = r0 + lane;
        uint64_t gq = 0, hq = 0;
        if (rl < hi) {
            gq = (uint64_t)quantise(grad[rl], scg);
            if (HCH) hq = (uint64_t)quantise(hess[rl], sch);
        }
        sum_g += (int64_t)gq;
        sum_h += (int64_t)hq;
        // lane's 16 rows of its feature: r0 % 64 == 0, so base % 16 == 0; with
        // base < hi <= n <= ld and ld % 16 == 0 the 16-byte load stays in the row
        const int64_t base = r0 + HFL * rg;
        const uint4 bv = base < hi ? *reinterpret_cast<const uint4*>(col + base) : make_uint4(0, 0, 0, 0);
        const uint32_t w[4] = {bv.x, bv.y, bv.z, bv.w};
        const int nv = (int)min((int64_t)HFL, max((int64_t)0, hi - base));
#define YABT_ROOT_STEP(J)                                                        \
        {                                                                        \
            const uint64_t gj = row_bcast64<J>(gq), hj = HCH ? row_bcast64<J>(hq) : 0; \
            const int b = (int)((w[(J) >> 2] >> (8 * ((J) & 3))) & 0xffu);       \
            if (fok && (J) < nv && b != d) hist_add<HCH>(L, b, fl, gj, hj);       \
        }
        YABT_ROOT_STEP(0) YABT_ROOT_STEP(1) YABT_ROOT_STEP(2) YABT_ROOT_STEP(3)
        YABT_ROOT_STEP(4) YABT_ROOT_STEP(5) YABT_ROOT_STEP(6) YABT_ROOT_STEP(7)
        YABT_ROOT_STEP(8) YABT_ROOT_STEP(9) YABT_ROOT_STEP(10) YABT_ROOT_STEP(11)
        YABT_ROOT_STEP(12) YABT_ROOT_STEP(13) YABT_ROOT_STEP(14) YABT_ROOT_STEP(15)
#undef YABT_ROOT_STEP
    }
    if (totals) {
        sum_g = wave_sum<int64_t>(sum_g);
        sum_h = wave_sum<int64_t>(sum_h);
        if (lane == 0) {
            atomicAdd((unsigned long long*)&q_tot->tot_g, (unsigned long long)sum_g);
            atomicAdd((unsigned long long*)&q_tot->tot_h, (unsigned long long)sum_h);
        }
    }
    __syncthreads();
    hist_flush<HCH>(L, out, F, f0);
}

// count_mode 0: all three channels; 1: no h channel when q->const_h.
static __global__ void __launch_bounds__(HBLOCK) k_hist_root(const uint8_t* __restrict__ bins_fm, int64_t ld,
                                                      const float* __restrict__ grad,
                                                      const float* __restrict__ hess, int64_t n, int F,
                                                      const Quant* q, double scg_v, double sch_v,
                                                      const int32_t* __restrict__ dflt, Quant* q_tot,
                                                      int64_t* out, int chunks, int count_mode,
                                                      const int32_t* done) {
    const int32_t dn = done ? *done : 0;
    const double scg = q ? q->scg : scg_v, sch = q ? q->sch : sch_v;
    const bool no_h = count_mode && q && q->const_h;
    if (dn) return;
    __shared__ HistLds L;
    if (no_h)
        hist_root_body<false>(L, bins_fm, ld, grad, hess, n, F, scg, sch, dflt, q_tot, out, chunks);
    else
        hist_root_body<true>(L, bins_fm, ld, grad, hess, n, F, scg, sch, dflt, q_tot, out, chunks);
}

// Rows of one node for a gather launch.
struct HistJob {
    int32_t active;
    int32_t pad;
    const uint32_t* rows;      // row ids of the node at positions [lo, hi)
    int64_t lo, hi;
    int64_t* out;              // [3][F][256], cleared beforehand, added into
};

// Chunks of a gather launch over m rows.
__host__ __device__ inline int gather_chunks(int64_t m) {
    const int64_t c = (m + GATHER_MIN_ROWS - 1) / GATHER_MIN_ROWS;
    return (int)(c < GATHER_MAX_CHUNKS ? c : GATHER_MAX_CHUNKS);
}

// Histogram of the rows listed at rows[lo:hi], bins gathered from the
// row-major copy.  Grid: tiles * GATHER_MAX_CHUNKS blocks (chunk-minor); a
// node uses ceil(m / GATHER_MIN_ROWS) chunks, the other blocks exit at once.
// Each wave loads the row ids, g and h of its next 64 rows one step ahead, so
// the dependent row-id -> g/h loads overlap the LDS clear and the adds.
template <bool HCH>
__device__ __forceinline__ void hist_gather_body(HistLds& L, const uint8_t* __restrict__ bins_rm, int64_t ld,
                                                 const float* __restrict__ grad, const float* __restrict__ hess,
                                                 int F, double scg, double sch, const int32_t* __restrict__ dflt,
                                                 const uint32_t* __restrict__ rows, int64_t jlo, int64_t jhi,
                                                 int64_t* out) {
    const int tile = blockIdx.x / GATHER_MAX_CHUNKS, chunk = blockIdx.x % GATHER_MAX_CHUNKS;
    const int f0 = tile * HFL;
    const int64_t m = jhi - jlo;
    if (f0 >= F || m <= 0) return;
    const int nch = gather_chunks(m);
    if (chunk >= nch) return;
    const int64_t per = ((m + nch - 1) / nch + WAVE - 1) / WAVE * WAVE;
    const int64_t lo = jlo + (int64_t)chunk * per, hi = min(jhi, lo + per);
    if (lo >= hi) return;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int fl = lane & (HFL - 1), rg = lane / HFL;
    const int f = f0 + fl;
    const bool fok = f < F;
    const int d = (fok && dflt) ? dflt[f] : -1;
    int64_t i0 = lo + (int64_t)wave * WAVE;
    uint32_t r = 0;
    float gx = 0.0f, hx = 0.0f;
    if (i0 + lane < hi) {
        r = rows[i0 + lane];
        gx = grad[r];
        if (HCH) hx = hess[r];
    }
    hist_clear<HCH>(L);
    __syncthreads();
    const uint8_t* fbase = bins_rm + f0 + (fok ? fl : 0);
    for (; i0 < hi; i0 += HSTEP) {
        const uint64_t gq = (uint64_t)quantise(gx, scg), hq = HCH ? (uint64_t)quantise(hx, sch) : 0;
        const int nv = (int)min((int64_t)HFL, max((int64_t)0, hi - (i0 + HFL * rg)));
        int bj[HFL];
#define YABT_GATHER_LOAD(J)                                                       \
        {                                                                         \
            const uint32_t rj = row_bcast32<J>(r);                                \
            bj[J] = (fok && (J) < nv) ? (int)fbase[(size_t)rj * ld] : -1;         \
        }
        YABT_GATHER_LOAD(0) YABT_GATHER_LOAD(1) YABT_GATHER_LOAD(2) YABT_GATHER_LOAD(3)
        YABT_GATHER_LOAD(4) YABT_GATHER_LOAD(5) YABT_GATHER_LOAD(6) YABT_GATHER_LOAD(7)
        YABT_GATHER_LOAD(8) YABT_GATHER_LOAD(9) YABT_GATHER_LOAD(10) YABT_GATHER_LOAD(11)
        YABT_GATHER_LOAD(12) YABT_GATHER_LOAD(13) YABT_GATHER_LOAD(14) YABT_GATHER_LOAD(15)
#undef YABT_GATHER_LOAD
        // next step's rows
        const int64_t in = i0 + HSTEP + lane;
        uint32_t rn = 0;
        float gn = 0.0f, hn = 0.0f;
        if (in < hi) {
            rn = rows[in];
            gn = grad[rn];
            if (HCH) hn = hess[rn];
        }
#define YABT_GATHER_ADD(J)                                                        \
        {                                                                         \
            const uint64_t gj = row_bcast64<J>(gq), hj = HCH ? row_bcast64<J>(hq) : 0; \
            if (bj[J] >= 0 && bj[J] != d) hist_add<HCH>(L, bj[J], fl, gj, hj);    \
        }
        YABT_GATHER_ADD(0) YABT_GATHER_ADD(1) YABT_GATHER_ADD(2) YABT_GATHER_ADD(3)
        YABT_GATHER_ADD(4) YABT_GATHER_ADD(5) YABT_GATHER_ADD(6) YABT_GATHER_ADD(7)
        YABT_GATHER_ADD(8) YABT_GATHER_ADD(9) YABT_GATHER_ADD(10) YABT_GATHER_ADD(11)
        YABT_GATHER_ADD(12) YABT_GATHER_ADD(13) YABT_GATHER_ADD(14) YABT_GATHER_ADD(15)
#undef YABT_GATHER_ADD
        r = rn;
        gx = gn;
        hx = hn;
    }
    __syncthreads();
    hist_flush<HCH>(L, out, F, f0);
}

// job->active == 0 or *done != 0 (done may be NULL): nothing to do.
static __global__ void __launch_bounds__(HBLOCK) k_hist_gather(const uint8_t* __restrict__ bins_rm, int64_t ld,
                                                        const float* __restrict__ grad,
                                                        const float* __restrict__ hess, int F, const Quant* q,
                                                        double scg_v, double sch_v,
                                                        const int32_t* __restrict__ dflt, const HistJob* job,
                                                        int count_mode, const int32_t* done) {
    // independent loads first: the job record, the done flag, the shifts
    const HistJob jb = *job;
    const int32_t dn = done ? *done : 0;
    const double scg = q ? q->scg : scg_v, sch = q ? q->sch : sch_v;
    const bool no_h = count_mode && q && q->const_h;
    if (dn || !jb.active) return;
    __shared__ HistLds L;
    if (no_h)
        hist_gather_body<false>(L, bins_rm, ld, grad, hess, F, scg, sch, dflt, jb.rows, jb.lo, jb.hi, jb.out);
    else
        hist_gather_body<true>(L, bins_rm, ld, grad, hess, F, scg, sch, dflt, jb.rows, jb.lo, jb.hi, jb.out);
}

}  // namespace yabt
