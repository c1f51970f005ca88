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

// ---------------------------------------------------------------------------
// Packed count channel.  The count rides in the low bits of one 64-bit LDS
// word next to q (q(h), or q(g) without the h channel): every row adds
// (q << cb) + 1, so a sum over R rows is (sum q) << cb + R, exact while
// R < 2^cb and |sum q| < 2^(63 - cb).  With |q| <= 2^(61 - k) (n <= 2^k, the
// standard shift) both hold for windows of R <= 2^w rows, w = (k + 1) / 2,
// cb = w + 1; after each window every thread moves its 4 entries into
// registers (exact integer unpack) and clears them.  Two LDS atomics per
// update instead of three (one without the h channel).
// ---------------------------------------------------------------------------

constexpr int HENT = NB * HFL / HBLOCK;       // entries per thread in an unpack

// Packed-word LDS of the gather (see hist_gather_packed); its callers keep it
// in a union with HistLds, which the final flush reuses.
struct HistLdsP {
    unsigned long long g[NB * HFL];           // sum q(g) (with the h channel)
    unsigned long long p[NB * HFL];           // packed (q << cb) + 1
};

// Final flush of the packed kernels: thread t holds cells i = t + k HBLOCK
// (bin i / HFL, feature f0 + i % HFL) with sums g, h and counts c.  They go
// through the block's LDS (a HistLds, 80 KB, which the kernels' LDS unions
// hold) transposed to [feature][bin], so that a wave's global atomics cover
// 64 consecutive bins of one feature: four 128-byte lines per instruction
// instead of sixteen.  Feature fl's bin b sits at fl NB + (b ^ 2 fl): the
// swizzle spreads the 16 features a half-wave writes for two bins over 32
// distinct bank pairs (unswizzled they share one), and stays inside each
// aligned group of 64 bins, so a wave's reads still cover 64 consecutive
// bins.  The caller has finished with its own LDS layout (a barrier before
// the call); cells without rows and features >= F are skipped.
template <bool HCH>
__device__ __forceinline__ void flush_cells(HistLds& T, const uint64_t (&g)[HENT], const int64_t (&h)[HENT],
                                            const uint32_t (&c)[HENT], int64_t* out, int F, int f0) {
#pragma unroll
    for (int k = 0; k < HENT; ++k) {
        const int i = threadIdx.x + k * HBLOCK;
        const int fl = i % HFL;
        const int j = fl * NB + ((i / HFL) ^ (2 * fl));
        T.g[j] = g[k];
        if (HCH) T.h[j] = (unsigned long long)h[k];
        T.c[j] = c[k];
    }
    __syncthreads();
    const size_t plane = (size_t)F * NB;
#pragma unroll
    for (int k = 0; k < HENT; ++k) {
        const int j = threadIdx.x + k * HBLOCK;
        const int fl = j / NB;
        const int fi = f0 + fl;
        const uint32_t cj = T.c[j];
        if (fi >= F || cj == 0) continue;
        const size_t at = (size_t)fi * NB + (size_t)((j % NB) ^ (2 * fl));
        atomicAdd((unsigned long long*)(out + at), T.g[j]);
        if (HCH) atomicAdd((unsigned long long*)(out + plane + at), T.h[j]);
        atomicAdd((unsigned long long*)(out + 2 * plane + at), (unsigned long long)cj);
    }
}

// log2 of the packing window for n rows, or -1 when a window would be
// shorter than one block step (then the three-word layout is used).
__host__ __device__ inline int pack_window_log2(int64_t n) {
    int k = 0;
    while (k < 62 && ((int64_t)1 << k) < n) ++k;
    const int w = (k + 1) / 2;
    return w >= 10 ? (w > 16 ? 16 : w) : -1;   // 2^10 rows = one block step
}

// LDS of the streaming root histogram: 256 bins x 32 words of 8 bytes.  Word
// fl of a bin is sum q(g) of feature f0 + fl (with the h channel), word
// 16 + fl the packed (q << cb) + 1 of feature f0 + fl.  A bin's words span
// 256 bytes, so the byte address of an entry is (bin << 8) | (fl << 3)
// (+ 128 for the packed word): one byte permute of the loaded bin word
// builds it.  Within the 16 lanes of a row group the 16 features hit 16
// distinct bank pairs whatever the bins are.
struct HistLdsR {
    unsigned long long w[NB * 2 * HFL];
};

constexpr int ROOT_PW = HFL;                  // word offset of the packed words in a bin row

// Byte J of `word` placed in bits 8..15 over `lo` (bits 0..7).
template <int J>
__device__ __forceinline__ uint32_t bin_addr(uint32_t word, uint32_t lo) {
    return __builtin_amdgcn_perm(word, lo, 0x0c0c0000u | ((4u + J) << 8));
}

// SKIP: dflt is given (rows in a feature's default bin are not added).
// Lanes of features >= F read feature f0's column and add into their own LDS
// columns, which the flush ignores, so the adds need no feature test.  Each
// wave loads the next step's g, h and bins before adding the current step.
template <bool HCH, bool SKIP>
__device__ __forceinline__ void hist_root_packed(HistLdsR& L, const uint8_t* __restrict__ bins_fm, int64_t ld,
                                                 const float* __restrict__ grad, const float* __restrict__ hess,
                                                 int64_t n, int F, double scg, double sch,
                                                 const int32_t* __restrict__ dflt, Quant* q_tot, int64_t* out,
                                                 int chunks, int wlog) {
    const int tile = blockIdx.x / chunks, chunk = blockIdx.x % chunks;
    const int f0 = tile * HFL;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int fl = lane & (HFL - 1), rg = lane / HFL;
    const int f = f0 + fl;
    const bool fok = f < F;
    const int64_t per = ((n + chunks - 1) / chunks + HSTEP - 1) / HSTEP * HSTEP;
    const int64_t lo = (int64_t)chunk * per, hi = min(n, lo + per);
    if (f0 >= F || lo >= hi) return;
    const int d = (SKIP && fok) ? dflt[f] : -1;
    const bool totals = q_tot != nullptr && tile == 0;
    const int cb = wlog + 1;
    const uint64_t cmask = ((uint64_t)1 << cb) - 1;
    const int64_t win_steps = (int64_t)1 << (wlog - 10);
    for (int i = threadIdx.x; i < NB * 2 * HFL; i += HBLOCK) L.w[i] = 0;
    const uint32_t lbase = (uint32_t)fl << 3;
    char* const lds = reinterpret_cast<char*>(L.w);
    int64_t qa[HENT];
    uint32_t ca[HENT];
#pragma unroll
    for (int k = 0; k < HENT; ++k) {
        qa[k] = 0;
        ca[k] = 0;
    }
    const uint8_t* col = bins_fm + (size_t)(fok ? f : f0) * ld;
    // r0 % 64 == 0, so base % 16 == 0; base < hi <= n <= ld, ld % 16 == 0:
    // the 16-byte load stays inside the row
    float gx = 0.0f, hx = 0.0f;
    uint4 bv = make_uint4(0, 0, 0, 0);
    {
        const int64_t r0 = lo + (int64_t)wave * WAVE;
        if (r0 + lane < hi) {
            gx = grad[r0 + lane];
            if (HCH) hx = hess[r0 + lane];
        }
        if (r0 + HFL * rg < hi) bv = *reinterpret_cast<const uint4*>(col + r0 + HFL * rg);
    }
    __syncthreads();
    int64_t sum_g = 0, sum_h = 0;
    const int64_t steps = (hi - lo + HSTEP - 1) / HSTEP;   // the same in every wave: barriers below
    for (int64_t s = 0; s < steps; ++s) {
        const int64_t r0 = lo + s * HSTEP + (int64_t)wave * WAVE;
        // next step's inputs
        float gn = 0.0f, hn = 0.0f;
        uint4 bn = make_uint4(0, 0, 0, 0);
        {
            const int64_t r1 = r0 + HSTEP;
            if (r1 + lane < hi) {
                gn = grad[r1 + lane];
                if (HCH) hn = hess[r1 + lane];
            }
            if (r1 + HFL * rg < hi) bn = *reinterpret_cast<const uint4*>(col + r1 + HFL * rg);
        }
        const bool rok = r0 + lane < hi;
        const int64_t gq = rok ? quantise(gx, scg) : 0;
        const int64_t hq = (HCH && rok) ? quantise(hx, sch) : 0;
        sum_g += gq;
        sum_h += hq;
        const uint64_t gw = HCH ? (uint64_t)gq : ((uint64_t)gq << cb) + 1;
        const uint64_t pw = HCH ? ((uint64_t)hq << cb) + 1 : 0;
        const uint32_t wv[4] = {bv.x, bv.y, bv.z, bv.w};
#define YABT_PACK_ADD(J)                                                         \
        {                                                                        \
            char* const at = lds + bin_addr<(J) & 3>(wv[(J) >> 2], lbase);       \
            unsigned long long* const pw_at = reinterpret_cast<unsigned long long*>(at + 8 * ROOT_PW); \
            if (HCH) {                                                           \
                atomicAdd(reinterpret_cast<unsigned long long*>(at), (unsigned long long)gj); \
                atomicAdd(pw_at, (unsigned long long)pj);                        \
            } else {                                                             \
                atomicAdd(pw_at, (unsigned long long)gj);                        \
            }                                                                    \
        }
#define YABT_PACK_STEP(J, TAIL)                                                  \
        {                                                                        \
            const uint64_t gj = row_bcast64<J>(gw);                              \
            const uint64_t pj = HCH ? row_bcast64<J>(pw) : 0;                     \
            if (!(TAIL) || (J) < nv) {                                           \
                if (SKIP) {                                                      \
                    const int b = (int)((wv[(J) >> 2] >> (8 * ((J) & 3))) & 0xffu); \
                    if (b != d) YABT_PACK_ADD(J)                                 \
                } else {                                                         \
                    YABT_PACK_ADD(J)                                             \
                }                                                                \
            }                                                                    \
        }
        if (r0 + WAVE <= hi) {   // wave-uniform: all 64 rows valid
            constexpr int nv = HFL;
            YABT_PACK_STEP(0, 0) YABT_PACK_STEP(1, 0) YABT_PACK_STEP(2, 0) YABT_PACK_STEP(3, 0)
            YABT_PACK_STEP(4, 0) YABT_PACK_STEP(5, 0) YABT_PACK_STEP(6, 0) YABT_PACK_STEP(7, 0)
            YABT_PACK_STEP(8, 0) YABT_PACK_STEP(9, 0) YABT_PACK_STEP(10, 0) YABT_PACK_STEP(11, 0)
            YABT_PACK_STEP(12, 0) YABT_PACK_STEP(13, 0) YABT_PACK_STEP(14, 0) YABT_PACK_STEP(15, 0)
        } else if (r0 < hi) {
            const int nv = (int)min((int64_t)HFL, max((int64_t)0, hi - (r0 + HFL * rg)));
            YABT_PACK_STEP(0, 1) YABT_PACK_STEP(1, 1) YABT_PACK_STEP(2, 1) YABT_PACK_STEP(3, 1)
            YABT_PACK_STEP(4, 1) YABT_PACK_STEP(5, 1) YABT_PACK_STEP(6, 1) YABT_PACK_STEP(7, 1)
            YABT_PACK_STEP(8, 1) YABT_PACK_STEP(9, 1) YABT_PACK_STEP(10, 1) YABT_PACK_STEP(11, 1)
            YABT_PACK_STEP(12, 1) YABT_PACK_STEP(13, 1) YABT_PACK_STEP(14, 1) YABT_PACK_STEP(15, 1)
        }
#undef YABT_PACK_STEP
#undef YABT_PACK_ADD
        if ((s + 1) % win_steps == 0 || s + 1 == steps) {
            __syncthreads();
#pragma unroll
            for (int k = 0; k < HENT; ++k) {
                const int i = threadIdx.x + k * HBLOCK;
                const int pi = (i / HFL) * (2 * HFL) + ROOT_PW + (i % HFL);
                const uint64_t v = L.w[pi];
                L.w[pi] = 0;
                const uint64_t c = v & cmask;
                qa[k] += (int64_t)(v - c) >> cb;
                ca[k] += (uint32_t)c;
            }
            __syncthreads();
        }
        gx = gn;
        hx = hn;
        bv = bn;
    }
    if (totals) {
        sum_g = wave_sum<int64_t>(sum_g);
        sum_h = wave_sum<int64_t>(sum_h);
        if (lane == 0) {
            atomicAdd((unsigned long long*)&q_tot->tot_g, (unsigned long long)sum_g);
            atomicAdd((unsigned long long*)&q_tot->tot_h, (unsigned long long)sum_h);
        }
    }
    uint64_t gv[HENT];
#pragma unroll
    for (int k = 0; k < HENT; ++k) {
        const int i = threadIdx.x + k * HBLOCK;
        gv[k] = HCH ? L.w[(i / HFL) * (2 * HFL) + (i % HFL)] : (uint64_t)qa[k];
    }
    __syncthreads();   // every g cell read before the LDS is rewritten
    flush_cells<HCH>(*reinterpret_cast<HistLds*>(&L), gv, qa, ca, out, F, f0);
}

// count_mode 0: all three channels; 1: no h channel when q->const_h.
// SKIP: dflt is given (a separate kernel, so that the loops without the
// default-bin test are compiled on their own).
template <bool SKIP>
static __global__ __attribute__((unused)) void __launch_bounds__(HBLOCK) k_hist_root(const uint8_t* __restrict__ bins_fm, int64_t ld,
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
    __shared__ union {
        HistLds u;
        HistLdsR p;
    } L;
    const int wlog = pack_window_log2(n);
    if (wlog >= 0) {
        if (no_h)
            hist_root_packed<false, SKIP>(L.p, bins_fm, ld, grad, hess, n, F, scg, sch, dflt, q_tot, out, chunks,
                                          wlog);
        else
            hist_root_packed<true, SKIP>(L.p, bins_fm, ld, grad, hess, n, F, scg, sch, dflt, q_tot, out, chunks,
                                         wlog);
    } else if (no_h) {
        hist_root_body<false>(L.u, bins_fm, ld, grad, hess, n, F, scg, sch, dflt, q_tot, out, chunks);
    } else {
        hist_root_body<true>(L.u, bins_fm, ld, grad, hess, n, F, scg, sch, dflt, q_tot, out, chunks);
    }
}

// Launch k_hist_root over `tiles * chunks` blocks (the instantiation with
// the default-bin test only when dflt is given).
static __attribute__((unused)) void launch_hist_root(int tiles, int chunks, hipStream_t stream,
                                                     const uint8_t* bins_fm, int64_t ld, const float* grad,
                                                     const float* hess, int64_t n, int F, const Quant* q,
                                                     double scg, double sch, const int32_t* dflt, Quant* q_tot,
                                                     int64_t* out, int count_mode, const int32_t* done) {
    if (dflt)
        k_hist_root<true><<<tiles * chunks, HBLOCK, 0, stream>>>(bins_fm, ld, grad, hess, n, F, q, scg, sch, dflt,
                                                                 q_tot, out, chunks, count_mode, done);
    else
        k_hist_root<false><<<tiles * chunks, HBLOCK, 0, stream>>>(bins_fm, ld, grad, hess, n, F, q, scg, sch,
                                                                  nullptr, q_tot, out, chunks, count_mode, done);
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
// row-major copy: chunk `chunk` of the node's rows for features
// [16 tile, 16 tile + 16).  A node uses gather_chunks(m) chunks; other chunk
// numbers return at once.
// Each wave loads the row ids, g and h of its next 64 rows one step ahead, so
// the dependent row-id -> g/h loads overlap the LDS clear and the adds.
template <bool HCH>
__device__ __forceinline__ void hist_gather_body(HistLds& L, const uint8_t* __restrict__ bins_rm, int64_t ld,
                                                 const float* __restrict__ grad, const float* __restrict__ hess,
                                                 int F, double scg, double sch, const int32_t* __restrict__ dflt,
                                                 const uint32_t* __restrict__ rows, int64_t jlo, int64_t jhi,
                                                 int64_t* out, int tile, int chunk) {
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

// Packed-word form of hist_gather_body (see hist_root_packed), with a
// three-stage software pipeline per wave: at step s the wave adds step s,
// loads g, h and the bins of step s + 1 (its row ids are already in
// registers) and the row ids of step s + 2.
template <bool HCH, bool SKIP>
__device__ __forceinline__ void hist_gather_packed(HistLdsP& L, const uint8_t* __restrict__ bins_rm, int64_t ld,
                                                   const float* __restrict__ grad, const float* __restrict__ hess,
                                                   int F, double scg, double sch, const int32_t* __restrict__ dflt,
                                                   const uint32_t* __restrict__ rows, int64_t jlo, int64_t jhi,
                                                   int64_t* out, int wlog, int tile, int chunk) {
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
    const int d = (SKIP && fok) ? dflt[f] : -1;
    const int cb = wlog + 1;
    const uint64_t cmask = ((uint64_t)1 << cb) - 1;
    const int64_t win_steps = (int64_t)1 << (wlog - 10);
    // lanes of features >= F gather feature f0's byte and add into their own
    // LDS columns, which the flush ignores
    const uint8_t* fbase = bins_rm + f0 + (fok ? fl : 0);
    const int64_t w0 = lo + (int64_t)wave * WAVE;   // this wave's rows at step s: w0 + s * HSTEP + [0, 64)
    // stage inputs: row ids of steps 0 and 1, g/h/bins of step 0
    uint32_t r0 = 0, r1 = 0;
    if (w0 + lane < hi) r0 = rows[w0 + lane];
    if (w0 + HSTEP + lane < hi) r1 = rows[w0 + HSTEP + lane];
    for (int i = threadIdx.x; i < NB * HFL; i += HBLOCK) {
        if (HCH) L.g[i] = 0;
        L.p[i] = 0;
    }
    int64_t qa[HENT];
    uint32_t ca[HENT];
#pragma unroll
    for (int k = 0; k < HENT; ++k) {
        qa[k] = 0;
        ca[k] = 0;
    }
    float gx = 0.0f, hx = 0.0f;
    uint32_t bj[HFL];
#define YABT_GATHER_BINS(J, R, BASE)                                             \
    {                                                                            \
        const uint32_t rj = row_bcast32<J>(R);                                   \
        bj[J] = ((BASE) + HFL * rg + (J) < hi) ? (uint32_t)fbase[(size_t)rj * ld] : 0u; \
    }
    if (w0 + lane < hi) {
        gx = grad[r0];
        if (HCH) hx = hess[r0];
    }
    YABT_GATHER_BINS(0, r0, w0) YABT_GATHER_BINS(1, r0, w0) YABT_GATHER_BINS(2, r0, w0)
    YABT_GATHER_BINS(3, r0, w0) YABT_GATHER_BINS(4, r0, w0) YABT_GATHER_BINS(5, r0, w0)
    YABT_GATHER_BINS(6, r0, w0) YABT_GATHER_BINS(7, r0, w0) YABT_GATHER_BINS(8, r0, w0)
    YABT_GATHER_BINS(9, r0, w0) YABT_GATHER_BINS(10, r0, w0) YABT_GATHER_BINS(11, r0, w0)
    YABT_GATHER_BINS(12, r0, w0) YABT_GATHER_BINS(13, r0, w0) YABT_GATHER_BINS(14, r0, w0)
    YABT_GATHER_BINS(15, r0, w0)
    __syncthreads();
    const int64_t steps = (hi - lo + HSTEP - 1) / HSTEP;   // the same in every wave: barriers below
    for (int64_t s = 0; s < steps; ++s) {
        const int64_t i0 = w0 + s * HSTEP, i1 = i0 + HSTEP, i2 = i1 + HSTEP;
        // stage: row ids of step s + 2
        uint32_t r2 = 0;
        if (i2 + lane < hi) r2 = rows[i2 + lane];
        // stage: g, h and bins of step s + 1
        float gn = 0.0f, hn = 0.0f;
        if (i1 + lane < hi) {
            gn = grad[r1];
            if (HCH) hn = hess[r1];
        }
        uint32_t bn[HFL];
#define YABT_GATHER_NEXT(J)                                                      \
        {                                                                        \
            const uint32_t rj = row_bcast32<J>(r1);                              \
            bn[J] = (i1 + HFL * rg + (J) < hi) ? (uint32_t)fbase[(size_t)rj * ld] : 0u; \
        }
        YABT_GATHER_NEXT(0) YABT_GATHER_NEXT(1) YABT_GATHER_NEXT(2) YABT_GATHER_NEXT(3)
        YABT_GATHER_NEXT(4) YABT_GATHER_NEXT(5) YABT_GATHER_NEXT(6) YABT_GATHER_NEXT(7)
        YABT_GATHER_NEXT(8) YABT_GATHER_NEXT(9) YABT_GATHER_NEXT(10) YABT_GATHER_NEXT(11)
        YABT_GATHER_NEXT(12) YABT_GATHER_NEXT(13) YABT_GATHER_NEXT(14) YABT_GATHER_NEXT(15)
#undef YABT_GATHER_NEXT
        // step s
        const bool rok = i0 + lane < hi;
        const int64_t gq = rok ? quantise(gx, scg) : 0;
        const int64_t hq = (HCH && rok) ? quantise(hx, sch) : 0;
        const uint64_t gw = HCH ? (uint64_t)gq : ((uint64_t)gq << cb) + 1;
        const uint64_t pw = HCH ? ((uint64_t)hq << cb) + 1 : 0;
#define YABT_GATHER_STEP(J, TAIL)                                                \
        {                                                                        \
            const uint64_t gj = row_bcast64<J>(gw);                              \
            const uint64_t pj = HCH ? row_bcast64<J>(pw) : 0;                     \
            const int b = (int)bj[J];                                            \
            if ((!(TAIL) || (J) < nv) && (!SKIP || b != d)) {                    \
                const int at = b * HFL + fl;                                     \
                if (HCH) {                                                       \
                    atomicAdd(&L.g[at], (unsigned long long)gj);                 \
                    atomicAdd(&L.p[at], (unsigned long long)pj);                 \
                } else {                                                         \
                    atomicAdd(&L.p[at], (unsigned long long)gj);                 \
                }                                                                \
            }                                                                    \
        }
        if (i0 + WAVE <= hi) {   // wave-uniform: all 64 rows valid
            constexpr int nv = HFL;
            YABT_GATHER_STEP(0, 0) YABT_GATHER_STEP(1, 0) YABT_GATHER_STEP(2, 0) YABT_GATHER_STEP(3, 0)
            YABT_GATHER_STEP(4, 0) YABT_GATHER_STEP(5, 0) YABT_GATHER_STEP(6, 0) YABT_GATHER_STEP(7, 0)
            YABT_GATHER_STEP(8, 0) YABT_GATHER_STEP(9, 0) YABT_GATHER_STEP(10, 0) YABT_GATHER_STEP(11, 0)
            YABT_GATHER_STEP(12, 0) YABT_GATHER_STEP(13, 0) YABT_GATHER_STEP(14, 0) YABT_GATHER_STEP(15, 0)
        } else if (i0 < hi) {
            const int nv = (int)min((int64_t)HFL, max((int64_t)0, hi - (i0 + HFL * rg)));
            YABT_GATHER_STEP(0, 1) YABT_GATHER_STEP(1, 1) YABT_GATHER_STEP(2, 1) YABT_GATHER_STEP(3, 1)
            YABT_GATHER_STEP(4, 1) YABT_GATHER_STEP(5, 1) YABT_GATHER_STEP(6, 1) YABT_GATHER_STEP(7, 1)
            YABT_GATHER_STEP(8, 1) YABT_GATHER_STEP(9, 1) YABT_GATHER_STEP(10, 1) YABT_GATHER_STEP(11, 1)
            YABT_GATHER_STEP(12, 1) YABT_GATHER_STEP(13, 1) YABT_GATHER_STEP(14, 1) YABT_GATHER_STEP(15, 1)
        }
#undef YABT_GATHER_STEP
        if ((s + 1) % win_steps == 0 || s + 1 == steps) {
            __syncthreads();
#pragma unroll
            for (int k = 0; k < HENT; ++k) {
                const int i = threadIdx.x + k * HBLOCK;
                const uint64_t v = L.p[i];
                L.p[i] = 0;
                const uint64_t c = v & cmask;
                qa[k] += (int64_t)(v - c) >> cb;
                ca[k] += (uint32_t)c;
            }
            __syncthreads();
        }
        r1 = r2;
        gx = gn;
        hx = hn;
#pragma unroll
        for (int J = 0; J < HFL; ++J) bj[J] = bn[J];
    }
#undef YABT_GATHER_BINS
    uint64_t gv[HENT];
#pragma unroll
    for (int k = 0; k < HENT; ++k) gv[k] = HCH ? L.g[threadIdx.x + k * HBLOCK] : (uint64_t)qa[k];
    __syncthreads();   // every g cell read before the LDS is rewritten
    flush_cells<HCH>(*reinterpret_cast<HistLds*>(&L), gv, qa, ca, out, F, f0);
}

// job->active == 0 or *done != 0 (done may be NULL): nothing to do.  wlog:
// pack_window_log2(n) for the n rows the shifts were chosen for.
static __global__ __attribute__((unused)) void __launch_bounds__(HBLOCK) k_hist_gather(const uint8_t* __restrict__ bins_rm, int64_t ld,
                                                        const float* __restrict__ grad,
                                                        const float* __restrict__ hess, int F, const Quant* q,
                                                        double scg_v, double sch_v,
                                                        const int32_t* __restrict__ dflt, const HistJob* job,
                                                        int count_mode, const int32_t* done, int wlog) {
    // independent loads first: the job record, the done flag, the shifts
    const HistJob jb = *job;
    const int32_t dn = done ? *done : 0;
    const double scg = q ? q->scg : scg_v, sch = q ? q->sch : sch_v;
    const bool no_h = count_mode && q && q->const_h;
    if (dn || !jb.active) return;
    const int tile = blockIdx.x / GATHER_MAX_CHUNKS, chunk = blockIdx.x % GATHER_MAX_CHUNKS;
    __shared__ union {
        HistLds u;
        HistLdsP p;
    } L;
    if (wlog >= 0) {
        if (no_h) {
            if (dflt)
                hist_gather_packed<false, true>(L.p, bins_rm, ld, grad, hess, F, scg, sch, dflt, jb.rows, jb.lo,
                                                jb.hi, jb.out, wlog, tile, chunk);
            else
                hist_gather_packed<false, false>(L.p, bins_rm, ld, grad, hess, F, scg, sch, dflt, jb.rows, jb.lo,
                                                 jb.hi, jb.out, wlog, tile, chunk);
        } else {
            if (dflt)
                hist_gather_packed<true, true>(L.p, bins_rm, ld, grad, hess, F, scg, sch, dflt, jb.rows, jb.lo,
                                               jb.hi, jb.out, wlog, tile, chunk);
            else
                hist_gather_packed<true, false>(L.p, bins_rm, ld, grad, hess, F, scg, sch, dflt, jb.rows, jb.lo,
                                                jb.hi, jb.out, wlog, tile, chunk);
        }
    } else if (no_h) {
        hist_gather_body<false>(L.u, bins_rm, ld, grad, hess, F, scg, sch, dflt, jb.rows, jb.lo, jb.hi, jb.out, tile, chunk);
    } else {
        hist_gather_body<true>(L.u, bins_rm, ld, grad, hess, F, scg, sch, dflt, jb.rows, jb.lo, jb.hi, jb.out, tile, chunk);
    }
}

}  // namespace yabt
