// gfx950 kernels for YABT's best-first (leaf-wise) tree growth.
//
// The path replaced is yabt/_cgrow/grow.c `cgrow` (grow.c:243-427) as called by
// yabt/grow_c.py `grow_tree_c` (grow_c.py:336-452).  One call grows one tree
// entirely on the device: the host enqueues a fixed sequence of launches and
// every launch reads what it has to do from device-resident job records that
// the previous launch wrote, so there is no host round trip per split.
//
// Arithmetic (identical to oracle/grow_oracle.c OR_MODE_FIXED):
//   * g and h are quantised once per call to int64 fixed point with one
//     power-of-two scale each (quant_shift); node histograms are exact integer
//     sums, so accumulation order, the row order inside a node and sibling
//     subtraction (grow.c:355-369) are all exact and deterministic;
//   * the split scan evaluates grow.c's double-precision Newton gain
//     (grow.c:157-176) on the exact prefix sums, with its tie-breaks (lowest
//     bin, then lowest feature, grow.c:170,181-192);
//   * leaf gains are stored as fp32 and the best leaf is picked with strict
//     '>' from 0 (grow.c:284-330), node values use feature 0's 256 bins
//     (grow.c:302-308,371-379).
// Build with -ffp-contract=off: no multiply-add may be fused.
//
// Launch sequence of one tree (all on the caller's stream):
//   k_setup                 max|g|,max|h| -> shifts, table init, clear slot 0
//   k_hist_root             streaming feature-major histogram of all rows
//   k_scan<ROOT>            split scan of the root + controller (first split)
//   repeat max_leaves-1 times (every kernel exits at once when the tree is done):
//     k_part_count          per-block left counts; clear the new slot
//     k_part_scatter        stable partition of the parent's segment
//     k_hist_gather         histogram of the smaller child (row-major gather)
//     k_scan<SPLIT>         sibling = parent - child (in place), scan both
//                           children, controller picks the next split
//
// HBM layout (see yabt_grow_workspace_bytes for the carve):
//   bins_fm (F, ld_fm) u8     feature-major, ld_fm % 16 == 0 (root stream, partition)
//   bins_rm (n, ld_rm) u8     row-major copy, ld_rm % 16 == 0 (child gathers)
//   rows[2] (n) u32           ping-pong row lists; a node at depth d keeps its
//                             rows at [seg_lo, seg_hi) of rows[d & 1] (root: identity)
//   hist   (L, 3, F, 256) i64 one slot per live leaf: the built child takes a new
//                             slot, the sibling is written over its parent's slot

#include "common.h"
#include "yabt_hip.h"

#include <climits>
#include <stdio.h>
#include <string.h>

namespace yabt {

// ---------------------------------------------------------------------------
// device-resident records
// ---------------------------------------------------------------------------

struct Quant {
    int32_t sg, sh;            // shifts
    double scg, sch;           // 2^sg, 2^sh
    double ig, ih;             // 2^-sg, 2^-sh
    uint32_t maxg_bits, maxh_bits;
    int32_t nonfinite;
    uint32_t ticket;
};

struct PartJob {
    int32_t active;
    int32_t f, b;
    int32_t build_left;        // out: 1 if the left child is the one to build
    const uint32_t* src;       // nullptr: row id == position (root)
    uint32_t* dst;
    int64_t s, e;              // parent segment
    int64_t mid;               // out: first right position
    int64_t* zero_ptr;         // slot cleared for the next build
    int64_t zero_count;
};

struct HistJob {
    int32_t active;
    int32_t pad;
    const uint32_t* rows;      // rows of the node, positions [lo, hi)
    int64_t lo, hi;
    int64_t* out;              // [3][F][256], pre-cleared, atomically accumulated
};

struct ScanRec {
    double sel;                // gain * boost[f]
    double gain;               // true gain
    int32_t b;                 // -1: no valid bin
    int32_t pad;
};

struct GrowState {
    int32_t n_nodes, n_leaves, n_active;
    int32_t done;
    int32_t status;
    int32_t k, nid, nl, nr;
    int32_t parent_slot, new_slot;
    uint32_t scan_ticket;
    PartJob part;
    HistJob hist;
};

struct GrowArgs {
    const uint8_t* bins_fm;
    int64_t ld_fm;
    const uint8_t* bins_rm;
    int64_t ld_rm;
    const float* grad;
    const float* hess;
    const uint8_t* fmask;
    const float* imat;
    float ib;
    int use_imat;
    const int32_t* nbins;
    int64_t n;
    int F;
    float lam, gamma, mcw, lr;
    int msl;
    int max_leaves, max_depth;
    // workspace
    GrowState* st;
    Quant* q;
    uint32_t* rows0;
    uint32_t* rows1;
    uint32_t* part_cnt;
    int64_t* hist;
    int32_t* slot_of;
    uint8_t* path;
    int32_t* leaf_node;
    float* leaf_gain;
    int32_t* leaf_f;
    int32_t* leaf_b;
    int64_t* seg_lo;
    int64_t* seg_hi;
    ScanRec* rec;
    int64_t* tot;
    // outputs (device)
    int64_t* feature;
    int64_t* thr_bin;
    int64_t* left;
    int64_t* right;
    float* value;
    int64_t* depth;
    int32_t* out_status;
};

constexpr int BLOCK = 256;
constexpr int PART_IPT = 16;                    // items per thread per tile
constexpr int PART_TILE = BLOCK * PART_IPT;     // 4096 rows
constexpr int PART_MAX_BLOCKS = 1024;
constexpr int HIST_FT = 16;                     // features per histogram tile
constexpr int ROOT_RPT = 16;                    // rows per thread per step (root)
constexpr int GATHER_MIN_ROWS = 4096;           // rows per gather block, at least
constexpr int GATHER_MAX_CHUNKS = 128;

__device__ __forceinline__ size_t slot_elems(int F) { return (size_t)3 * (size_t)F * NB; }

__device__ __forceinline__ bool job_done(const GrowState* st) {
    return st != nullptr && *(volatile const int32_t*)&st->done != 0;
}

// ---------------------------------------------------------------------------
// block helpers
// ---------------------------------------------------------------------------

// Block-wide exclusive scan of one u32 per thread (BLOCK threads = 4 waves).
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* s_wave, uint32_t* total) {
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x >> 6;
    uint32_t ex = wave_excl_scan_u32(v, lane);
    if (lane == WAVE - 1) s_wave[w] = ex + v;
    __syncthreads();
    uint32_t off = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < BLOCK / WAVE; ++i) {
        if (i < w) off += s_wave[i];
        tot += s_wave[i];
    }
    __syncthreads();
    *total = tot;
    return off + ex;
}

template <typename T>
__device__ __forceinline__ T block_sum(T v, T* s_red) {
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x >> 6;
#pragma unroll
    for (int d = WAVE / 2; d > 0; d >>= 1) v += __shfl_xor(v, d, WAVE);
    if (lane == 0) s_red[w] = v;
    __syncthreads();
    T t = 0;
#pragma unroll
    for (int i = 0; i < BLOCK / WAVE; ++i) t += s_red[i];
    __syncthreads();
    return t;
}

// (key, idx) is better than (k2, i2) iff key > k2, or equal keys and idx < i2.
__device__ __forceinline__ bool better(double k1, int i1, double k2, int i2) {
    return k1 > k2 || (k1 == k2 && i1 < i2);
}

// Block argmax over per-thread candidates; invalid candidates carry idx = INT_MAX.
__device__ void block_argmax(double& key, int& idx, double* s_key, int* s_idx) {
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x >> 6;
#pragma unroll
    for (int d = WAVE / 2; d > 0; d >>= 1) {
        double ok = __shfl_xor(key, d, WAVE);
        int oi = __shfl_xor(idx, d, WAVE);
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
    for (int i = 1; i < BLOCK / WAVE; ++i)
        if (better(s_key[i], s_idx[i], key, idx)) {
            key = s_key[i];
            idx = s_idx[i];
        }
    __syncthreads();
}

// Last-block-done: returns true in exactly one block, after every block of
// the grid has passed this point; that block then sees all their writes.
__device__ bool last_block(uint32_t* ticket) {
    __shared__ int s_last;
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t t = atomicAdd(ticket, 1u);
        s_last = (t == gridDim.x - 1);
    }
    __syncthreads();
    if (s_last) {
        __threadfence();
        if (threadIdx.x == 0) *ticket = 0;
    }
    return s_last != 0;
}

// ---------------------------------------------------------------------------
// quantisation setup
// ---------------------------------------------------------------------------

__device__ void quant_reduce(const float* grad, const float* hess, int64_t n, Quant* q) {
    __shared__ float s_m[2][BLOCK / WAVE];
    __shared__ int s_nf;
    if (threadIdx.x == 0) s_nf = 0;
    __syncthreads();
    float mg = 0.0f, mh = 0.0f;
    int nf = 0;
    for (int64_t i = (int64_t)blockIdx.x * BLOCK + threadIdx.x; i < n; i += (int64_t)gridDim.x * BLOCK) {
        const float a = grad[i], c = hess[i];
        if (!isfinite(a) || !isfinite(c)) nf = 1;
        mg = fmaxf(mg, fabsf(a));
        mh = fmaxf(mh, fabsf(c));
    }
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x >> 6;
#pragma unroll
    for (int d = WAVE / 2; d > 0; d >>= 1) {
        mg = fmaxf(mg, __shfl_xor(mg, d, WAVE));
        mh = fmaxf(mh, __shfl_xor(mh, d, WAVE));
    }
    if (nf) atomicOr(&s_nf, 1);
    if (lane == 0) {
        s_m[0][w] = mg;
        s_m[1][w] = mh;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < BLOCK / WAVE; ++i) {
            mg = fmaxf(mg, s_m[0][i]);
            mh = fmaxf(mh, s_m[1][i]);
        }
        // non-negative floats order like their bit patterns
        atomicMax(&q->maxg_bits, __float_as_uint(mg));
        atomicMax(&q->maxh_bits, __float_as_uint(mh));
        if (s_nf) atomicOr(&q->nonfinite, 1);
    }
}

__device__ void quant_finish(Quant* q, int64_t n) {
    const float mg = __uint_as_float(q->maxg_bits), mh = __uint_as_float(q->maxh_bits);
    q->sg = quant_shift(mg, n);
    q->sh = quant_shift(mh, n);
    q->scg = ldexp(1.0, q->sg);
    q->sch = ldexp(1.0, q->sh);
    q->ig = ldexp(1.0, -q->sg);
    q->ih = ldexp(1.0, -q->sh);
}

__global__ void k_quant_clear(Quant* q) {
    q->maxg_bits = 0;
    q->maxh_bits = 0;
    q->nonfinite = 0;
    q->ticket = 0;
}

// Stand-alone quantisation (used by the histogram entry point).
__global__ void __launch_bounds__(BLOCK) k_quant(const float* grad, const float* hess, int64_t n, Quant* q) {
    quant_reduce(grad, hess, n, q);
    if (last_block(&q->ticket) && threadIdx.x == 0) quant_finish(q, n);
}

// Tree setup: quantisation, node-table init, root slot clear, state init.
__global__ void __launch_bounds__(BLOCK) k_setup(GrowArgs A) {
    quant_reduce(A.grad, A.hess, A.n, A.q);
    const int N = 2 * A.max_leaves + 1;
    const int64_t tid = (int64_t)blockIdx.x * BLOCK + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * BLOCK;
    for (int64_t i = tid; i < N; i += stride) {
        A.feature[i] = LEAF;
        A.thr_bin[i] = 0;
        A.left[i] = -1;
        A.right[i] = -1;
        A.value[i] = 0.0f;
        A.depth[i] = 0;
        A.seg_lo[i] = 0;
        A.seg_hi[i] = 0;
        A.slot_of[i] = -1;
    }
    for (int64_t i = tid; i < (int64_t)N * A.F; i += stride) A.path[i] = 0;
    const int64_t ne = (int64_t)slot_elems(A.F);
    for (int64_t i = tid; i < ne; i += stride) A.hist[i] = 0;
    if (last_block(&A.q->ticket) && threadIdx.x == 0) {
        GrowState* st = A.st;
        quant_finish(A.q, A.n);
        st->status = 0;
        st->done = 0;
        if (A.q->nonfinite) {
            st->status = -1;
            st->done = 1;
            A.out_status[0] = -1;
        }
        st->n_nodes = 1;
        st->n_leaves = 1;
        st->n_active = 1;
        st->scan_ticket = 0;
        st->part.active = 0;
        st->hist.active = 0;
        A.seg_lo[0] = 0;
        A.seg_hi[0] = A.n;
        A.slot_of[0] = 0;
    }
}

// ---------------------------------------------------------------------------
// histograms
// ---------------------------------------------------------------------------

// LDS sub-histogram of FT features: exact int64 g/h sums and u32 counts.
template <int FT>
struct HistLds {
    unsigned long long g[FT * NB];
    unsigned long long h[FT * NB];
    uint32_t c[FT * NB];
};

template <int FT>
__device__ __forceinline__ void lds_clear(HistLds<FT>& L) {
    for (int i = threadIdx.x; i < FT * NB; i += BLOCK) {
        L.g[i] = 0;
        L.h[i] = 0;
        L.c[i] = 0;
    }
}

template <int FT>
__device__ __forceinline__ void lds_add(HistLds<FT>& L, int at, int64_t gq, int64_t hq) {
    atomicAdd(&L.g[at], (unsigned long long)gq);
    atomicAdd(&L.h[at], (unsigned long long)hq);
    atomicAdd(&L.c[at], 1u);
}

// Add the block's LDS histogram into out[3][F][256]; empty bins are skipped.
template <int FT>
__device__ __forceinline__ void lds_flush(HistLds<FT>& L, int64_t* out, int F, int f0, int ft) {
    const size_t plane = (size_t)F * NB;
    for (int i = threadIdx.x; i < ft * NB; i += BLOCK) {
        const uint32_t c = L.c[i];
        if (c == 0) continue;
        const size_t at = (size_t)(f0 + i / NB) * NB + (i % NB);
        atomicAdd((unsigned long long*)(out + at), L.g[i]);
        atomicAdd((unsigned long long*)(out + plane + at), L.h[i]);
        atomicAdd((unsigned long long*)(out + 2 * plane + at), (unsigned long long)c);
    }
}

// Streaming histogram of rows [0, n) from the feature-major layout.
// Grid: n_tiles * chunks blocks, chunks % 8 == 0, block -> (tile = bid / chunks,
// chunk = bid % chunks) so every tile of a row chunk runs on the same XCD and
// the chunk's g/h lines are fetched into that XCD's L2 once.
template <int FT>
__global__ void __launch_bounds__(BLOCK) k_hist_root(const uint8_t* __restrict__ bins_fm, int64_t ld,
                                                     const float* __restrict__ grad,
                                                     const float* __restrict__ hess, int64_t n, int F,
                                                     const Quant* __restrict__ q, double scg_v, double sch_v,
                                                     int64_t* out, int chunks, const GrowState* st) {
    if (job_done(st)) return;
    __shared__ HistLds<FT> L;
    const int tile = blockIdx.x / chunks, chunk = blockIdx.x % chunks;
    const int f0 = tile * FT;
    const int ft = min(FT, F - f0);
    const int64_t step = (int64_t)BLOCK * ROOT_RPT;
    const int64_t per = ((n + chunks - 1) / chunks + step - 1) / step * step;
    const int64_t lo = (int64_t)chunk * per, hi = min(n, lo + per);
    if (ft <= 0 || lo >= hi) return;
    lds_clear(L);
    __syncthreads();
    const double scg = q ? q->scg : scg_v, sch = q ? q->sch : sch_v;
    for (int64_t r0 = lo + (int64_t)threadIdx.x * ROOT_RPT; r0 < hi; r0 += step) {
        int64_t gq[ROOT_RPT], hq[ROOT_RPT];
        const int nv = (int)min((int64_t)ROOT_RPT, hi - r0);
        if (nv == ROOT_RPT) {
            const float4* g4 = reinterpret_cast<const float4*>(grad + r0);
            const float4* h4 = reinterpret_cast<const float4*>(hess + r0);
#pragma unroll
            for (int v = 0; v < ROOT_RPT / 4; ++v) {
                const float4 a = g4[v], c = h4[v];
                gq[4 * v + 0] = quantise(a.x, scg);
                gq[4 * v + 1] = quantise(a.y, scg);
                gq[4 * v + 2] = quantise(a.z, scg);
                gq[4 * v + 3] = quantise(a.w, scg);
                hq[4 * v + 0] = quantise(c.x, sch);
                hq[4 * v + 1] = quantise(c.y, sch);
                hq[4 * v + 2] = quantise(c.z, sch);
                hq[4 * v + 3] = quantise(c.w, sch);
            }
        } else {
#pragma unroll
            for (int j = 0; j < ROOT_RPT; ++j) {
                gq[j] = j < nv ? quantise(grad[r0 + j], scg) : 0;
                hq[j] = j < nv ? quantise(hess[r0 + j], sch) : 0;
            }
        }
        for (int f = 0; f < ft; ++f) {
            // r0 % 16 == 0 and ld % 16 == 0, r0 < n <= ld: the 16-byte load stays in the row
            const uint4 bv = *reinterpret_cast<const uint4*>(bins_fm + (size_t)(f0 + f) * ld + r0);
            const uint32_t w4[4] = {bv.x, bv.y, bv.z, bv.w};
            const int base = f * NB;
            if (nv == ROOT_RPT) {
#pragma unroll
                for (int j = 0; j < ROOT_RPT; ++j)
                    lds_add(L, base + (int)((w4[j >> 2] >> (8 * (j & 3))) & 0xffu), gq[j], hq[j]);
            } else {
                for (int j = 0; j < nv; ++j)
                    lds_add(L, base + (int)((w4[j >> 2] >> (8 * (j & 3))) & 0xffu), gq[j], hq[j]);
            }
        }
    }
    __syncthreads();
    lds_flush(L, out, F, f0, ft);
}

// Histogram of the rows listed at positions [lo, hi) of job->rows, read
// through the row-major copy.  Grid: n_tiles * GATHER_MAX_CHUNKS blocks; the
// number of chunks in use shrinks with the node so small nodes flush little.
template <int FT>
__global__ void __launch_bounds__(BLOCK) k_hist_gather(const uint8_t* __restrict__ bins_rm, int64_t ld,
                                                       const float* __restrict__ grad,
                                                       const float* __restrict__ hess, int F,
                                                       const Quant* __restrict__ q, double scg_v, double sch_v,
                                                       const HistJob* job, const GrowState* st) {
    if (job_done(st)) return;
    if (!job->active) return;
    __shared__ HistLds<FT> L;
    const int chunks_max = GATHER_MAX_CHUNKS;
    const int tile = blockIdx.x / chunks_max, chunk = blockIdx.x % chunks_max;
    const int f0 = tile * FT;
    const int ft = min(FT, F - f0);
    const int64_t jlo = job->lo, jhi = job->hi, m = jhi - jlo;
    if (ft <= 0 || m <= 0) return;
    const int64_t want = (m + GATHER_MIN_ROWS - 1) / GATHER_MIN_ROWS;
    const int nch = (int)min((int64_t)chunks_max, want);
    if (chunk >= nch) return;
    const int64_t per = (m + nch - 1) / nch;
    const int64_t lo = jlo + (int64_t)chunk * per, hi = min(jhi, lo + per);
    if (lo >= hi) return;
    lds_clear(L);
    __syncthreads();
    const double scg = q ? q->scg : scg_v, sch = q ? q->sch : sch_v;
    const uint32_t* rows = job->rows;
    for (int64_t i = lo + threadIdx.x; i < hi; i += BLOCK) {
        const uint32_t r = rows[i];
        const int64_t gq = quantise(grad[r], scg), hq = quantise(hess[r], sch);
        // ld % 16 == 0 and f0 % 16 == 0: aligned 16-byte load inside the row
        const uint4 bv = *reinterpret_cast<const uint4*>(bins_rm + (size_t)r * ld + f0);
        const uint32_t w4[4] = {bv.x, bv.y, bv.z, bv.w};
        if (ft == FT) {
#pragma unroll
            for (int f = 0; f < FT; ++f)
                lds_add(L, f * NB + (int)((w4[f >> 2] >> (8 * (f & 3))) & 0xffu), gq, hq);
        } else {
            for (int f = 0; f < ft; ++f)
                lds_add(L, f * NB + (int)((w4[f >> 2] >> (8 * (f & 3))) & 0xffu), gq, hq);
        }
    }
    __syncthreads();
    lds_flush(L, job->out, F, f0, ft);
}

// ---------------------------------------------------------------------------
// partition (stable; membership equals grow.c:201-217's two-pointer result)
// ---------------------------------------------------------------------------

struct PartRange {
    int nblk;
    int64_t lo, hi;
};

__device__ __forceinline__ PartRange part_range(int64_t s, int64_t e) {
    PartRange r;
    const int64_t m = e - s;
    const int64_t tiles = (m + PART_TILE - 1) / PART_TILE;
    r.nblk = (int)min((int64_t)gridDim.x, max(tiles, (int64_t)1));
    const int64_t tpb = (tiles + r.nblk - 1) / r.nblk;
    r.lo = s + (int64_t)blockIdx.x * tpb * PART_TILE;
    r.hi = min(e, r.lo + tpb * PART_TILE);
    if (r.lo > e) r.lo = e;
    return r;
}

__device__ __forceinline__ uint32_t part_row(const PartJob& J, int64_t i) {
    return J.src ? J.src[i] : (uint32_t)i;
}

__global__ void __launch_bounds__(BLOCK) k_part_count(const uint8_t* __restrict__ bins_fm, int64_t ld,
                                                      PartJob* jp, uint32_t* cnt, const GrowState* st) {
    if (job_done(st)) return;
    const PartJob J = *jp;
    if (!J.active) return;
    if (J.zero_ptr)
        for (int64_t i = (int64_t)blockIdx.x * BLOCK + threadIdx.x; i < J.zero_count;
             i += (int64_t)gridDim.x * BLOCK)
            J.zero_ptr[i] = 0;
    const PartRange R = part_range(J.s, J.e);
    if ((int)blockIdx.x >= R.nblk) return;
    const uint8_t* col = bins_fm + (size_t)J.f * ld;
    uint32_t c = 0;
    for (int64_t i = R.lo + threadIdx.x; i < R.hi; i += BLOCK) c += (int)col[part_row(J, i)] <= J.b;
    __shared__ uint32_t s_red[BLOCK / WAVE];
    c = block_sum<uint32_t>(c, s_red);
    if (threadIdx.x == 0) cnt[blockIdx.x] = c;
}

__global__ void __launch_bounds__(BLOCK) k_part_scatter(const uint8_t* __restrict__ bins_fm, int64_t ld,
                                                        PartJob* jp, const uint32_t* cnt, HistJob* hj,
                                                        const GrowState* st) {
    if (job_done(st)) return;
    const PartJob J = *jp;
    if (!J.active) return;
    const PartRange R = part_range(J.s, J.e);
    if ((int)blockIdx.x >= R.nblk) return;
    __shared__ uint32_t s_red[BLOCK / WAVE];
    // lefts in earlier blocks and in all blocks
    uint64_t before = 0, total = 0;
    for (int j = threadIdx.x; j < R.nblk; j += BLOCK) {
        const uint64_t c = cnt[j];
        total += c;
        if (j < (int)blockIdx.x) before += c;
    }
    __shared__ uint64_t s_red64[BLOCK / WAVE];
    before = block_sum<uint64_t>(before, s_red64);
    total = block_sum<uint64_t>(total, s_red64);
    const int64_t mid = J.s + (int64_t)total;
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        const int bl = (mid - J.s) <= (J.e - mid);
        jp->mid = mid;
        jp->build_left = bl;
        if (hj) {
            hj->rows = J.dst;
            hj->lo = bl ? J.s : mid;
            hj->hi = bl ? mid : J.e;
            hj->active = 1;
        }
    }
    const uint8_t* col = bins_fm + (size_t)J.f * ld;
    int64_t run_l = (int64_t)before;                       // lefts placed before this tile
    int64_t run_r = (R.lo - J.s) - (int64_t)before;        // rights placed before this tile
    for (int64_t t0 = R.lo; t0 < R.hi; t0 += PART_TILE) {
        const int64_t a = t0 + (int64_t)threadIdx.x * PART_IPT;
        uint32_t rid[PART_IPT];
        uint32_t flags = 0, nv = 0;
#pragma unroll
        for (int j = 0; j < PART_IPT; ++j) {
            const int64_t i = a + j;
            if (i < R.hi) {
                rid[j] = part_row(J, i);
                flags |= ((int)col[rid[j]] <= J.b ? 1u : 0u) << j;
                ++nv;
            }
        }
        const uint32_t nl = __popc(flags), nr = nv - nl;
        uint32_t tl, tr;
        const uint32_t ol = block_excl_scan(nl, s_red, &tl);
        const uint32_t orr = block_excl_scan(nr, s_red, &tr);
        int64_t pl = J.s + run_l + ol, pr = mid + run_r + orr;
#pragma unroll
        for (int j = 0; j < PART_IPT; ++j) {
            if ((uint32_t)j < nv) {
                if ((flags >> j) & 1u) J.dst[pl++] = rid[j];
                else J.dst[pr++] = rid[j];
            }
        }
        run_l += tl;
        run_r += tr;
    }
}

// ---------------------------------------------------------------------------
// split scan
// ---------------------------------------------------------------------------

struct ScanParams {
    double lam, gamma, mcw;
    int msl;
};

// One wave scans feature f of one node: lane l owns bins 4l..4l+3.
// qg/qh/qc point at the feature's 256 bins.  Returns the record in every lane;
// *t256 receives the (g, h) totals over all 256 bins (used for node values).
__device__ ScanRec scan_feature(const int64_t g4[4], const int64_t h4[4], const int64_t c4[4], int nb,
                                double ig, double ih, const ScanParams& sp, double bo, int lane,
                                int64_t* t256g, int64_t* t256h) {
    int64_t pg[4], ph[4], pc[4];
    pg[0] = g4[0];
    ph[0] = h4[0];
    pc[0] = c4[0];
#pragma unroll
    for (int j = 1; j < 4; ++j) {
        pg[j] = pg[j - 1] + g4[j];
        ph[j] = ph[j - 1] + h4[j];
        pc[j] = pc[j - 1] + c4[j];
    }
    const int64_t og = wave_excl_scan(pg[3], lane);
    const int64_t oh = wave_excl_scan(ph[3], lane);
    const int64_t oc = wave_excl_scan(pc[3], lane);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        pg[j] += og;
        ph[j] += oh;
        pc[j] += oc;
    }
    *t256g = __shfl(pg[3], WAVE - 1, WAVE);
    *t256h = __shfl(ph[3], WAVE - 1, WAVE);
    // totals over the feature's used bins b < nb (grow.c:151-156)
    int64_t Gt = 0, Ht = 0, Ct = 0;
    if (nb > 0) {
        const int jj = (nb - 1) & 3, src = (nb - 1) >> 2;
        int64_t vg = pg[0], vh = ph[0], vc = pc[0];
#pragma unroll
        for (int j = 1; j < 4; ++j)
            if (jj == j) {
                vg = pg[j];
                vh = ph[j];
                vc = pc[j];
            }
        Gt = __shfl(vg, src, WAVE);
        Ht = __shfl(vh, src, WAVE);
        Ct = __shfl(vc, src, WAVE);
    }
    const double G = (double)Gt * ig, H = (double)Ht * ih;
    const double parent = G * G / (H + sp.lam);
    ScanRec r;
    r.sel = -INFINITY;
    r.gain = -INFINITY;
    r.b = -1;
    r.pad = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int b = 4 * lane + j;
        if (b + 1 < nb) {
            const int64_t cl = pc[j], cr = Ct - pc[j];
            const double GL = (double)pg[j] * ig, GR = (double)(Gt - pg[j]) * ig;
            const double HL = (double)ph[j] * ih, HR = (double)(Ht - ph[j]) * ih;
            if (cl >= sp.msl && cr >= sp.msl && HL >= sp.mcw && HR >= sp.mcw) {
                const double gain =
                    0.5 * (GL * GL / (HL + sp.lam) + GR * GR / (HR + sp.lam) - parent) - sp.gamma;
                const double sel = gain * bo;
                if (sel > r.sel) {
                    r.sel = sel;
                    r.gain = gain;
                    r.b = b;
                }
            }
        }
    }
    // wave argmax: larger sel, then lower bin; lanes without a valid bin lose
#pragma unroll
    for (int d = WAVE / 2; d > 0; d >>= 1) {
        const double os = __shfl_xor(r.sel, d, WAVE);
        const double og2 = __shfl_xor(r.gain, d, WAVE);
        const int ob = __shfl_xor(r.b, d, WAVE);
        const bool take = ob >= 0 && (r.b < 0 || os > r.sel || (os == r.sel && ob < r.b));
        if (take) {
            r.sel = os;
            r.gain = og2;
            r.b = ob;
        }
    }
    return r;
}

// boost[f] = 1 + ib * max(0, max_{p on path} imat[p][f]) in fp32 (grow.c:111-122)
__device__ float path_boost(const uint8_t* path, const float* imat, float ib, int F, int f, int lane) {
    float m = 0.0f;
    for (int p = lane; p < F; p += WAVE)
        if (path[p]) {
            const float v = imat[(size_t)p * F + f];
            if (v > m) m = v;
        }
#pragma unroll
    for (int d = WAVE / 2; d > 0; d >>= 1) {
        const float o = __shfl_xor(m, d, WAVE);
        if (o > m) m = o;
    }
    return 1.0f + ib * m;
}

__device__ __forceinline__ void load_bins(const int64_t* slot, int F, int f, int lane, int64_t g4[4],
                                          int64_t h4[4], int64_t c4[4]) {
    const size_t plane = (size_t)F * NB, at = (size_t)f * NB + 4 * lane;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        g4[j] = slot[at + j];
        h4[j] = slot[plane + at + j];
        c4[j] = slot[2 * plane + at + j];
    }
}

// Feature-major reduction of one node's records (grow.c:181-192).
__device__ void reduce_records(const ScanRec* rec, int F, double* gain, int* f_out, int* b_out) {
    __shared__ double s_key[BLOCK / WAVE];
    __shared__ int s_idx[BLOCK / WAVE];
    double key = -INFINITY;
    int idx = INT_MAX;
    for (int f = threadIdx.x; f < F; f += BLOCK) {
        const ScanRec r = rec[f];
        if (r.b >= 0 && better(r.sel, f, key, idx)) {
            key = r.sel;
            idx = f;
        }
    }
    block_argmax(key, idx, s_key, s_idx);
    if (idx == INT_MAX) {
        *gain = -INFINITY;
        *f_out = -1;
        *b_out = -1;
    } else {
        *gain = rec[idx].gain;
        *f_out = idx;
        *b_out = rec[idx].b;
    }
}

__device__ float node_value(int64_t tg, int64_t th, const Quant* q, float lr, float lam) {
    const double G = (double)tg * q->ig, H = (double)th * q->ih;
    return (float)(-lr * G / (H + lam));
}

// Pick the next split (grow.c:321-350) or finish the tree.  One block.
__device__ void controller_next(const GrowArgs& A) {
    GrowState* st = A.st;
    __shared__ double s_key[BLOCK / WAVE];
    __shared__ int s_idx[BLOCK / WAVE];
    __shared__ int s_k;
    const int n_active = st->n_active;
    if (st->n_leaves >= A.max_leaves) {
        if (threadIdx.x == 0) s_k = -1;
    } else {
        double key = -INFINITY;
        int idx = INT_MAX;
        for (int a = threadIdx.x; a < n_active; a += BLOCK) {
            const float g = A.leaf_gain[a];
            if (g > 0.0f && better((double)g, a, key, idx)) {
                key = (double)g;
                idx = a;
            }
        }
        block_argmax(key, idx, s_key, s_idx);
        if (threadIdx.x == 0) s_k = (idx == INT_MAX) ? -1 : idx;
    }
    __syncthreads();
    const int k = s_k;
    if (k < 0) {
        if (threadIdx.x == 0) {
            st->done = 1;
            st->part.active = 0;
            st->hist.active = 0;
            A.out_status[0] = st->n_nodes;
        }
        return;
    }
    const int nid = A.leaf_node[k];
    const int f = A.leaf_f[k], b = A.leaf_b[k];
    const int nl = st->n_nodes, nr = st->n_nodes + 1;
    const int64_t d = A.depth[nid];
    // children inherit the parent's path plus f (grow.c:347-350)
    const uint8_t* pp = A.path + (size_t)nid * A.F;
    uint8_t* pl = A.path + (size_t)nl * A.F;
    uint8_t* pr = A.path + (size_t)nr * A.F;
    for (int j = threadIdx.x; j < A.F; j += BLOCK) {
        const uint8_t v = (j == f) ? (uint8_t)1 : pp[j];
        pl[j] = v;
        pr[j] = v;
    }
    if (threadIdx.x == 0) {
        st->k = k;
        st->nid = nid;
        st->nl = nl;
        st->nr = nr;
        st->n_nodes = nl + 2;
        st->n_leaves += 1;
        st->parent_slot = A.slot_of[nid];
        st->new_slot = st->n_leaves - 1;
        A.depth[nl] = d + 1;
        A.depth[nr] = d + 1;
        A.feature[nid] = f;
        A.thr_bin[nid] = b;
        A.left[nid] = nl;
        A.right[nid] = nr;
        A.value[nid] = 0.0f;
        PartJob& J = st->part;
        J.f = f;
        J.b = b;
        J.s = A.seg_lo[nid];
        J.e = A.seg_hi[nid];
        J.src = (d == 0) ? nullptr : ((d & 1) ? A.rows1 : A.rows0);
        J.dst = ((d + 1) & 1) ? A.rows1 : A.rows0;
        J.zero_ptr = A.hist + (size_t)st->new_slot * slot_elems(A.F);
        J.zero_count = (int64_t)slot_elems(A.F);
        J.mid = 0;
        J.build_left = 1;
        J.active = 1;
        st->hist.out = J.zero_ptr;
        st->hist.active = 0;  // set by k_part_scatter once the segment is known
    }
}

template <bool ROOT>
__global__ void __launch_bounds__(BLOCK) k_scan(GrowArgs A) {
    GrowState* st = A.st;
    if (job_done(st)) return;
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x >> 6;
    const int f = blockIdx.x * (BLOCK / WAVE) + w;
    const ScanParams sp = {(double)A.lam, (double)A.gamma, (double)A.mcw, A.msl};
    const Quant* q = A.q;
    if (f < A.F) {
        const int nb = max(0, min(NB, A.nbins[f]));
        const bool use = A.fmask[f] != 0;
        if (ROOT) {
            int64_t g4[4], h4[4], c4[4], tg, th;
            load_bins(A.hist, A.F, f, lane, g4, h4, c4);
            ScanRec r = scan_feature(g4, h4, c4, nb, q->ig, q->ih, sp, 1.0, lane, &tg, &th);
            if (!use) {
                r.sel = -INFINITY;
                r.gain = -INFINITY;
                r.b = -1;
            }
            if (lane == 0) {
                A.rec[f] = r;
                if (f == 0) {
                    A.tot[0] = tg;
                    A.tot[1] = th;
                }
            }
        } else {
            const int nl = st->nl, nr = st->nr;
            const int bl = st->part.build_left;
            int64_t* hp = A.hist + (size_t)st->parent_slot * slot_elems(A.F);
            const int64_t* hn = A.hist + (size_t)st->new_slot * slot_elems(A.F);
            // sibling = parent - built child, written over the parent's slot
            int64_t bg[4], bh[4], bc[4], sg4[4], sh4[4], sc4[4];
            load_bins(hn, A.F, f, lane, bg, bh, bc);
            load_bins(hp, A.F, f, lane, sg4, sh4, sc4);
            const size_t plane = (size_t)A.F * NB, at = (size_t)f * NB + 4 * lane;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                sg4[j] -= bg[j];
                sh4[j] -= bh[j];
                sc4[j] -= bc[j];
                hp[at + j] = sg4[j];
                hp[plane + at + j] = sh4[j];
                hp[2 * plane + at + j] = sc4[j];
            }
            const float bo = (A.use_imat && use) ? path_boost(A.path + (size_t)nl * A.F, A.imat, A.ib, A.F, f, lane)
                                                 : 1.0f;
            for (int c = 0; c < 2; ++c) {
                const bool built = (c == 0) == (bl != 0);
                int64_t tg, th;
                ScanRec r = built ? scan_feature(bg, bh, bc, nb, q->ig, q->ih, sp, (double)bo, lane, &tg, &th)
                                  : scan_feature(sg4, sh4, sc4, nb, q->ig, q->ih, sp, (double)bo, lane, &tg, &th);
                if (!use) {
                    r.sel = -INFINITY;
                    r.gain = -INFINITY;
                    r.b = -1;
                }
                if (lane == 0) {
                    A.rec[(size_t)c * A.F + f] = r;
                    if (f == 0) {
                        A.tot[2 * c + 0] = tg;
                        A.tot[2 * c + 1] = th;
                    }
                }
            }
            (void)nr;
        }
    }
    if (!last_block(&st->scan_ticket)) return;

    // ---- controller (one block) ----
    __shared__ double s_gain[2];
    __shared__ int s_f[2], s_b[2];
    if (ROOT) {
        double g0;
        int f0, b0;
        reduce_records(A.rec, A.F, &g0, &f0, &b0);
        if (threadIdx.x == 0) {
            if (0 >= A.max_depth) g0 = -INFINITY;
            A.value[0] = node_value(A.tot[0], A.tot[1], q, A.lr, A.lam);
            A.leaf_node[0] = 0;
            A.leaf_gain[0] = (float)g0;
            A.leaf_f[0] = f0;
            A.leaf_b[0] = b0;
            st->n_nodes = 1;
            st->n_leaves = 1;
            st->n_active = 1;
        }
        __syncthreads();
        controller_next(A);
        return;
    }
    for (int c = 0; c < 2; ++c) {
        double g;
        int bf, bb;
        reduce_records(A.rec + (size_t)c * A.F, A.F, &g, &bf, &bb);
        if (threadIdx.x == 0) {
            s_gain[c] = g;
            s_f[c] = bf;
            s_b[c] = bb;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const int nl = st->nl, nr = st->nr, k = st->k;
        const int64_t d = A.depth[nl];
        const int bl = st->part.build_left;
        const int64_t mid = st->part.mid;
        A.seg_lo[nl] = st->part.s;
        A.seg_hi[nl] = mid;
        A.seg_lo[nr] = mid;
        A.seg_hi[nr] = st->part.e;
        A.slot_of[bl ? nl : nr] = st->new_slot;
        A.slot_of[bl ? nr : nl] = st->parent_slot;
        A.value[nl] = node_value(A.tot[0], A.tot[1], q, A.lr, A.lam);
        A.value[nr] = node_value(A.tot[2], A.tot[3], q, A.lr, A.lam);
        double gl = s_gain[0], gr = s_gain[1];
        if (d >= A.max_depth) {
            gl = -INFINITY;
            gr = -INFINITY;
        }
        A.leaf_node[k] = nl;
        A.leaf_gain[k] = (float)gl;
        A.leaf_f[k] = s_f[0];
        A.leaf_b[k] = s_b[0];
        const int na = st->n_active;
        A.leaf_node[na] = nr;
        A.leaf_gain[na] = (float)gr;
        A.leaf_f[na] = s_f[1];
        A.leaf_b[na] = s_b[1];
        st->n_active = na + 1;
        st->part.active = 0;
        st->hist.active = 0;
    }
    __syncthreads();
    controller_next(A);
}

// ---------------------------------------------------------------------------
// leaf ids, apply, transpose
// ---------------------------------------------------------------------------

// out[row] = leaf node id, from each leaf's segment of the final row lists.
// Grid (chunks, nodes).
__global__ void __launch_bounds__(BLOCK) k_leaf_ids(const int64_t* feature, const int64_t* depth,
                                                    const int64_t* seg_lo, const int64_t* seg_hi,
                                                    const uint32_t* rows0, const uint32_t* rows1,
                                                    const int32_t* out_status, int64_t* out) {
    const int nid = blockIdx.y;
    if (nid >= out_status[0] || feature[nid] != LEAF) return;
    const int64_t lo = seg_lo[nid], hi = seg_hi[nid], d = depth[nid];
    const uint32_t* rows = (d == 0) ? nullptr : ((d & 1) ? rows1 : rows0);
    for (int64_t i = lo + (int64_t)blockIdx.x * BLOCK + threadIdx.x; i < hi; i += (int64_t)gridDim.x * BLOCK) {
        const int64_t r = rows ? (int64_t)rows[i] : i;
        out[r] = nid;
    }
}

// Row routing on raw X (n, F) row-major, x[f] <= threshold goes left
// (grow.c:223-239, tree.py:97-116).
__global__ void __launch_bounds__(BLOCK) k_apply(const float* __restrict__ X, int64_t ldx,
                                                 const int64_t* __restrict__ feature,
                                                 const float* __restrict__ threshold,
                                                 const int64_t* __restrict__ left,
                                                 const int64_t* __restrict__ right, int64_t n, int max_steps,
                                                 int64_t* out) {
    for (int64_t r = (int64_t)blockIdx.x * BLOCK + threadIdx.x; r < n; r += (int64_t)gridDim.x * BLOCK) {
        const float* x = X + (size_t)r * ldx;
        int64_t node = 0;
        for (int s = 0; s < max_steps; ++s) {
            const int64_t f = feature[node];
            if (f < 0) break;
            node = (x[f] <= threshold[node]) ? left[node] : right[node];
        }
        out[r] = node;
    }
}

// (F, ld_fm) feature-major -> (n, ld_rm) row-major, 64x64 byte tiles via LDS.
__global__ void __launch_bounds__(BLOCK) k_transpose(const uint8_t* __restrict__ src, int64_t ld_src, int64_t n,
                                                     int F, uint8_t* __restrict__ dst, int64_t ld_dst) {
    __shared__ uint8_t t[64][65];
    const int64_t r0 = (int64_t)blockIdx.x * 64;
    const int f0 = blockIdx.y * 64;
    for (int i = threadIdx.x; i < 64 * 64; i += BLOCK) {
        const int fi = i / 64, ri = i % 64;
        const int64_t r = r0 + ri;
        const int f = f0 + fi;
        t[fi][ri] = (r < n && f < F) ? src[(size_t)f * ld_src + r] : (uint8_t)0;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 64 * 64; i += BLOCK) {
        const int ri = i / 64, fi = i % 64;
        const int64_t r = r0 + ri;
        const int f = f0 + fi;
        if (r < n && f < ld_dst) dst[(size_t)r * ld_dst + f] = t[fi][ri];
    }
}

__global__ void k_fill_i64(int64_t* p, int64_t v, int64_t count) {
    for (int64_t i = (int64_t)blockIdx.x * BLOCK + threadIdx.x; i < count; i += (int64_t)gridDim.x * BLOCK)
        p[i] = v;
}

__global__ void k_set_hist_job(HistJob* j, const uint32_t* rows, int64_t lo, int64_t hi, int64_t* out) {
    j->active = 1;
    j->rows = rows;
    j->lo = lo;
    j->hi = hi;
    j->out = out;
}

__global__ void k_set_part_job(PartJob* j, const uint32_t* src, uint32_t* dst, int64_t s, int64_t e, int f, int b) {
    j->active = 1;
    j->f = f;
    j->b = b;
    j->src = src;
    j->dst = dst;
    j->s = s;
    j->e = e;
    j->mid = 0;
    j->build_left = 1;
    j->zero_ptr = nullptr;
    j->zero_count = 0;
}

__global__ void k_zero_u32(uint32_t* p) { *p = 0; }

__global__ void k_copy_mid(const PartJob* j, int64_t* out) { out[0] = j->mid; }

// Stand-alone scan of one histogram with explicit shifts and boosts.
__global__ void __launch_bounds__(BLOCK) k_scan_one(const int64_t* hist, int F, const int32_t* nbins,
                                                    const uint8_t* fmask, const float* boost, int sg, int sh,
                                                    ScanParams sp, ScanRec* rec, uint32_t* ticket,
                                                    double* out_gain, int32_t* out_fb) {
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x >> 6;
    const int f = blockIdx.x * (BLOCK / WAVE) + w;
    if (f < F) {
        int64_t g4[4], h4[4], c4[4], tg, th;
        load_bins(hist, F, f, lane, g4, h4, c4);
        const int nb = max(0, min(NB, nbins[f]));
        ScanRec r = scan_feature(g4, h4, c4, nb, ldexp(1.0, -sg), ldexp(1.0, -sh), sp,
                                 (double)(boost ? boost[f] : 1.0f), lane, &tg, &th);
        if (!fmask[f]) {
            r.sel = -INFINITY;
            r.gain = -INFINITY;
            r.b = -1;
        }
        if (lane == 0) rec[f] = r;
    }
    if (!last_block(ticket)) return;
    double g;
    int bf, bb;
    reduce_records(rec, F, &g, &bf, &bb);
    if (threadIdx.x == 0) {
        out_gain[0] = g;
        out_fb[0] = bf;
        out_fb[1] = bb;
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

thread_local char g_err[512] = "";

int fail(int code, const char* msg) {
    snprintf(g_err, sizeof g_err, "%s", msg);
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    snprintf(g_err, sizeof g_err, "%s: %s", what, hipGetErrorString(e));
    return -100;
}

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

struct Carve {
    char* base;
    size_t off;
    template <typename T>
    T* take(size_t count) {
        off = align_up(off, 256);
        T* p = base ? reinterpret_cast<T*>(base + off) : nullptr;
        off += count * sizeof(T);
        return p;
    }
};

size_t carve_grow(char* base, int64_t n, int F, int max_leaves, GrowArgs* A) {
    Carve c{base, 0};
    const size_t N = (size_t)(2 * max_leaves + 1);
    GrowArgs tmp;
    GrowArgs& a = A ? *A : tmp;
    a.st = c.take<GrowState>(1);
    a.q = c.take<Quant>(1);
    a.rows0 = c.take<uint32_t>((size_t)(n > 0 ? n : 1));
    a.rows1 = c.take<uint32_t>((size_t)(n > 0 ? n : 1));
    a.part_cnt = c.take<uint32_t>(PART_MAX_BLOCKS);
    a.hist = c.take<int64_t>((size_t)max_leaves * 3 * (size_t)F * NB);
    a.slot_of = c.take<int32_t>(N);
    a.path = c.take<uint8_t>(N * (size_t)F);
    a.leaf_node = c.take<int32_t>(N);
    a.leaf_gain = c.take<float>(N);
    a.leaf_f = c.take<int32_t>(N);
    a.leaf_b = c.take<int32_t>(N);
    a.seg_lo = c.take<int64_t>(N);
    a.seg_hi = c.take<int64_t>(N);
    a.rec = c.take<ScanRec>((size_t)2 * F);
    a.tot = c.take<int64_t>(4);
    return align_up(c.off, 256);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int launch_grid(int64_t work, int per_block, int cap) {
    int64_t g = (work + per_block - 1) / per_block;
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return (int)g;
}

int root_chunks(int64_t n, int tiles) {
    // ~2 resident blocks per CU on 256 CUs; chunks a multiple of 8 (one XCD each)
    int want = (512 + tiles - 1) / tiles;
    const int64_t max_useful = (n + (int64_t)BLOCK * ROOT_RPT - 1) / ((int64_t)BLOCK * ROOT_RPT);
    if (want > max_useful) want = (int)max_useful;
    if (want < 1) want = 1;
    return (want + 7) / 8 * 8;
}

}  // namespace yabt

using namespace yabt;

extern "C" {

const char* yabt_last_error(void) { return g_err; }

size_t yabt_grow_workspace_bytes(int64_t n, int F, int max_leaves) {
    if (n < 0 || F < 1 || max_leaves < 1) return 0;
    return carve_grow(nullptr, n, F, max_leaves, nullptr);
}

int yabt_grow(const uint8_t* bins_fm, int64_t ld_fm, const uint8_t* bins_rm, int64_t ld_rm, const float* grad,
              const float* hess, const uint8_t* fmask, const float* imat, float ib, int use_imat,
              const int32_t* nbins, int64_t n, int F, float lam, float gamma, float mcw, int msl, float lr,
              int max_leaves, int max_depth, void* workspace, size_t workspace_bytes, int64_t* out_feature,
              int64_t* out_thr_bin, int64_t* out_left, int64_t* out_right, float* out_value,
              int64_t* out_depth, int32_t* out_status, hipStream_t stream) {
    if (F < 1 || n < 0 || n > 0xFFFFFFFFll || max_leaves < 1 || max_leaves > 32767)
        return fail(-2, "yabt_grow: bad sizes (need F >= 1, 0 <= n < 2^32, 1 <= max_leaves <= 32767)");
    if (ld_fm < n || ld_fm % 16 || ld_rm < F || ld_rm % 16)
        return fail(-2, "yabt_grow: leading dimensions must be multiples of 16 covering n (bins_fm) and F (bins_rm)");
    if (!bins_fm || !bins_rm || !grad || !hess || !fmask || !nbins || (use_imat && !imat) || !workspace ||
        !out_feature || !out_thr_bin || !out_left || !out_right || !out_value || !out_depth || !out_status)
        return fail(-2, "yabt_grow: null pointer argument");
    if (!aligned16(bins_fm) || !aligned16(bins_rm) || !aligned16(grad) || !aligned16(hess))
        return fail(-2, "yabt_grow: bins, grad and hess must be 16-byte aligned");
    GrowArgs A;
    memset(&A, 0, sizeof A);
    const size_t need = carve_grow((char*)workspace, n, F, max_leaves, &A);
    if (workspace_bytes < need) return fail(-2, "yabt_grow: workspace too small");
    A.bins_fm = bins_fm;
    A.ld_fm = ld_fm;
    A.bins_rm = bins_rm;
    A.ld_rm = ld_rm;
    A.grad = grad;
    A.hess = hess;
    A.fmask = fmask;
    A.imat = imat;
    A.ib = ib;
    A.use_imat = use_imat ? 1 : 0;
    A.nbins = nbins;
    A.n = n;
    A.F = F;
    A.lam = lam;
    A.gamma = gamma;
    A.mcw = mcw;
    A.lr = lr;
    A.msl = msl;
    A.max_leaves = max_leaves;
    A.max_depth = max_depth;
    A.feature = out_feature;
    A.thr_bin = out_thr_bin;
    A.left = out_left;
    A.right = out_right;
    A.value = out_value;
    A.depth = out_depth;
    A.out_status = out_status;

    const int tiles = (F + HIST_FT - 1) / HIST_FT;
    const int setup_grid = launch_grid(n, BLOCK * 16, 1024);
    k_quant_clear<<<1, 1, 0, stream>>>(A.q);
    k_setup<<<setup_grid, BLOCK, 0, stream>>>(A);
    const int rc = root_chunks(n, tiles);
    k_hist_root<HIST_FT><<<tiles * rc, BLOCK, 0, stream>>>(bins_fm, ld_fm, grad, hess, n, F, A.q, 0.0, 0.0, A.hist, rc,
                                                           A.st);
    const int scan_grid = (F + BLOCK / WAVE - 1) / (BLOCK / WAVE);
    k_scan<true><<<scan_grid, BLOCK, 0, stream>>>(A);
    const int pgrid = launch_grid(n, PART_TILE, PART_MAX_BLOCKS);
    for (int it = 1; it < max_leaves; ++it) {
        k_part_count<<<pgrid, BLOCK, 0, stream>>>(bins_fm, ld_fm, &A.st->part, A.part_cnt, A.st);
        k_part_scatter<<<pgrid, BLOCK, 0, stream>>>(bins_fm, ld_fm, &A.st->part, A.part_cnt, &A.st->hist, A.st);
        k_hist_gather<HIST_FT><<<tiles * GATHER_MAX_CHUNKS, BLOCK, 0, stream>>>(bins_rm, ld_rm, grad, hess, F, A.q,
                                                                                0.0, 0.0, &A.st->hist, A.st);
        k_scan<false><<<scan_grid, BLOCK, 0, stream>>>(A);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "yabt_grow launch");
    return 0;
}

// Per-row leaf ids of the tree the last yabt_grow call on this workspace grew.
int yabt_grow_leaf_ids(void* workspace, int64_t n, int F, int max_leaves, const int64_t* feature,
                       const int64_t* depth, const int32_t* status, int64_t* out, hipStream_t stream) {
    if (!workspace || !feature || !depth || !status || !out || n < 0 || F < 1 || max_leaves < 1)
        return fail(-2, "yabt_grow_leaf_ids: bad arguments");
    if (n == 0) return 0;
    GrowArgs A;
    memset(&A, 0, sizeof A);
    carve_grow((char*)workspace, n, F, max_leaves, &A);
    const int N = 2 * max_leaves + 1;
    dim3 grid(launch_grid(n, BLOCK * 8, 256), N);
    k_leaf_ids<<<grid, BLOCK, 0, stream>>>(feature, depth, A.seg_lo, A.seg_hi, A.rows0, A.rows1, status, out);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : hip_fail(e, "yabt_grow_leaf_ids launch");
}

int yabt_transpose_bins(const uint8_t* bins_fm, int64_t ld_fm, int64_t n, int F, uint8_t* bins_rm, int64_t ld_rm,
                        hipStream_t stream) {
    if (!bins_fm || !bins_rm || n < 0 || F < 1 || ld_fm < n || ld_rm < F)
        return fail(-2, "yabt_transpose_bins: bad arguments");
    if (n == 0) return 0;
    dim3 grid((unsigned)((n + 63) / 64), (unsigned)((ld_rm + 63) / 64));
    k_transpose<<<grid, BLOCK, 0, stream>>>(bins_fm, ld_fm, n, F, bins_rm, ld_rm);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : hip_fail(e, "yabt_transpose_bins launch");
}

size_t yabt_hist_workspace_bytes(void) { return align_up(sizeof(Quant), 256) + align_up(sizeof(HistJob), 256); }

// Exact fixed-point node histogram: out[3][F][256] int64 = (sum q(g), sum q(h),
// count) over rows[0:m] (rows == NULL: all n rows, streamed feature-major).
// out_shifts[2] receives (sg, sh) of or_quant_shift over all n rows.
int yabt_hist(const uint8_t* bins_fm, int64_t ld_fm, const uint8_t* bins_rm, int64_t ld_rm, const float* grad,
              const float* hess, int64_t n, int F, const uint32_t* rows, int64_t m, void* workspace,
              int64_t* out, int32_t* out_shifts, hipStream_t stream) {
    if (F < 1 || n < 0 || n > 0xFFFFFFFFll || !grad || !hess || !out || !workspace || !out_shifts)
        return fail(-2, "yabt_hist: bad arguments");
    if (rows ? (!bins_rm || ld_rm < F || ld_rm % 16 || !aligned16(bins_rm) || m < 0)
             : (!bins_fm || ld_fm < n || ld_fm % 16 || !aligned16(bins_fm)))
        return fail(-2, "yabt_hist: bins layout (pointer, alignment or leading dimension) invalid");
    if (!aligned16(grad) || !aligned16(hess)) return fail(-2, "yabt_hist: grad and hess must be 16-byte aligned");
    Carve c{(char*)workspace, 0};
    Quant* q = c.take<Quant>(1);
    HistJob* job = c.take<HistJob>(1);
    k_quant_clear<<<1, 1, 0, stream>>>(q);
    k_quant<<<launch_grid(n, BLOCK * 16, 1024), BLOCK, 0, stream>>>(grad, hess, n, q);
    const int64_t ne = 3 * (int64_t)F * NB;
    k_fill_i64<<<launch_grid(ne, BLOCK, 1024), BLOCK, 0, stream>>>(out, 0, ne);
    const int tiles = (F + HIST_FT - 1) / HIST_FT;
    if (!rows) {
        const int rc = root_chunks(n, tiles);
        if (n > 0)
            k_hist_root<HIST_FT><<<tiles * rc, BLOCK, 0, stream>>>(bins_fm, ld_fm, grad, hess, n, F, q, 0.0, 0.0, out,
                                                                   rc, nullptr);
    } else if (m > 0) {
        k_set_hist_job<<<1, 1, 0, stream>>>(job, rows, 0, m, out);
        k_hist_gather<HIST_FT><<<tiles * GATHER_MAX_CHUNKS, BLOCK, 0, stream>>>(bins_rm, ld_rm, grad, hess, F, q,
                                                                                0.0, 0.0, job, nullptr);
    }
    hipError_t e = hipMemcpyAsync(out_shifts, &q->sg, 2 * sizeof(int32_t), hipMemcpyDeviceToDevice, stream);
    if (e != hipSuccess) return hip_fail(e, "yabt_hist shifts copy");
    e = hipGetLastError();
    return e == hipSuccess ? 0 : hip_fail(e, "yabt_hist launch");
}

// Single-launch variant of yabt_hist with caller-given shifts that adds into
// `out` without clearing it (rows == NULL: one streaming kernel launch).
int yabt_hist_accumulate(const uint8_t* bins_fm, int64_t ld_fm, const uint8_t* bins_rm, int64_t ld_rm,
                         const float* grad, const float* hess, int64_t n, int F, const uint32_t* rows, int64_t m,
                         int sg, int sh, void* workspace, int64_t* out, hipStream_t stream) {
    if (F < 1 || n < 0 || n > 0xFFFFFFFFll || !grad || !hess || !out || (rows && !workspace))
        return fail(-2, "yabt_hist_accumulate: bad arguments");
    if (rows ? (!bins_rm || ld_rm < F || ld_rm % 16 || !aligned16(bins_rm) || m < 0)
             : (!bins_fm || ld_fm < n || ld_fm % 16 || !aligned16(bins_fm)))
        return fail(-2, "yabt_hist_accumulate: bins layout (pointer, alignment or leading dimension) invalid");
    if (!aligned16(grad) || !aligned16(hess))
        return fail(-2, "yabt_hist_accumulate: grad and hess must be 16-byte aligned");
    const double scg = ldexp(1.0, sg), sch = ldexp(1.0, sh);
    const int tiles = (F + HIST_FT - 1) / HIST_FT;
    if (!rows) {
        const int rc = root_chunks(n, tiles);
        if (n > 0)
            k_hist_root<HIST_FT><<<tiles * rc, BLOCK, 0, stream>>>(bins_fm, ld_fm, grad, hess, n, F, nullptr, scg, sch,
                                                                   out, rc, nullptr);
    } else if (m > 0) {
        Carve c{(char*)workspace, 0};
        c.take<Quant>(1);
        HistJob* job = c.take<HistJob>(1);
        k_set_hist_job<<<1, 1, 0, stream>>>(job, rows, 0, m, out);
        k_hist_gather<HIST_FT><<<tiles * GATHER_MAX_CHUNKS, BLOCK, 0, stream>>>(bins_rm, ld_rm, grad, hess, F, nullptr,
                                                                                scg, sch, job, nullptr);
    }
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : hip_fail(e, "yabt_hist_accumulate launch");
}

size_t yabt_best_split_workspace_bytes(int F) {
    return F < 1 ? 0 : align_up((size_t)F * sizeof(ScanRec), 256) + 256;
}

// Best split of one exact histogram (grow.c:129-197 on fixed-point sums).
// out_gain[0] = true gain (-inf if none); out_fb[0..1] = (feature, bin).
int yabt_best_split(const int64_t* hist, int F, const int32_t* nbins, const uint8_t* fmask, const float* boost,
                    int sg, int sh, double lam, double gamma, double mcw, int msl, void* workspace,
                    double* out_gain, int32_t* out_fb, hipStream_t stream) {
    if (!hist || F < 1 || !nbins || !fmask || !workspace || !out_gain || !out_fb)
        return fail(-2, "yabt_best_split: bad arguments");
    Carve c{(char*)workspace, 0};
    ScanRec* rec = c.take<ScanRec>((size_t)F);
    uint32_t* ticket = c.take<uint32_t>(1);
    k_zero_u32<<<1, 1, 0, stream>>>(ticket);
    const ScanParams sp = {lam, gamma, mcw, msl};
    k_scan_one<<<(F + 3) / 4, BLOCK, 0, stream>>>(hist, F, nbins, fmask, boost, sg, sh, sp, rec, ticket, out_gain,
                                                  out_fb);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : hip_fail(e, "yabt_best_split launch");
}

size_t yabt_partition_workspace_bytes(void) {
    return align_up(sizeof(PartJob), 256) + align_up(PART_MAX_BLOCKS * sizeof(uint32_t), 256);
}

// Stable partition of rows_in[0:m] (NULL: positions 0..m-1) by
// bins_fm[f][row] <= b into rows_out; out_mid[0] = number of left rows.
int yabt_partition(const uint8_t* bins_fm, int64_t ld_fm, int64_t n, int f, int b, const uint32_t* rows_in,
                   int64_t m, uint32_t* rows_out, void* workspace, int64_t* out_mid, hipStream_t stream) {
    if (!bins_fm || !rows_out || !workspace || !out_mid || m < 0 || f < 0 || ld_fm < n || m > 0xFFFFFFFFll ||
        (!rows_in && m > n))
        return fail(-2, "yabt_partition: bad arguments");
    Carve c{(char*)workspace, 0};
    PartJob* job = c.take<PartJob>(1);
    uint32_t* cnt = c.take<uint32_t>(PART_MAX_BLOCKS);
    k_set_part_job<<<1, 1, 0, stream>>>(job, rows_in, rows_out, 0, m, f, b);
    if (m > 0) {
        const int g = launch_grid(m, PART_TILE, PART_MAX_BLOCKS);
        k_part_count<<<g, BLOCK, 0, stream>>>(bins_fm, ld_fm, job, cnt, nullptr);
        k_part_scatter<<<g, BLOCK, 0, stream>>>(bins_fm, ld_fm, job, cnt, nullptr, nullptr);
    }
    k_copy_mid<<<1, 1, 0, stream>>>(job, out_mid);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : hip_fail(e, "yabt_partition launch");
}

// Leaf (node) index per row of raw X (n, ldx) row-major (capply, grow.c:223-239).
int yabt_apply(const float* X, int64_t ldx, int64_t n, int F, const int64_t* feature, const float* threshold,
               const int64_t* left, const int64_t* right, int n_nodes, int64_t* out_node, hipStream_t stream) {
    if (!X || ldx < F || n < 0 || F < 1 || !feature || !threshold || !left || !right || n_nodes < 1 || !out_node)
        return fail(-2, "yabt_apply: bad arguments");
    if (n == 0) return 0;
    k_apply<<<launch_grid(n, BLOCK, 4096), BLOCK, 0, stream>>>(X, ldx, feature, threshold, left, right, n, n_nodes,
                                                               out_node);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : hip_fail(e, "yabt_apply launch");
}

}  // extern "C"
