// Reference-arithmetic best-first growth on gfx950: the trees of
// yabt/_cgrow/grow.c `cgrow` (grow.c:243-427), bit for bit.
//
// yabt_grow (grow.hip) sums exact fixed-point values; its trees equal cgrow's
// except where cgrow's own fp32 rounding decides a split.  This grower
// reproduces cgrow's arithmetic instead:
//   * a node histogram is the fp32 sum, per (feature, bin), of the node's rows
//     in the order cgrow's rows[] array holds them (grow.c:37-62): one block
//     per feature streams the node's rows in that order, buckets each tile by
//     bin with a stable counting sort in LDS, and one thread per bin keeps the
//     bin's running sums (the sparse builder, grow.c:68-107, likewise);
//   * rows[] follows cgrow's in-place two-pointer partition (grow.c:201-217),
//     which is a fixed permutation of the node's rows, computed in parallel
//     (see "partition" below);
//   * the larger child is parent - smaller child in fp32 (grow.c:355-369);
//   * the split scan sums the bins in double in bin order and evaluates
//     grow.c's gain expression and tie-breaks (grow.c:129-197); node values
//     come from feature 0's 256 bins summed in double (grow.c:302-308,
//     371-379); interaction boosts are grow.c's fp32 compute_boost
//     (grow.c:111-122);
//   * the leaf table, its fp32 gains and the first-maximum selection
//     (grow.c:284-407) run on the host between splits: one device round trip
//     per split.
//
// Partition.  With positions relative to the node start, m rows, and
//   p_k = position of the k-th row going right, counted from the left,
//   q_k = position of the k-th row going left, counted from the right, q_0 = m,
//   K   = #{k : p_k < q_k},
// the two-pointer loop sends
//   * the right row of rank r to q_{r-1} - 1 if r <= K, or if r = K + 1 and
//     its position is below q_K; every other right row moves one place left;
//   * the left row of rank t to p_t if t <= K; every other left row stays.
//
// Workspace (yabt_grow_ref_workspace_bytes): rows and a copy (n u32), the
// partition's flags / ranks / p / q arrays, the built child's g and h in row
// order, and one (3, F, 256) fp32 histogram per node.

#include "common.h"
#include "host.h"
#include "yabt_hip.h"

#include <math.h>
#include <string.h>

#include <atomic>
#include <vector>

namespace yabt {
namespace ref {

constexpr int RB = 256;            // threads per block
constexpr int PT = 2048;           // partition rows per block
constexpr int WT = 4096;           // histogram rows per tile
constexpr int ST = NB + 1;         // bucket starts per (feature, tile)

struct Job {
    int64_t s, e;                  // parent segment
    int64_t nl;                    // rows going left
    int32_t build_left;
    int64_t cs, ce;                // built child's segment
};

struct ChildRes {
    double gain;                   // best true gain (-inf if none)
    int32_t f, b;
    float value;
    int32_t seq;                   // the round that wrote this record (written last)
};

struct Res {
    ChildRes c[2];
    int64_t mid;
    int32_t build_left;
    int32_t pad;
};

struct Ws {
    uint32_t* rows;
    uint32_t* rows_tmp;
    uint8_t* flag;
    uint32_t* rank;
    uint32_t* p;
    uint32_t* q;
    uint32_t* blk;                 // per-block left counts, then their exclusive prefix
    float* G;
    float* H;
    uint16_t* perm;                // (fgroup, ld_perm): per tile, positions bucketed by bin
    uint16_t* xperm;               // (fgroup, ld_perm): sparse builder, per tile, rows outside the default bin
    uint16_t* starts;              // (fgroup, n_tiles, 257): per tile, bucket starts
    int64_t n_tiles, ld_perm;
    int fgroup;                    // features bucketed per pass
    double* expl;                  // (F, 3): sparse builder's explicit g, h sums, default-bin rows
    double* tot;                   // (2): sparse builder's node g, h sums
    float* hist;                   // (N, 3, F, 256)
    double* fsel;                  // (2, F)
    double* fgain;                 // (2, F)
    int32_t* fb;                   // (2, F)
    uint8_t* path;                 // (N, F)
    int64_t* segs;                 // (N, 3): leaf node, start, end
    Job* job;
    size_t bytes;
};

// The workspace for feature groups of fgroup features.
Ws carve(char* base, int64_t n, int F, int max_leaves, bool sparse, int fgroup) {
    Carve c{base, 0};
    Ws w;
    const int64_t N = 2 * (int64_t)max_leaves + 1;
    const int64_t nn = n > 0 ? n : 1;
    w.n_tiles = (nn + WT - 1) / WT;
    w.ld_perm = w.n_tiles * WT;
    w.fgroup = fgroup;
    w.rows = c.take<uint32_t>(nn);
    w.rows_tmp = c.take<uint32_t>(nn);
    w.flag = c.take<uint8_t>(nn);
    w.rank = c.take<uint32_t>(nn);
    w.p = c.take<uint32_t>(nn);
    w.q = c.take<uint32_t>(nn);
    w.blk = c.take<uint32_t>((nn + PT - 1) / PT + 1);
    w.G = c.take<float>(nn);
    w.H = c.take<float>(nn);
    w.perm = c.take<uint16_t>((size_t)fgroup * (size_t)w.ld_perm);
    w.xperm = sparse ? c.take<uint16_t>((size_t)fgroup * (size_t)w.ld_perm) : nullptr;
    w.starts = c.take<uint16_t>((size_t)fgroup * (size_t)w.n_tiles * ST);
    w.expl = c.take<double>(3 * (size_t)F);
    w.tot = c.take<double>(2);
    w.hist = c.take<float>((size_t)N * 3 * F * NB);
    w.fsel = c.take<double>(2 * (size_t)F);
    w.fgain = c.take<double>(2 * (size_t)F);
    w.fb = c.take<int32_t>(2 * (size_t)F);
    w.path = c.take<uint8_t>((size_t)N * F);
    w.segs = c.take<int64_t>((size_t)N * 3);
    w.job = c.take<Job>(1);
    w.bytes = c.off;
    return w;
}

// The recommended feature group: every feature at once while the bucket
// buffers stay within GROUP_BUDGET bytes, else as many as fit.
constexpr size_t GROUP_BUDGET = (size_t)8 << 30;

int recommended_group(int64_t n, int F, int max_leaves, bool sparse) {
    const size_t one = carve(nullptr, n, F, max_leaves, sparse, 1).bytes;
    const size_t two = carve(nullptr, n, F, max_leaves, sparse, 2).bytes;
    const size_t per = two - one;                  // bucket buffers of one more feature (+ alignment)
    return (int)max((size_t)1, min((size_t)F, GROUP_BUDGET / max(per, (size_t)1)));
}

// The largest feature group whose workspace fits in `bytes` (0: none does).
int group_for(size_t bytes, int64_t n, int F, int max_leaves, bool sparse) {
    int lo = 0, hi = F;
    while (lo < hi) {
        const int mid = (lo + hi + 1) / 2;
        if (carve(nullptr, n, F, max_leaves, sparse, mid).bytes <= bytes) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// ---------------------------------------------------------------------------
// setup
// ---------------------------------------------------------------------------

__global__ void __launch_bounds__(RB) k_init(uint32_t* rows, int64_t n, uint8_t* path, int64_t path_n,
                                             int64_t* feature, int64_t* thr_bin, int64_t* left, int64_t* right,
                                             float* value, int64_t* depth, int N) {
    const int64_t tid = (int64_t)blockIdx.x * RB + threadIdx.x, stride = (int64_t)gridDim.x * RB;
    for (int64_t i = tid; i < n; i += stride) rows[i] = (uint32_t)i;
    for (int64_t i = tid; i < path_n; i += stride) path[i] = 0;
    for (int64_t i = tid; i < N; i += stride) {
        feature[i] = LEAF;
        thr_bin[i] = 0;
        left[i] = -1;
        right[i] = -1;
        value[i] = 0.0f;
        depth[i] = 0;
    }
}

// ---------------------------------------------------------------------------
// partition in cgrow's order
// ---------------------------------------------------------------------------

// Flags (row goes left) and the left count of each PT-row block.
__global__ void __launch_bounds__(RB) k_part_flags(const uint8_t* __restrict__ bins_fm, int64_t ld, int f, int b,
                                                   const uint32_t* __restrict__ rows, int64_t s, int64_t m,
                                                   uint8_t* __restrict__ flag, uint32_t* __restrict__ blk) {
    __shared__ uint32_t s_red[RB / WAVE];
    const uint8_t* col = bins_fm + (size_t)f * ld;
    const int64_t x0 = (int64_t)blockIdx.x * PT;
    uint32_t cnt = 0;
    for (int j = threadIdx.x; j < PT; j += RB) {
        const int64_t x = x0 + j;
        if (x < m) {
            const uint8_t l = (int)col[rows[s + x]] <= b ? 1 : 0;
            flag[x] = l;
            cnt += l;
        }
    }
    cnt = block_sum<RB, uint32_t>(cnt, s_red);
    if (threadIdx.x == 0) blk[blockIdx.x] = cnt;
}

// One block: exclusive prefix of the block counts; the job record.
__global__ void __launch_bounds__(RB) k_part_offsets(uint32_t* blk, int nblk, Job* job, int64_t s, int64_t e) {
    __shared__ uint32_t s_w[RB / WAVE];
    uint32_t carry = 0;
    for (int i0 = 0; i0 < nblk; i0 += RB) {
        const int i = i0 + threadIdx.x;
        const uint32_t v = i < nblk ? blk[i] : 0u;
        uint32_t tot;
        const uint32_t ex = block_excl_scan<RB, uint32_t>(v, s_w, &tot);
        if (i < nblk) blk[i] = carry + ex;
        carry += tot;
    }
    if (threadIdx.x == 0) {
        const int64_t m = e - s;
        job->s = s;
        job->e = e;
        job->nl = carry;
        job->build_left = (int64_t)carry <= m - (int64_t)carry ? 1 : 0;
        job->cs = job->build_left ? s : s + (int64_t)carry;
        job->ce = job->build_left ? s + (int64_t)carry : e;
    }
}

// Ranks: rank[x] = left rows before x; p (right rows, from the left) and q
// (left rows, from the right) hold positions.
__global__ void __launch_bounds__(RB) k_part_rank(const uint8_t* __restrict__ flag, const uint32_t* __restrict__ blk,
                                                  const Job* __restrict__ job, int64_t m, uint32_t* __restrict__ rank,
                                                  uint32_t* __restrict__ p, uint32_t* __restrict__ q) {
    __shared__ uint32_t s_w[RB / WAVE];
    const uint32_t nl = (uint32_t)job->nl;
    const int64_t x0 = (int64_t)blockIdx.x * PT;
    uint32_t carry = blk[blockIdx.x];
    for (int j0 = 0; j0 < PT; j0 += RB) {
        const int64_t x = x0 + j0 + threadIdx.x;
        const uint32_t l = x < m ? flag[x] : 0u;
        uint32_t tot;
        const uint32_t ex = carry + block_excl_scan<RB, uint32_t>(l, s_w, &tot);
        if (x < m) {
            rank[x] = ex;
            if (l) q[nl - ex - 1] = (uint32_t)x;
            else p[(uint32_t)x - ex] = (uint32_t)x;
        }
        carry += tot;
    }
}

// Destinations of the two-pointer loop; rows_tmp[s + dest] = rows[s + x].
// Block 0 also records the children's path masks and node bookkeeping.
__global__ void __launch_bounds__(RB) k_part_permute(const uint8_t* __restrict__ flag,
                                                     const uint32_t* __restrict__ rank, const uint32_t* __restrict__ p,
                                                     const uint32_t* __restrict__ q, const Job* __restrict__ job,
                                                     const uint32_t* __restrict__ rows, uint32_t* __restrict__ rows_tmp,
                                                     int64_t s, int64_t m, uint8_t* path, int F, int nid, int f,
                                                     int nl_id, int nr_id) {
    const int64_t nl = job->nl;
    // K = #{k : p_k < q_k}: p rises and q falls, and p_k < q_k exactly when
    // the k-th left row from the right lies at or after nl, so K is the
    // number of left rows in [nl, m): nl minus the left rows before nl
    const int64_t K = nl < m ? nl - (int64_t)rank[nl] : 0;
    const int64_t qK = K == 0 ? m : (int64_t)q[K - 1];
    for (int64_t x = (int64_t)blockIdx.x * RB + threadIdx.x; x < m; x += (int64_t)gridDim.x * RB) {
        const int64_t lb = rank[x];
        int64_t dest;
        if (flag[x]) {
            const int64_t t = nl - lb;                 // rank from the right, 1-based
            dest = t <= K ? (int64_t)p[t - 1] : x;
        } else {
            const int64_t r = x - lb + 1;              // rank from the left, 1-based
            if (r <= K) dest = (r == 1 ? m : (int64_t)q[r - 2]) - 1;
            else if (r == K + 1 && x < qK) dest = qK - 1;
            else dest = x - 1;
        }
        rows_tmp[s + dest] = rows[s + x];
    }
    if (blockIdx.x == 0) {
        for (int j = threadIdx.x; j < F; j += RB) {
            const uint8_t v = (uint8_t)(path[(size_t)nid * F + j] | (j == f ? 1 : 0));
            path[(size_t)nl_id * F + j] = v;
            path[(size_t)nr_id * F + j] = v;
        }
    }
}

// rows[s:e) = rows_tmp[s:e); the built child's g, h in its row order.
__global__ void __launch_bounds__(RB) k_part_commit(uint32_t* __restrict__ rows, const uint32_t* __restrict__ rows_tmp,
                                                    const Job* __restrict__ job, int64_t s, int64_t m,
                                                    const float* __restrict__ grad, const float* __restrict__ hess,
                                                    float* __restrict__ G, float* __restrict__ H) {
    const int64_t cs = job->cs, ce = job->ce;
    for (int64_t x = (int64_t)blockIdx.x * RB + threadIdx.x; x < m; x += (int64_t)gridDim.x * RB) {
        const int64_t i = s + x;
        const uint32_t r = rows_tmp[i];
        rows[i] = r;
        if (i >= cs && i < ce) {
            G[i - cs] = grad[r];
            H[i - cs] = hess[r];
        }
    }
}

// ---------------------------------------------------------------------------
// histogram: cgrow's row-order fp32 chains, bucketed per tile
// ---------------------------------------------------------------------------
//
// cgrow adds each row into its (feature, bin) cell in fp32, in rows[] order
// (grow.c:37-62).  The node's rows are cut into tiles of WT rows in that
// order.  k_walk_sort buckets every (feature, tile) by bin, stably, in
// parallel over the whole device; k_walk_chain then runs one block per
// feature over the tiles in order, thread b adding bin b's run of each tile
// to its fp32 accumulators, so every cell is cgrow's sequential sum.
//
// Sparse builder (grow.c:68-107, default bins dbin): the default bin gets no
// run; its thread instead adds, in double and in row order, the tile's rows
// outside the default bin; block F adds the node's g and h in double in row
// order; k_hist_default combines them.

// Segment [cs, cs + m): the job's built child, or [0, n) for the root (job null).
struct Seg {
    int64_t cs, m;
};

__device__ __forceinline__ Seg seg_of(const Job* job, int64_t n) {
    if (!job) return Seg{0, n};
    return Seg{job->cs, job->ce - job->cs};
}

constexpr int SW = RB / WAVE;             // waves per sort / chain block
constexpr int SSUB = WT / SW;             // rows per wave per tile (sort)
constexpr int SGR = SSUB / WAVE;          // 64-row groups per wave per tile (sort)
constexpr int TPT = WT / RB;              // rows per thread per tile

// Bin of the node's row at position x: row x for the root (rows[] is the
// identity there, grow.c:289), rows[cs + x] for a built child.
template <bool ROOT>
__device__ __forceinline__ uint32_t node_bin(const uint8_t* __restrict__ bins_fm, int64_t ld_fm,
                                            const uint8_t* __restrict__ bins_rm, int64_t ld_rm,
                                            const uint32_t* __restrict__ rows, int64_t cs, int f, int64_t x) {
    if (ROOT) return bins_fm[(size_t)f * (size_t)ld_fm + (size_t)x];
    return bins_rm[(size_t)rows[cs + x] * (size_t)ld_rm + f];
}

// Stable bucketing of one tile of one feature (block (f, t)): perm[f][t*WT +
// k] lists the tile's positions bin by bin, each bin in row order, and
// starts[f][t][b] is where bin b's run begins (starts[...][256] = the run
// total).  The lanes of a wave sharing a bin are found by an LDS atomic OR of
// each lane's bit into s_peer[w][bin] (order-free), read back and cleared; a
// row's rank is the number of those lanes below it plus the wave's running
// count s_cnt[w][bin].  Sparse builder (dbin): the default bin gets no run,
// and xperm lists the tile's other positions in row order.
template <bool ROOT, bool SPARSE>
__global__ void __launch_bounds__(RB) k_walk_sort(const uint8_t* __restrict__ bins_fm, int64_t ld_fm,
                                                  const uint8_t* __restrict__ bins_rm, int64_t ld_rm,
                                                  const uint32_t* __restrict__ rows, const Job* __restrict__ job,
                                                  int64_t n, int fg0, const int32_t* __restrict__ dbin,
                                                  uint16_t* __restrict__ perm, uint16_t* __restrict__ xperm,
                                                  int64_t ld_perm, uint16_t* __restrict__ starts, int64_t n_tiles) {
    __shared__ uint8_t s_bin[WT];
    __shared__ uint64_t s_peer[SW][NB];
    __shared__ uint32_t s_cnt[SW][NB];
    __shared__ uint16_t s_perm[WT];
    __shared__ uint16_t s_xperm[SPARSE ? WT : 1];
    __shared__ uint32_t s_scan[SW];
    __shared__ uint32_t s_xoff[SW + 1];
    const Seg sg = seg_of(job, n);
    const int fl = blockIdx.x, f = fg0 + fl;       // buffers by group position, bins by feature
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), w = tid / WAVE;
    const int df = SPARSE ? dbin[f] : -1;
    for (int64_t t = blockIdx.y; t * WT < sg.m; t += gridDim.y) {
    const int64_t t0 = t * WT;
    const int tn = (int)min((int64_t)WT, sg.m - t0);
    for (int i = tid; i < SW * NB; i += RB) {
        (&s_cnt[0][0])[i] = 0;
        (&s_peer[0][0])[i] = 0;
    }
#pragma unroll
    for (int j = 0; j < TPT; ++j) {
        const int x = j * RB + tid;
        if (x < tn) s_bin[x] = (uint8_t)node_bin<ROOT>(bins_fm, ld_fm, bins_rm, ld_rm, rows, sg.cs, f, t0 + x);
    }
    __syncthreads();
    uint32_t rk[SGR], xr[SGR];
    uint8_t qb[SGR];
    uint32_t xrun = 0;
#pragma unroll
    for (int q = 0; q < SGR; ++q) {
        const int x = w * SSUB + q * WAVE + lane;
        const bool v = x < tn;
        const uint32_t bin = v ? (uint32_t)s_bin[x] : 0u;
        qb[q] = (uint8_t)bin;
        if (v) atomicOr(&s_peer[w][bin], 1ull << lane);
        __builtin_amdgcn_wave_barrier();
        const uint64_t peers = v ? s_peer[w][bin] : 0ull;
        const uint32_t base = v ? s_cnt[w][bin] : 0u;
        __builtin_amdgcn_wave_barrier();
        const uint32_t r = lane_prefix(peers);
        if (v) s_peer[w][bin] = 0ull;
        if (v && r == 0) s_cnt[w][bin] = base + (uint32_t)__popcll(peers);
        __builtin_amdgcn_wave_barrier();
        rk[q] = base + r;
        if (SPARSE) {
            const uint64_t xb = __ballot(v && (int)bin != df);
            xr[q] = xrun + lane_prefix(xb);
            xrun += (uint32_t)__popcll(xb);
        }
    }
    if (SPARSE && lane == 0) s_xoff[w] = xrun;
    __syncthreads();
    // bucket starts (sparse: no room for the default bin) and wave bases
    uint16_t* st_out = starts + ((size_t)fl * (size_t)n_tiles + (size_t)t) * ST;
    {
        const int b = tid;
        uint32_t c[SW];
        uint32_t tb = 0;
#pragma unroll
        for (int u = 0; u < SW; ++u) {
            c[u] = s_cnt[u][b];
            tb += c[u];
        }
        if (SPARSE && b == df) tb = 0;
        uint32_t total;
        const uint32_t st = block_excl_scan<RB, uint32_t>(tb, s_scan, &total);
        st_out[b] = (uint16_t)st;
        if (b == NB - 1) st_out[NB] = (uint16_t)(st + tb);
        uint32_t run = st;
#pragma unroll
        for (int u = 0; u < SW; ++u) {
            s_cnt[u][b] = run;
            run += c[u];
        }
        if (SPARSE && tid == 0) {
            uint32_t o = 0;
#pragma unroll
            for (int u = 0; u < SW; ++u) {
                const uint32_t v = s_xoff[u];
                s_xoff[u] = o;
                o += v;
            }
            s_xoff[SW] = o;
        }
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < SGR; ++q) {
        const int x = w * SSUB + q * WAVE + lane;
        if (x < tn && (!SPARSE || (int)qb[q] != df)) {
            s_perm[s_cnt[w][qb[q]] + rk[q]] = (uint16_t)x;
            if (SPARSE) s_xperm[s_xoff[w] + xr[q]] = (uint16_t)x;
        }
    }
    __syncthreads();
    const int total = SPARSE ? (int)s_xoff[SW] : tn;
    uint16_t* po = perm + (size_t)fl * (size_t)ld_perm + (size_t)t0;
    for (int k = tid; k < total; k += RB) po[k] = s_perm[k];
    if (SPARSE) {
        uint16_t* xo = xperm + (size_t)fl * (size_t)ld_perm + (size_t)t0;
        for (int k = tid; k < total; k += RB) xo[k] = s_xperm[k];
    }
    __syncthreads();
    }
}

// Sequential fp32 sums of the pairs s_gh[idx[k]], k in [lo, hi).
__device__ __forceinline__ void run_f32(const float2* s_gh, const uint16_t* idx, uint32_t lo, uint32_t hi,
                                        float& ag, float& ah) {
    uint32_t k = lo;
    for (; k + 8 <= hi; k += 8) {
        uint32_t i[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) i[j] = idx[k + j];
        float2 p[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) p[j] = s_gh[i[j]];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            ag += p[j].x;
            ah += p[j].y;
        }
    }
    for (; k < hi; ++k) {
        const float2 p = s_gh[idx[k]];
        ag += p.x;
        ah += p.y;
    }
}

// Sequential double sums of the fp32 pairs s_gh[idx[k]] (idx null: s_gh[k]),
// k in [0, hi).
__device__ __forceinline__ void run_f64(const float2* s_gh, const uint16_t* idx, uint32_t hi, double& ag,
                                        double& ah) {
    uint32_t k = 0;
    for (; k + 8 <= hi; k += 8) {
        float2 p[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) p[j] = s_gh[idx ? (uint32_t)idx[k + j] : k + j];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            ag += (double)p[j].x;
            ah += (double)p[j].y;
        }
    }
    for (; k < hi; ++k) {
        const float2 p = s_gh[idx ? (uint32_t)idx[k] : k];
        ag += (double)p.x;
        ah += (double)p.y;
    }
}

// One tile of a chain block, TPT entries per thread, loaded a tile ahead.
struct ChainTile {
    float g[TPT], h[TPT];
    uint32_t idx[TPT], xidx[TPT];
    uint32_t st, st_end;
};

template <bool SPARSE>
__device__ __forceinline__ void chain_load(ChainTile& c, const float* __restrict__ G, const float* __restrict__ H,
                                           const uint16_t* __restrict__ pf, const uint16_t* __restrict__ xf,
                                           const uint16_t* __restrict__ sf, bool totals, int64_t t, int64_t m) {
    const int64_t t0 = t * WT;
#pragma unroll
    for (int j = 0; j < TPT; ++j) {
        const int64_t x = t0 + j * RB + threadIdx.x;
        if (x < m) {
            c.g[j] = G[x];
            c.h[j] = H[x];
            if (!totals) {
                c.idx[j] = pf[x];
                if (SPARSE) c.xidx[j] = xf[x];
            }
        }
    }
    if (!totals) {
        c.st = sf[(size_t)t * ST + threadIdx.x];
        if (threadIdx.x == 0) c.st_end = sf[(size_t)t * ST + NB];
    }
}

// The chains (block f, thread b = bin): the node's tiles in order, each
// tile's g, h and bucketed positions staged in LDS, bin b's run added in fp32
// in row order (grow.c:55-59); the count cell is cgrow's chain of 1.0f adds,
// which is min(count, 2^24) exactly.  Sparse builder: the default bin's
// thread adds the tile's other rows in double in row order (xperm), and
// block F adds the node's g and h in double in row order (grow.c:85-97);
// k_hist_default combines them.  G, H hold the node's g, h by position.
template <bool SPARSE>
__global__ void __launch_bounds__(RB) k_walk_chain(const float* __restrict__ G, const float* __restrict__ H,
                                                   const Job* __restrict__ job, int64_t n, int F, int fg0, int nf,
                                                   const int32_t* __restrict__ dbin,
                                                   const uint16_t* __restrict__ perm,
                                                   const uint16_t* __restrict__ xperm, int64_t ld_perm,
                                                   const uint16_t* __restrict__ starts, int64_t n_tiles,
                                                   float* __restrict__ hist_base, size_t hsz, int slot_l, int slot_r,
                                                   double* __restrict__ eout, double* __restrict__ tot) {
    __shared__ float2 s_gh[WT];
    __shared__ uint16_t s_idx[WT];
    __shared__ uint16_t s_xidx[SPARSE ? WT : 1];
    __shared__ uint16_t s_st[ST];
    const Seg sg = seg_of(job, n);
    const int64_t m = sg.m;
    const int tid = threadIdx.x;
    const int fl = blockIdx.x, f = fg0 + fl;       // buffers by group position, cells by feature
    const bool totals = SPARSE && fl == nf;        // the extra block of the first group
    const int df = (SPARSE && !totals) ? dbin[f] : -1;
    const size_t fo = (size_t)(totals ? 0 : fl);
    const uint16_t* pf = perm + fo * (size_t)ld_perm;
    const uint16_t* xf = SPARSE ? xperm + fo * (size_t)ld_perm : nullptr;
    const uint16_t* sf = starts + fo * (size_t)n_tiles * ST;
    float ag = 0.0f, ah = 0.0f;
    double eg = 0.0, eh = 0.0;
    int64_t cnt = 0;
    ChainTile nxt;
    if (m > 0) chain_load<SPARSE>(nxt, G, H, pf, xf, sf, totals, 0, m);
    for (int64_t t = 0, t0 = 0; t0 < m; ++t, t0 += WT) {
        const int tn = (int)min((int64_t)WT, m - t0);
#pragma unroll
        for (int j = 0; j < TPT; ++j) {
            const int x = j * RB + tid;
            if (x < tn) {
                s_gh[x] = make_float2(nxt.g[j], nxt.h[j]);
                if (!totals) {
                    s_idx[x] = (uint16_t)nxt.idx[j];
                    if (SPARSE) s_xidx[x] = (uint16_t)nxt.xidx[j];
                }
            }
        }
        if (!totals) {
            s_st[tid] = (uint16_t)nxt.st;
            if (tid == 0) s_st[NB] = (uint16_t)nxt.st_end;
        }
        __syncthreads();
        if (t0 + WT < m) chain_load<SPARSE>(nxt, G, H, pf, xf, sf, totals, t + 1, m);
        if (totals) {
            if (tid == 0) run_f64(s_gh, nullptr, (uint32_t)tn, eg, eh);
        } else if (SPARSE && tid == df) {
            const uint32_t nx = s_st[NB];      // the tile's rows outside the default bin
            run_f64(s_gh, s_xidx, nx, eg, eh);
            cnt += (int64_t)tn - nx;
        } else {
            const uint32_t lo = s_st[tid], hi = s_st[tid + 1];
            run_f32(s_gh, s_idx, lo, hi, ag, ah);
            cnt += hi - lo;
        }
        __syncthreads();
    }
    if (totals) {
        if (tid == 0) {
            tot[0] = eg;
            tot[1] = eh;
        }
        return;
    }
    const int slot = (!job || job->build_left) ? slot_l : slot_r;
    float* hist = hist_base + (size_t)slot * hsz;
    if (SPARSE && tid == df) {
        eout[3 * (size_t)f] = eg;
        eout[3 * (size_t)f + 1] = eh;
        eout[3 * (size_t)f + 2] = (double)cnt;
    } else {
        hist[(size_t)0 * F * NB + (size_t)f * NB + tid] = ag;
        hist[(size_t)1 * F * NB + (size_t)f * NB + tid] = ah;
        hist[(size_t)2 * F * NB + (size_t)f * NB + tid] = (float)min(cnt, (int64_t)1 << 24);
    }
}

// Sparse builder's default-bin cells (grow.c:101-106): 0 + (float)(node sum -
// explicit sum) for g and h, 0 + (float)(rows in the default bin) for the count.
__global__ void __launch_bounds__(RB) k_hist_default(const int32_t* __restrict__ dbin,
                                                     const double* __restrict__ eout, const double* __restrict__ tot,
                                                     int F, float* __restrict__ hist_base, size_t hsz,
                                                     const Job* __restrict__ job, int slot_l, int slot_r) {
    const int f = blockIdx.x * RB + threadIdx.x;
    if (f >= F) return;
    const int slot = (!job || job->build_left) ? slot_l : slot_r;
    float* hist = hist_base + (size_t)slot * hsz;
    const size_t at = (size_t)f * NB + dbin[f];
    hist[(size_t)0 * F * NB + at] = 0.0f + (float)(tot[0] - eout[3 * (size_t)f]);
    hist[(size_t)1 * F * NB + at] = 0.0f + (float)(tot[1] - eout[3 * (size_t)f + 1]);
    hist[(size_t)2 * F * NB + at] = 0.0f + (float)eout[3 * (size_t)f + 2];
}

// ---------------------------------------------------------------------------
// split scan (grow.c:129-197), one wave per (feature, child)
// ---------------------------------------------------------------------------

// Exponent bounds of a set of fp32 values, for deciding when double sums of
// them are exact in any order: every value is a multiple of 2^lsb and below
// 2^(top + 1) in magnitude.  Non-finite values make the set inexact.
struct ExpRange {
    int lsb, top;
    bool finite;
};

__device__ __forceinline__ void exp_range_add(ExpRange& r, float x) {
    const uint32_t u = __float_as_uint(x);
    const int ex = (int)((u >> 23) & 0xffu);
    const uint32_t mant = u & 0x7fffffu;
    if (ex == 0xff) {
        r.finite = false;
        return;
    }
    if (ex == 0 && mant == 0) return;                  // +-0 adds nothing
    const uint32_t m24 = ex == 0 ? mant : (mant | 0x800000u);
    const int e0 = ex == 0 ? -149 : ex - 150;          // weight of the mantissa's bit 0
    const int lsb = e0 + __builtin_ctz(m24);
    const int top = e0 + 31 - __builtin_clz(m24);
    r.lsb = min(r.lsb, lsb);
    r.top = max(r.top, top);
}

// Wave-wide: true when every partial sum of up to 256 of the wave's values
// (any subset, so any order of addition) is exactly representable in double:
// all are multiples of 2^lsb and |sum| < 256 * 2^(top + 1) = 2^(top + 9), so
// top + 9 - lsb <= 53 suffices.
__device__ __forceinline__ bool wave_sums_exact(ExpRange r) {
#pragma unroll
    for (int d = WAVE / 2; d > 0; d >>= 1) {
        r.lsb = min(r.lsb, __shfl_xor(r.lsb, d, WAVE));
        r.top = max(r.top, __shfl_xor(r.top, d, WAVE));
        r.finite = r.finite && __shfl_xor((int)r.finite, d, WAVE);
    }
    return r.finite && (r.top < r.lsb || r.top + 9 - r.lsb <= 53);
}

struct ScanParams {
    const int32_t* nbins;
    const uint8_t* fmask;
    const float* imat;
    float ib;
    int use_imat;
    double lam, gamma, mcw;
    int msl;
    int F;
};

// The pick's inputs and the split record it writes.
struct PickArgs {
    float lr;
    double lam;
    float* out_value;
    Res* res;
    const Job* job;                // null at the root
    int nid, split_f, split_b;     // the split (nid < 0 at the root)
    int32_t seq;                   // round number stamped on the records
    int64_t child_depth;
    int64_t *out_feature, *out_thr_bin, *out_left, *out_right, *out_depth;
};

// One child's feature-major first maximum (grow.c:183-192), node value from
// feature 0's 256 bins summed in double (grow.c:302-308, 371-379), and (for
// the left child of a split) the split's node record (grow.c:340-350,
// 381-386).  One wave.
__device__ void ref_pick(const float* __restrict__ hist, size_t hsz, int node0, int node1, int c, int F,
                         const double* __restrict__ fsel, const double* __restrict__ fgain,
                         const int32_t* __restrict__ fb, const PickArgs& A, float* s_g, float* s_h) {
    const int node = c == 0 ? node0 : node1;
    const int lane = threadIdx.x;
    {
        const float* hg = hist + (size_t)node * hsz;
        const float* hh = hg + (size_t)F * NB;
        for (int b = lane; b < NB; b += WAVE) {
            s_g[b] = hg[b];
            s_h[b] = hh[b];
        }
    }
    __syncthreads();
    if (lane == 0 && A.nid >= 0 && c == 0) {
        A.out_feature[A.nid] = A.split_f;
        A.out_thr_bin[A.nid] = A.split_b;
        A.out_left[A.nid] = node0;
        A.out_right[A.nid] = node1;
        A.out_value[A.nid] = 0.0f;
        A.out_depth[node0] = A.child_depth;
        A.out_depth[node1] = A.child_depth;
    }
    // lanes take features in increasing order with grow.c's strict >, then
    // the largest sel, lowest f wins
    double best_sel = -INFINITY, best_true = -INFINITY;
    int bf = -1, bb = -1;
    for (int f = lane; f < F; f += WAVE) {
        const int b = fb[(size_t)c * F + f];
        const double s = fsel[(size_t)c * F + f];
        if (b >= 0 && s > best_sel) {
            best_sel = s;
            best_true = fgain[(size_t)c * F + f];
            bf = f;
            bb = b;
        }
    }
#pragma unroll
    for (int d = WAVE / 2; d > 0; d >>= 1) {
        const double os = __shfl_xor(best_sel, d, WAVE);
        const double ot = __shfl_xor(best_true, d, WAVE);
        const int of = __shfl_xor(bf, d, WAVE);
        const int ob = __shfl_xor(bb, d, WAVE);
        if (of >= 0 && (bf < 0 || os > best_sel || (os == best_sel && of < bf))) {
            best_sel = os;
            best_true = ot;
            bf = of;
            bb = ob;
        }
    }
    if (lane == 0) {
        double G = 0.0, H = 0.0;
        for (int b0 = 0; b0 < NB; b0 += 8) {
            float vg[8], vh[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                vg[j] = s_g[b0 + j];
                vh[j] = s_h[b0 + j];
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                G += vg[j];
                H += vh[j];
            }
        }
        const float v = (float)(-A.lr * G / (H + A.lam));
        A.out_value[node] = v;
        // A.res is host memory mapped for the device: the record's fields,
        // a system-scope fence, then the round number the host waits for
        volatile ChildRes& r = A.res->c[c];
        r.gain = bf < 0 ? -INFINITY : best_true;
        r.f = bf;
        r.b = bb;
        r.value = v;
        if (c == 0) {
            volatile Res* R = A.res;
            R->mid = A.job ? A.job->s + A.job->nl : 0;
            R->build_left = A.job ? A.job->build_left : 0;
        }
        __threadfence_system();
        r.seq = A.seq;
    }
    __syncthreads();
}

// One wave per (feature, child): the split scan (grow.c:129-197).  At a split
// (parent >= 0) the subtracted child's block first forms its feature's bins
// as parent - built child in fp32 (grow.c:361,368) and stores them.
__global__ void __launch_bounds__(WAVE) k_scan_feature(float* __restrict__ hist, size_t hsz, int node0, int node1,
                                                       int parent, const uint8_t* __restrict__ path, ScanParams P,
                                                       double* __restrict__ fsel, double* __restrict__ fgain,
                                                       int32_t* __restrict__ fb, PickArgs A) {
    __shared__ float s_in[3][NB];
    __shared__ double s_gl[NB], s_hl[NB], s_cl[NB];
    const int f = blockIdx.x, c = blockIdx.y, lane = threadIdx.x;
    const int node = c == 0 ? node0 : node1;
    const int F = P.F;
    double best_sel = -INFINITY, best_true = -INFINITY;
    int best_b = -1;
    const bool sub = parent >= 0 && node == (A.job->build_left ? node1 : node0);
    if (sub) {
        const int built = A.job->build_left ? node0 : node1;
        const size_t plane = (size_t)F * NB;
        const float* hp = hist + (size_t)parent * hsz + (size_t)f * NB;
        const float* hb = hist + (size_t)built * hsz + (size_t)f * NB;
        float* ho = hist + (size_t)node * hsz + (size_t)f * NB;
        for (int b = lane; b < NB; b += WAVE) {
#pragma unroll
            for (int ch = 0; ch < 3; ++ch) {
                const float v = hp[ch * plane + b] - hb[ch * plane + b];
                ho[ch * plane + b] = v;
                s_in[ch][b] = v;
            }
        }
    }
    if (P.fmask[f]) {
        const int nb = min(max(P.nbins[f], 1), NB);
        if (!sub) {
            const float* hg = hist + (size_t)node * hsz + (size_t)f * NB;
            const float* hh = hg + (size_t)F * NB;
            const float* hc = hh + (size_t)F * NB;
            for (int b = lane; b < NB; b += WAVE) {
                s_in[0][b] = hg[b];
                s_in[1][b] = hh[b];
                s_in[2][b] = hc[b];
            }
        }
        __syncthreads();
        // the prefix sums in double, in bin order (grow.c:146-160).  When
        // every partial sum of the node's bins is exact in double, the prefix
        // is the exact one whatever the order of the additions, so the wave
        // scans it in parallel (4 bins per lane); otherwise lane 0 adds the
        // bins in order as cgrow does.
        ExpRange rg{1 << 20, -(1 << 20), true}, rh = rg;
        float vg[4], vh[4], vc[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int b = 4 * lane + j;
            vg[j] = b < nb ? s_in[0][b] : 0.0f;
            vh[j] = b < nb ? s_in[1][b] : 0.0f;
            vc[j] = b < nb ? s_in[2][b] : 0.0f;
            exp_range_add(rg, vg[j]);
            exp_range_add(rh, vh[j]);
        }
        // counts are integers below 2^24: their sums are always exact
        const bool exact = wave_sums_exact(rg) && wave_sums_exact(rh);
        if (exact) {
            double pg[4], ph[4], pc[4];
            double ag = 0.0, ah = 0.0, ac = 0.0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                ag += (double)vg[j];
                ah += (double)vh[j];
                ac += (double)vc[j];
                pg[j] = ag;
                ph[j] = ah;
                pc[j] = ac;
            }
            const double og = wave_excl_scan<double>(ag, lane);
            const double oh = wave_excl_scan<double>(ah, lane);
            const double oc = wave_excl_scan<double>(ac, lane);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int b = 4 * lane + j;
                if (b < nb) {
                    s_gl[b] = og + pg[j];
                    s_hl[b] = oh + ph[j];
                    s_cl[b] = oc + pc[j];
                }
            }
        } else if (lane == 0) {
            double G = 0.0, H = 0.0, C = 0.0;
            for (int b0 = 0; b0 < nb; b0 += 8) {
                float wg[8], wh[8], wc[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int b = min(b0 + j, nb - 1);
                    wg[j] = s_in[0][b];
                    wh[j] = s_in[1][b];
                    wc[j] = s_in[2][b];
                }
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (b0 + j < nb) {
                        G += wg[j];
                        H += wh[j];
                        C += wc[j];
                        s_gl[b0 + j] = G;
                        s_hl[b0 + j] = H;
                        s_cl[b0 + j] = C;
                    }
            }
        }
        __syncthreads();
        // compute_boost (grow.c:111-122): 1 + ib * max(0, max over the path
        // of imat[p][f]); the maximum is taken lane-parallel (max is exact)
        float mx = 0.0f;
        if (P.use_imat) {
            for (int p = lane; p < F; p += WAVE)
                if (path[(size_t)node * F + p]) {
                    const float v = P.imat[(size_t)p * F + f];
                    if (v > mx) mx = v;
                }
#pragma unroll
            for (int d = WAVE / 2; d > 0; d >>= 1) {
                const float o = __shfl_xor(mx, d, WAVE);
                if (o > mx) mx = o;
            }
        }
        const double bo = P.use_imat ? (double)(1.0f + P.ib * mx) : 1.0;
        const double Gt = s_gl[nb - 1], Ht = s_hl[nb - 1], Ct = s_cl[nb - 1];
        const double parent = Gt * Gt / (Ht + P.lam);
        for (int b = lane; b < nb - 1; b += WAVE) {
            const double GL = s_gl[b], HL = s_hl[b], CL = s_cl[b];
            const double GR = Gt - GL, HR = Ht - HL, CR = Ct - CL;
            if (CL >= P.msl && CR >= P.msl && HL >= P.mcw && HR >= P.mcw) {
                const double gain = 0.5 * (GL * GL / (HL + P.lam) + GR * GR / (HR + P.lam) - parent) - P.gamma;
                const double sel = gain * bo;
                if (sel > best_sel) {           // lanes visit b in increasing order
                    best_sel = sel;
                    best_true = gain;
                    best_b = b;
                }
            }
        }
        // the first maximum over b: largest sel, then smallest b
#pragma unroll
        for (int d = WAVE / 2; d > 0; d >>= 1) {
            const double os = __shfl_xor(best_sel, d, WAVE);
            const double ot = __shfl_xor(best_true, d, WAVE);
            const int ob = __shfl_xor(best_b, d, WAVE);
            const bool take = ob >= 0 && (best_b < 0 || os > best_sel || (os == best_sel && ob < best_b));
            if (take) {
                best_sel = os;
                best_true = ot;
                best_b = ob;
            }
        }
    }
    if (lane == 0) {
        fsel[(size_t)c * F + f] = best_sel;
        fgain[(size_t)c * F + f] = best_true;
        fb[(size_t)c * F + f] = best_b;
    }
}

// One wave per child: ref_pick after every scan block is done.
__global__ void __launch_bounds__(WAVE) k_scan_pick(const float* __restrict__ hist, size_t hsz, int node0, int node1,
                                                    int F, const double* __restrict__ fsel,
                                                    const double* __restrict__ fgain, const int32_t* __restrict__ fb,
                                                    PickArgs A) {
    __shared__ float s_g[NB], s_h[NB];
    ref_pick(hist, hsz, node0, node1, blockIdx.x, F, fsel, fgain, fb, A, s_g, s_h);
}

// Per-row leaf ids from the final rows[] and the leaves' segments.
__global__ void __launch_bounds__(RB) k_leaf_rows(const uint32_t* __restrict__ rows, const int64_t* __restrict__ seg,
                                                  int n_leaf, int64_t* __restrict__ out) {
    const int k = blockIdx.y;
    if (k >= n_leaf) return;
    const int64_t node = seg[3 * k], s = seg[3 * k + 1], e = seg[3 * k + 2];
    for (int64_t i = s + (int64_t)blockIdx.x * RB + threadIdx.x; i < e; i += (int64_t)gridDim.x * RB)
        out[rows[i]] = node;
}

__global__ void k_set_status(int32_t* out, int v) { out[0] = v; }

__global__ void __launch_bounds__(RB) k_rows_out(const uint32_t* __restrict__ rows, int64_t n, int64_t* __restrict__ out) {
    for (int64_t i = (int64_t)blockIdx.x * RB + threadIdx.x; i < n; i += (int64_t)gridDim.x * RB) out[i] = rows[i];
}

// ---------------------------------------------------------------------------
// host driver
// ---------------------------------------------------------------------------

struct Grower {
    const uint8_t* bins_fm;
    int64_t ld_fm;
    const uint8_t* bins_rm;
    int64_t ld_rm;
    const float* grad;
    const float* hess;
    int64_t n;
    int F;
    Ws w;
    size_t hsz;
    const int32_t* dbin;           // sparse builder's default bins, or null
    hipStream_t st;

    // Histogram of the job's built child (at most m_max rows) into node
    // slot_l (left child built) or slot_r; job null: all rows into slot_l.
    // With default bins, the sparse builder's arithmetic (grow.c:68-107).
    void hist(const Job* job, int64_t m_max, int slot_l, int slot_r, const float* G, const float* H) {
        const int64_t tiles = min((int64_t)65535, max((int64_t)1, (m_max + WT - 1) / WT));
        const uint32_t* rows = w.rows;
        for (int fg0 = 0; fg0 < F; fg0 += w.fgroup) {
            const int nf = min(w.fgroup, F - fg0);
            const dim3 sgrid((unsigned)nf, (unsigned)tiles);
#define YABT_SORT(ROOT, SPARSE)                                                                                      \
    k_walk_sort<ROOT, SPARSE><<<sgrid, RB, 0, st>>>(bins_fm, ld_fm, bins_rm, ld_rm, rows, job, n, fg0, dbin, w.perm, \
                                                    w.xperm, w.ld_perm, w.starts, w.n_tiles)
            if (!job) {
                if (dbin) YABT_SORT(true, true); else YABT_SORT(true, false);
            } else {
                if (dbin) YABT_SORT(false, true); else YABT_SORT(false, false);
            }
#undef YABT_SORT
            // the sparse builder's node totals: one more block with the first group
            const unsigned cgrid = (unsigned)nf + (dbin && fg0 == 0 ? 1u : 0u);
            if (dbin)
                k_walk_chain<true><<<cgrid, RB, 0, st>>>(G, H, job, n, F, fg0, nf, dbin, w.perm, w.xperm, w.ld_perm,
                                                         w.starts, w.n_tiles, w.hist, hsz, slot_l, slot_r, w.expl,
                                                         w.tot);
            else
                k_walk_chain<false><<<cgrid, RB, 0, st>>>(G, H, job, n, F, fg0, nf, dbin, w.perm, w.xperm,
                                                          w.ld_perm, w.starts, w.n_tiles, w.hist, hsz, slot_l, slot_r,
                                                          w.expl, w.tot);
        }
        if (dbin)
            k_hist_default<<<(F + RB - 1) / RB, RB, 0, st>>>(dbin, w.expl, w.tot, F, w.hist, hsz, job, slot_l, slot_r);
    }
};

}  // namespace ref
}  // namespace yabt

using namespace yabt;
using namespace yabt::ref;

extern "C" {

size_t yabt_grow_ref_workspace_bytes(int64_t n, int F, int max_leaves, int sparse) {
    if (n < 0 || n > 0xFFFFFFFFll || F < 1 || max_leaves < 1 || max_leaves > 32767) return 0;
    return carve(nullptr, n, F, max_leaves, sparse != 0, recommended_group(n, F, max_leaves, sparse != 0)).bytes;
}

size_t yabt_grow_ref_workspace_min_bytes(int64_t n, int F, int max_leaves, int sparse) {
    if (n < 0 || n > 0xFFFFFFFFll || F < 1 || max_leaves < 1 || max_leaves > 32767) return 0;
    return carve(nullptr, n, F, max_leaves, sparse != 0, 1).bytes;
}

int yabt_grow_ref(const uint8_t* bins_fm, int64_t ld_fm, const uint8_t* bins_rm, int64_t ld_rm, const float* grad,
                  const float* hess, const uint8_t* fmask, const float* imat, float ib, int use_imat,
                  const int32_t* nbins, const int32_t* default_bin, int64_t n, int F, float lam, float gamma,
                  float mcw, int msl, float lr, int max_leaves, int max_depth, void* workspace,
                  size_t workspace_bytes, int64_t* out_feature,
                  int64_t* out_thr_bin, int64_t* out_left, int64_t* out_right, float* out_value, int64_t* out_depth,
                  int64_t* out_leaf_of_row, int64_t* out_rows, int32_t* out_n_nodes, hipStream_t stream) {
    if (n < 0 || n > 0xFFFFFFFFll || F < 1 || max_leaves < 1 || max_leaves > 32767)
        return fail(-2, "yabt_grow_ref: bad sizes");
    if (!grad || !hess || !fmask || !nbins || !workspace || !out_feature || !out_thr_bin || !out_left || !out_right ||
        !out_value || !out_depth || !out_n_nodes || (use_imat && !imat))
        return fail(-2, "yabt_grow_ref: null pointer argument");
    if (n > 0 && (!bins_fm || !bins_rm || ld_fm < n || ld_rm < F || ld_rm % 16 || !aligned16(bins_rm)))
        return fail(-2, "yabt_grow_ref: bins layout (pointer, alignment or leading dimension) invalid");
    const bool sparse = default_bin != nullptr;
    const int fgroup = group_for(workspace_bytes, n, F, max_leaves, sparse);
    if (fgroup < 1) return fail(-2, "yabt_grow_ref: workspace too small");
    if (default_bin) {   // the kernels index bin tables with it: check it first
        std::vector<int32_t> db(F);
        hipError_t e = hipMemcpyAsync(db.data(), default_bin, (size_t)F * sizeof(int32_t), hipMemcpyDeviceToHost, stream);
        if (e == hipSuccess) e = hipStreamSynchronize(stream);
        if (e != hipSuccess) return hip_fail(e, "yabt_grow_ref: default_bin copy");
        for (int f = 0; f < F; ++f)
            if (db[f] < 0 || db[f] >= NB) return fail(-2, "yabt_grow_ref: default_bin entries must be in [0, 255]");
    }

    Grower g;
    g.bins_fm = bins_fm;
    g.ld_fm = ld_fm;
    g.bins_rm = bins_rm;
    g.ld_rm = ld_rm;
    g.grad = grad;
    g.hess = hess;
    g.n = n;
    g.F = F;
    g.w = carve((char*)workspace, n, F, max_leaves, sparse, fgroup);
    g.hsz = (size_t)3 * F * NB;
    g.dbin = default_bin;
    g.st = stream;
    const Ws& w = g.w;
    const int N = 2 * max_leaves + 1;

    Res* h_res = nullptr;
    hipError_t he = hipHostMalloc((void**)&h_res, sizeof(Res), hipHostMallocMapped | hipHostMallocCoherent);
    if (he != hipSuccess) return hip_fail(he, "yabt_grow_ref: pinned result buffer");
    struct Free {
        Res* p;
        ~Free() { (void)hipHostFree(p); }
    } free_res{h_res};

    k_init<<<launch_grid(max((int64_t)N * F, n), RB, 1024), RB, 0, stream>>>(
        w.rows, n, w.path, (int64_t)N * F, out_feature, out_thr_bin, out_left, out_right, out_value, out_depth, N);

    ScanParams P;
    P.nbins = nbins;
    P.fmask = fmask;
    P.imat = imat;
    P.ib = ib;
    P.use_imat = use_imat;
    P.lam = (double)lam;
    P.gamma = (double)gamma;
    P.mcw = (double)mcw;
    P.msl = msl;
    P.F = F;

    // host copy of cgrow's leaf table (grow.c:284-287) and node segments
    std::vector<int64_t> node_start(N, 0), node_end(N, 0), node_depth(N, 0);
    std::vector<int64_t> leaf_node(N), leaf_f(N), leaf_b(N);
    std::vector<float> leaf_gain(N);
    Res* d_res = nullptr;   // the device's address of h_res
    he = hipHostGetDevicePointer((void**)&d_res, h_res, 0);
    if (he != hipSuccess) return hip_fail(he, "yabt_grow_ref: mapped result buffer");
    h_res->c[0].seq = h_res->c[1].seq = -1;
    // The pick writes each child's record into h_res and stamps it with the
    // round number last; the host spins on the stamps (checking the stream
    // for errors, and for completion without a stamp) instead of a copy and
    // a stream synchronisation.
    auto sync_res = [&](int32_t seq, int children) -> int {
        volatile Res* R = h_res;
        for (uint64_t spin = 0;; ++spin) {
            bool ok = true;
            for (int c = 0; c < children; ++c) ok = ok && R->c[c].seq == seq;
            if (ok) {
                std::atomic_thread_fence(std::memory_order_acquire);
                return 0;
            }
            if ((spin & 1023) == 1023) {
                const hipError_t e = hipStreamQuery(stream);
                if (e == hipSuccess) {
                    ok = true;
                    for (int c = 0; c < children; ++c) ok = ok && R->c[c].seq == seq;
                    if (ok) return 0;
                    return fail(-4, "yabt_grow_ref: stream finished without the split result");
                }
                if (e != hipErrorNotReady) return hip_fail(e, "yabt_grow_ref: split");
            }
        }
    };

    // root
    node_end[0] = n;
    g.hist(nullptr, n, 0, 0, grad, hess);
    PickArgs A;
    A.lr = lr;
    A.lam = (double)lam;
    A.out_value = out_value;
    A.res = d_res;
    A.seq = 0;
    A.job = nullptr;
    A.nid = -1;
    A.split_f = A.split_b = 0;
    A.child_depth = 0;
    A.out_feature = out_feature;
    A.out_thr_bin = out_thr_bin;
    A.out_left = out_left;
    A.out_right = out_right;
    A.out_depth = out_depth;
    k_scan_feature<<<dim3(F, 1), WAVE, 0, stream>>>(w.hist, g.hsz, 0, 0, -1, w.path, P, w.fsel, w.fgain, w.fb, A);
    k_scan_pick<<<1, WAVE, 0, stream>>>(w.hist, g.hsz, 0, 0, F, w.fsel, w.fgain, w.fb, A);
    int rc = launch_status("yabt_grow_ref launch");
    if (rc) return rc;
    if ((rc = sync_res(0, 1))) return rc;
    double g0 = h_res->c[0].gain;
    if (0 >= max_depth) g0 = -INFINITY;
    leaf_node[0] = 0;
    leaf_gain[0] = (float)g0;
    leaf_f[0] = h_res->c[0].f;
    leaf_b[0] = h_res->c[0].b;
    int n_active = 1, n_leaves = 1, n_nodes = 1;
    std::vector<char> split(N, 0);

    while (n_leaves < max_leaves) {             // grow.c:321-408
        int best_k = -1;
        float best_g = 0.0f;
        for (int k = 0; k < n_active; ++k)
            if (leaf_gain[k] > best_g) {
                best_g = leaf_gain[k];
                best_k = k;
            }
        if (best_k < 0) break;
        const int nid = (int)leaf_node[best_k];
        const int f = (int)leaf_f[best_k], b = (int)leaf_b[best_k];
        const int64_t s = node_start[nid], e = node_end[nid], m = e - s;
        const int nl = n_nodes, nr = n_nodes + 1;
        n_nodes += 2;
        const int64_t d = node_depth[nid] + 1;
        split[nid] = 1;

        // partition rows[s:e) in cgrow's order; the smaller child's g, h
        const int pblk = (int)max((int64_t)1, (m + PT - 1) / PT);
        k_part_flags<<<pblk, RB, 0, stream>>>(bins_fm, ld_fm, f, b, w.rows, s, m, w.flag, w.blk);
        k_part_offsets<<<1, RB, 0, stream>>>(w.blk, pblk, w.job, s, e);
        k_part_rank<<<pblk, RB, 0, stream>>>(w.flag, w.blk, w.job, m, w.rank, w.p, w.q);
        k_part_permute<<<launch_grid(m, RB * 4, 4096), RB, 0, stream>>>(w.flag, w.rank, w.p, w.q, w.job, w.rows,
                                                                      w.rows_tmp, s, m, w.path, F, nid, f, nl, nr);
        k_part_commit<<<launch_grid(m, RB * 4, 4096), RB, 0, stream>>>(w.rows, w.rows_tmp, w.job, s, m, grad, hess, w.G,
                                                                     w.H);
        // the smaller child (ties left, grow.c:355) has at most m / 2 rows;
        // the other is parent - built (grow.c:361,368)
        g.hist(w.job, m / 2, nl, nr, w.G, w.H);
        A.job = w.job;
        A.seq = n_leaves;               // 1, 2, ... one per split
        A.nid = nid;
        A.split_f = f;
        A.split_b = b;
        A.child_depth = d;
        k_scan_feature<<<dim3(F, 2), WAVE, 0, stream>>>(w.hist, g.hsz, nl, nr, nid, w.path, P, w.fsel, w.fgain,
                                                        w.fb, A);
        k_scan_pick<<<2, WAVE, 0, stream>>>(w.hist, g.hsz, nl, nr, F, w.fsel, w.fgain, w.fb, A);
        if ((rc = launch_status("yabt_grow_ref launch"))) return rc;
        if ((rc = sync_res(A.seq, 2))) return rc;
        const int64_t mid = h_res->mid;
        node_start[nl] = s;
        node_end[nl] = mid;
        node_start[nr] = mid;
        node_end[nr] = e;
        node_depth[nl] = d;
        node_depth[nr] = d;
        n_leaves += 1;
        double glg = h_res->c[0].gain, grg = h_res->c[1].gain;
        if (d >= max_depth) glg = grg = -INFINITY;
        leaf_node[best_k] = nl;
        leaf_gain[best_k] = (float)glg;
        leaf_f[best_k] = h_res->c[0].f;
        leaf_b[best_k] = h_res->c[0].b;
        leaf_node[n_active] = nr;
        leaf_gain[n_active] = (float)grg;
        leaf_f[n_active] = h_res->c[1].f;
        leaf_b[n_active] = h_res->c[1].b;
        n_active += 1;
    }

    // outputs: node count, per-row leaf ids, cgrow's final rows[]
    k_set_status<<<1, 1, 0, stream>>>(out_n_nodes, n_nodes);
    std::vector<int64_t> segs;   // read by the copy below until the final synchronisation
    if (out_leaf_of_row && n > 0) {
        for (int i = 0; i < n_nodes; ++i)
            if (!split[i]) {
                segs.push_back(i);
                segs.push_back(node_start[i]);
                segs.push_back(node_end[i]);
            }
        const int n_leaf = (int)(segs.size() / 3);
        hipError_t e = hipMemcpyAsync(w.segs, segs.data(), segs.size() * sizeof(int64_t), hipMemcpyHostToDevice, stream);
        if (e != hipSuccess) return hip_fail(e, "yabt_grow_ref: leaf segments");
        k_leaf_rows<<<dim3((unsigned)launch_grid(n, RB * 4, 256), (unsigned)n_leaf), RB, 0, stream>>>(w.rows, w.segs,
                                                                                                   n_leaf,
                                                                                                   out_leaf_of_row);
    }
    if (out_rows && n > 0) k_rows_out<<<launch_grid(n, RB * 4, 4096), RB, 0, stream>>>(w.rows, n, out_rows);
    if ((rc = launch_status("yabt_grow_ref launch"))) return rc;
    const hipError_t e = hipStreamSynchronize(stream);
    return e == hipSuccess ? 0 : hip_fail(e, "yabt_grow_ref: final synchronisation");
}

}  // extern "C"
