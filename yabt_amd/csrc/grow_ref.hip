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
//     (grow.c:284-407) run on the host.  A leaf's split, its children's rows
//     (in cgrow's order) and histograms depend only on the leaf's own rows,
//     so the host computes up to KR splits per round -- planned by running
//     the leaf table ahead through the splits already computed -- and
//     commits them in cgrow's best-first order: one device round trip per
//     round.  A node at depth d keeps its rows at [s, e) of row array
//     d % RA, so a computed split never moves its leaf's rows (the lookahead
//     goes at most RA - 1 levels below a committed leaf) and cgrow's final
//     rows[] is the final leaves' segments of their arrays.
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
// Workspace (yabt_grow_ref_workspace_bytes): RA row arrays (n u32), the
// partition's flags / ranks / p / q arrays and the built children's g and h
// by position, the bucket lists, and one (3, F, 256) fp32 histogram per
// slot: the root's and the two children of every computed split.

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
constexpr int KR = 16;             // splits computed per round, at most
constexpr int RA = 16;             // row arrays: a node at depth d uses array d % RA
constexpr int PEND_PER_LEAF = 3;   // computed splits per leaf of the budget, at most

// One split of a round (the root's histogram: a pseudo-job with the whole
// row range as its built child).  The host fills the split; k_part_offsets
// fills the partition's outcome.
struct Job {
    int32_t f, b;                  // the split
    int32_t src, dst;              // row arrays of the leaf (depth % RA) and of its children
    int32_t slot_p, slot_l, slot_r;    // histogram / path slots: the leaf (-1: none), its children
    int32_t build_left;            // the smaller child, ties left (grow.c:355)
    int64_t s, e;                  // the leaf's segment
    int64_t nl;                    // rows going left
    int64_t cs, ce;                // built child's segment
};

// A round as the kernels see it: its splits, their partition blocks and the
// sort tiles of their built children (prefix sums), the round number.
struct Round {
    int32_t K;
    int32_t seq;
    int32_t boff[KR + 1];
    int32_t toff[KR + 1];
    Job job[KR];
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

// Job k of `R` for flattened block or tile index x of prefix sums off[0..K].
__device__ __forceinline__ int job_of(const int32_t* off, int K, int64_t x) {
    int k = 0;
    while (k + 1 < K && off[k + 1] <= x) ++k;
    return k;
}

struct Ws {
    uint32_t* rows;                // RA arrays of rows_ld ids: depth % RA
    int64_t rows_ld;
    uint8_t* flag;
    uint32_t* rank;
    uint32_t* p;
    uint32_t* q;
    uint32_t* blk;                 // per-block left counts, then their exclusive prefix
    float* G;                      // built children's g, h by position
    float* H;
    uint16_t* perm;                // (fgroup, ld_perm): per tile, positions bucketed by bin
    uint16_t* xperm;               // (fgroup, ld_perm): sparse builder, per tile, rows outside the default bin
    uint16_t* starts;              // (fgroup, n_tiles, 257): per tile, bucket starts
    int64_t n_tiles, ld_perm;
    int fgroup;                    // features bucketed per pass
    double* expl;                  // (KR, F, 3): sparse builder's explicit g, h sums, default-bin rows
    double* tot;                   // (KR, 2): sparse builder's node g, h sums
    float* hist;                   // (slots, 3, F, 256)
    int slots;                     // the root's and 2 per computed split
    int pend_cap;                  // computed splits, at most
    double* fsel;                  // (2 KR, F)
    double* fgain;                 // (2 KR, F)
    int32_t* fb;                   // (2 KR, F)
    uint8_t* path;                 // (slots, F)
    int64_t* segs;                 // (N, 4): leaf node, start, end, row array
    Round* round;
    size_t bytes;
};

// The workspace for feature groups of fgroup features.
Ws carve(char* base, int64_t n, int F, int max_leaves, bool sparse, int fgroup) {
    Carve c{base, 0};
    Ws w;
    const int64_t N = 2 * (int64_t)max_leaves + 1;
    const int64_t nn = n > 0 ? n : 1;
    // a round's built children hold at most half of each leaf's rows: at
    // most n / 2 rows in at most n / (2 WT) + KR tiles; the root's n rows in
    // n / WT tiles
    w.n_tiles = (nn + WT - 1) / WT + KR;
    w.ld_perm = w.n_tiles * WT;
    w.fgroup = fgroup;
    w.pend_cap = PEND_PER_LEAF * max_leaves + KR;
    w.slots = 1 + 2 * w.pend_cap;
    w.rows_ld = (nn + 63) / 64 * 64;
    w.rows = c.take<uint32_t>((size_t)RA * (size_t)w.rows_ld);
    w.flag = c.take<uint8_t>(nn);
    w.rank = c.take<uint32_t>(nn);
    w.p = c.take<uint32_t>(nn);
    w.q = c.take<uint32_t>(nn);
    w.blk = c.take<uint32_t>((nn + PT - 1) / PT + KR + 1);
    w.G = c.take<float>(nn);
    w.H = c.take<float>(nn);
    w.perm = c.take<uint16_t>((size_t)fgroup * (size_t)w.ld_perm);
    w.xperm = sparse ? c.take<uint16_t>((size_t)fgroup * (size_t)w.ld_perm) : nullptr;
    w.starts = c.take<uint16_t>((size_t)fgroup * (size_t)w.n_tiles * ST);
    w.expl = c.take<double>((size_t)KR * 3 * (size_t)F);
    w.tot = c.take<double>((size_t)KR * 2);
    w.hist = c.take<float>((size_t)w.slots * 3 * F * NB);
    w.fsel = c.take<double>((size_t)2 * KR * F);
    w.fgain = c.take<double>((size_t)2 * KR * F);
    w.fb = c.take<int32_t>((size_t)2 * KR * F);
    w.path = c.take<uint8_t>((size_t)w.slots * F);
    w.segs = c.take<int64_t>((size_t)N * 4);
    w.round = c.take<Round>(1);
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

__global__ void __launch_bounds__(RB) k_init(uint32_t* rows, int64_t n, uint8_t* path, int F) {
    const int64_t tid = (int64_t)blockIdx.x * RB + threadIdx.x, stride = (int64_t)gridDim.x * RB;
    for (int64_t i = tid; i < n; i += stride) rows[i] = (uint32_t)i;     // grow.c:289
    for (int64_t i = tid; i < F; i += stride) path[i] = 0;               // the root's path
}

// ---------------------------------------------------------------------------
// partition in cgrow's order, every split of a round
// ---------------------------------------------------------------------------
//
// Job k's partition blocks are R->boff[k] .. R->boff[k + 1] - 1, PT rows each
// of its leaf's segment; flags, ranks, p and q are indexed by position (the
// leaves of a round have disjoint segments), p and q hold positions relative
// to the leaf's start.

// Flags (row goes left) and the left count of each PT-row block.  The
// round's job table comes as the kernel argument Rv (no copy of its own
// ahead of the round); block 0 stores it at Rd for the round's other kernels.
__global__ void __launch_bounds__(RB) k_part_flags(const uint8_t* __restrict__ bins_fm, int64_t ld, const Round Rv,
                                                   Round* __restrict__ Rd, const uint32_t* __restrict__ rows,
                                                   int64_t rows_ld, uint8_t* __restrict__ flag,
                                                   uint32_t* __restrict__ blk) {
    __shared__ uint32_t s_red[RB / WAVE];
    if (blockIdx.x == 0) {
        static_assert(sizeof(Round) % 4 == 0, "the job table in words");
        const uint32_t* src = reinterpret_cast<const uint32_t*>(&Rv);
        uint32_t* dst = reinterpret_cast<uint32_t*>(Rd);
        for (int i = threadIdx.x; i < (int)(sizeof(Round) / 4); i += RB) dst[i] = src[i];
    }
    const Round* R = &Rv;
    const int k = job_of(R->boff, R->K, blockIdx.x);
    const Job& J = R->job[k];
    const int64_t s = J.s, m = J.e - J.s;
    const uint32_t* src = rows + (size_t)J.src * (size_t)rows_ld;
    const uint8_t* col = bins_fm + (size_t)J.f * ld;
    const int b = J.b;
    const int64_t x0 = (int64_t)(blockIdx.x - R->boff[k]) * PT;
    uint32_t cnt = 0;
    for (int j = threadIdx.x; j < PT; j += RB) {
        const int64_t x = x0 + j;
        if (x < m) {
            const uint8_t l = (int)col[src[s + x]] <= b ? 1 : 0;
            flag[s + x] = l;
            cnt += l;
        }
    }
    cnt = block_sum<RB, uint32_t>(cnt, s_red);
    if (threadIdx.x == 0) blk[blockIdx.x] = cnt;
}

// Block k: exclusive prefix of job k's block counts; the partition's outcome.
__global__ void __launch_bounds__(RB) k_part_offsets(uint32_t* blk, Round* R) {
    __shared__ uint32_t s_w[RB / WAVE];
    const int k = blockIdx.x;
    Job& J = R->job[k];
    const int b0 = R->boff[k], nblk = R->boff[k + 1] - b0;
    uint32_t carry = 0;
    for (int i0 = 0; i0 < nblk; i0 += RB) {
        const int i = i0 + threadIdx.x;
        const uint32_t v = i < nblk ? blk[b0 + i] : 0u;
        uint32_t tot;
        const uint32_t ex = block_excl_scan<RB, uint32_t>(v, s_w, &tot);
        if (i < nblk) blk[b0 + i] = carry + ex;
        carry += tot;
    }
    if (threadIdx.x == 0) {
        const int64_t m = J.e - J.s;
        J.nl = carry;
        J.build_left = (int64_t)carry <= m - (int64_t)carry ? 1 : 0;
        J.cs = J.build_left ? J.s : J.s + (int64_t)carry;
        J.ce = J.build_left ? J.s + (int64_t)carry : J.e;
    }
}

// Ranks: rank[x] = left rows before x; p (right rows, from the left) and q
// (left rows, from the right) hold positions.
__global__ void __launch_bounds__(RB) k_part_rank(const uint8_t* __restrict__ flag, const uint32_t* __restrict__ blk,
                                                  const Round* __restrict__ R, uint32_t* __restrict__ rank,
                                                  uint32_t* __restrict__ p, uint32_t* __restrict__ q) {
    __shared__ uint32_t s_w[RB / WAVE];
    const int k = job_of(R->boff, R->K, blockIdx.x);
    const Job& J = R->job[k];
    const int64_t s = J.s, m = J.e - J.s;
    const uint32_t nl = (uint32_t)J.nl;
    const int64_t x0 = (int64_t)(blockIdx.x - R->boff[k]) * PT;
    uint32_t carry = blk[blockIdx.x];
    for (int j0 = 0; j0 < PT; j0 += RB) {
        const int64_t x = x0 + j0 + threadIdx.x;
        const uint32_t l = x < m ? flag[s + x] : 0u;
        uint32_t tot;
        const uint32_t ex = carry + block_excl_scan<RB, uint32_t>(l, s_w, &tot);
        if (x < m) {
            rank[s + x] = ex;
            if (l) q[s + nl - ex - 1] = (uint32_t)x;
            else p[s + (uint32_t)x - ex] = (uint32_t)x;
        }
        carry += tot;
    }
}

// Destinations of the two-pointer loop: the children's array at s + dest gets
// the leaf's row at s + x, and the built child's g, h go to the same
// position.  Block 0 of a job records the children's path masks.
__global__ void __launch_bounds__(RB) k_part_permute(const uint8_t* __restrict__ flag,
                                                     const uint32_t* __restrict__ rank, const uint32_t* __restrict__ p,
                                                     const uint32_t* __restrict__ q, const Round* __restrict__ R,
                                                     uint32_t* __restrict__ rows, int64_t rows_ld,
                                                     const float* __restrict__ grad, const float* __restrict__ hess,
                                                     float* __restrict__ G, float* __restrict__ H, uint8_t* path,
                                                     int F) {
    const int k = job_of(R->boff, R->K, blockIdx.x);
    const Job& J = R->job[k];
    const int64_t s = J.s, m = J.e - J.s, nl = J.nl, cs = J.cs, ce = J.ce;
    const uint32_t* src = rows + (size_t)J.src * (size_t)rows_ld;
    uint32_t* dst = rows + (size_t)J.dst * (size_t)rows_ld;
    // K = #{k : p_k < q_k}: p rises and q falls, and p_k < q_k exactly when
    // the k-th left row from the right lies at or after nl, so K is the
    // number of left rows in [nl, m): nl minus the left rows before nl
    const int64_t K = nl < m ? nl - (int64_t)rank[s + nl] : 0;
    const int64_t qK = K == 0 ? m : (int64_t)q[s + K - 1];
    const int64_t x0 = (int64_t)(blockIdx.x - R->boff[k]) * PT;
    for (int j = threadIdx.x; j < PT; j += RB) {
        const int64_t x = x0 + j;
        if (x >= m) break;
        const int64_t lb = rank[s + x];
        int64_t dest;
        if (flag[s + x]) {
            const int64_t t = nl - lb;                 // rank from the right, 1-based
            dest = t <= K ? (int64_t)p[s + t - 1] : x;
        } else {
            const int64_t r = x - lb + 1;              // rank from the left, 1-based
            if (r <= K) dest = (r == 1 ? m : (int64_t)q[s + r - 2]) - 1;
            else if (r == K + 1 && x < qK) dest = qK - 1;
            else dest = x - 1;
        }
        const uint32_t row = src[s + x];
        const int64_t at = s + dest;
        dst[at] = row;
        if (at >= cs && at < ce) {
            G[at] = grad[row];
            H[at] = hess[row];
        }
    }
    if (blockIdx.x == R->boff[k]) {
        for (int jf = threadIdx.x; jf < F; jf += RB) {
            const uint8_t v = (uint8_t)(path[(size_t)J.slot_p * F + jf] | (jf == J.f ? 1 : 0));
            path[(size_t)J.slot_l * F + jf] = v;
            path[(size_t)J.slot_r * F + jf] = v;
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
// parallel over the whole device; a chain kernel then runs one block per
// (feature, split) over the tiles in order, adding bin b's run of each tile
// to its fp32 accumulators, so every cell is cgrow's sequential sum.
// Dense (k_walk_chain_dense): the tile's g and h permuted into bucket order
// in LDS, one thread per (bin, channel).
//
// Sparse builder (grow.c:68-107, default bins dbin; k_walk_chain<true>): the
// default bin gets no run; its thread instead adds, in double and in row
// order, the tile's rows outside the default bin; block F adds the node's g
// and h in double in row order; k_hist_default combines them.

constexpr int SW = RB / WAVE;             // waves per sort / chain block
constexpr int SSUB = WT / SW;             // rows per wave per tile (sort)
constexpr int SGR = SSUB / WAVE;          // 64-row groups per wave per tile (sort)
constexpr int TPT = WT / RB;              // rows per thread per tile

// Bin of the node's row at position x: row x for the root (rows[] is the
// identity there, grow.c:289), rows[cs + x] of the children's array for a
// built child.
template <bool ROOT>
__device__ __forceinline__ uint32_t node_bin(const uint8_t* __restrict__ bins_fm, int64_t ld_fm,
                                            const uint8_t* __restrict__ bins_rm, int64_t ld_rm,
                                            const uint32_t* __restrict__ rows, int64_t cs, int f, int64_t x) {
    if (ROOT) return bins_fm[(size_t)f * (size_t)ld_fm + (size_t)x];
    return bins_rm[(size_t)rows[cs + x] * (size_t)ld_rm + f];
}

// Stable bucketing of one tile of one feature (block (f, t), t a tile of
// the round's built children: job k's tiles are R->toff[k] ..
// R->toff[k + 1] - 1, the ones past its child's rows idle): perm[f][t*WT + k]
// lists the tile's positions bin by bin, each bin in row order, and
// starts[f][t][b] is where bin b's run begins (starts[...][256] = the run
// total).  The lanes of a wave sharing a bin are found by an LDS atomic OR of
// each lane's bit into s_peer[w][bin] (order-free), read back and cleared; a
// row's rank is the number of those lanes below it plus the wave's running
// count s_cnt[w][bin].  Sparse builder (dbin): the default bin gets no run,
// and xperm lists the tile's other positions in row order.
template <bool ROOT, bool SPARSE>
__global__ void __launch_bounds__(RB, SPARSE ? 5 : 8) k_walk_sort(const uint8_t* __restrict__ bins_fm, int64_t ld_fm,
                                                  const uint8_t* __restrict__ bins_rm, int64_t ld_rm,
                                                  const uint32_t* __restrict__ rows, int64_t rows_ld,
                                                  const Round* __restrict__ R, int fg0,
                                                  const int32_t* __restrict__ dbin, uint16_t* __restrict__ perm,
                                                  uint16_t* __restrict__ xperm, int64_t ld_perm,
                                                  uint16_t* __restrict__ starts, int64_t n_tiles) {
    __shared__ uint8_t s_bin[WT];
    __shared__ uint64_t s_peer[SW][NB];            // once the tile is ranked: its bucketed positions
    __shared__ uint32_t s_cnt[SW][NB];
    __shared__ uint16_t s_xperm[SPARSE ? WT : 1];
    static_assert(sizeof(s_peer) == WT * sizeof(uint16_t), "the bucketed positions fill the peer masks' space");
    uint16_t* s_perm = reinterpret_cast<uint16_t*>(&s_peer[0][0]);
    __shared__ uint32_t s_scan[SW];
    __shared__ uint32_t s_xoff[SW + 1];
    const int fl = blockIdx.x, f = fg0 + fl;       // buffers by group position, bins by feature
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), w = tid / WAVE;
    const int df = SPARSE ? dbin[f] : -1;
    const int K = R->K;
    for (int64_t t = blockIdx.y; t < R->toff[K]; t += gridDim.y) {
    const int kj = job_of(R->toff, K, t);
    const Job& J = R->job[kj];
    const int64_t cs = J.cs, m = J.ce - J.cs;
    const int64_t t0 = (t - R->toff[kj]) * WT;      // the tile's first row in the child
    if (t0 >= m) continue;                          // uniform across the block
    const uint32_t* crow = rows + (size_t)J.dst * (size_t)rows_ld;
    const int tn = (int)min((int64_t)WT, m - t0);
    for (int i = tid; i < SW * NB; i += RB) {
        (&s_cnt[0][0])[i] = 0;
        (&s_peer[0][0])[i] = 0;
    }
#pragma unroll 2
    for (int j = 0; j < TPT; ++j) {
        const int x = j * RB + tid;
        if (x < tn) s_bin[x] = (uint8_t)node_bin<ROOT>(bins_fm, ld_fm, bins_rm, ld_rm, crow, cs, f, t0 + x);
    }
    __syncthreads();
    // per group: the rank (bits 0-9), the sparse rank outside the default bin
    // (bits 10-19) and the bin (bits 24-31) in one register
    uint32_t pk[SGR];
    uint32_t xrun = 0;
#pragma unroll
    for (int q = 0; q < SGR; ++q) {
        const int x = w * SSUB + q * WAVE + lane;
        const bool v = x < tn;
        const uint32_t bin = v ? (uint32_t)s_bin[x] : 0u;
        if (v) atomicOr(&s_peer[w][bin], 1ull << lane);
        __builtin_amdgcn_wave_barrier();
        const uint64_t peers = v ? s_peer[w][bin] : 0ull;
        const uint32_t base = v ? s_cnt[w][bin] : 0u;
        __builtin_amdgcn_wave_barrier();
        const uint32_t r = lane_prefix(peers);
        if (v) s_peer[w][bin] = 0ull;
        if (v && r == 0) s_cnt[w][bin] = base + (uint32_t)__popcll(peers);
        __builtin_amdgcn_wave_barrier();
        pk[q] = (base + r) | (bin << 24);
        if (SPARSE) {
            const uint64_t xb = __ballot(v && (int)bin != df);
            pk[q] |= (xrun + lane_prefix(xb)) << 10;
            xrun += (uint32_t)__popcll(xb);
        }
        // packed here, not where it is used: otherwise its three parts stay
        // live in registers of their own through the remaining groups
        asm volatile("" : "+v"(pk[q]));
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
        const uint32_t bin = pk[q] >> 24;
        if (x < tn && (!SPARSE || (int)bin != df)) {
            s_perm[s_cnt[w][bin] + (pk[q] & 1023u)] = (uint16_t)x;
            if (SPARSE) s_xperm[s_xoff[w] + ((pk[q] >> 10) & 1023u)] = (uint16_t)x;
        }
    }
    __syncthreads();
    const int total = SPARSE ? (int)s_xoff[SW] : tn;
    uint16_t* po = perm + (size_t)fl * (size_t)ld_perm + (size_t)t * WT;
    for (int k = tid; k < total; k += RB) po[k] = s_perm[k];
    if (SPARSE) {
        uint16_t* xo = xperm + (size_t)fl * (size_t)ld_perm + (size_t)t * WT;
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

// The sequential double sum S <- RN(S + (double)x_k), k = 0 .. tn - 1 in
// order, of each channel of the fp32 pairs s_gh[k] (cgrow's node totals,
// grow.c:85-97), computed by the whole block with the same result.  A step
// rounds only when the exact partial sum does not fit a double's 53 bits,
// and with fp32 addends that is rare (an addend far below |S|, or |S|
// growing past a binade with its lowest bit set); the steps before the first
// rounding give the exact sum, which any order computes.  So, in fixed point
// with unit u = 2^(Emax - 61), where 2^Emax bounds |S| + sum |x_k| (every
// exact partial sum below 2^62 u): each thread takes its share of the
// elements as integers x_k / u, a block scan gives every exact prefix, and
// the first element that is not a multiple of u or whose exact prefix does
// not fit a double is added on its own as cgrow adds it; the tile then
// starts again from the new S.  S is kept as S_int u + S_lo, |S_lo| < u: a
// prefix T u + S_lo has S_lo's lowest bit, so it fits if |T| < 2^(l + 53 -
// log2 u), l the exponent of that bit; with S_lo = 0 it fits if T's odd
// part is below 2^53.  After TSE_TRIES restarts in one tile the remaining
// elements are added one by one by one thread.  Every thread holds the same S.
constexpr int TSE_TRIES = 8;
// Element k of the sum: channel ch of s_gh[k], or of s_gh[idx[k]] with IDX.
template <bool IDX>
__device__ __forceinline__ float tse_x(const float2* s_gh, const uint16_t* idx, int ch, int k) {
    const float2 p = s_gh[IDX ? (int)idx[k] : k];
    return ch ? p.y : p.x;
}

// The exponent of x's lowest set bit (x finite, nonzero).
__device__ __forceinline__ int tse_lsb_exp(double x) {
    const uint64_t b = (uint64_t)__double_as_longlong(x) & 0x7fffffffffffffffull;
    const int e = (int)(b >> 52);
    uint64_t m = b & 0x000fffffffffffffull;
    if (e == 0) return -1074 + __builtin_ctzll(m);
    m |= 0x0010000000000000ull;
    return e - 1075 + __builtin_ctzll(m);
}

// Both channels at once (g: c = 0, h: c = 1), so that they share the
// block's passes and barriers; each channel restarts on its own.  s_wave:
// 2 x RB / WAVE words, s_k, s_s, s_m: two each.
template <bool IDX>
__device__ void tile_sum_exact(const float2* s_gh, const uint16_t* idx, int tn, double (&S)[2], int64_t* s_wave,
                               int* s_k, double* s_s, double* s_m) {
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), w = tid / WAVE;
    constexpr int NW = RB / WAVE;
    int k0[2] = {0, 0}, tries[2] = {0, 0};
    for (;;) {
        bool act[2];
#pragma unroll
        for (int c = 0; c < 2; ++c) act[c] = k0[c] < tn;
        if (!act[0] && !act[1]) return;
        // a channel with many restarts: its rest one by one (threads 0 and 1)
#pragma unroll
        for (int c = 0; c < 2; ++c)
            if (act[c] && tries[c] >= TSE_TRIES) {
                if (tid == c) {
                    double a = S[c];
                    for (int k = k0[c]; k < tn; ++k) a += (double)tse_x<IDX>(s_gh, idx, c, k);
                    s_s[c] = a;
                }
            }
        __syncthreads();
#pragma unroll
        for (int c = 0; c < 2; ++c)
            if (act[c] && tries[c] >= TSE_TRIES) {
                S[c] = s_s[c];
                k0[c] = tn;
                act[c] = false;
            }
        __syncthreads();
        if (!act[0] && !act[1]) return;
        int kb[2], ke[2];
        double am[2] = {0.0, 0.0};
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int cnt = tn - k0[c], per = (cnt + RB - 1) / RB;
            kb[c] = k0[c] + tid * per;
            ke[c] = min(tn, kb[c] + per);
            if (act[c])
                for (int k = kb[c]; k < ke[c]; ++k) am[c] += fabs((double)tse_x<IDX>(s_gh, idx, c, k));
#pragma unroll
            for (int d = WAVE / 2; d > 0; d >>= 1) am[c] += __shfl_xor(am[c], d, WAVE);
        }
        if (tid < 2) s_m[tid] = 0.0;
        __syncthreads();
        if (lane == 0) {
            atomicAdd(&s_m[0], am[0]);
            atomicAdd(&s_m[1], am[1]);
        }
        __syncthreads();
        double M[2];
#pragma unroll
        for (int c = 0; c < 2; ++c) M[c] = (fabs(S[c]) + s_m[c]) * (1.0 + 0x1p-30);
        int ue[2];
        double sc[2], Slo[2];
        int64_t Sint[2], TL[2];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            if (act[c] && M[c] == 0.0) {      // S and the rest are zeros
                k0[c] = tn;
                act[c] = false;
            }
            if (act[c] && !(M[c] <= 0x1p1000)) {   // inf, NaN or near them: the rest one by one
                tries[c] = TSE_TRIES;
                act[c] = false;               // (this round does nothing for c)
            }
            int Emax = 0;
            if (act[c]) (void)frexp(M[c], &Emax);   // 2^(Emax - 1) <= M < 2^Emax
            ue[c] = Emax - 61;                // u = 2^ue: |partial sums| < 2^Emax = 2^61 u
            sc[c] = ldexp(1.0, -ue[c]);
            Sint[c] = act[c] ? (int64_t)(S[c] * sc[c]) : 0;   // exact scale, truncated
            Slo[c] = act[c] ? S[c] - ldexp((double)Sint[c], ue[c]) : 0.0;
            TL[c] = 0;
            if (Slo[c] != 0.0) {
                const int sh = tse_lsb_exp(Slo[c]) + 53 - ue[c];
                TL[c] = sh > 0 ? ((int64_t)1 << sh) - 1 : 0;
            }
        }
        auto fits = [&](int c, int64_t T) -> bool {
            if (Slo[c] != 0.0) return (T < 0 ? -T : T) <= TL[c];
            if (T == 0) return true;
            uint64_t t = (uint64_t)(T < 0 ? -T : T);
            t >>= __builtin_ctzll(t);
            return t < ((uint64_t)1 << 53);
        };
        auto unit = [&](int c, int k, int64_t& r) -> bool {   // x_k / u, if an integer
            const double v = (double)tse_x<IDX>(s_gh, idx, c, k) * sc[c];
            if (v != rint(v) || fabs(v) >= 0x1p62) return false;
            r = (int64_t)v;
            return true;
        };
        int64_t loc[2] = {0, 0};
#pragma unroll
        for (int c = 0; c < 2; ++c)
            if (act[c])
                for (int k = kb[c]; k < ke[c]; ++k) {
                    int64_t r = 0;
                    if (unit(c, k, r)) loc[c] += r;
                }
        // exclusive scans of both channels' sums over the block
        int64_t ex[2], total[2];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int64_t e = wave_incl_scan_i64(loc[c], lane) - loc[c];
            if (lane == WAVE - 1) s_wave[c * NW + w] = e + loc[c];
            ex[c] = e;
        }
        __syncthreads();
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            int64_t off = 0, tot = 0;
#pragma unroll
            for (int i = 0; i < NW; ++i) {
                const int64_t v = s_wave[c * NW + i];
                if (i < w) off += v;
                tot += v;
            }
            ex[c] += off;
            total[c] = tot;
        }
        int bad[2] = {INT_MAX, INT_MAX};
        int64_t Tbad[2] = {0, 0};
#pragma unroll
        for (int c = 0; c < 2; ++c)
            if (act[c]) {
                int64_t T = Sint[c] + ex[c];
                for (int k = kb[c]; k < ke[c]; ++k) {
                    int64_t r = 0;
                    if (!unit(c, k, r) || !fits(c, T + r)) {
                        bad[c] = k;
                        Tbad[c] = T;          // the exact prefix before element k
                        break;
                    }
                    T += r;
                }
            }
        // first failures of both channels over the block
        const int m0 = wave_min_i32(bad[0]), m1 = wave_min_i32(bad[1]);
        if (tid < 2) s_k[tid] = INT_MAX;
        __syncthreads();                      // (also: every wave has read s_wave)
        if (lane == 0) {
            atomicMin(&s_k[0], m0);
            atomicMin(&s_k[1], m1);
        }
        __syncthreads();
        const int kf[2] = {s_k[0], s_k[1]};
#pragma unroll
        for (int c = 0; c < 2; ++c)
            if (act[c] && kf[c] != INT_MAX && kb[c] <= kf[c] && kf[c] < ke[c])   // cgrow's add of element kf
                s_s[c] = (ldexp((double)Tbad[c], ue[c]) + Slo[c]) + (double)tse_x<IDX>(s_gh, idx, c, kf[c]);
        __syncthreads();
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            if (!act[c]) continue;
            if (kf[c] == INT_MAX) {           // no rounding in the rest: the exact sum
                S[c] = ldexp((double)(Sint[c] + total[c]), ue[c]) + Slo[c];
                k0[c] = tn;
            } else {
                S[c] = s_s[c];
                k0[c] = kf[c] + 1;
                ++tries[c];
            }
        }
        __syncthreads();                      // s_s, s_k and s_m are rewritten next round
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

// The chains with default bins (block f, thread b = bin; SPARSE; dense
// chains run in k_walk_chain_dense): the node's tiles in order, each tile's
// g, h and bucketed positions staged in LDS, bin b's run added in fp32 in row
// order (grow.c:55-59); the count cell is cgrow's chain of 1.0f adds, which
// is min(count, 2^24) exactly.  The default bin's thread adds the tile's
// other rows in double in row order (xperm), and block F adds the node's g
// and h in double in row order (grow.c:85-97); k_hist_default combines them.
// G, H hold the node's g, h by position.
// Block (f, k): job k's built child (its tiles R->toff[k] ..); G, H hold the
// g, h of the child's rows at their positions.
template <bool SPARSE>
__global__ void __launch_bounds__(RB) k_walk_chain(const float* __restrict__ Gb, const float* __restrict__ Hb,
                                                   const Round* __restrict__ R, int F, int fg0, int nf,
                                                   const int32_t* __restrict__ dbin,
                                                   const uint16_t* __restrict__ perm,
                                                   const uint16_t* __restrict__ xperm, int64_t ld_perm,
                                                   const uint16_t* __restrict__ starts, int64_t n_tiles,
                                                   float* __restrict__ hist_base, size_t hsz,
                                                   double* __restrict__ eout_b, double* __restrict__ tot_b) {
    __shared__ __align__(16) float2 s_gh[WT];
    __shared__ uint16_t s_idx[WT];
    __shared__ uint16_t s_xidx[SPARSE ? WT : 1];
    __shared__ uint16_t s_st[ST];
    __shared__ int64_t s_tw[2 * (RB / WAVE)];         // the totals block's scans
    __shared__ int s_tk[2];
    __shared__ double s_ts[2], s_tm[2];
    const int kj = blockIdx.y;
    const Job& J = R->job[kj];
    const int64_t m = J.ce - J.cs;
    const int64_t tile0 = R->toff[kj];
    const float* G = Gb + J.cs;
    const float* H = Hb + J.cs;
    double* eout = eout_b + (size_t)kj * 3 * F;
    double* tot = tot_b + (size_t)kj * 2;
    const int tid = threadIdx.x;
    const int fl = blockIdx.x, f = fg0 + fl;       // buffers by group position, cells by feature
    const bool totals = SPARSE && fl == nf;        // the extra block of the first group
    const int df = (SPARSE && !totals) ? dbin[f] : -1;
    const size_t fo = (size_t)(totals ? 0 : fl);
    const uint16_t* pf = perm + fo * (size_t)ld_perm + (size_t)tile0 * WT;
    const uint16_t* xf = SPARSE ? xperm + fo * (size_t)ld_perm + (size_t)tile0 * WT : nullptr;
    const uint16_t* sf = starts + (fo * (size_t)n_tiles + (size_t)tile0) * ST;
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
            // the node's g and h in double in row order, by the whole block
            double S2[2] = {eg, eh};
            tile_sum_exact<false>(s_gh, nullptr, tn, S2, s_tw, s_tk, s_ts, s_tm);
            eg = S2[0];
            eh = S2[1];
        } else {
            if (SPARSE && tid == df) {
                cnt += (int64_t)tn - s_st[NB];
            } else {
                const uint32_t lo = s_st[tid], hi = s_st[tid + 1];
                run_f32(s_gh, s_idx, lo, hi, ag, ah);
                cnt += hi - lo;
            }
            if (SPARSE) {
                // the tile's rows outside the default bin (xidx, in row
                // order), their g and h in double, by the whole block
                double S2[2] = {eg, eh};
                tile_sum_exact<true>(s_gh, s_xidx, (int)s_st[NB], S2, s_tw, s_tk, s_ts, s_tm);
                eg = S2[0];
                eh = S2[1];
            }
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
    const int slot = J.build_left ? J.slot_l : J.slot_r;
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

// Sequential fp32 sum of s[k], k in [lo, hi) (hi <= WT): blocks of 16 read 8
// ahead of the adds, so that a long run (a bin that holds most of a tile, as
// the features on a node's path do) waits about one LDS latency per 16
// values rather than per 8; the block's last prefetch reads inside the
// array whether or not it is used.
__device__ __forceinline__ void run_f32_one(const float* s, uint32_t lo, uint32_t hi, float& acc) {
    uint32_t k = lo;
    const uint32_t nb = (hi - lo) / 16;
    if (nb > 0) {
        float a[8], b[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) a[u] = s[k + u];
        for (uint32_t blk = 0; blk < nb; ++blk) {
#pragma unroll
            for (int u = 0; u < 8; ++u) b[u] = s[k + 8 + u];
#pragma unroll
            for (int u = 0; u < 8; ++u) acc += a[u];
            const uint32_t kn = min(k + 16, (uint32_t)(WT - 8));
#pragma unroll
            for (int u = 0; u < 8; ++u) a[u] = s[kn + u];
#pragma unroll
            for (int u = 0; u < 8; ++u) acc += b[u];
            k += 16;
        }
    }
    if (k + 8 <= hi) {
        float p[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) p[u] = s[k + u];
#pragma unroll
        for (int u = 0; u < 8; ++u) acc += p[u];
        k += 8;
    }
    for (; k < hi; ++k) acc += s[k];
}

constexpr int CB = 2 * RB;           // threads of a dense chain block: bin b's g chain, then its h chain
constexpr int CPT = WT / CB;         // positions per thread per tile

// One tile of a dense chain block, CPT positions per thread, loaded a tile ahead.
struct DenseTile {
    float g[CPT], h[CPT];
    uint32_t idx[CPT];
    uint32_t st;                     // threads 0 .. NB: bucket start (NB: the run total)
};

__device__ __forceinline__ void dense_load(DenseTile& c, const float* __restrict__ G, const float* __restrict__ H,
                                           const uint16_t* __restrict__ pf, const uint16_t* __restrict__ sf,
                                           int64_t t, int64_t m) {
    const int64_t t0 = t * WT;
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int64_t x = t0 + j * CB + threadIdx.x;
        if (x < m) {
            c.g[j] = G[x];
            c.h[j] = H[x];
            c.idx[j] = pf[x];
        }
    }
    if (threadIdx.x <= NB) c.st = sf[(size_t)t * ST + threadIdx.x];
}

// Dense chains (no default bins): block (f, k), thread b (< NB) adds bin b's
// g and thread NB + b its h, each in fp32 in row order (grow.c:55-59), from
// the tile's pairs permuted into bucket order in LDS (channel by channel,
// so a bin's run is contiguous); the count cell is cgrow's chain of 1.0f
// adds, min(count, 2^24).  A bin's two channels run in different waves:
// one dependent add per row and thread.
__global__ void __launch_bounds__(CB) k_walk_chain_dense(const float* __restrict__ Gb, const float* __restrict__ Hb,
                                                         const Round* __restrict__ R, int F, int fg0,
                                                         const uint16_t* __restrict__ perm, int64_t ld_perm,
                                                         const uint16_t* __restrict__ starts, int64_t n_tiles,
                                                         float* __restrict__ hist_base, size_t hsz) {
    __shared__ __align__(16) float2 s_gh[WT];
    __shared__ float s_ch[2][WT];    // g, h in bucket order
    __shared__ uint16_t s_st[ST];
    const int kj = blockIdx.y;
    const Job& J = R->job[kj];
    const int64_t m = J.ce - J.cs;
    const int64_t tile0 = R->toff[kj];
    const float* G = Gb + J.cs;
    const float* H = Hb + J.cs;
    const int tid = threadIdx.x, ch = tid / NB, b = tid % NB;
    const int fl = blockIdx.x, f = fg0 + fl;       // buffers by group position, cells by feature
    const uint16_t* pf = perm + (size_t)fl * (size_t)ld_perm + (size_t)tile0 * WT;
    const uint16_t* sf = starts + ((size_t)fl * (size_t)n_tiles + (size_t)tile0) * ST;
    float acc = 0.0f;
    int64_t cnt = 0;
    DenseTile nxt;
    if (m > 0) dense_load(nxt, G, H, pf, sf, 0, m);
    for (int64_t t = 0, t0 = 0; t0 < m; ++t, t0 += WT) {
        const int tn = (int)min((int64_t)WT, m - t0);
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int x = j * CB + tid;
            if (x < tn) s_gh[x] = make_float2(nxt.g[j], nxt.h[j]);
        }
        if (tid <= NB) s_st[tid] = (uint16_t)nxt.st;
        __syncthreads();
        // bucket order: entry k of the lists is position idx (every read
        // issued before the first write)
        float2 v[CPT];
#pragma unroll
        for (int j = 0; j < CPT; ++j) v[j] = s_gh[j * CB + tid < tn ? nxt.idx[j] : 0u];
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int k = j * CB + tid;
            if (k < tn) {
                s_ch[0][k] = v[j].x;
                s_ch[1][k] = v[j].y;
            }
        }
        __syncthreads();
        if (t0 + WT < m) dense_load(nxt, G, H, pf, sf, t + 1, m);
        const uint32_t lo = s_st[b], hi = s_st[b + 1];
        run_f32_one(s_ch[ch], lo, hi, acc);
        cnt += hi - lo;
        __syncthreads();
    }
    const int slot = J.build_left ? J.slot_l : J.slot_r;
    float* hist = hist_base + (size_t)slot * hsz;
    hist[(size_t)ch * F * NB + (size_t)f * NB + b] = acc;
    if (ch == 0) hist[(size_t)2 * F * NB + (size_t)f * NB + b] = (float)min(cnt, (int64_t)1 << 24);
}

// ---------------------------------------------------------------------------
// the root's histogram from a per-fit rank table
// ---------------------------------------------------------------------------
//
// The root's rows are 0 .. n - 1 in order (grow.c:289) and a fit's bins do
// not change between its trees, so the bucketing of every (feature, WT-row
// tile) of the root is the same for each tree of a fit.  k_root_rank computes
// it once: for each position its rank inside its bin's run in its tile (runs
// in row order, as k_walk_sort's), and each tile's run starts.  Each tree's
// root then runs only the chains, k_rank_chain: one block per feature, thread
// b = bin b, the tiles in order; a tile's g, h go into an LDS table T[rank][bin]
// (a window of ranks at a time: RW of 256 bins, more of fewer), so that step r
// of every thread reads its run's r-th entry from one row of T -- consecutive
// cells across a wave, no bank conflicts -- and adds it in fp32 as cgrow does
// (grow.c:55-59).

constexpr int RW = 32;             // ranks per window of k_rank_chain's LDS table at 256 bins

// The rank table of yabt_ref_root_order: ranks (uint16, F x ld_rank, position
// t * WT + x of feature f at f * ld_rank + t * WT + x), the run starts
// (uint16, F x tiles x ST, as k_walk_sort's), each (feature, tile)'s longest
// run (uint16, F x tiles) and its largest bin present (uint8, F x tiles).
struct RootOrder {
    uint16_t* rank;
    uint16_t* starts;
    uint16_t* maxrun;
    uint8_t* maxbin;
    int64_t ld_rank;
    int64_t tiles;
};

__host__ __device__ inline size_t root_order_carve(char* base, int64_t n, int F, RootOrder* o) {
    const int64_t tiles = (n + WT - 1) / WT > 0 ? (n + WT - 1) / WT : 1;
    const int64_t ld = tiles * WT;
    const size_t rank_bytes = ((size_t)F * (size_t)ld * sizeof(uint16_t) + 255) / 256 * 256;
    const size_t st_bytes = ((size_t)F * (size_t)tiles * ST * sizeof(uint16_t) + 255) / 256 * 256;
    const size_t mx_bytes = ((size_t)F * (size_t)tiles * sizeof(uint16_t) + 255) / 256 * 256;
    const size_t mb_bytes = ((size_t)F * (size_t)tiles + 255) / 256 * 256;
    if (o) {
        o->rank = (uint16_t*)base;
        o->starts = (uint16_t*)(base + rank_bytes);
        o->maxrun = (uint16_t*)(base + rank_bytes + st_bytes);
        o->maxbin = (uint8_t*)(base + rank_bytes + st_bytes + mx_bytes);
        o->ld_rank = ld;
        o->tiles = tiles;
    }
    return rank_bytes + st_bytes + mx_bytes + mb_bytes;
}

// Block (f, t): the ranks and run starts of feature f's tile t (tiles grid-
// strided over y), bucketed as in k_walk_sort.
__global__ void __launch_bounds__(RB, 8) k_root_rank(const uint8_t* __restrict__ bins_fm, int64_t ld_fm, int64_t n,
                                                  RootOrder o) {
    __shared__ uint8_t s_bin[WT];
    __shared__ uint64_t s_peer[SW][NB];
    __shared__ uint32_t s_cnt[SW][NB];
    __shared__ uint32_t s_scan[SW];
    __shared__ uint32_t s_max, s_mb;
    const int f = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & (WAVE - 1), w = tid / WAVE;
    for (int64_t t = blockIdx.y; t < o.tiles; t += gridDim.y) {
        const int64_t t0 = t * WT;
        const int tn = (int)max((int64_t)0, min((int64_t)WT, n - t0));
        for (int i = tid; i < SW * NB; i += RB) {
            (&s_cnt[0][0])[i] = 0;
            (&s_peer[0][0])[i] = 0;
        }
        if (tid == 0) {
            s_max = 0;
            s_mb = 0;
        }
#pragma unroll
        for (int j = 0; j < TPT; ++j) {
            const int x = j * RB + tid;
            if (x < tn) s_bin[x] = bins_fm[(size_t)f * (size_t)ld_fm + (size_t)(t0 + x)];
        }
        __syncthreads();
        uint32_t pk[SGR];   // per group: the rank (bits 0-9) and the bin (bits 24-31)
#pragma unroll
        for (int q = 0; q < SGR; ++q) {
            const int x = w * SSUB + q * WAVE + lane;
            const bool v = x < tn;
            const uint32_t bin = v ? (uint32_t)s_bin[x] : 0u;
            if (v) atomicOr(&s_peer[w][bin], 1ull << lane);
            __builtin_amdgcn_wave_barrier();
            const uint64_t peers = v ? s_peer[w][bin] : 0ull;
            const uint32_t base = v ? s_cnt[w][bin] : 0u;
            __builtin_amdgcn_wave_barrier();
            const uint32_t r = lane_prefix(peers);
            if (v) s_peer[w][bin] = 0ull;
            if (v && r == 0) s_cnt[w][bin] = base + (uint32_t)__popcll(peers);
            __builtin_amdgcn_wave_barrier();
            pk[q] = (base + r) | (bin << 24);
            asm volatile("" : "+v"(pk[q]));   // packed here, not at its use
        }
        __syncthreads();
        {
            const int b = tid;
            uint32_t c[SW];
            uint32_t tb = 0;
#pragma unroll
            for (int u = 0; u < SW; ++u) {
                c[u] = s_cnt[u][b];
                tb += c[u];
            }
            uint32_t total;
            atomicMax(&s_max, tb);
            if (tb) atomicMax(&s_mb, (uint32_t)b);
            const uint32_t st = block_excl_scan<RB, uint32_t>(tb, s_scan, &total);
            if (tid == 0) {
                o.maxrun[(size_t)f * (size_t)o.tiles + (size_t)t] = (uint16_t)s_max;
                o.maxbin[(size_t)f * (size_t)o.tiles + (size_t)t] = (uint8_t)s_mb;
            }
            uint16_t* st_out = o.starts + ((size_t)f * (size_t)o.tiles + (size_t)t) * ST;
            st_out[b] = (uint16_t)st;
            if (b == NB - 1) st_out[NB] = (uint16_t)(st + tb);
            // wave u's share of bin b starts c[0] + .. + c[u - 1] into the run
            uint32_t run = 0;
#pragma unroll
            for (int u = 0; u < SW; ++u) {
                s_cnt[u][b] = run;
                run += c[u];
            }
        }
        __syncthreads();
        uint16_t* ro = o.rank + (size_t)f * (size_t)o.ld_rank + (size_t)t0;
#pragma unroll
        for (int q = 0; q < SGR; ++q) {
            const int x = w * SSUB + q * WAVE + lane;
            if (x < tn) ro[x] = (uint16_t)(s_cnt[w][pk[q] >> 24] + (pk[q] & 1023u));
        }
        __syncthreads();
    }
}

// k_rank_chain's producers: RPROD threads, each loading RQ groups of four
// positions of a tile.  Many producers with few positions each keep several
// tiles in flight within the registers (RING tiles ahead).
constexpr int RPROD = 2 * RB;
constexpr int RQ = WT / (4 * RPROD);
constexpr int RPT = 4 * RQ;                  // positions per producer and tile
constexpr int RING = 3;
static_assert(RQ * 4 * RPROD == WT, "a tile in whole groups of four per producer");

// One tile's positions for a producer thread of k_rank_chain, RQ groups of
// four: entry j = 4 q + k is position t WT + q 4 RPROD + 4 slot + k, so a
// wave's 16-byte loads of g (and of h) cover 1 KB in one piece and its loads
// of ranks and bins 512 and 256 bytes.  The tile keeps the loaded words as
// they are: unpacking them at load time would wait for the loads there, and
// the loads are meant to run under earlier tiles' work.
struct RankTile {
    float4 g[RQ], h[RQ];
    uint2 r[RQ];                   // ranks, 16 bits each; 0xffff: past the rows
    uint32_t bw[RQ];               // bins, 8 bits each
};

__device__ __forceinline__ float rt_g(const RankTile& c, int j) {
    const float4 v = c.g[j >> 2];
    return (j & 3) == 0 ? v.x : (j & 3) == 1 ? v.y : (j & 3) == 2 ? v.z : v.w;
}
__device__ __forceinline__ float rt_h(const RankTile& c, int j) {
    const float4 v = c.h[j >> 2];
    return (j & 3) == 0 ? v.x : (j & 3) == 1 ? v.y : (j & 3) == 2 ? v.z : v.w;
}
__device__ __forceinline__ uint32_t rt_rank(const RankTile& c, int j) {
    const uint32_t w = (j & 2) ? c.r[j >> 2].y : c.r[j >> 2].x;
    return (j & 1) ? (w >> 16) : (w & 0xffffu);
}
__device__ __forceinline__ uint32_t rt_bin(const RankTile& c, int j) { return (c.bw[j >> 2] >> (8 * (j & 3))) & 0xffu; }

// A whole tile ((t + 1) WT <= n) with 16-byte aligned g, h and bins: loads
// only, no branch (a branch joining a second way of filling the tile would
// make the compiler wait for these loads right here).
__device__ __forceinline__ void rank_tile_load_vec(RankTile& c, const float* __restrict__ g,
                                                   const float* __restrict__ h, const uint8_t* __restrict__ bn,
                                                   const uint16_t* __restrict__ rk, int64_t t, int slot) {
    const int64_t x0 = t * WT + 4 * (int64_t)slot;
#pragma unroll
    for (int q = 0; q < RQ; ++q) c.g[q] = *reinterpret_cast<const float4*>(g + x0 + q * 4 * RPROD);
#pragma unroll
    for (int q = 0; q < RQ; ++q) c.h[q] = *reinterpret_cast<const float4*>(h + x0 + q * 4 * RPROD);
#pragma unroll
    for (int q = 0; q < RQ; ++q) c.r[q] = *reinterpret_cast<const uint2*>(rk + x0 + q * 4 * RPROD);
#pragma unroll
    for (int q = 0; q < RQ; ++q) c.bw[q] = *reinterpret_cast<const uint32_t*>(bn + x0 + q * 4 * RPROD);
}

// Any tile, one position at a time (the last, partial tile, or unaligned data).
__device__ __forceinline__ void rank_tile_load_any(RankTile& c, const float* __restrict__ g,
                                                   const float* __restrict__ h, const uint8_t* __restrict__ bn,
                                                   const uint16_t* __restrict__ rk, int64_t t, int64_t n, int slot) {
#pragma unroll
    for (int q = 0; q < RQ; ++q) {
        const int64_t x = t * WT + (int64_t)q * 4 * RPROD + 4 * (int64_t)slot;
        float gv[4] = {0.0f, 0.0f, 0.0f, 0.0f}, hv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        uint32_t rv[4] = {0xffffu, 0xffffu, 0xffffu, 0xffffu}, bv = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if (x + k < n) {
                gv[k] = g[x + k];
                hv[k] = h[x + k];
                rv[k] = rk[x + k];
                bv |= (uint32_t)bn[x + k] << (8 * k);
            }
        }
        c.g[q] = make_float4(gv[0], gv[1], gv[2], gv[3]);
        c.h[q] = make_float4(hv[0], hv[1], hv[2], hv[3]);
        c.r[q] = make_uint2(rv[0] | (rv[1] << 16), rv[2] | (rv[3] << 16));
        c.bw[q] = bv;
    }
}

// One window of a tile's entries, g and h in separate tables: a producer
// writes each value as it was loaded (pairing g with h for one 8-byte store
// would have the compiler permute the loaded registers right after the
// loads, which waits for them).  Cell (r, b) is at (r << lg) + b, where
// 2^lg >= 1 + the feature's largest bin: a window holds RW NB >> lg ranks, so
// a feature of few bins (long runs per tile) takes a tile in one window.
struct RankTable {
    float g[RW * NB];
    float h[RW * NB];
};

// A producer's window [w0, w0 + rw) of its tile's entries into T[rank - w0][bin]
// (rw = RW NB >> lg; a bin past 2^lg, which the rank table rules out, is
// dropped rather than written into another rank's cells).
__device__ __forceinline__ void rank_stage(const RankTile& c, RankTable& T, uint32_t w0, uint32_t rw, int lg) {
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
        // a rank below w0 wraps above rw; past the rows the rank is 0xffff
        const uint32_t rank = rt_rank(c, j), r = rank - w0;
        const uint32_t b = rt_bin(c, j);
        if (rank != 0xffffu && r < rw && (b >> lg) == 0) {
            T.g[(r << lg) + b] = rt_g(c, j);
            T.h[(r << lg) + b] = rt_h(c, j);
        }
    }
}

// Block f: the root's fp32 cells of feature f, cgrow's row-order chains
// (grow.c:37-62); the count cell is cgrow's chain of 1.0f adds,
// min(count, 2^24).  Threads 0 .. RB - 1 are the consumers, thread b adding
// bin b's run of each tile in rank order from an LDS table T[rank][bin]
// (2^lg bins a rank, lg from the largest bin of the feature's tiles);
// threads RB .. RB + RPROD - 1 are the producers, filling the other of two
// tables with the next tile meanwhile (window 0 of every tile; a tile whose
// longest run passes the window has its further windows staged and added in turn,
// its positions reloaded).  The producers' next tiles load RING tiles ahead:
// a step is shorter than a load's latency under load.  VEC:
// g, h and the bins are 16-byte aligned (every feature's column:
// ld_fm % 16 == 0).
template <bool VEC>
__global__ void __launch_bounds__(RB + RPROD) k_rank_chain(const float* __restrict__ g, const float* __restrict__ h,
                                                       const uint8_t* __restrict__ bins_fm, int64_t ld_fm, int64_t n,
                                                       RootOrder o, float* __restrict__ hist, int F) {
    __shared__ RankTable T[2];
    __shared__ uint32_t s_mb;
    const int f = blockIdx.x;
    const bool prod = threadIdx.x >= RB;
    const int lt = prod ? (int)threadIdx.x - RB : (int)threadIdx.x;   // consumers: the bin; producers: the slot
    const uint8_t* bn = bins_fm + (size_t)f * (size_t)ld_fm;
    const uint16_t* rk = o.rank + (size_t)f * (size_t)o.ld_rank;
    const uint16_t* sf = o.starts + (size_t)f * (size_t)o.tiles * ST;
    const uint16_t* mx = o.maxrun + (size_t)f * (size_t)o.tiles;
    const int64_t tiles = (n + WT - 1) / WT;
    const int64_t full = VEC ? n / WT : 0;      // tiles the producers load with 16-byte loads
    {
        if (threadIdx.x == 0) s_mb = 0;
        __syncthreads();
        uint32_t m = 0;
        const uint8_t* mb = o.maxbin + (size_t)f * (size_t)o.tiles;
        for (int64_t t = threadIdx.x; t < tiles; t += blockDim.x) m = max(m, (uint32_t)mb[t]);
        atomicMax(&s_mb, m);
        __syncthreads();
    }
    const int lg = 32 - __builtin_clz(__builtin_amdgcn_readfirstlane((int)s_mb) | 1);   // 2^lg > the largest bin
    const uint32_t rw = (uint32_t)(RW * NB) >> lg;                                     // ranks per window
    // consumers: at 256 bins (both) thread lt runs both chains of bin lt;
    // below, thread lt runs the one chain of channel cch = lt >> lg (0: g,
    // 1: h) of bin cb = lt mod 2^lg, and threads from 2^(lg + 1) on idle
    const bool both = lg == 8;
    const int cb = both ? lt : (lt & ((1 << lg) - 1));
    const int cch = both ? 0 : (lt >> lg);
    const bool live = prod || cch < 2;
    float ag = 0.0f, ah = 0.0f;   // both: g and h; else: channel cch in ag
    int64_t cnt = 0;
    // consumer: window [w0, w0 + rw) of tile t's run of its bin from table Tb;
    // steps to the tile's longest run in the window (uniform); past this
    // thread's run a step adds +0.0f, which leaves the sums' bits unchanged (a
    // sum that starts at +0.0f is never -0.0f).  Both chains: eight ranks'
    // reads in flight, then their adds.
    auto run2 = [&](const RankTable& Tb, uint32_t len, uint32_t mr, uint32_t w0) {
        const uint32_t kend = min(len > w0 ? len - w0 : 0u, rw);
        const uint32_t kmax = min(mr - w0, rw);
        for (uint32_t r = 0; r < kmax; r += 8) {
            float vg[8], vh[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                vg[u] = Tb.g[((r + u) << 8) + lt];
                vh[u] = Tb.h[((r + u) << 8) + lt];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const bool in = r + u < kend;
                ag += in ? vg[u] : 0.0f;
                ah += in ? vh[u] : 0.0f;
            }
        }
    };
    // One chain (tb: the channel's table at the bin's column), sixteen ranks a
    // turn in two register sets: each set's next reads are issued before the
    // other set's adds (the accumulator passes through the asm after the
    // reads, so the adds cannot move above them); groups past the window
    // read a clamped group in it, unused.
    auto run1 = [&](const float* tb, uint32_t len, uint32_t mr, uint32_t w0) {
        const uint32_t kend = min(len > w0 ? len - w0 : 0u, rw);
        const uint32_t kmax = min(mr - w0, rw);
        if (kmax == 0) return;
        float a[8], b[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) a[u] = tb[u << lg];
        for (uint32_t r = 0; r < kmax; r += 16) {
            const uint32_t rb = min(r + 8, rw - 8), ra = min(r + 16, rw - 8);
#pragma unroll
            for (int u = 0; u < 8; ++u) b[u] = tb[(rb + u) << lg];
            asm volatile("" : "+v"(ag) : : "memory");
#pragma unroll
            for (int u = 0; u < 8; ++u) ag += r + u < kend ? a[u] : 0.0f;
#pragma unroll
            for (int u = 0; u < 8; ++u) a[u] = tb[(ra + u) << lg];
            asm volatile("" : "+v"(ag) : : "memory");
#pragma unroll
            for (int u = 0; u < 8; ++u) ag += r + 8 + u < kend ? b[u] : 0.0f;
        }
    };
    auto run = [&](const RankTable& Tb, uint32_t len, uint32_t mr, uint32_t w0) {
        if (both)
            run2(Tb, len, mr, w0);
        else
            run1((cch ? Tb.h : Tb.g) + cb, len, mr, w0);
    };
    auto load = [&](RankTile& c, int64_t t) {
        if (t < full)
            rank_tile_load_vec(c, g, h, bn, rk, t, lt);
        else
            rank_tile_load_any(c, g, h, bn, rk, t, n, lt);
    };
    // every thread: tile t's longest run, RING tiles ahead in mrs[t % RING];
    // consumers: their bin's run start and end in the tile, in se[t % RING]
    // (a load used in the step it is issued would put a memory latency on
    // every tile's path)
    uint32_t mrs[RING], se[RING];
    const uint16_t* sfl = sf + (prod ? 0 : cb);   // consumers' start entries: tile t at sfl[t ST], its end at sfl[t ST + 1]
    auto meta = [&](int k, int64_t t) {
        if (t < tiles) {
            mrs[k] = mx[t];
            if (!prod) se[k] = (uint32_t)sfl[(size_t)t * ST] | ((uint32_t)sfl[(size_t)t * ST + 1] << 16);
        }
    };
#pragma unroll
    for (int k = 0; k < RING; ++k) meta(k, k);
    // producers: tile 0's window 0, and the ring (tiles 1 .. RING)
    RankTile ring[RING];
    if (prod && tiles > 0) {
        RankTile c;
        load(c, 0);
        rank_stage(c, T[0], 0, rw, lg);
    }
    if (prod && full > 0) {
#pragma unroll
        for (int k = 0; k < RING; ++k) rank_tile_load_vec(ring[k], g, h, bn, rk, min((int64_t)(1 + k), full - 1), lt);
    }
    __syncthreads();
    // step t: the consumers add tile t's window 0 from T[t & 1] while the
    // producers stage tile t + 1's from ring slot R (then reload R with tile
    // t + 1 + RING); then tile t's further windows, if any
    auto step = [&](int64_t t, RankTile& R, int k) {
        if (t >= tiles) return;
        const uint32_t mr = (uint32_t)__builtin_amdgcn_readfirstlane((int)mrs[k]);
        uint32_t len = 0;
        if (!prod) len = (se[k] >> 16) - (se[k] & 0xffffu);
        meta(k, t + RING);
        if (!prod) {
            if (live) run(T[t & 1], len, mr, 0);
            cnt += len;
        } else if (t + 1 < tiles) {
            if (t + 1 < full) {
                rank_stage(R, T[(t + 1) & 1], 0, rw, lg);
            } else {
                RankTile c;
                rank_tile_load_any(c, g, h, bn, rk, t + 1, n, lt);
                rank_stage(c, T[(t + 1) & 1], 0, rw, lg);
            }
        }
        if (prod && full > 0) rank_tile_load_vec(R, g, h, bn, rk, min(t + 1 + RING, full - 1), lt);
        __syncthreads();
        for (uint32_t w0 = rw; w0 < mr; w0 += rw) {
            if (prod) {
                RankTile c;
                load(c, t);
                rank_stage(c, T[t & 1], w0, rw, lg);
            }
            __syncthreads();
            if (!prod && live) run(T[t & 1], len, mr, w0);
            __syncthreads();
        }
    };
    for (int64_t t = 0; t < tiles; t += RING) {
#pragma unroll
        for (int k = 0; k < RING; ++k) step(t + k, ring[k], k);
    }
    // below 256 bins the chains' sums meet in LDS (T[0], free after the last
    // step's barrier): s_o[ch NB + bin], the counts at T[0].h; bins from 2^lg
    // on are empty
    float* s_o = T[0].g;
    __syncthreads();
    if (!both && !prod && cch < 2) s_o[cch * NB + cb] = ag;
    if (!both && !prod && cch == 0) T[0].h[cb] = (float)min(cnt, (int64_t)1 << 24);
    __syncthreads();
    if (!prod) {
        float vg = ag, vh = ah, vc = (float)min(cnt, (int64_t)1 << 24);
        if (!both) {
            const bool in = (lt >> lg) == 0;
            vg = in ? s_o[lt] : 0.0f;
            vh = in ? s_o[NB + lt] : 0.0f;
            vc = in ? T[0].h[lt] : 0.0f;
        }
        hist[(size_t)f * NB + lt] = vg;
        hist[(size_t)F * NB + (size_t)f * NB + lt] = vh;
        hist[(size_t)2 * F * NB + (size_t)f * NB + lt] = vc;
    }
}

inline void launch_rank_chain(const float* g, const float* h, const uint8_t* bins_fm, int64_t ld_fm, int64_t n,
                              const RootOrder& o, float* hist, int F, hipStream_t stream) {
    const bool vec = ((uintptr_t)g % 16 == 0) && ((uintptr_t)h % 16 == 0) && ((uintptr_t)bins_fm % 16 == 0) &&
                     (ld_fm % 16 == 0);
    if (vec)
        k_rank_chain<true><<<F, RB + RPROD, 0, stream>>>(g, h, bins_fm, ld_fm, n, o, hist, F);
    else
        k_rank_chain<false><<<F, RB + RPROD, 0, stream>>>(g, h, bins_fm, ld_fm, n, o, hist, F);
}

// Sparse builder's default-bin cells (grow.c:101-106): 0 + (float)(node sum -
// explicit sum) for g and h, 0 + (float)(rows in the default bin) for the count.
// Block (., k): job k's built child.
__global__ void __launch_bounds__(RB) k_hist_default(const int32_t* __restrict__ dbin,
                                                     const double* __restrict__ eout_b,
                                                     const double* __restrict__ tot_b, int F,
                                                     float* __restrict__ hist_base, size_t hsz,
                                                     const Round* __restrict__ R) {
    const int f = blockIdx.x * RB + threadIdx.x;
    if (f >= F) return;
    const Job& J = R->job[blockIdx.y];
    const double* eout = eout_b + (size_t)blockIdx.y * 3 * F;
    const double* tot = tot_b + (size_t)blockIdx.y * 2;
    const int slot = J.build_left ? J.slot_l : J.slot_r;
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

// One child's feature-major first maximum (grow.c:183-192) and node value
// from feature 0's 256 bins summed in double (grow.c:302-308, 371-379),
// written to the round's record for the host.  One wave; child y of the
// round is child y % nc of job y / nc (nc = 1 at the root, else 2).
__device__ void ref_pick(const float* __restrict__ hist, size_t hsz, const Round* __restrict__ R, int y, int nc,
                         int F, const double* __restrict__ fsel, const double* __restrict__ fgain,
                         const int32_t* __restrict__ fb, float lr, double lam, Res* res, float* s_g, float* s_h) {
    const int kj = y / nc, c = y % nc;
    const Job& J = R->job[kj];
    const int node = c == 0 ? J.slot_l : J.slot_r;
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
    // lanes take features in increasing order with grow.c's strict >, then
    // the largest sel, lowest f wins
    double best_sel = -INFINITY, best_true = -INFINITY;
    int bf = -1, bb = -1;
    for (int f = lane; f < F; f += WAVE) {
        const int b = fb[(size_t)y * F + f];
        const double s = fsel[(size_t)y * F + f];
        if (b >= 0 && s > best_sel) {
            best_sel = s;
            best_true = fgain[(size_t)y * F + f];
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
        const float v = (float)(-lr * G / (H + lam));
        // res is host memory mapped for the device: the record's fields, a
        // system-scope fence, then the round number the host waits for
        volatile ChildRes& r = res[kj].c[c];
        r.gain = bf < 0 ? -INFINITY : best_true;
        r.f = bf;
        r.b = bb;
        r.value = v;
        if (c == 0) {
            volatile Res* rk = res + kj;
            rk->mid = J.s + J.nl;
            rk->build_left = J.build_left;
        }
        __threadfence_system();
        r.seq = R->seq;
    }
    __syncthreads();
}

// One wave per (feature, child): the split scan (grow.c:129-197); child y of
// the round is child y % nc of job y / nc (nc = 1 at the root, else 2).  At
// a split the subtracted child's block first forms its feature's bins as
// parent - built child in fp32 (grow.c:361,368) and stores them.
__global__ void __launch_bounds__(WAVE) k_scan_feature(float* __restrict__ hist, size_t hsz,
                                                       const Round* __restrict__ R, int nc,
                                                       const uint8_t* __restrict__ path, ScanParams P,
                                                       double* __restrict__ fsel, double* __restrict__ fgain,
                                                       int32_t* __restrict__ fb) {
    __shared__ float s_in[3][NB];
    __shared__ double s_gl[NB], s_hl[NB], s_cl[NB];
    const int f = blockIdx.x, y = blockIdx.y, lane = threadIdx.x;
    const Job& J = R->job[y / nc];
    const int c = y % nc;
    const int node = c == 0 ? J.slot_l : J.slot_r;
    const int parent = J.slot_p;
    const int F = P.F;
    double best_sel = -INFINITY, best_true = -INFINITY;
    int best_b = -1;
    const bool sub = parent >= 0 && c == (J.build_left ? 1 : 0);
    if (sub) {
        const int built = J.build_left ? J.slot_l : J.slot_r;
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
        fsel[(size_t)y * F + f] = best_sel;
        fgain[(size_t)y * F + f] = best_true;
        fb[(size_t)y * F + f] = best_b;
    }
}

// One wave per child of the round: ref_pick after every scan block is done.
__global__ void __launch_bounds__(WAVE) k_scan_pick(const float* __restrict__ hist, size_t hsz,
                                                    const Round* __restrict__ R, int nc, int F,
                                                    const double* __restrict__ fsel,
                                                    const double* __restrict__ fgain, const int32_t* __restrict__ fb,
                                                    float lr, double lam, Res* res) {
    __shared__ float s_g[NB], s_h[NB];
    ref_pick(hist, hsz, R, blockIdx.x, nc, F, fsel, fgain, fb, lr, lam, res, s_g, s_h);
}

// Per-row leaf ids and cgrow's final rows[] from the final leaves' segments:
// leaf k is node seg[4k] with rows [seg[4k+1], seg[4k+2]) of row array
// seg[4k+3].  Either output may be null.
__global__ void __launch_bounds__(RB) k_leaf_rows(const uint32_t* __restrict__ rows, int64_t rows_ld,
                                                  const int64_t* __restrict__ seg, int n_leaf,
                                                  int64_t* __restrict__ out_leaf, int64_t* __restrict__ out_rows) {
    const int k = blockIdx.y;
    if (k >= n_leaf) return;
    const int64_t node = seg[4 * k], s = seg[4 * k + 1], e = seg[4 * k + 2];
    const uint32_t* r = rows + (size_t)seg[4 * k + 3] * (size_t)rows_ld;
    for (int64_t i = s + (int64_t)blockIdx.x * RB + threadIdx.x; i < e; i += (int64_t)gridDim.x * RB) {
        const uint32_t row = r[i];
        if (out_leaf) out_leaf[row] = node;
        if (out_rows) out_rows[i] = row;
    }
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

    // Histograms of the round's K built children (the root: every row), in
    // `tiles` sort tiles; G, H: their g, h by position.  With default bins,
    // the sparse builder's arithmetic (grow.c:68-107).
    void hist(bool root, int K, int64_t tiles, const float* G, const float* H) {
        const unsigned ty = (unsigned)min((int64_t)65535, max((int64_t)1, tiles));
        for (int fg0 = 0; fg0 < F; fg0 += w.fgroup) {
            const int nf = min(w.fgroup, F - fg0);
            const dim3 sgrid((unsigned)nf, ty);
#define YABT_SORT(ROOT, SPARSE)                                                                             \
    k_walk_sort<ROOT, SPARSE><<<sgrid, RB, 0, st>>>(bins_fm, ld_fm, bins_rm, ld_rm, w.rows, w.rows_ld, w.round, \
                                                    fg0, dbin, w.perm, w.xperm, w.ld_perm, w.starts, w.n_tiles)
            if (root) {
                if (dbin) YABT_SORT(true, true); else YABT_SORT(true, false);
            } else {
                if (dbin) YABT_SORT(false, true); else YABT_SORT(false, false);
            }
#undef YABT_SORT
            // the sparse builder's node totals: one more block with the first group
            const dim3 cgrid((unsigned)nf + (dbin && fg0 == 0 ? 1u : 0u), (unsigned)K);
            if (dbin)
                k_walk_chain<true><<<cgrid, RB, 0, st>>>(G, H, w.round, F, fg0, nf, dbin, w.perm, w.xperm, w.ld_perm,
                                                         w.starts, w.n_tiles, w.hist, hsz, w.expl, w.tot);
            else
                k_walk_chain_dense<<<cgrid, CB, 0, st>>>(G, H, w.round, F, fg0, w.perm, w.ld_perm, w.starts,
                                                         w.n_tiles, w.hist, hsz);
        }
        if (dbin)
            k_hist_default<<<dim3((F + RB - 1) / RB, (unsigned)K), RB, 0, st>>>(dbin, w.expl, w.tot, F, w.hist, hsz,
                                                                              w.round);
    }
};

// A computed split, on the host.  Leaves name their origin as 2 p + c (child
// c of split p) or -1 (the root).
struct HSplit {
    int origin;
    int f, b, depth;               // the split; depth of its children
    int slot_p;
    int64_t s, e, mid;
    int child_pend[2];             // the children's computed splits (-1: none)
    int child_node[2];             // the children's node ids once committed (-1: not committed)
    float cgain[2];                // the children's table gains (depth cap applied)
    int cf[2], cb[2];              // the children's best splits
    float cval[2];                 // the children's values
};

// A leaf as a split candidate.
struct LeafView {
    int f, b, depth, slot, arr;
    int64_t s, e;
};

}  // namespace ref
}  // namespace yabt

using namespace yabt;
using namespace yabt::ref;

extern "C" {

size_t yabt_ref_root_order_bytes(int64_t n, int F) {
    if (n < 0 || n > 0xFFFFFFFFll || F < 1) return 0;
    return root_order_carve(nullptr, n, F, nullptr);
}

int yabt_ref_root_order(const uint8_t* bins_fm, int64_t ld_fm, int64_t n, int F, void* out, size_t out_bytes,
                        hipStream_t stream) {
    if (n < 0 || n > 0xFFFFFFFFll || F < 1) return fail(-2, "yabt_ref_root_order: bad sizes");
    if (!out || (n > 0 && (!bins_fm || ld_fm < n))) return fail(-2, "yabt_ref_root_order: bad pointer or layout");
    if (out_bytes < root_order_carve(nullptr, n, F, nullptr))
        return fail(-2, "yabt_ref_root_order: output buffer too small");
    if (n == 0) return 0;
    RootOrder o;
    root_order_carve((char*)out, n, F, &o);
    const unsigned ty = (unsigned)min((int64_t)65535, o.tiles);
    k_root_rank<<<dim3((unsigned)F, ty), RB, 0, stream>>>(bins_fm, ld_fm, n, o);
    return launch_status("yabt_ref_root_order launch");
}

int yabt_ref_root_hist(const uint8_t* bins_fm, int64_t ld_fm, const float* grad, const float* hess, int64_t n, int F,
                       const void* root_order, size_t root_order_bytes, float* out, hipStream_t stream) {
    if (n < 0 || n > 0xFFFFFFFFll || F < 1) return fail(-2, "yabt_ref_root_hist: bad sizes");
    if (!out || !root_order || (n > 0 && (!bins_fm || !grad || !hess || ld_fm < n)))
        return fail(-2, "yabt_ref_root_hist: bad pointer or layout");
    if (root_order_bytes < root_order_carve(nullptr, n, F, nullptr))
        return fail(-2, "yabt_ref_root_hist: root_order smaller than yabt_ref_root_order_bytes(n, F)");
    RootOrder o;
    root_order_carve((char*)const_cast<void*>(root_order), n, F, &o);
    launch_rank_chain(grad, hess, bins_fm, ld_fm, n, o, out, F, stream);
    return launch_status("yabt_ref_root_hist launch");
}

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
                  size_t workspace_bytes, const void* root_order, int64_t* out_feature,
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
    const int L = max_leaves;

    // host staging of a round, and the round's records in mapped host memory,
    // both from the library's pinned pool; every return waits for the stream
    // before they go back: enqueued picks write h_res and enqueued copies read
    // h_round until they have run
    struct Held {
        PinnedHold round, res;
        hipStream_t s;
        ~Held() {
            if (round.p || res.p) (void)hipStreamSynchronize(s);
        }
    } held;
    held.s = stream;
    if (int prc = held.round.take(sizeof(Round), hipHostMallocDefault)) return prc;
    if (int prc = held.res.take(KR * sizeof(Res), hipHostMallocMapped | hipHostMallocCoherent)) return prc;
    Round* h_round = static_cast<Round*>(held.round.p);
    Res* h_res = static_cast<Res*>(held.res.p);
    hipError_t he = hipSuccess;
    Res* d_res = nullptr;   // the device's address of h_res
    he = hipHostGetDevicePointer((void**)&d_res, h_res, 0);
    if (he != hipSuccess) return hip_fail(he, "yabt_grow_ref: mapped result buffer");
    for (int k = 0; k < KR; ++k) h_res[k].c[0].seq = h_res[k].c[1].seq = -1;

    k_init<<<launch_grid(n > F ? n : F, RB, 1024), RB, 0, stream>>>(w.rows, n, w.path, F);

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

    // The picks write each child's record into h_res and stamp it with the
    // round number last; the host spins on the stamps (checking the stream
    // for errors, and for completion without a stamp) instead of a copy and
    // a stream synchronisation.
    auto sync_res = [&](int32_t seq, int jobs, int children) -> int {
        volatile Res* R = h_res;
        auto all = [&]() {
            for (int k = 0; k < jobs; ++k)
                for (int c = 0; c < children; ++c)
                    if (R[k].c[c].seq != seq) return false;
            return true;
        };
        for (SpinWait sw;;) {
            if (all()) {
                std::atomic_thread_fence(std::memory_order_acquire);
                return 0;
            }
            if (sw.stream_check()) {
                const hipError_t e = hipStreamQuery(stream);
                if (e == hipSuccess) {
                    if (all()) return 0;
                    return fail(-4, "yabt_grow_ref: stream finished without the round's results");
                }
                if (e != hipErrorNotReady) return hip_fail(e, "yabt_grow_ref: round");
            }
        }
    };
    auto launch_round = [&]() -> int {
        const hipError_t e = hipMemcpyAsync(w.round, h_round, sizeof(Round), hipMemcpyHostToDevice, stream);
        return e == hipSuccess ? 0 : hip_fail(e, "yabt_grow_ref: round copy");
    };

    // the root: one pseudo-job whose built child is every row
    int rc = 0;
    {
        Round& R = *h_round;
        memset(&R, 0, sizeof R);
        R.K = 1;
        R.seq = 0;
        R.toff[1] = (int32_t)max((int64_t)1, (n + WT - 1) / WT);
        Job& J = R.job[0];
        J.f = -1;
        J.slot_p = -1;
        J.slot_l = 0;
        J.slot_r = 0;
        J.build_left = 1;
        J.s = 0;
        J.e = n;
        J.nl = n;
        J.cs = 0;
        J.ce = n;
        if ((rc = launch_round())) return rc;
        if (root_order && !sparse && n > 0) {
            RootOrder o;
            root_order_carve((char*)const_cast<void*>(root_order), n, F, &o);
            launch_rank_chain(grad, hess, bins_fm, ld_fm, n, o, w.hist, F, stream);
        } else {
            g.hist(true, 1, R.toff[1], grad, hess);
        }
        k_scan_feature<<<dim3(F, 1), WAVE, 0, stream>>>(w.hist, g.hsz, w.round, 1, w.path, P, w.fsel, w.fgain, w.fb);
        k_scan_pick<<<1, WAVE, 0, stream>>>(w.hist, g.hsz, w.round, 1, F, w.fsel, w.fgain, w.fb, lr, (double)lam,
                                             d_res);
        if ((rc = launch_status("yabt_grow_ref launch"))) return rc;
        if ((rc = sync_res(0, 1, 1))) return rc;
    }
    const double root_gain = h_res[0].c[0].gain;
    const int root_f = h_res[0].c[0].f, root_b = h_res[0].c[0].b;

    // node arrays (cgrow's outputs), written on the host as splits commit
    std::vector<int64_t> o_feature(N, LEAF), o_thr(N, 0), o_left(N, -1), o_right(N, -1), o_depth(N, 0);
    std::vector<float> o_value(N, 0.0f);
    o_value[0] = h_res[0].c[0].value;

    std::vector<HSplit> sp;
    sp.reserve((size_t)w.pend_cap);
    auto view = [&](int src) -> LeafView {
        LeafView v;
        if (src < 0) {
            v.f = root_f;
            v.b = root_b;
            v.depth = 0;
            v.slot = 0;
            v.s = 0;
            v.e = n;
        } else {
            const HSplit& q = sp[(size_t)(src >> 1)];
            const int c = src & 1;
            v.f = q.cf[c];
            v.b = q.cb[c];
            v.depth = q.depth;
            v.slot = 1 + 2 * (src >> 1) + c;
            v.s = c ? q.mid : q.s;
            v.e = c ? q.e : q.mid;
        }
        v.arr = v.depth % RA;
        return v;
    };
    // cgrow's leaf table (grow.c:284-287): gain, computed split, origin, node id
    std::vector<float> t_gain(N, 0.0f);
    std::vector<int> t_pend(N, -1), t_src(N, -1), t_node(N, -1);
    t_gain[0] = (float)(0 >= max_depth ? -INFINITY : root_gain);
    t_src[0] = -1;
    t_node[0] = 0;
    int na = 1, nn = 1;
    // the first maximum of the fp32 gains above 0.0f (grow.c:322-330)
    auto argmax = [](const std::vector<float>& gain, int cnt) {
        int best = -1;
        float bg = 0.0f;
        for (int a = 0; a < cnt; ++a)
            if (gain[a] > bg) {
                bg = gain[a];
                best = a;
            }
        return best;
    };
    std::vector<float> p_gain(N);
    std::vector<int> p_pend(N), p_src(N), p_level(N);
    std::vector<char> p_moved(N);

    for (int32_t seq = 1;; ++seq) {
        // replay: commit the best leaf while its split is computed
        int best = -1;
        while (na < L) {
            best = argmax(t_gain, na);
            if (best < 0 || t_pend[best] < 0) break;
            const int p = t_pend[best];
            HSplit& q = sp[(size_t)p];
            const int nid = t_node[best], nl = nn, nr = nn + 1;
            // the split's node record (grow.c:338-350, 371-386)
            o_feature[nid] = q.f;
            o_thr[nid] = q.b;
            o_left[nid] = nl;
            o_right[nid] = nr;
            o_value[nid] = 0.0f;
            o_depth[nl] = o_depth[nr] = q.depth;
            o_value[nl] = q.cval[0];
            o_value[nr] = q.cval[1];
            q.child_node[0] = nl;
            q.child_node[1] = nr;
            // left child replaces the split leaf, right child is appended
            // (grow.c:393-407)
            t_gain[best] = q.cgain[0];
            t_pend[best] = q.child_pend[0];
            t_src[best] = 2 * p;
            t_node[best] = nl;
            t_gain[na] = q.cgain[1];
            t_pend[na] = q.child_pend[1];
            t_src[na] = 2 * p + 1;
            t_node[na] = nr;
            nn += 2;
            ++na;
            best = -1;
        }
        if (best < 0) break;   // no leaf with a positive gain, or the budget is spent
        // plan: the table run ahead -- a leaf whose split is computed gives
        // way to its children, a leaf without one is taken for the round.
        // Only leaves at most one computed split below a committed leaf are
        // taken (level <= RA - 2): a split at depth d writes row array
        // (d + 1) % RA, so one level more would overwrite the rows of a
        // committed leaf that may stay a leaf.
        for (int a = 0; a < na; ++a) {
            p_gain[a] = t_gain[a];
            p_pend[a] = t_pend[a];
            p_src[a] = t_src[a];
            p_level[a] = 0;
            p_moved[a] = 0;
        }
        Round& R = *h_round;
        memset(&R, 0, sizeof R);
        R.seq = seq;
        int j = 0, nas = na, nls = na;
        const int np0 = (int)sp.size();
        while (nls + j < L && j < KR) {
            const int a = argmax(p_gain, nas);
            if (a < 0) break;
            const int p = p_pend[a];
            if (p >= 0) {
                const HSplit& q = sp[(size_t)p];
                const int lv = p_level[a] + 1;
                p_gain[a] = q.cgain[0];
                p_pend[a] = q.child_pend[0];
                p_src[a] = 2 * p;
                p_level[a] = lv;
                p_moved[a] = 1;
                p_gain[nas] = q.cgain[1];
                p_pend[nas] = q.child_pend[1];
                p_src[nas] = 2 * p + 1;
                p_level[nas] = lv;
                p_moved[nas] = 1;
                ++nas;
                ++nls;
                continue;
            }
            if (p_level[a] > RA - 2) {
                p_gain[a] = -INFINITY;   // not taken; the simulation goes on below it
                continue;
            }
            // computed splits: every round may need one for the leaf it is
            // blocked on, at most L - na more; extras keep np + L - na <=
            // pend_cap - 1 (so the first of a round always fits)
            const int np = (int)sp.size();
            if (np >= w.pend_cap) return fail(-5, "yabt_grow_ref: computed splits exceed the workspace");
            if (j > 0 && np + L - na > w.pend_cap - 1) break;
            const LeafView v = view(p_src[a]);
            HSplit q;
            q.origin = p_src[a];
            q.f = v.f;
            q.b = v.b;
            q.depth = v.depth + 1;
            q.slot_p = v.slot;
            q.s = v.s;
            q.e = v.e;
            q.mid = v.s;
            q.child_pend[0] = q.child_pend[1] = -1;
            q.child_node[0] = q.child_node[1] = -1;
            sp.push_back(q);
            if (q.origin >= 0) sp[(size_t)(q.origin >> 1)].child_pend[q.origin & 1] = np;
            if (!p_moved[a]) t_pend[a] = np;    // a committed leaf's entry
            p_gain[a] = -INFINITY;
            Job& J = R.job[j];
            J.f = v.f;
            J.b = v.b;
            J.src = v.arr;
            J.dst = (v.depth + 1) % RA;
            J.slot_p = v.slot;
            J.slot_l = 1 + 2 * np;
            J.slot_r = 2 + 2 * np;
            J.s = v.s;
            J.e = v.e;
            const int64_t m = v.e - v.s;
            R.boff[j + 1] = R.boff[j] + (int32_t)max((int64_t)1, (m + PT - 1) / PT);
            R.toff[j + 1] = R.toff[j] + (int32_t)max((int64_t)1, (m / 2 + WT - 1) / WT);
            ++j;
        }
        if (j == 0) break;
        R.K = j;
        // partition (the job table goes in with its first kernel),
        // histograms of the built children, both children's scans
        const int nblk = R.boff[j];
        k_part_flags<<<nblk, RB, 0, stream>>>(bins_fm, ld_fm, R, w.round, w.rows, w.rows_ld, w.flag, w.blk);
        k_part_offsets<<<j, RB, 0, stream>>>(w.blk, w.round);
        k_part_rank<<<nblk, RB, 0, stream>>>(w.flag, w.blk, w.round, w.rank, w.p, w.q);
        k_part_permute<<<nblk, RB, 0, stream>>>(w.flag, w.rank, w.p, w.q, w.round, w.rows, w.rows_ld, grad, hess,
                                                 w.G, w.H, w.path, F);
        g.hist(false, j, R.toff[j], w.G, w.H);
        k_scan_feature<<<dim3(F, 2 * j), WAVE, 0, stream>>>(w.hist, g.hsz, w.round, 2, w.path, P, w.fsel, w.fgain,
                                                             w.fb);
        k_scan_pick<<<2 * j, WAVE, 0, stream>>>(w.hist, g.hsz, w.round, 2, F, w.fsel, w.fgain, w.fb, lr,
                                                 (double)lam, d_res);
        if ((rc = launch_status("yabt_grow_ref launch"))) return rc;
        if ((rc = sync_res(seq, j, 2))) return rc;
        for (int k = 0; k < j; ++k) {
            HSplit& q = sp[(size_t)(np0 + k)];
            q.mid = h_res[k].mid;
            for (int c = 0; c < 2; ++c) {
                const ChildRes& r = h_res[k].c[c];
                q.cgain[c] = (float)(q.depth >= max_depth ? -INFINITY : r.gain);
                q.cf[c] = r.f;
                q.cb[c] = r.b;
                q.cval[c] = r.value;
            }
        }
    }

    // outputs: the node arrays, per-row leaf ids, cgrow's final rows[]
    const int32_t n_nodes = nn;
    hipError_t e = hipSuccess;
    auto put = [&](void* dst, const void* src, size_t bytes) {
        if (e == hipSuccess) e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream);
    };
    put(out_feature, o_feature.data(), (size_t)N * sizeof(int64_t));
    put(out_thr_bin, o_thr.data(), (size_t)N * sizeof(int64_t));
    put(out_left, o_left.data(), (size_t)N * sizeof(int64_t));
    put(out_right, o_right.data(), (size_t)N * sizeof(int64_t));
    put(out_value, o_value.data(), (size_t)N * sizeof(float));
    put(out_depth, o_depth.data(), (size_t)N * sizeof(int64_t));
    put(out_n_nodes, &n_nodes, sizeof(int32_t));
    std::vector<int64_t> segs;   // read by the copy below until the final synchronisation
    if ((out_leaf_of_row || out_rows) && n > 0) {
        for (int a = 0; a < na; ++a) {
            const LeafView v = view(t_src[a]);
            segs.push_back(t_node[a]);
            segs.push_back(v.s);
            segs.push_back(v.e);
            segs.push_back(v.arr);
        }
        const int n_leaf = (int)(segs.size() / 4);
        put(w.segs, segs.data(), segs.size() * sizeof(int64_t));
        if (e == hipSuccess)
            k_leaf_rows<<<dim3((unsigned)launch_grid(n, RB * 4, 256), (unsigned)n_leaf), RB, 0, stream>>>(
                w.rows, w.rows_ld, w.segs, n_leaf, out_leaf_of_row, out_rows);
    }
    if (e != hipSuccess) return hip_fail(e, "yabt_grow_ref: outputs");
    if ((rc = launch_status("yabt_grow_ref launch"))) return rc;
    e = hipStreamSynchronize(stream);
    return e == hipSuccess ? 0 : hip_fail(e, "yabt_grow_ref: final synchronisation");
}

}  // extern "C"
