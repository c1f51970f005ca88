// gfx950 best-first (leaf-wise) tree growth, one tree per call.
//
// Replaces yabt/_cgrow/grow.c `cgrow` (grow.c:243-427) as called by
// yabt/grow_c.py `grow_tree_c` (grow_c.py:336-452).  The host enqueues a fixed
// launch sequence; every launch reads what to do from device-resident records
// written by the previous launch, so no split needs a host round trip.
//
// Arithmetic (bit-identical to oracle/grow_oracle.c OR_MODE_FIXED):
//   * g and h are quantised once per call to int64 fixed point (quant_shift);
//     node histograms are exact integer sums, so the accumulation order, the
//     row order inside a node and sibling subtraction (grow.c:355-369) are
//     exact and the result is deterministic;
//   * the split scan evaluates grow.c's double-precision Newton gain on the
//     exact prefix sums with grow.c's tie-breaks (scan.h);
//   * leaf gains are stored in fp32 and the best leaf is the first maximum
//     above 0 (grow.c:322-330); node values come from the node totals, which
//     equal feature 0's 256 bins (grow.c:302-308, 371-379).
//
// Launch sequence of one tree (caller's stream):
//   k_quant_clear, k_setup   max|g|,|h| -> shifts; table init; clear slot 0
//   k_hist_root              streaming histogram of all rows (+ root totals)
//   k_scan<ROOT>             default-bin fill, scan, controller: first split
//   max_leaves - 1 times (each kernel returns at once once the tree is done):
//     k_split_partition      one pass: children's rows to the other row list,
//                            written through two atomic cursors (left, right)
//     k_hist_gather          histogram of the smaller child
//     k_scan<SPLIT>          fill, sibling = parent - child in place, scan
//                            both children, controller picks the next split
//
// The left child's size is known exactly before partitioning (the count prefix
// at the chosen bin), so the partition needs no counting pass and the smaller
// child (ties left, grow.c:355) is chosen when the split is chosen.
//
// HBM layout:
//   bins_fm (F, ld_fm) u8     feature-major: root stream, partitions
//   bins_rm (n, ld_rm) u8     row-major copy: gathered child histograms
//   rows0/rows1 (n) u32       a node at depth d >= 1 keeps its rows at
//                             [seg_lo, seg_hi) of rows[d & 1]; the root is
//                             the identity and is never stored
//   hist (L, 3, F, 256) i64   one slot per live leaf: the built child takes a
//                             new slot, the sibling overwrites its parent's

#include "common.h"
#include "hist.h"
#include "host.h"
#include "scan.h"
#include "yabt_hip.h"

#include <string.h>

namespace yabt {

constexpr int SB = 256;                        // threads per scan / partition / setup block
constexpr int PART_IPT = 16;                   // rows per thread per partition tile
constexpr int PART_TILE = SB * PART_IPT;
constexpr int PART_MAX_BLOCKS = 1024;

// Best split of one live leaf (grow.c's leaf_node/leaf_gain/leaf_f/leaf_b
// table, grow.c:284-287, plus the node's exact totals).
struct LeafRec {
    float gain;                // (float) true gain, -inf if none (grow.c:316,394,404)
    int32_t node, f, b;
    int32_t depth, slot;       // node depth, histogram slot
    int64_t s, e;              // node segment in its row list
    int64_t tot[3];            // node totals: sum q(g), sum q(h), rows
    int64_t left[3];           // totals of bins <= b of feature f
};

struct SplitJob {
    int32_t k, nid, nl, nr;
    int32_t f, b;
    int32_t build_left;        // 1: the left child is built, the right is subtracted
    int32_t parent_slot, new_slot;
    int32_t depth;             // children's depth
    const uint32_t* src;       // parent's rows (nullptr: identity)
    uint32_t* dst;             // children's rows
    int64_t s, e, mid;
    int64_t tot[3];            // parent totals
    int64_t left[3];           // left-child totals
    int64_t* new_hist;         // the built child's slot (cleared by the previous scan launch)
    unsigned long long cursor[2];   // next write position, left / right
};

struct GrowState {
    int32_t n_nodes, n_leaves, n_active;
    int32_t done;
    int32_t status;
    uint32_t scan_ticket;
    int32_t active;            // a split job is pending
    int32_t pad;
    SplitJob job;
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
    const int32_t* dflt;
    int64_t n;
    int F;
    float lam, gamma, mcw, lr;
    int msl;
    int max_leaves, max_depth;
    GrowState* st;
    Quant* q;
    uint32_t* rows0;
    uint32_t* rows1;
    int64_t* hist;
    uint8_t* path;
    LeafRec* leaf;
    int64_t* seg_lo;
    int64_t* seg_hi;
    ScanRec* rec;
    int64_t* feature;
    int64_t* thr_bin;
    int64_t* left;
    int64_t* right;
    float* value;
    int64_t* depth;
    int32_t* out_status;
};

__device__ __forceinline__ size_t slot_elems(int F) { return (size_t)3 * (size_t)F * NB; }

__device__ __forceinline__ bool tree_done(const GrowState* st) { return *(volatile const int32_t*)&st->done != 0; }

// ---------------------------------------------------------------------------
// setup
// ---------------------------------------------------------------------------

__global__ void __launch_bounds__(SB) k_setup(GrowArgs A) {
    quant_reduce<SB>(A.grad, A.hess, A.n, A.q);
    const int N = 2 * A.max_leaves + 1;
    const int64_t tid = (int64_t)blockIdx.x * SB + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * SB;
    for (int64_t i = tid; i < N; i += stride) {
        A.feature[i] = LEAF;
        A.thr_bin[i] = 0;
        A.left[i] = -1;
        A.right[i] = -1;
        A.value[i] = 0.0f;
        A.depth[i] = 0;
        A.seg_lo[i] = 0;
        A.seg_hi[i] = 0;
    }
    for (int64_t i = tid; i < (int64_t)N * A.F; i += stride) A.path[i] = 0;
    const int64_t ne = (int64_t)slot_elems(A.F);
    for (int64_t i = tid; i < ne; i += stride) A.hist[i] = 0;
}

// One thread, after k_setup: shifts and tree state.
__global__ void k_setup_finish(GrowArgs A) {
    GrowState* st = A.st;
    quant_finish(A.q, A.n);
    st->status = 0;
    st->done = 0;
    st->active = 0;
    st->hist.active = 0;
    st->scan_ticket = 0;
    st->n_nodes = 1;
    st->n_leaves = 1;
    st->n_active = 1;
    if (A.q->nonfinite) {
        st->status = -1;
        st->done = 1;
        A.out_status[0] = -1;
    }
    A.seg_lo[0] = 0;
    A.seg_hi[0] = A.n;
}

// ---------------------------------------------------------------------------
// partition: one pass, two atomic write cursors
// ---------------------------------------------------------------------------

// Rows of [s, e) with bin <= b go to [s, mid), the others to [mid, e) of the
// children's row list.  Each block compacts a tile in order and reserves its
// output ranges with one atomic add per side, so rows stay grouped by tile;
// the order inside a child does not affect any result (sums are exact).
__global__ void __launch_bounds__(SB) k_split_partition(const uint8_t* __restrict__ bins_fm, int64_t ld,
                                                        GrowState* st) {
    if (tree_done(st) || !st->active) return;
    SplitJob& J = st->job;
    const int64_t s = J.s, e = J.e;
    const int fcol = J.f, b = J.b;
    const uint32_t* src = J.src;
    uint32_t* dst = J.dst;
    const int64_t m = e - s;
    const int64_t tiles = (m + PART_TILE - 1) / PART_TILE;
    const int nblk = (int)min((int64_t)gridDim.x, max(tiles, (int64_t)1));
    if ((int)blockIdx.x >= nblk) return;
    const int64_t tpb = (tiles + nblk - 1) / nblk;
    const int64_t lo = s + (int64_t)blockIdx.x * tpb * PART_TILE;
    const int64_t hi = min(e, lo + tpb * PART_TILE);
    const uint8_t* col = bins_fm + (size_t)fcol * ld;
    __shared__ uint32_t s_wave[SB / WAVE];
    __shared__ unsigned long long s_base[2];
    for (int64_t t0 = lo; t0 < hi; t0 += PART_TILE) {
        const int64_t a = t0 + (int64_t)threadIdx.x * PART_IPT;
        uint32_t rid[PART_IPT];
        uint32_t flags = 0, nv = 0;
#pragma unroll
        for (int j = 0; j < PART_IPT; ++j) {
            const int64_t i = a + j;
            if (i < hi) {
                rid[j] = src ? src[i] : (uint32_t)i;
                flags |= ((int)col[rid[j]] <= b ? 1u : 0u) << j;
                ++nv;
            }
        }
        const uint32_t nl = __popc(flags), nr = nv - nl;
        uint32_t tl, tr;
        const uint32_t ol = block_excl_scan<SB, uint32_t>(nl, s_wave, &tl);
        const uint32_t orr = block_excl_scan<SB, uint32_t>(nr, s_wave, &tr);
        if (threadIdx.x == 0) {
            s_base[0] = atomicAdd(&J.cursor[0], (unsigned long long)tl);
            s_base[1] = atomicAdd(&J.cursor[1], (unsigned long long)tr);
        }
        __syncthreads();
        uint64_t pl = s_base[0] + ol, pr = s_base[1] + orr;
#pragma unroll
        for (int j = 0; j < PART_IPT; ++j) {
            if ((uint32_t)j < nv) {
                if ((flags >> j) & 1u) dst[pl++] = rid[j];
                else dst[pr++] = rid[j];
            }
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// split scan + controller
// ---------------------------------------------------------------------------

__device__ __forceinline__ float node_value(const int64_t tot[3], const Quant* q, float lr, float lam) {
    const double G = (double)tot[0] * q->ig, H = (double)tot[1] * q->ih;
    return (float)(-lr * G / (H + lam));
}

__device__ __forceinline__ void leaf_from_record(LeafRec& L, const ScanRec* rec, int bf, bool capped) {
    if (bf >= 0) {
        const ScanRec& r = rec[bf];
        L.gain = (float)(capped ? -INFINITY : r.gain);
        L.f = bf;
        L.b = r.b;
        L.left[0] = r.left[0];
        L.left[1] = r.left[1];
        L.left[2] = r.left[2];
    } else {
        L.gain = -INFINITY;
        L.f = -1;
        L.b = -1;
        L.left[0] = L.left[1] = L.left[2] = 0;
    }
}

// Pick the next split (grow.c:321-350) and write its job, or finish the tree.
__device__ void select_next(const GrowArgs& A) {
    GrowState* st = A.st;
    __shared__ double s_key[SB / WAVE];
    __shared__ int s_idx[SB / WAVE];
    const int n_active = st->n_active, n_leaves = st->n_leaves;
    int k = -1;
    if (n_leaves < A.max_leaves) {
        double key = -INFINITY;
        int idx = INT_MAX;
        for (int a = threadIdx.x; a < n_active; a += SB) {
            const float g = A.leaf[a].gain;
            if (g > 0.0f && better((double)g, a, key, idx)) {
                key = (double)g;
                idx = a;
            }
        }
        block_argmax<SB>(key, idx, s_key, s_idx);
        k = idx == INT_MAX ? -1 : idx;
    }
    if (k < 0) {
        if (threadIdx.x == 0) {
            st->done = 1;
            st->active = 0;
            st->hist.active = 0;
            A.out_status[0] = st->n_nodes;
        }
        return;
    }
    const LeafRec L = A.leaf[k];
    const int nid = L.node, nl = st->n_nodes, nr = nl + 1;
    // children inherit the parent's path plus f (grow.c:347-350)
    const uint8_t* pp = A.path + (size_t)nid * A.F;
    for (int j = threadIdx.x; j < A.F; j += SB) {
        const uint8_t v = (j == L.f) ? (uint8_t)1 : pp[j];
        A.path[(size_t)nl * A.F + j] = v;
        A.path[(size_t)nr * A.F + j] = v;
    }
    if (threadIdx.x != 0) return;
    const int64_t d = L.depth, s = L.s, e = L.e;
    const int64_t cl = L.left[2], c = L.tot[2];
    const int bl = cl <= c - cl;
    const int new_slot = n_leaves;           // slots 0..n_leaves-1 are live
    A.depth[nl] = d + 1;
    A.depth[nr] = d + 1;
    A.feature[nid] = L.f;
    A.thr_bin[nid] = L.b;
    A.left[nid] = nl;
    A.right[nid] = nr;
    A.value[nid] = 0.0f;
    st->n_nodes = nl + 2;
    st->n_leaves = n_leaves + 1;
    SplitJob& J = st->job;
    J.k = k;
    J.nid = nid;
    J.nl = nl;
    J.nr = nr;
    J.f = L.f;
    J.b = L.b;
    J.build_left = bl;
    J.parent_slot = L.slot;
    J.new_slot = new_slot;
    J.depth = (int32_t)(d + 1);
    J.src = (d == 0) ? nullptr : ((d & 1) ? A.rows1 : A.rows0);
    J.dst = ((d + 1) & 1) ? A.rows1 : A.rows0;
    J.s = s;
    J.e = e;
    J.mid = s + cl;
    for (int i = 0; i < 3; ++i) {
        J.tot[i] = L.tot[i];
        J.left[i] = L.left[i];
    }
    J.new_hist = A.hist + (size_t)new_slot * slot_elems(A.F);
    J.cursor[0] = (unsigned long long)s;
    J.cursor[1] = (unsigned long long)(s + cl);
    HistJob& H = st->hist;
    H.rows = J.dst;
    H.lo = bl ? s : s + cl;
    H.hi = bl ? s + cl : e;
    H.out = J.new_hist;
    H.active = 1;
    st->active = 1;
}

template <bool ROOT>
__global__ void __launch_bounds__(SB) k_scan(GrowArgs A) {
    GrowState* st = A.st;
    if (tree_done(st)) return;
    const Quant* q = A.q;
    const bool derive = q->const_h != 0;     // no count channel: counts = h / hq_const
    const int64_t hqc = q->hq_const;
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    const int f = blockIdx.x * (SB / WAVE) + w;
    const ScanParams sp = {(double)A.lam, (double)A.gamma, (double)A.mcw, A.msl};
    {
        // the next split builds its child into slot n_leaves (select_next): clear it now
        const int next_slot = st->n_leaves;
        if (next_slot < A.max_leaves) {
            int64_t* z = A.hist + (size_t)next_slot * slot_elems(A.F);
            const int64_t ne = (int64_t)slot_elems(A.F);
            for (int64_t i = (int64_t)blockIdx.x * SB + threadIdx.x; i < ne; i += (int64_t)gridDim.x * SB) z[i] = 0;
        }
    }
    if (f < A.F) {
        const int nb = max(0, min(NB, A.nbins[f]));
        const bool use = A.fmask[f] != 0;
        const int d = A.dflt ? A.dflt[f] : -1;
        const size_t plane = (size_t)A.F * NB, at = (size_t)f * NB + 4 * lane;
        int64_t t256[3];
        if (ROOT) {
            const int64_t tot[3] = {q->tot_g, q->tot_h, A.n};
            int64_t g4[4], h4[4], c4[4];
            load_bins(A.hist, A.F, f, lane, g4, h4, c4);
            fill_default(g4, h4, c4, d, tot, !derive, lane);
            if (d >= 0 && (d >> 2) == lane) store_bins(A.hist, A.F, f, lane, g4, h4, c4);
            if (derive)
#pragma unroll
                for (int j = 0; j < 4; ++j) c4[j] = h4[j] / hqc;
            ScanRec r = scan_feature(g4, h4, c4, nb, q->ig, q->ih, sp, 1.0, lane, t256);
            if (!use) no_split(r);
            if (lane == 0) A.rec[f] = r;
        } else {
            const SplitJob& J = st->job;
            const int bl = J.build_left;
            int64_t* hp = A.hist + (size_t)J.parent_slot * slot_elems(A.F);
            int64_t* hn = A.hist + (size_t)J.new_slot * slot_elems(A.F);
            int64_t btot[3];
            for (int i = 0; i < 3; ++i) btot[i] = bl ? J.left[i] : J.tot[i] - J.left[i];
            int64_t bg[4], bh[4], bc[4], sg4[4], sh4[4], sc4[4];
            load_bins(hn, A.F, f, lane, bg, bh, bc);
            load_bins(hp, A.F, f, lane, sg4, sh4, sc4);
            fill_default(bg, bh, bc, d, btot, !derive, lane);
            if (d >= 0 && (d >> 2) == lane) store_bins(hn, A.F, f, lane, bg, bh, bc);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                sg4[j] -= bg[j];
                sh4[j] -= bh[j];
                sc4[j] -= bc[j];
                hp[at + j] = sg4[j];
                hp[plane + at + j] = sh4[j];
                hp[2 * plane + at + j] = sc4[j];
            }
            if (derive)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    bc[j] = bh[j] / hqc;
                    sc4[j] = sh4[j] / hqc;
                }
            const float bo = (A.use_imat && use) ? path_boost(A.path + (size_t)J.nl * A.F, A.imat, A.ib, A.F, f, lane)
                                                 : 1.0f;
            for (int c = 0; c < 2; ++c) {
                const bool built = (c == 0) == (bl != 0);
                ScanRec r = built ? scan_feature(bg, bh, bc, nb, q->ig, q->ih, sp, (double)bo, lane, t256)
                                  : scan_feature(sg4, sh4, sc4, nb, q->ig, q->ih, sp, (double)bo, lane, t256);
                if (!use) no_split(r);
                if (lane == 0) A.rec[(size_t)c * A.F + f] = r;
            }
        }
    }
    if (!last_block(&st->scan_ticket)) return;

    // ---- controller (one block) ----
    __shared__ int s_bf[2];
    for (int c = 0; c < (ROOT ? 1 : 2); ++c) {
        const int bf = reduce_records<SB>(A.rec + (size_t)c * A.F, A.F);
        if (threadIdx.x == 0) s_bf[c] = bf;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        if (ROOT) {
            LeafRec L;
            L.node = 0;
            L.depth = 0;
            L.slot = 0;
            L.s = 0;
            L.e = A.n;
            L.tot[0] = q->tot_g;
            L.tot[1] = q->tot_h;
            L.tot[2] = A.n;
            leaf_from_record(L, A.rec, s_bf[0], 0 >= A.max_depth);
            A.leaf[0] = L;
            A.value[0] = node_value(L.tot, q, A.lr, A.lam);
            st->n_nodes = 1;
            st->n_leaves = 1;
            st->n_active = 1;
        } else {
            const SplitJob& J = st->job;
            const bool capped = J.depth >= A.max_depth;
            LeafRec Ll, Lr;
            Ll.node = J.nl;
            Lr.node = J.nr;
            Ll.depth = Lr.depth = J.depth;
            Ll.s = J.s;
            Ll.e = J.mid;
            Lr.s = J.mid;
            Lr.e = J.e;
            Ll.slot = J.build_left ? J.new_slot : J.parent_slot;
            Lr.slot = J.build_left ? J.parent_slot : J.new_slot;
            for (int i = 0; i < 3; ++i) {
                Ll.tot[i] = J.left[i];
                Lr.tot[i] = J.tot[i] - J.left[i];
            }
            leaf_from_record(Ll, A.rec, s_bf[0], capped);
            leaf_from_record(Lr, A.rec + A.F, s_bf[1], capped);
            A.seg_lo[J.nl] = J.s;
            A.seg_hi[J.nl] = J.mid;
            A.seg_lo[J.nr] = J.mid;
            A.seg_hi[J.nr] = J.e;
            A.value[J.nl] = node_value(Ll.tot, q, A.lr, A.lam);
            A.value[J.nr] = node_value(Lr.tot, q, A.lr, A.lam);
            const int na = st->n_active;
            A.leaf[J.k] = Ll;            // left child replaces the split leaf
            A.leaf[na] = Lr;             // right child is appended (grow.c:393-407)
            st->n_active = na + 1;
            st->active = 0;
            st->hist.active = 0;
        }
    }
    __syncthreads();
    select_next(A);
}

// out[row] = leaf node id, from each leaf's segment of the final row lists.
// Grid (chunks, nodes).
__global__ void __launch_bounds__(SB) k_leaf_ids(const int64_t* feature, const int64_t* depth, const int64_t* seg_lo,
                                                 const int64_t* seg_hi, const uint32_t* rows0, const uint32_t* rows1,
                                                 const int32_t* out_status, int64_t* out) {
    const int nid = blockIdx.y;
    if (nid >= out_status[0] || feature[nid] != LEAF) return;
    const int64_t lo = seg_lo[nid], hi = seg_hi[nid], d = depth[nid];
    const uint32_t* rows = (d == 0) ? nullptr : ((d & 1) ? rows1 : rows0);
    for (int64_t i = lo + (int64_t)blockIdx.x * SB + threadIdx.x; i < hi; i += (int64_t)gridDim.x * SB)
        out[rows ? (int64_t)rows[i] : i] = nid;
}

size_t carve_grow(char* base, int64_t n, int F, int max_leaves, GrowArgs* A) {
    Carve c{base, 0};
    const size_t N = (size_t)(2 * max_leaves + 1);
    GrowArgs tmp;
    GrowArgs& a = A ? *A : tmp;
    a.st = c.take<GrowState>(1);
    a.q = c.take<Quant>(1);
    a.rows0 = c.take<uint32_t>((size_t)(n > 0 ? n : 1));
    a.rows1 = c.take<uint32_t>((size_t)(n > 0 ? n : 1));
    a.hist = c.take<int64_t>((size_t)max_leaves * 3 * (size_t)F * NB);
    a.path = c.take<uint8_t>(N * (size_t)F);
    a.leaf = c.take<LeafRec>(N);
    a.seg_lo = c.take<int64_t>(N);
    a.seg_hi = c.take<int64_t>(N);
    a.rec = c.take<ScanRec>((size_t)2 * F);
    return align_up(c.off, 256);
}

}  // namespace yabt

using namespace yabt;

extern "C" {

size_t yabt_grow_workspace_bytes(int64_t n, int F, int max_leaves) {
    if (n < 0 || F < 1 || max_leaves < 1) return 0;
    return carve_grow(nullptr, n, F, max_leaves, nullptr);
}

int yabt_grow(const uint8_t* bins_fm, int64_t ld_fm, const uint8_t* bins_rm, int64_t ld_rm, const float* grad,
              const float* hess, const uint8_t* fmask, const float* imat, float ib, int use_imat, const int32_t* nbins,
              const int32_t* default_bin, int64_t n, int F, float lam, float gamma, float mcw, int msl, float lr,
              int max_leaves, int max_depth, void* workspace, size_t workspace_bytes, int64_t* out_feature,
              int64_t* out_thr_bin, int64_t* out_left, int64_t* out_right, float* out_value, int64_t* out_depth,
              int32_t* out_status, hipStream_t stream) {
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
    A.dflt = default_bin;
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

    const int tiles = (F + HFL - 1) / HFL;
    k_quant_clear<<<1, 1, 0, stream>>>(A.q);
    k_setup<<<launch_grid(n, SB * 16, 1024), SB, 0, stream>>>(A);
    k_setup_finish<<<1, 1, 0, stream>>>(A);
    const int rc = root_chunks(n, tiles);
    k_hist_root<<<tiles * rc, HBLOCK, 0, stream>>>(bins_fm, ld_fm, grad, hess, n, F, A.q, 0.0, 0.0, A.dflt, A.q,
                                                   A.hist, rc, 1, &A.st->done);
    const int scan_grid = (F + SB / WAVE - 1) / (SB / WAVE);
    k_scan<true><<<scan_grid, SB, 0, stream>>>(A);
    const int pgrid = launch_grid(n, PART_TILE, PART_MAX_BLOCKS);
    for (int it = 1; it < max_leaves; ++it) {
        k_split_partition<<<pgrid, SB, 0, stream>>>(bins_fm, ld_fm, A.st);
        k_hist_gather<<<tiles * GATHER_MAX_CHUNKS, HBLOCK, 0, stream>>>(bins_rm, ld_rm, grad, hess, F, A.q, 0.0,
                                                                        0.0, A.dflt, &A.st->hist, 1, &A.st->done);
        k_scan<false><<<scan_grid, SB, 0, stream>>>(A);
    }
    return launch_status("yabt_grow launch");
}

int yabt_grow_leaf_ids(void* workspace, int64_t n, int F, int max_leaves, const int64_t* feature,
                       const int64_t* depth, const int32_t* status, int64_t* out, hipStream_t stream) {
    if (!workspace || !feature || !depth || !status || !out || n < 0 || F < 1 || max_leaves < 1 ||
        max_leaves > 32767)
        return fail(-2, "yabt_grow_leaf_ids: bad arguments");
    if (n == 0) return 0;
    GrowArgs A;
    memset(&A, 0, sizeof A);
    carve_grow((char*)workspace, n, F, max_leaves, &A);
    dim3 grid(launch_grid(n, SB * 8, 256), 2 * max_leaves + 1);
    k_leaf_ids<<<grid, SB, 0, stream>>>(feature, depth, A.seg_lo, A.seg_hi, A.rows0, A.rows1, status, out);
    return launch_status("yabt_grow_leaf_ids launch");
}

}  // extern "C"
