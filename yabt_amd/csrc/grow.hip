// gfx950 best-first (leaf-wise) tree growth, one tree per call.
//
// Replaces yabt/_cgrow/grow.c `cgrow` (grow.c:243-427) as called by
// yabt/grow_c.py `grow_tree_c` (grow_c.py:336-452).  The host enqueues a fixed
// launch sequence; every launch reads what to do from device-resident records
// written by the previous launch, so no split needs a host round trip.
//
// Arithmetic (bit-identical to oracle/grow_oracle.c OR_MODE_FIXED):
//   * g and h are quantised once per call to int64 fixed point with the
//     contract of common.h (hist_shift or wide_shift, chosen per call);
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
//   k_quant_clear, k_setup   max|g|,|h|; table init; clear slot 0
//   k_quant_resid            quantisation residuals -> contract, shifts,
//                            constant-hessian detection (common.h)
//   k_setup_finish           tree state
//   k_hist_root              streaming histogram of all rows (+ root totals)
//   k_scan<ROOT>             default-bin fill, scan, controller: first split
//   max_leaves - 1 times (each kernel returns at once once the tree is done):
//     k_split_partition      clear the built child's slot; one pass: the
//                            children's rows to the other row list, written
//                            through one atomic packed (left, right) count
//     k_hist_gather          histogram of the smaller child
//     k_scan<SPLIT>          fill, sibling = parent - child, scan both
//                            children (one wave each), the last block picks
//                            the next split
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
constexpr int SCAN_FEATS = 4;                  // features per scan block

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
    int64_t* new_hist;         // the built child's slot, cleared by the partition launch
    unsigned long long placed;      // rows placed: left count in the low 32 bits, right in the high 32
    unsigned long long pad1;
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
    const uint32_t* counts;              // per-fit bin counts (F, 256), or NULL
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
    float* gains;              // leaf[a].gain, contiguous (read by every scan block at launch)
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
// partition: one pass, one packed atomic count per tile
// ---------------------------------------------------------------------------

// Rows of [s, e) with bin <= b go to [s, mid), the others to [mid, e) of the
// children's row list.  A block takes tiles of PART_TILE rows; a thread holds
// rows t0 + j * SB + tid (j < PART_IPT), so each of its loads is coalesced
// across the block and all row-id loads, then all bin loads, are in flight
// together.  Waves compact with ballots and lane prefixes; the block reserves
// its output ranges with one atomic add per side, so the order inside a child
// depends on the schedule, which no result does (sums are exact).
// Every block first clears its share of the slot the gather adds into next.
__global__ void __launch_bounds__(SB) k_split_partition(const uint8_t* __restrict__ bins_fm, int64_t ld,
                                                        GrowState* st, int64_t slot_n) {
    // independent loads first
    const int32_t done = st->done, active = st->active;
    SplitJob& J = st->job;
    const int64_t s = J.s, e = J.e;
    const int fcol = J.f, b = J.b;
    const uint32_t* src = J.src;
    uint32_t* dst = J.dst;
    int64_t* z = J.new_hist;
    if (done || !active) return;
    for (int64_t i = (int64_t)blockIdx.x * SB + threadIdx.x; i < slot_n; i += (int64_t)gridDim.x * SB) z[i] = 0;
    const int64_t m = e - s;
    const int64_t tiles = (m + PART_TILE - 1) / PART_TILE;
    const int nblk = (int)min((int64_t)gridDim.x, max(tiles, (int64_t)1));
    if ((int)blockIdx.x >= nblk) return;
    const int64_t tpb = (tiles + nblk - 1) / nblk;
    const int64_t lo = s + (int64_t)blockIdx.x * tpb * PART_TILE;
    const int64_t hi = min(e, lo + tpb * PART_TILE);
    const uint8_t* col = bins_fm + (size_t)fcol * ld;
    const int w = threadIdx.x / WAVE;
    __shared__ uint32_t s_cnt[SB / WAVE][2];
    __shared__ unsigned long long s_base[SB / WAVE][2];
    for (int64_t t0 = lo; t0 < hi; t0 += PART_TILE) {
        uint32_t rid[PART_IPT];
#pragma unroll
        for (int j = 0; j < PART_IPT; ++j) {
            const int64_t i = min(t0 + (int64_t)j * SB + threadIdx.x, hi - 1);
            rid[j] = src ? src[i] : (uint32_t)i;
        }
        uint32_t bv[PART_IPT];
#pragma unroll
        for (int j = 0; j < PART_IPT; ++j) bv[j] = col[rid[j]];
        uint32_t left = 0, valid = 0, nl = 0, nv = 0;
#pragma unroll
        for (int j = 0; j < PART_IPT; ++j) {
            const bool v = t0 + (int64_t)j * SB + threadIdx.x < hi;
            const bool l = v && (int)bv[j] <= b;
            valid |= (v ? 1u : 0u) << j;
            left |= (l ? 1u : 0u) << j;
            nl += (uint32_t)__popcll(__ballot(l));
            nv += (uint32_t)__popcll(__ballot(v));
        }
        if ((threadIdx.x & (WAVE - 1)) == 0) {
            s_cnt[w][0] = nl;
            s_cnt[w][1] = nv - nl;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            uint32_t tl = 0, tr = 0;
            for (int i = 0; i < SB / WAVE; ++i) {
                tl += s_cnt[i][0];
                tr += s_cnt[i][1];
            }
            // one atomic reserves both children's places (a child holds at
            // most n < 2^32 rows: the left half never carries)
            const unsigned long long old =
                atomicAdd(&J.placed, (unsigned long long)tl | ((unsigned long long)tr << 32));
            unsigned long long bl = (unsigned long long)J.s + (old & 0xFFFFFFFFull);
            unsigned long long br = (unsigned long long)J.mid + (old >> 32);
            for (int i = 0; i < SB / WAVE; ++i) {
                s_base[i][0] = bl;
                s_base[i][1] = br;
                bl += s_cnt[i][0];
                br += s_cnt[i][1];
            }
        }
        __syncthreads();
        uint64_t pl = s_base[w][0], pr = s_base[w][1];
#pragma unroll
        for (int j = 0; j < PART_IPT; ++j) {
            const bool v = (valid >> j) & 1u, l = (left >> j) & 1u;
            const uint64_t ml = __ballot(l), mr = __ballot(v && !l);
            if (l) dst[pl + lane_prefix(ml)] = rid[j];
            else if (v) dst[pr + lane_prefix(mr)] = rid[j];
            pl += (uint64_t)__popcll(ml);
            pr += (uint64_t)__popcll(mr);
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

// r: the node's best record, or nullptr when no feature has a valid split.
__device__ __forceinline__ void leaf_from_record(LeafRec& L, const ScanRec* r, bool capped) {
    if (r) {
        L.gain = (float)(capped ? -INFINITY : r->gain);
        L.f = r->f;
        L.b = r->b;
        L.left[0] = r->left[0];
        L.left[1] = r->left[1];
        L.left[2] = r->left[2];
    } else {
        L.gain = -INFINITY;
        L.f = -1;
        L.b = -1;
        L.left[0] = L.left[1] = L.left[2] = 0;
    }
}

constexpr int GAIN_REGS = 4;                   // leaf gains a scan thread preloads

// Pick the next split (grow.c:321-350) and write its job, or finish the tree.
// gpre[i] holds gains[threadIdx.x + i * NT] as read at launch for the n_pre
// leaves that existed then, -inf for skip_idx (the split leaf); leaves past
// the preload are read here.  The leaves written since, s_new_idx[0..n_new),
// compete with their records s_new.
template <int NT>
__device__ void select_next(const GrowArgs& A, const float* gpre, int n_pre, int skip_idx, const LeafRec* s_new,
                            const int* s_new_idx, int n_new) {
    GrowState* st = A.st;
    __shared__ double s_key[NT / WAVE];
    __shared__ int s_idx[NT / WAVE];
    __shared__ LeafRec s_L;
    const int n_leaves = st->n_leaves;
    int k = -1;
    if (n_leaves < A.max_leaves) {
        double key = -INFINITY;
        int idx = INT_MAX;
#pragma unroll
        for (int i = 0; i < GAIN_REGS; ++i) {
            const int a = threadIdx.x + i * NT;
            const float g = gpre[i];
            if (a < n_pre && g > 0.0f && better((double)g, a, key, idx)) {
                key = (double)g;
                idx = a;
            }
        }
        for (int a = GAIN_REGS * NT + threadIdx.x; a < n_pre; a += NT) {
            const float g = A.gains[a];
            if (a != skip_idx && g > 0.0f && better((double)g, a, key, idx)) {
                key = (double)g;
                idx = a;
            }
        }
        block_argmax<NT>(key, idx, s_key, s_idx);
        for (int j = 0; j < n_new; ++j) {
            const float g = s_new[j].gain;
            if (g > 0.0f && better((double)g, s_new_idx[j], key, idx)) {
                key = (double)g;
                idx = s_new_idx[j];
            }
        }
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
    // the chosen leaf's record: one of the new ones, or a load
    if (threadIdx.x == 0) {
        if (k == s_new_idx[0]) s_L = s_new[0];
        else if (n_new > 1 && k == s_new_idx[1]) s_L = s_new[1];
        else s_L = A.leaf[k];
    }
    __syncthreads();
    const LeafRec& L = s_L;
    const int nid = L.node, nl = st->n_nodes, nr = nl + 1;
    if (A.use_imat) {
        // children inherit the parent's path plus f (grow.c:347-350); only the
        // interaction boost reads the paths
        const uint8_t* pp = A.path + (size_t)nid * A.F;
        for (int j = threadIdx.x; j < A.F; j += NT) {
            const uint8_t v = (j == L.f) ? (uint8_t)1 : pp[j];
            A.path[(size_t)nl * A.F + j] = v;
            A.path[(size_t)nr * A.F + j] = v;
        }
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
    // rows1 = rows0 + (rows1 - rows0): pointer arithmetic instead of a select,
    // which the compiler would turn into a two-entry table in scratch memory
    const ptrdiff_t r1 = A.rows1 - A.rows0;
    J.src = (d == 0) ? nullptr : A.rows0 + (d & 1) * r1;
    J.dst = A.rows0 + ((d + 1) & 1) * r1;
    J.s = s;
    J.e = e;
    J.mid = s + cl;
    for (int i = 0; i < 3; ++i) {
        J.tot[i] = L.tot[i];
        J.left[i] = L.left[i];
    }
    J.new_hist = A.hist + (size_t)new_slot * slot_elems(A.F);
    J.placed = 0;
    J.pad1 = 0;
    HistJob& H = st->hist;
    H.rows = J.dst;
    H.lo = bl ? s : s + cl;
    H.hi = bl ? s + cl : e;
    H.out = J.new_hist;
    H.active = 1;
    st->active = 1;
}

// Scan launch: SCAN_FEATS features per block; the split form gives each
// feature two waves, one per child (wave w: feature w % SCAN_FEATS, child
// w / SCAN_FEATS).  Each block publishes its best record per child (thread 0
// stores them and alone issues the release fence, so the fence covers only
// those stores); the histogram stores follow the ticket.  The last block to
// take a ticket is the controller.
template <bool ROOT>
__global__ void __launch_bounds__(ROOT ? SCAN_FEATS * WAVE : 2 * SCAN_FEATS * WAVE) k_scan(GrowArgs A) {
    constexpr int NT = ROOT ? SCAN_FEATS * WAVE : 2 * SCAN_FEATS * WAVE;
    constexpr int NC = ROOT ? 1 : 2;
    GrowState* st = A.st;
    const Quant* q = A.q;
    const SplitJob& J = st->job;
    // independent loads first
    const int32_t done = st->done;
    const bool derive = q->const_h != 0;     // no h channel: sum q(h) = count * hq_const
    const int64_t hqc = q->hq_const;
    const int bl = ROOT ? 1 : J.build_left;
    // leaf gains for the controller's next-split choice (every block loads
    // them; only the last block uses them)
    const int n_pre = ROOT ? 0 : st->n_active;
    const int skip_idx = ROOT ? -1 : J.k;
    float gpre[GAIN_REGS];
#pragma unroll
    for (int i = 0; i < GAIN_REGS; ++i) {
        const int a = threadIdx.x + i * NT;
        const float g = A.gains[min(a, 2 * A.max_leaves)];
        gpre[i] = (a < n_pre && a != skip_idx) ? g : -INFINITY;
    }
    const int parent_slot = ROOT ? 0 : J.parent_slot, new_slot = ROOT ? 0 : J.new_slot;
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    const int f = blockIdx.x * SCAN_FEATS + (w % SCAN_FEATS);
    const int c = w / SCAN_FEATS;
    const bool fok = f < A.F;
    const int fc = min(f, A.F - 1);          // unconditional loads: issued together
    const int nb_f = A.nbins[fc];
    const uint8_t use_f = A.fmask[fc];
    const int d_f = A.dflt ? A.dflt[fc] : -1;
    if (done) return;
    const int nb = fok ? max(0, min(NB, nb_f)) : 0;
    const bool use = fok && use_f != 0;
    const int d = fok ? d_f : -1;
    const ScanParams sp = {(double)A.lam, (double)A.gamma, (double)A.mcw, A.msl};
    const bool has_h = !derive;
    const bool built = ROOT || (c == 0) == (bl != 0);     // this wave scans the built child (the root: slot 0)
    int64_t* hp = A.hist + (size_t)parent_slot * slot_elems(A.F);
    int64_t* hn = A.hist + (size_t)new_slot * slot_elems(A.F);
    __shared__ ScanRec s_rec[NT / WAVE];
    __shared__ int s_last;
    int64_t g4[4], h4[4], c4[4];
    if (fok) {
        int64_t tot[3];
        if (ROOT) {
            tot[0] = q->tot_g;
            tot[1] = derive ? A.n * hqc : q->tot_h;
            tot[2] = A.n;
        } else {
            for (int i = 0; i < 3; ++i) tot[i] = bl ? J.left[i] : J.tot[i] - J.left[i];
        }
        load_bins(hn, A.F, f, lane, g4, h4, c4, has_h);
        fill_default(g4, h4, c4, d, tot, has_h, lane);
        if (!built) {
            int64_t pg[4], ph[4], pc[4];
            load_bins(hp, A.F, f, lane, pg, ph, pc, has_h);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                g4[j] = pg[j] - g4[j];
                h4[j] = ph[j] - h4[j];
                c4[j] = pc[j] - c4[j];
            }
        }
        int64_t hs[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) hs[j] = derive ? c4[j] * hqc : h4[j];
        const float bo = (!ROOT && A.use_imat && use)
                             ? path_boost(A.path + (size_t)J.nl * A.F, A.imat, A.ib, A.F, f, lane)
                             : 1.0f;
        int64_t t256[3];
        ScanRec r = scan_feature(g4, hs, c4, nb, q->ig, q->ih, sp, (double)bo, lane, t256);
        if (!use) no_split(r);
        r.f = f;
        if (lane == 0) s_rec[w] = r;
    } else if (lane == 0) {
        no_split(s_rec[w]);
        s_rec[w].f = -1;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int cc = 0; cc < NC; ++cc) {
            int bi = cc * SCAN_FEATS;
            for (int i = 1; i < SCAN_FEATS; ++i) {
                const ScanRec& o = s_rec[cc * SCAN_FEATS + i];
                if (rec_beats(o.sel, o.f, o.b, s_rec[bi].sel, s_rec[bi].f, s_rec[bi].b)) bi = cc * SCAN_FEATS + i;
            }
            publish_record(&A.rec[(size_t)cc * gridDim.x + blockIdx.x], s_rec[bi]);
        }
        record_published();
        const uint32_t t = atomicAdd(&st->scan_ticket, 1u);
        s_last = (t == gridDim.x - 1);
    }
    __syncthreads();
    const bool last = s_last != 0;
    if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    // every wave of the block has loaded its bins (barriers above): store
    if (fok) {
        if (built) {
            if (d >= 0 && (d >> 2) == lane) store_bins(hn, A.F, f, lane, g4, h4, c4, has_h);
        } else {
            store_bins(hp, A.F, f, lane, g4, h4, c4, has_h);
        }
    }
    if (!last) return;
    if (threadIdx.x == 0) st->scan_ticket = 0;

    // ---- controller (one block) ----
    __shared__ ScanRec s_best[NC];
    if (w < NC) {
        const ScanRec r = wave_best_record(A.rec + (size_t)w * gridDim.x, gridDim.x, lane);
        if (lane == 0) s_best[w] = r;
    }
    __shared__ LeafRec s_new[2];
    __shared__ int s_new_idx[2];
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
            L.tot[1] = derive ? A.n * hqc : q->tot_h;
            L.tot[2] = A.n;
            leaf_from_record(L, s_best[0].b >= 0 ? &s_best[0] : nullptr, 0 >= A.max_depth);
            A.leaf[0] = L;
            A.gains[0] = L.gain;
            A.value[0] = node_value(L.tot, q, A.lr, A.lam);
            st->n_nodes = 1;
            st->n_leaves = 1;
            st->n_active = 1;
            s_new[0] = L;
            s_new_idx[0] = 0;
            s_new_idx[1] = -1;
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
            leaf_from_record(Ll, s_best[0].b >= 0 ? &s_best[0] : nullptr, capped);
            leaf_from_record(Lr, s_best[1].b >= 0 ? &s_best[1] : nullptr, capped);
            A.seg_lo[J.nl] = J.s;
            A.seg_hi[J.nl] = J.mid;
            A.seg_lo[J.nr] = J.mid;
            A.seg_hi[J.nr] = J.e;
            A.value[J.nl] = node_value(Ll.tot, q, A.lr, A.lam);
            A.value[J.nr] = node_value(Lr.tot, q, A.lr, A.lam);
            const int na = st->n_active;
            A.leaf[J.k] = Ll;            // left child replaces the split leaf
            A.leaf[na] = Lr;             // right child is appended (grow.c:393-407)
            A.gains[J.k] = Ll.gain;
            A.gains[na] = Lr.gain;
            st->n_active = na + 1;
            st->active = 0;
            st->hist.active = 0;
            s_new[0] = Ll;
            s_new[1] = Lr;
            s_new_idx[0] = J.k;
            s_new_idx[1] = na;
        }
    }
    __syncthreads();
    select_next<NT>(A, gpre, n_pre, skip_idx, s_new, s_new_idx, ROOT ? 1 : 2);
}

// out[row] = leaf node id, from each leaf's segment of the final row lists.
// Grid (chunks, nodes).  Segments are clamped to [0, n) and row ids >= n are
// dropped, so a workspace that no longer holds this tree's rows (grown over
// since, with another n) cannot write outside `out`.
__global__ void __launch_bounds__(SB) k_leaf_ids(const int64_t* feature, const int64_t* depth, const int64_t* seg_lo,
                                                 const int64_t* seg_hi, const uint32_t* rows0, const uint32_t* rows1,
                                                 const int32_t* out_status, int64_t n, int64_t* out) {
    const int nid = blockIdx.y;
    if (nid >= out_status[0] || feature[nid] != LEAF) return;
    const int64_t lo = max((int64_t)0, seg_lo[nid]), hi = min(n, seg_hi[nid]), d = depth[nid];
    const uint32_t* rows = (d == 0) ? nullptr : ((d & 1) ? rows1 : rows0);
    for (int64_t i = lo + (int64_t)blockIdx.x * SB + threadIdx.x; i < hi; i += (int64_t)gridDim.x * SB) {
        const int64_t r = rows ? (int64_t)rows[i] : i;
        if (r < n) out[r] = nid;
    }
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
    a.gains = c.take<float>(N);
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
              const int32_t* default_bin, const uint32_t* bin_counts, int64_t n, int F, float lam, float gamma,
              float mcw, int msl, float lr,
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
    A.counts = bin_counts;
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
    launch_quant_resid(stream, grad, hess, n, A.q);
    k_setup_finish<<<1, 1, 0, stream>>>(A);
    launch_hist_root(stream, bins_fm, ld_fm, grad, hess, n, F, A.q, 0.0, 0.0, 0, A.dflt, A.counts, A.q, A.hist, 1,
                     &A.st->done);
    const int scan_grid = (F + SCAN_FEATS - 1) / SCAN_FEATS;
    k_scan<true><<<scan_grid, SCAN_FEATS * WAVE, 0, stream>>>(A);
    const int pgrid = launch_grid(n, PART_TILE, PART_MAX_BLOCKS);
    const int64_t slot_n = (int64_t)3 * F * NB;
    for (int it = 1; it < max_leaves; ++it) {
        k_split_partition<<<pgrid, SB, 0, stream>>>(bins_fm, ld_fm, A.st, slot_n);
        k_hist_gather<<<tiles * GATHER_MAX_CHUNKS, HBLOCK, 0, stream>>>(bins_rm, ld_rm, grad, hess, F, A.q, 0.0,
                                                                        0.0, A.dflt, &A.st->hist, 1, &A.st->done,
                                                                        0);
        k_scan<false><<<scan_grid, 2 * SCAN_FEATS * WAVE, 0, stream>>>(A);
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
    k_leaf_ids<<<grid, SB, 0, stream>>>(feature, depth, A.seg_lo, A.seg_hi, A.rows0, A.rows1, status, n, out);
    return launch_status("yabt_grow_leaf_ids launch");
}

}  // extern "C"
