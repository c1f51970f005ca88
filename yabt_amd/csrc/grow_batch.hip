// Best-first growth in rounds on gfx950: yabt_grow's trees (exact fixed-point
// sums, cgrow's best-first order, grow.c:243-427) with several splits
// computed per round.
//
// A leaf's best split and the histograms of its children depend only on the
// leaf's rows, not on when the leaf is split.  So a round computes several
// splits at once -- one partition launch, one histogram launch over every
// built child, one scan launch over every child -- and the scan's last block
// (the controller, one wave, working in LDS) then replays cgrow's leaf table
// (grow.c:321-408: first maximum of the fp32 gains above 0, left child
// replaces the split slot, right child appended, node ids in that order)
// over the computed splits, committing them until the leaf it would split
// next has no computed split.  It then plans the next round by running the
// same table further ahead: a leaf whose split is computed (committed or
// not) gives way to its children, whose best splits are known, and a leaf
// without one is taken for the round, until KMAX are taken or the leaves
// committed and taken fill the leaf budget.  Splits are taken at any depth
// below the committed tree, so in trees grown deep-first (fresh children
// often beat the older leaves) a round follows every branch one level down.
//
// Rows: a node at depth d >= 1 keeps its rows at [s, e) of row list d & 1
// (the root: the identity), written by its parent's split and intact until
// the node itself is split (only its ancestors, split before it, and its
// descendants, split after it, write inside [s, e)).  The rows of a final
// leaf whose computed split was never committed are the rows of the
// uncomputed nodes below it; the per-row leaf ids are written from those.
// Committed splits get exactly yabt_grow's node arrays, values and per-row
// leaf ids (same sums, same scan, same order); the others are never read.
//
// Launches: k_setup, k_quant_resid (the contract, common.h), k_setup_finish,
// k_hist_root, k_scan<true> (root, plans
// round 1), then per round k_part, k_gather, k_scan<false>, and at the end
// k_leaf_plan, k_leaf_ids (per-row leaf ids).
// The controller writes the round count and the done flag to mapped host
// memory; the host keeps at most LOOKAHEAD rounds in flight and stops when
// the tree is done.
//
// HBM layout: bins feature-major (partitions) and row-major (gathers); two
// lists of n uint32 row ids; hist: (PEND_PER_LEAF L + KMAX + 1, 3, F, 256)
// int64 slots, one per computed split plus the root's.

#include "common.h"
#include "hist.h"
#include "host.h"
#include "scan.h"
#include "yabt_hip.h"

#include <limits.h>
#include <string.h>

#include <atomic>

namespace yabt {
namespace rnd {

constexpr int SB = 256;                          // threads of the partition / setup blocks
constexpr int PART_IPT_WIDE = 16;                // rows per thread per partition tile: rounds
constexpr int PART_IPT_NARROW = 8;               //   of more / fewer than PART_WIDE_ROWS rows
constexpr int64_t PART_WIDE_ROWS = 1 << 20;
constexpr int PART_BLOCKS = 2048;
constexpr int SCAN_FEATS = 4;                    // features per scan block
constexpr int KMAX = 16;                         // splits computed per round, at most
constexpr int GBLOCKS = 256;                     // gather blocks of a launch, about (multiple of XCDS)
constexpr int XCDS = 8;                          // dies of the device; blocks go to them in turn
constexpr int CT = 2 * SCAN_FEATS * WAVE;        // threads of a split-scan block (the controller)
constexpr int LOOKAHEAD = 2;                     // rounds the host keeps in flight
constexpr int MAX_LEAVES = 1024;                 // leaf table held in the controller's LDS
constexpr int TABLE_REGS = 4;                    // leaf-table entries per lane when the replay holds it in registers
constexpr int PEND_PER_LEAF = 3;                 // computed splits per leaf of the budget, at most
constexpr int LEAF_CHUNK = 8192;                 // rows per leaf-id block
constexpr int LEAF_PLAN = 1024;                  // threads of the leaf-id planning block
// index bits of a packed planning candidate: candidates are the leaves and
// both children of every computed split, below 2^PICK_IDX_BITS
constexpr int PICK_IDX_BITS = 13;
static_assert(MAX_LEAVES + 2 * (PEND_PER_LEAF * MAX_LEAVES + KMAX) <= (1 << PICK_IDX_BITS), "candidate indices");

// A computed split.  Leaves of the table name their origin as 2 p + c (child
// c of split p) or -1 (the root).
struct Pend {
    int32_t f, b, build_left, depth;     // depth of the children
    int32_t parent_slot, new_slot;
    int32_t child_pend[2];               // the children's computed splits, -1: none
    int32_t child_node[2];               // the children's node ids once committed, -1: not committed
    int32_t origin, pad;                 // the split leaf's origin
    const uint32_t* src;                 // the leaf's rows (null: the identity)
    uint32_t* dst;                       // the children's rows
    int64_t s, e, mid;
    int64_t tot[3], left[3];
    int64_t pad2;
    unsigned long long placed;           // rows placed: left count in the low 32 bits, right in the high 32
    unsigned long long pad1;
    ScanRec child[2];                    // the children's best records (b = -1: none)
};

// What the controller needs of a computed split, packed.
struct PendSum {
    float gain[2];                       // the children's table gains (depth cap applied)
    int16_t child_pend[2];               // the children's computed splits, -1: none
    int16_t origin;                      // the split leaf's origin (2 q + c, -1: the root)
    int16_t committed;                   // 1 once the split is committed
};

struct State {
    int32_t n_nodes, n_leaves, done;
    int32_t n_round;                     // splits computed this round
    int32_t n_pend;                      // Pend entries used
    int32_t round;                       // controllers run
    uint32_t scan_ticket;                // splits whose scan blocks have all finished
    int32_t pad;
    int32_t root_pend;                   // the root's computed split, -1: none
    float root_gain;                     // the root's table gain
    int32_t round_pend[KMAX];            // this round's Pend entries
    int64_t tile_off[KMAX + 1];          // partition tiles of this round's splits, prefix sums
    int32_t part_ipt;                    // rows per thread of this round's partition tiles
    int32_t pad4;
    int32_t unit_off[KMAX + 1];          // gather units of this round's built children, prefix sums
    int32_t pad3;
    int64_t unit_rows;                   // rows per gather unit (a child's last unit: the rest)
    uint32_t split_ticket[KMAX];         // scan blocks of each split finished
};

// A run of final-leaf rows for the leaf-id pass: positions [lo, hi) of a row
// list (rows null: the identity) all belong to node `label`; its chunks of
// LEAF_CHUNK rows are numbered from chunk0.
struct LeafRun {
    const uint32_t* rows;
    int64_t lo, hi;
    int64_t label;
};

// The host's view, in mapped host memory: one word, ((round + 1) << 1) |
// done, written with a single 32-bit store so that no fence has to order
// separate fields (0: no controller has run).
struct Flags {
    int32_t word;
    int32_t pad[3];
};

struct Args {
    const uint8_t* bins_fm;
    int64_t ld_fm;
    const uint8_t* bins_rm;
    int64_t ld_rm;
    const float* grad;
    const float* hess;
    float2* gh;                          // (n) (g, h) interleaved, written by k_setup: one load per gathered row
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
    int pend_cap;                        // Pend entries (and new slots) available
    State* st;
    Quant* q;
    uint32_t* rows;                      // two lists of rows_ld row ids
    int64_t rows_ld;
    int64_t* hist;
    int64_t* pieces;                     // gather_units(tiles) slots: one per gather unit
    uint8_t* pend_path;                  // (pend_cap, F) features on the path to each split's children
    int32_t* leaf_src;                   // cgrow's leaf table after the commits: each leaf's origin
    int32_t* leaf_node;                  // and node id (gains and computed splits follow from the origin)
    Pend* pend;
    PendSum* psum;
    ScanRec* rec;                        // (KMAX, 2, scan blocks)
    LeafRun* leaf_runs;                  // 2 pend_cap + 1 runs
    int32_t* leaf_chunk0;                // their first chunks, then the run count and the chunk count
    int leaf_chunk_cap;                  // chunks, at most
    int64_t* feature;
    int64_t* thr_bin;
    int64_t* left;
    int64_t* right;
    float* value;
    int64_t* depth;
    int32_t* out_status;
    Flags* flags;                        // device address of the mapped host flags
};

__device__ __forceinline__ size_t slot_elems(int F) { return (size_t)3 * (size_t)F * NB; }

// ---------------------------------------------------------------------------
// setup
// ---------------------------------------------------------------------------

__global__ void __launch_bounds__(SB) k_setup(Args A) {
    quant_reduce<SB>(A.grad, A.hess, A.n, A.q, A.gh);
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
    }
    const int64_t ne = (int64_t)slot_elems(A.F);
    for (int64_t i = tid; i < ne; i += stride) A.hist[i] = 0;
}

__global__ void k_setup_finish(Args A) {
    State* st = A.st;
    st->done = 0;
    st->n_round = 0;
    st->n_pend = 0;
    st->round = 0;
    st->scan_ticket = 0;
    for (int i = 0; i < KMAX; ++i) st->split_ticket[i] = 0;
    st->root_pend = -1;
    st->root_gain = -INFINITY;
    st->n_nodes = 1;
    st->n_leaves = 1;
    // every word of the status is written here, so the caller need not clear it
    A.out_status[0] = 0;
    A.out_status[1] = 0;
    A.out_status[2] = 0;
    if (A.q->nonfinite) {
        st->done = 1;
        A.out_status[0] = -1;
        A.out_status[1] = 0;
        A.out_status[2] = 0;
        A.flags->word = 1;   // done before any round
    }
}

// ---------------------------------------------------------------------------
// partition: every split of the round, tiles grid-strided
// ---------------------------------------------------------------------------

// Rows of [s, e) with bin <= b go to [s, mid), the others to [mid, e) of the
// children's row list.  A tile reserves its places in both children with one
// 64-bit atomic on the split's packed (left, right) count: a child holds at
// most n < 2^32 rows, so the left half never carries into the right.  (The
// order inside a child depends on the schedule, which no exact sum does.)
template <int IPT>
__device__ __forceinline__ void part_tiles(const uint8_t* __restrict__ bins_fm, int64_t ld, int64_t n, State* st,
                                           Pend* pend, int nr) {
    constexpr int TILE = SB * IPT;
    const int w = threadIdx.x / WAVE;
    __shared__ uint32_t s_cnt[SB / WAVE][2];
    __shared__ unsigned long long s_base[SB / WAVE][2];
    __shared__ int64_t s_toff[KMAX + 1];
    __shared__ int32_t s_rp[KMAX];
    // the round's tile offsets and Pend entries, loaded together
    if (threadIdx.x <= nr) s_toff[threadIdx.x] = st->tile_off[threadIdx.x];
    if (threadIdx.x < nr) s_rp[threadIdx.x] = st->round_pend[threadIdx.x];
    __syncthreads();
    const int64_t T = s_toff[nr];
    int j = 0;   // tiles t grow, so their splits j do
    for (int64_t t = blockIdx.x; t < T; t += gridDim.x) {
        while (j + 1 < nr && s_toff[j + 1] <= t) ++j;
        Pend& P = pend[s_rp[j]];
        const int64_t t0 = P.s + (t - s_toff[j]) * TILE;
        const int64_t hi = min(P.e, t0 + TILE);
        const uint8_t* col = bins_fm + (size_t)P.f * ld;
        const int b = P.b;
        const uint32_t* src = P.src;
        uint32_t* dst = P.dst;
        uint32_t rid[IPT];
#pragma unroll
        for (int k = 0; k < IPT; ++k) {
            const int64_t i = min(t0 + (int64_t)k * SB + threadIdx.x, hi - 1);
            rid[k] = src ? min(src[i], (uint32_t)(n - 1)) : (uint32_t)i;   // a row id stays a row id
        }
        uint32_t bv[IPT];
#pragma unroll
        for (int k = 0; k < IPT; ++k) bv[k] = col[rid[k]];
        uint32_t left = 0, valid = 0, nl = 0, nv = 0;
#pragma unroll
        for (int k = 0; k < IPT; ++k) {
            const bool v = t0 + (int64_t)k * SB + threadIdx.x < hi;
            const bool l = v && (int)bv[k] <= b;
            valid |= (v ? 1u : 0u) << k;
            left |= (l ? 1u : 0u) << k;
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
            const unsigned long long old =
                atomicAdd(&P.placed, (unsigned long long)tl | ((unsigned long long)tr << 32));
            unsigned long long bl = (unsigned long long)P.s + (old & 0xFFFFFFFFull);
            unsigned long long br = (unsigned long long)P.mid + (old >> 32);
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
        for (int k = 0; k < IPT; ++k) {
            const bool v = (valid >> k) & 1u, l = (left >> k) & 1u;
            const uint64_t ml = __ballot(l), mr = __ballot(v && !l);
            if (l) dst[pl + lane_prefix(ml)] = rid[k];
            else if (v) dst[pr + lane_prefix(mr)] = rid[k];
            pl += (uint64_t)__popcll(ml);
            pr += (uint64_t)__popcll(mr);
        }
        __syncthreads();
    }
}

__global__ void __launch_bounds__(SB) k_part(const uint8_t* __restrict__ bins_fm, int64_t ld, int64_t n, State* st,
                                             Pend* pend) {
    const int32_t done = st->done, nr = st->n_round;
    if (done || nr == 0) return;
    if (st->part_ipt == PART_IPT_WIDE)
        part_tiles<PART_IPT_WIDE>(bins_fm, ld, n, st, pend, nr);
    else
        part_tiles<PART_IPT_NARROW>(bins_fm, ld, n, st, pend, nr);
}

// ---------------------------------------------------------------------------
// gather: the built child of every split of the round, (split, chunk) units
// ---------------------------------------------------------------------------

// Gather units of a round, about: a multiple of XCDS near GBLOCKS / tiles,
// so that one unit per tile fills the device once.
__host__ __device__ inline int gather_target(int tiles) {
    const int g = GBLOCKS / XCDS / tiles;
    return XCDS * (g > 1 ? g : 1);
}
// Units a round may use, at most (blocks per tile of the gather launch).
__host__ __device__ inline int gather_units(int tiles) { return gather_target(tiles) + KMAX; }

// Rows per gather unit of a round of nr splits gathering R rows in all: whole
// waves, and large enough that the splits' units (ceil(rows / unit_rows)
// each, at most R / unit_rows + nr in all) stay within gather_target when it
// exceeds nr, and within gather_units always.
__host__ __device__ inline int64_t gather_unit_rows(int64_t R, int nr, int tiles) {
    const int t = gather_target(tiles);
    const int64_t d = t > nr ? t - nr : 1;
    const int64_t per = ((R + d - 1) / d + WAVE - 1) / WAVE * WAVE;
    return per > 0 ? per : WAVE;
}

// Each built child is cut into units of unit_rows rows (split j owns units
// unit_off[j] .. unit_off[j + 1]); block (tile, u) stores the histogram of
// unit u's rows in slot u of `pieces` -- no atomics, no clearing -- and the
// scan adds up a child's units.  Block ids go to the XCDS dies in turn and
// the blocks of one unit (every tile of the same rows) are numbered to land
// on one die, sharing its L2 for the rows' bins, ids and g, h.
__global__ void __launch_bounds__(HBLOCK) k_gather(const uint8_t* __restrict__ bins_rm, int64_t ld,
                                                   const float* __restrict__ grad, const float* __restrict__ hess,
                                                   const float2* __restrict__ gh,
                                                   int F, const Quant* q, const int32_t* __restrict__ dflt,
                                                   const State* st, const Pend* pend, int64_t* pieces) {
    const int32_t done = st->done, nr = st->n_round;
    const double scg = q->scg, sch = q->sch;
    const int wlog = q->wlog;
    const bool no_h = q->const_h != 0;
    if (done || nr == 0) return;
    // block id -> (unit, tile): die x = id % XCDS holds units x, x + XCDS, ...
    const int tiles = (F + HFL - 1) / HFL;
    const int x = blockIdx.x % XCDS, k = blockIdx.x / XCDS;
    const int tile = k % tiles, unit = (k / tiles) * XCDS + x;
    if (unit >= st->unit_off[nr]) return;
    int j = 0;
    while (j + 1 < nr && st->unit_off[j + 1] <= unit) ++j;
    const Pend& P = pend[st->round_pend[j]];
    const int64_t per = st->unit_rows;
    const int64_t c_lo = P.build_left ? P.s : P.mid, c_hi = P.build_left ? P.mid : P.e;
    const int64_t lo = c_lo + (int64_t)(unit - st->unit_off[j]) * per, hi = min(c_hi, lo + per);
    int64_t* out = pieces + (size_t)unit * slot_elems(F);
    __shared__ GatherLds L;
    if (no_h) {
        if (dflt)
            hist_gather_rows<false, true, true>(L, bins_rm, ld, grad, hess, F, scg, sch, dflt, P.dst, lo, hi, out,
                                                wlog, tile, gh);
        else
            hist_gather_rows<false, false, true>(L, bins_rm, ld, grad, hess, F, scg, sch, dflt, P.dst, lo, hi, out,
                                                 wlog, tile, gh);
    } else {
        if (dflt)
            hist_gather_rows<true, true, true>(L, bins_rm, ld, grad, hess, F, scg, sch, dflt, P.dst, lo, hi, out,
                                               wlog, tile, gh);
        else
            hist_gather_rows<true, false, true>(L, bins_rm, ld, grad, hess, F, scg, sch, dflt, P.dst, lo, hi, out,
                                                wlog, tile, gh);
    }
}

// ---------------------------------------------------------------------------
// scan + controller
// ---------------------------------------------------------------------------

__device__ __forceinline__ float node_value(const int64_t tot[3], const Quant* q, float lr, float lam) {
    const double G = (double)tot[0] * q->ig, H = (double)tot[1] * q->ih;
    return (float)(-lr * G / (H + lam));
}

// A child's table gain from its best record: the fp32 gain, -inf if it has
// no split or sits at the depth cap (grow.c:296-305).
__device__ __forceinline__ float rec_gain(const ScanRec& r, bool capped) {
    return (r.b >= 0 && !capped) ? (float)r.gain : -INFINITY;
}

// LDS written by one lane, then read by the others of the wave.
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// Inclusive prefix sum over the wave (32- or 64-bit integers).
template <typename T>
__device__ __forceinline__ T wave_incl_scan(T v, int lane) {
    static_assert(std::is_integral<T>::value && (sizeof(T) == 4 || sizeof(T) == 8), "integer scan");
    if constexpr (sizeof(T) == 4) return (T)wave_incl_scan_i32((int32_t)v, lane);
    else return (T)wave_incl_scan_i64((int64_t)v, lane);
}

// A leaf as a split candidate, from its origin (2 p + c, or -1: the root
// with record *root).
struct LeafV {
    int32_t f, b, depth, slot;
    int64_t s, e, tot[3], left[3];
};

__device__ __forceinline__ LeafV leaf_view(const Args& A, int src, const ScanRec* root) {
    LeafV v;
    const ScanRec* r;
    if (src < 0) {
        const Quant* q = A.q;
        v.depth = 0;
        v.slot = 0;
        v.s = 0;
        v.e = A.n;
        v.tot[0] = q->tot_g;
        v.tot[1] = q->const_h ? A.n * q->hq_const : q->tot_h;
        v.tot[2] = A.n;
        r = root;
    } else {
        const Pend& P = A.pend[src >> 1];
        const int c = src & 1;
        v.depth = P.depth;
        v.slot = ((c == 0) == (P.build_left != 0)) ? P.new_slot : P.parent_slot;
        v.s = c ? P.mid : P.s;
        v.e = c ? P.e : P.mid;
        for (int i = 0; i < 3; ++i) v.tot[i] = c ? P.tot[i] - P.left[i] : P.left[i];
        r = &P.child[c];
    }
    v.f = r->f;
    v.b = r->b;
    for (int i = 0; i < 3; ++i) v.left[i] = r->left[i];
    return v;
}

// The controller's LDS: cgrow's leaf table (entry a: leaf a), the computed
// splits' children, and the lists this controller fills.  The arrays live in
// the scan launch's dynamic LDS, sized by the leaf budget and the Pend
// capacity (table_bytes); the struct holds their addresses.
// LDS pointers (address space 3): accesses through them compile to ds_*
// instructions, where generic pointers would take the slower flat path.
#define YABT_LDS __attribute__((address_space(3)))

struct Table {
    YABT_LDS float* gain;                // [L]
    YABT_LDS int16_t* pend;              // [L] computed split, -1: none
    YABT_LDS int16_t* src;               // [L] origin
    YABT_LDS int16_t* node;              // [L] node id (the committed table)
    YABT_LDS float (*cgain)[2];          // [pend_cap] PendSum, per computed split
    YABT_LDS int16_t (*cpend)[2];        // [pend_cap]
    YABT_LDS int16_t* corigin;           // [pend_cap]
    YABT_LDS uint8_t* ccommit;           // [pend_cap]
    YABT_LDS float* ckey;                // [pend_cap] while planning: key of the split's node (+inf: not known)
    YABT_LDS float* cbud;                // [pend_cap] while planning: that key where the split counts for the budget
    YABT_LDS float* ckand;               // [L + 2 pend_cap] while planning: the listed candidates' keys
    YABT_LDS int16_t* cidx;              // [L + 2 pend_cap] and their indices
    YABT_LDS int16_t* commit_p;          // [L] this controller's commits: split, parent node
    YABT_LDS int16_t* commit_nid;        // [L]
    YABT_LDS int16_t* plan_src;          // [KMAX] this round's splits: origin
    YABT_LDS float* root_gain;           // the root's table gain and computed split
    YABT_LDS int32_t* root_pend;
};

// Carve of the controller's LDS at `base` into *T (base null: size only).
__host__ __device__ inline size_t table_carve(char* base, int L, int pend_cap, Table* T) {
    size_t off = 0;
    auto take = [&](size_t bytes) {
        off = (off + 15) / 16 * 16;
        char* p = base ? base + off : nullptr;
        off += bytes;
        return p;
    };
    char* gain = take(sizeof(float) * L);
    char* cgain = take(sizeof(float) * 2 * pend_cap);
    char* ckey = take(sizeof(float) * pend_cap);
    char* cbud = take(sizeof(float) * pend_cap);
    char* ckand = take(sizeof(float) * (L + 2 * (size_t)pend_cap));
    char* root_gain = take(sizeof(float));
    char* root_pend = take(sizeof(int32_t));
    char* pend = take(sizeof(int16_t) * L);
    char* src = take(sizeof(int16_t) * L);
    char* node = take(sizeof(int16_t) * L);
    char* cpend = take(sizeof(int16_t) * 2 * pend_cap);
    char* corigin = take(sizeof(int16_t) * pend_cap);
    char* commit_p = take(sizeof(int16_t) * L);
    char* commit_nid = take(sizeof(int16_t) * L);
    char* plan_src = take(sizeof(int16_t) * KMAX);
    char* cidx = take(sizeof(int16_t) * (L + 2 * (size_t)pend_cap));
    char* ccommit = take(pend_cap);
#if defined(__HIP_DEVICE_COMPILE__)
    // tested on base, not on T: a null test of the table's own address keeps
    // the table in private (scratch) memory
    if (base) {
        T->gain = (YABT_LDS float*)gain;
        T->cgain = (YABT_LDS float(*)[2])cgain;
        T->ckey = (YABT_LDS float*)ckey;
        T->cbud = (YABT_LDS float*)cbud;
        T->ckand = (YABT_LDS float*)ckand;
        T->root_gain = (YABT_LDS float*)root_gain;
        T->root_pend = (YABT_LDS int32_t*)root_pend;
        T->pend = (YABT_LDS int16_t*)pend;
        T->src = (YABT_LDS int16_t*)src;
        T->node = (YABT_LDS int16_t*)node;
        T->cpend = (YABT_LDS int16_t(*)[2])cpend;
        T->corigin = (YABT_LDS int16_t*)corigin;
        T->commit_p = (YABT_LDS int16_t*)commit_p;
        T->commit_nid = (YABT_LDS int16_t*)commit_nid;
        T->plan_src = (YABT_LDS int16_t*)plan_src;
        T->cidx = (YABT_LDS int16_t*)cidx;
        T->ccommit = (YABT_LDS uint8_t*)ccommit;
    }
#else
    (void)T;
    for (char* p : {gain, cgain, ckey, cbud, ckand, root_gain, root_pend, pend, src, node, cpend, corigin, commit_p,
                    commit_nid, plan_src, cidx, ccommit})
        (void)p;
#endif
    return (off + 15) / 16 * 16;
}

// First maximum of s_gain[0..na) above 0 (cgrow's strict > from 0.0f, the
// lowest index on ties), over one wave; -1: none.  Each lane keeps the first
// maximum above 0 of its entries (lane, lane + 64, ...), four LDS loads in
// flight; the table's is the lowest index among the lanes holding the wave's
// maximum.
__device__ __forceinline__ int wave_table_argmax(const YABT_LDS float* s_gain, int na, int lane) {
    float key = 0.0f;
    int idx = INT_MAX;
    constexpr int U = 4;
    for (int a0 = lane; a0 < na; a0 += U * WAVE) {
        float g[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int a = a0 + u * WAVE;
            g[u] = a < na ? s_gain[a] : -INFINITY;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (g[u] > key) {
                key = g[u];
                idx = a0 + u * WAVE;
            }
        }
    }
    const float m = wave_max_f32(key);
    if (!(m > 0.0f)) return -1;
    return wave_min_i32(key == m ? idx : INT_MAX);
}

// Position of the best entry of a compacted candidate list (largest key
// above 0, the lowest index on ties), over one wave; -1: none.
__device__ __forceinline__ int wave_list_argmax(const YABT_LDS float* keys, const YABT_LDS int16_t* ids, int m,
                                                int lane) {
    float key = 0.0f;
    int idx = INT_MAX, pos = INT_MAX;
    for (int i = lane; i < m; i += WAVE) {
        const float k = keys[i];
        const int x = ids[i];
        if (k > key || (k == key && k > 0.0f && x < idx)) {
            key = k;
            idx = x;
            pos = i;
        }
    }
    const float mx = wave_max_f32(key);
    if (!(mx > 0.0f)) return -1;
    const int wi = wave_min_i32(key == mx ? idx : INT_MAX);
    return wave_min_i32((key == mx && idx == wi) ? pos : INT_MAX);
}

// Table gain and computed split of the leaf with origin src.
__device__ __forceinline__ float gain_of(const Table& T, int src) {
    return src < 0 ? *T.root_gain : T.cgain[src >> 1][src & 1];
}
__device__ __forceinline__ int pend_of(const Table& T, int src) {
    return src < 0 ? *T.root_pend : (int)T.cpend[src >> 1][src & 1];
}

// Node arrays of commit i (split p of node nid, children nl, nl + 1); the
// parent's value is cleared afterwards (it may be a child of this batch).
__device__ __forceinline__ void write_commit(const Args& A, int p, int nid, int nl) {
    Pend& P = A.pend[p];
    const int nr = nl + 1;
    int64_t tl[3], tr[3];
    for (int i = 0; i < 3; ++i) {
        tl[i] = P.left[i];
        tr[i] = P.tot[i] - P.left[i];
    }
    A.feature[nid] = P.f;
    A.thr_bin[nid] = P.b;
    A.left[nid] = nl;
    A.right[nid] = nr;
    A.depth[nl] = P.depth;
    A.depth[nr] = P.depth;
    A.value[nl] = node_value(tl, A.q, A.lr, A.lam);
    A.value[nr] = node_value(tr, A.q, A.lr, A.lam);
    P.child_node[0] = nl;
    P.child_node[1] = nr;
    A.psum[p].committed = 1;
}

// The controller, one wave: T holds cgrow's leaf table as the previous
// round's commits left it (nn nodes, na leaves, gains and computed splits
// filled in from the origins) and the np computed splits' children.  Replay
// cgrow's leaf table over the computed splits, store it, plan the next round
// (or finish the tree), publish.
// root: the root's record while the root is an uncomputed leaf (the first
// controller), else null.
//
// Planning chooses the leaves whose splits the next round computes.  cgrow's
// coming pops, run ahead of the commits with every computed split expanded,
// come in the order of a key: the minimum of the gains on a leaf's path from
// the committed leaf it hangs from (a child enters the table only when its
// parent is popped, and the table always pops its maximum).  So the round
// takes `best` -- the leaf the commits stopped at, cgrow's next split -- and
// then the uncomputed leaves of largest key (committed leaves without a
// computed split, uncomputed children of uncommitted computed splits) while
// the leaves the run-ahead would hold at that pop (the committed ones, one
// more per computed split of larger key, one per leaf taken) fit the budget.
// Ties in key may be ordered otherwise than cgrow's table: the plan decides
// only which splits are computed when, never the tree (the commits replay
// cgrow's table exactly), and the split the commits wait for is always taken.
__device__ __forceinline__ void control(const Args& A, Table& T, int nn, int na, int np, const ScanRec* root, int lane) {
    State* st = A.st;
    const int L = A.max_leaves;
    const int nn0 = nn;
    // replay (grow.c:321-330): commit the best leaf while its split is computed
    int best = -1, ncm = 0;
    if (L <= TABLE_REGS * WAVE) {
        // the table in registers, entry u * 64 + lane in slot u of the lane.
        // A positive fp32 gain orders as its bits, so the best is a 32-bit
        // wave maximum of the lanes' best bits (non-positive and NaN gains
        // count as 0), and the lowest entry holding it is the lowest lane of
        // the first slot whose ballot is not empty: cgrow's first maximum
        // above 0.
        float tg[TABLE_REGS];
        int tp[TABLE_REGS], ts[TABLE_REGS], tn[TABLE_REGS];
#pragma unroll
        for (int u = 0; u < TABLE_REGS; ++u) {
            const int a = u * WAVE + lane;
            const bool in = a < na;
            tg[u] = in ? T.gain[a] : -INFINITY;
            tp[u] = in ? (int)T.pend[a] : -1;
            ts[u] = in ? (int)T.src[a] : 0;
            tn[u] = in ? (int)T.node[a] : 0;
        }
        auto bits = [](float g) { return g > 0.0f ? __float_as_uint(g) : 0u; };
        while (na < L) {
            uint32_t lb = 0;
#pragma unroll
            for (int u = 0; u < TABLE_REGS; ++u) lb = max(lb, bits(tg[u]));
            const uint32_t m = (uint32_t)__builtin_amdgcn_readfirstlane((int)wave_max_u32_v(lb));
            if (m == 0u) break;
            int ub = 0;
            uint64_t bal = 0;
#pragma unroll
            for (int u = TABLE_REGS - 1; u >= 0; --u) {
                const uint64_t b = __ballot(bits(tg[u]) == m);
                if (b != 0) {
                    ub = u;
                    bal = b;
                }
            }
            const int bl = __builtin_ctzll(bal);
            best = ub * WAVE + bl;
            int pv = tp[0], nv = tn[0];
#pragma unroll
            for (int u = 1; u < TABLE_REGS; ++u) {
                pv = ub == u ? tp[u] : pv;
                nv = ub == u ? tn[u] : nv;
            }
            const int p = __builtin_amdgcn_readlane(pv, bl);
            if (p < 0) break;
            const int nid = __builtin_amdgcn_readlane(nv, bl);
            const float g0 = T.cgain[p][0], g1 = T.cgain[p][1];
            const int c0 = T.cpend[p][0], c1 = T.cpend[p][1];
            // left child replaces the split leaf, right child is appended
            // (grow.c:393-407)
            const int un = na / WAVE, ln = na % WAVE;
#pragma unroll
            for (int u = 0; u < TABLE_REGS; ++u) {
                const bool atb = u == ub && lane == bl, atn = u == un && lane == ln;
                tg[u] = atb ? g0 : (atn ? g1 : tg[u]);
                tp[u] = atb ? c0 : (atn ? c1 : tp[u]);
                ts[u] = atb ? 2 * p : (atn ? 2 * p + 1 : ts[u]);
                tn[u] = atb ? nn : (atn ? nn + 1 : tn[u]);
            }
            if (lane == 0) {
                T.ccommit[p] = 1;
                T.commit_p[ncm] = (int16_t)p;
                T.commit_nid[ncm] = (int16_t)nid;
            }
            nn += 2;
            ++na;
            ++ncm;
            best = -1;
        }
#pragma unroll
        for (int u = 0; u < TABLE_REGS; ++u) {
            const int a = u * WAVE + lane;
            if (a < na) {
                T.gain[a] = tg[u];
                T.pend[a] = (int16_t)tp[u];
                T.src[a] = (int16_t)ts[u];
                T.node[a] = (int16_t)tn[u];
            }
        }
        wave_sync();
    }
    while (L > TABLE_REGS * WAVE && na < L) {
        best = wave_table_argmax(T.gain, na, lane);
        if (best < 0 || T.pend[best] < 0) break;
        const int p = T.pend[best];
        if (lane == 0) {
            T.ccommit[p] = 1;
            T.commit_p[ncm] = (int16_t)p;
            T.commit_nid[ncm] = T.node[best];
            // left child replaces the split leaf, right child is appended
            // (grow.c:393-407)
            T.gain[best] = T.cgain[p][0];
            T.pend[best] = T.cpend[p][0];
            T.src[best] = (int16_t)(2 * p);
            T.node[best] = (int16_t)nn;
            T.gain[na] = T.cgain[p][1];
            T.pend[na] = T.cpend[p][1];
            T.src[na] = (int16_t)(2 * p + 1);
            T.node[na] = (int16_t)(nn + 1);
        }
        nn += 2;
        ++na;
        ++ncm;
        best = -1;
        wave_sync();
    }
    // the commits' node arrays, then the cleared parent values
    for (int i = lane; i < ncm; i += WAVE) write_commit(A, T.commit_p[i], T.commit_nid[i], nn0 + 2 * i);
    // the wave's stores so far have completed (at this XCD's L2, where the
    // clears below go too)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    for (int i = lane; i < ncm; i += WAVE) A.value[T.commit_nid[i]] = 0.0f;
    // store the committed table
    for (int a = lane; a < na; a += WAVE) {
        A.leaf_src[a] = T.src[a];
        A.leaf_node[a] = T.node[a];
    }
    int status = 0, j = 0;
    int my_pick = -1;   // lane t: the candidate taken as the round's split t
    const int np0 = np;
    if (best >= 0) {
        // keys of the uncommitted computed splits' nodes: a committed leaf's
        // split takes the leaf's gain, then (index order: a split's parent
        // split has a lower index) a split below an uncommitted split q takes
        // min(key of q, the child's gain)
        for (int p = lane; p < np0; p += WAVE) T.ckey[p] = INFINITY;
        wave_sync();
        for (int a = lane; a < na; a += WAVE) {
            const int p = T.pend[a];
            if (p >= 0) T.ckey[p] = T.gain[a];
        }
        wave_sync();
        for (int c0 = 0; c0 < np0; c0 += WAVE) {
            const int p = c0 + lane;
            for (;;) {
                bool moved = false;
                if (p < np0 && !T.ccommit[p] && T.ckey[p] == INFINITY) {
                    const int o = T.corigin[p];
                    const float kq = o >= 0 ? T.ckey[o >> 1] : INFINITY;
                    if (o >= 0 && !T.ccommit[o >> 1] && kq != INFINITY) {
                        T.ckey[p] = fminf(kq, T.cgain[o >> 1][o & 1]);
                        moved = true;
                    }
                }
                wave_sync();
                if (__ballot(moved) == 0) break;
            }
        }
        // the candidates, compacted into (key, index) lists: leaf a is
        // candidate a, child c of split p candidate na + 2 p + c, and only
        // positive keys are listed (a pick needs a positive gain); and the
        // budget's entries: each uncommitted computed split's key, where it
        // adds a leaf to the run-ahead (only positive ones can count)
        int m = 0, mb = 0;
        auto append = [&](bool live, float key, int idx, YABT_LDS float* keys, YABT_LDS int16_t* ids, int& cnt) {
            const uint64_t bal = __ballot(live);
            const int pos = cnt + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                                 __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
            if (live) {
                keys[pos] = key;
                if (ids) ids[pos] = (int16_t)idx;
            }
            cnt += __popcll(bal);
        };
        for (int a0 = 0; a0 < na; a0 += WAVE) {
            const int a = a0 + lane;
            const float g = (a < na && a != best && T.pend[a] < 0) ? T.gain[a] : -INFINITY;
            append(g > 0.0f, g, a, T.ckand, T.cidx, m);
        }
        for (int p0 = 0; p0 < np0; p0 += WAVE) {
            const int p = p0 + lane;
            const bool in = p < np0;
            const float kp = in ? T.ckey[p] : -INFINITY;
            const bool live = in && !T.ccommit[p] && kp != INFINITY;
            append(live && kp > 0.0f, kp, p, T.cbud, nullptr, mb);
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const float kc = (live && T.cpend[p][c] == -1) ? fminf(kp, T.cgain[p][c]) : -INFINITY;
                append(kc > 0.0f, kc, na + 2 * p + c, T.ckand, T.cidx, m);
            }
        }
        wave_sync();
        // take best, then the largest keys (the lowest candidate on ties).
        // Short lists sit in registers, R entries per lane, each candidate
        // packed into 32 bits as its key's top bits (positive floats order as
        // unsigned integers) over its inverted index, so that a pick is one
        // 32-bit wave maximum.  Keys that agree in those bits are picked by
        // index and counted for the budget as equal: that changes which
        // splits a round computes, never the tree (the commits replay the
        // table).  Each lane keeps its best, the budget count is a ballot per
        // register, and lane t keeps the round's split t.
        constexpr int R = 4;
        constexpr uint32_t IDX = (1u << PICK_IDX_BITS) - 1;
        const bool in_regs = m <= R * WAVE && mb <= R * WAVE;
        uint32_t bk[R];   // budget keys, bucketed as the candidates' (0: none)
        uint32_t pc[R];
        uint32_t lb = 0;   // this lane's best packed candidate (0: none)
        auto lane_best = [&]() {
            lb = 0;
#pragma unroll
            for (int r = 0; r < R; ++r) lb = max(lb, pc[r]);
        };
        if (in_regs) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int i = lane + r * WAVE;
                // listed keys and budget entries are > 0
                pc[r] = i < m ? (__float_as_uint(T.ckand[i]) & ~IDX) | (IDX - (uint32_t)T.cidx[i]) : 0u;
                bk[r] = i < mb ? __float_as_uint(T.cbud[i]) & ~IDX : 0u;
            }
            lane_best();
        }
        if (in_regs) {
            // every pick at once: extraction t (the t-th largest candidate
            // after best) and the budget count at its key go to lane t, with
            // no scalar work between extractions; then the stopping rules
            // below, as the one-at-a-time loop applies them
            uint32_t pk = 0;   // lane t: extraction t
            int pe = 0;        // lane t: budget entries >= its key
            // a pick past the candidates or at na + t >= L stops the round
            // whatever its budget count, so those are not extracted
            const int t_end = min(KMAX, min(m, L - na - 1) + 1);
#pragma unroll 1
            for (int t = 1; t < t_end; ++t) {
                const uint32_t top = wave_max_u32_v(lb);
                const uint32_t key = top & ~IDX;
                int e = 0;
#pragma unroll
                for (int r = 0; r < R; ++r) e += __popcll(__ballot(bk[r] != 0u && bk[r] >= key));
                if (lane == t) {
                    pk = top;
                    pe = e;
                }
                if (top != 0u && lb == top) {   // its lane drops it and looks again
#pragma unroll
                    for (int r = 0; r < R; ++r)
                        if (pc[r] == top) pc[r] = 0u;
                    lane_best();
                }
            }
            for (;;) {
                if (np >= A.pend_cap) {
                    status = -5;
                    break;
                }
                if (j > 0 && np + L - na > A.pend_cap - 1) break;
                ++np;
                ++j;
                if (j >= KMAX) break;
                if (__builtin_amdgcn_readlane((int)pk, j) == 0) break;
                // the budget: leaves of the run-ahead when it pops this one
                if (na + __builtin_amdgcn_readlane(pe, j) + j >= L) break;
            }
            my_pick = lane == 0 ? best : (int)(IDX - (pk & IDX));
        } else {
            int cand = best, cpos = -1;
            for (;;) {
                if (np >= A.pend_cap) {
                    status = -5;
                    break;
                }
                if (j > 0 && np + L - na > A.pend_cap - 1) break;
                if (lane == j) my_pick = cand;
                if (cpos >= 0) {   // the list in LDS: taken
                    if (lane == 0) T.ckand[cpos] = -INFINITY;
                    wave_sync();
                }
                ++np;
                ++j;
                if (j >= KMAX) break;
                cpos = wave_list_argmax(T.ckand, T.cidx, m, lane);
                if (cpos < 0) break;
                cand = T.cidx[cpos];
                const float key = T.ckand[cpos];
                int e = 0;
                for (int i = lane; i < mb; i += WAVE) e += T.cbud[i] >= key ? 1 : 0;
                e = wave_sum<int>(e);
                if (na + e + j >= L) break;
            }
        }
    }
    // this round's splits, one per lane
    int64_t tiles = 0, gathered = 0;
    int f = -1, src = -1;
    if (lane < j) {
        src = my_pick < na ? T.src[my_pick] : my_pick - na;
        const int p = np0 + lane;
        const LeafV Lv = leaf_view(A, src, root);
        const int64_t cl = Lv.left[2], c = Lv.tot[2], m = Lv.e - Lv.s;
        const bool build_left = cl <= c - cl;        // the smaller child, ties left (grow.c:355)
        const int64_t built = build_left ? cl : c - cl;
        tiles = m;   // rows for now: tiles once the round's width is known
        gathered = built;
        f = Lv.f;
        Pend P;
        P.f = Lv.f;
        P.b = Lv.b;
        P.build_left = build_left ? 1 : 0;
        P.depth = Lv.depth + 1;
        P.parent_slot = Lv.slot;
        P.new_slot = p + 1;
        P.child_pend[0] = P.child_pend[1] = -1;
        P.child_node[0] = P.child_node[1] = -1;
        P.origin = src;
        P.pad = 0;
        P.src = (Lv.depth == 0) ? nullptr : A.rows + (size_t)(Lv.depth & 1) * A.rows_ld;
        P.dst = A.rows + (size_t)((Lv.depth + 1) & 1) * A.rows_ld;
        P.s = Lv.s;
        P.e = Lv.e;
        P.mid = Lv.s + cl;
        for (int i = 0; i < 3; ++i) {
            P.tot[i] = Lv.tot[i];
            P.left[i] = Lv.left[i];
        }
        P.pad2 = 0;
        P.placed = 0;
        P.pad1 = 0;
        P.child[0].b = P.child[1].b = -1;
        A.pend[p] = P;
        PendSum S;
        S.gain[0] = S.gain[1] = -INFINITY;
        S.child_pend[0] = S.child_pend[1] = -1;
        S.origin = (int16_t)src;
        S.committed = 0;
        A.psum[p] = S;
        st->round_pend[lane] = p;
        // the split's parent split names it (the root's: st->root_pend)
        if (src >= 0) {
            A.pend[src >> 1].child_pend[src & 1] = p;
            A.psum[src >> 1].child_pend[src & 1] = (int16_t)p;
        } else {
            st->root_pend = p;
        }
    }
    // partition tiles: wide when the round moves many rows
    const int ipt = wave_sum<int64_t>(tiles) > PART_WIDE_ROWS ? PART_IPT_WIDE : PART_IPT_NARROW;
    tiles = (tiles + (int64_t)SB * ipt - 1) / ((int64_t)SB * ipt);
    tiles = wave_incl_scan<int64_t>(tiles, lane);
    // gather units: the round's rows over about gather_target units per tile
    const int64_t R = wave_sum<int64_t>(gathered);
    const int64_t per = gather_unit_rows(R, j, (A.F + HFL - 1) / HFL);
    const int units = (int)wave_incl_scan<int64_t>((gathered + per - 1) / per, lane);
    if (lane < j) {
        st->tile_off[lane + 1] = tiles;
        st->unit_off[lane + 1] = units;
    }
    if (A.use_imat) {
        // the children's path: the leaf's path plus its split feature
        for (int i = 0; i < j; ++i) {
            const int si = __shfl(src, i, WAVE), fi = __shfl(f, i, WAVE);
            const uint8_t* pp = si < 0 ? nullptr : A.pend_path + (size_t)(si >> 1) * A.F;
            uint8_t* out = A.pend_path + (size_t)(np0 + i) * A.F;
            for (int c = lane; c < A.F; c += WAVE) out[c] = (c == fi) ? (uint8_t)1 : (pp ? pp[c] : (uint8_t)0);
        }
    }
    const int done = (status < 0 || j == 0) ? 1 : 0;
    if (lane == 0) {
        st->n_nodes = nn;
        st->n_leaves = na;
        st->n_pend = np;
        st->tile_off[0] = 0;
        st->unit_off[0] = 0;
        st->unit_rows = per;
        st->part_ipt = ipt;
        if (status < 0) {
            A.out_status[0] = status;
        } else if (done) {
            A.out_status[0] = nn;
        }
        if (done) {
            A.out_status[1] = st->round + 1;
            A.out_status[2] = np;
        }
        st->done = done;
        st->n_round = done ? 0 : j;
        const int r = st->round + 1;
        st->round = r;
        // the host's view: round and done in one store
        volatile Flags* fl = A.flags;
        fl->word = ((r + 1) << 1) | done;
    }
}

// Adds the bins of feature f (4 per lane) of slots r_begin, r_begin + step,
// ... <= r_end of `base` into g4, h4, c4, two slots' loads in flight.
__device__ __forceinline__ void add_slots(const int64_t* base, int F, int f, int lane, int r_begin, int r_end, int step,
                                          int64_t g4[4], int64_t h4[4], int64_t c4[4], bool has_h) {
    const size_t se = slot_elems(F);
    int r = r_begin;
    for (; r + step <= r_end; r += 2 * step) {
        int64_t ag[4], ah[4], ac[4], bg[4], bh[4], bc[4];
        load_bins(base + (size_t)r * se, F, f, lane, ag, ah, ac, has_h);
        load_bins(base + (size_t)(r + step) * se, F, f, lane, bg, bh, bc, has_h);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            g4[i] += ag[i] + bg[i];
            h4[i] += ah[i] + bh[i];
            c4[i] += ac[i] + bc[i];
        }
    }
    if (r <= r_end) {
        int64_t ag[4], ah[4], ac[4];
        load_bins(base + (size_t)r * se, F, f, lane, ag, ah, ac, has_h);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            g4[i] += ag[i];
            h4[i] += ah[i];
            c4[i] += ac[i];
        }
    }
}

// LDS of a split round's scan block: the exchange of the built child's
// piece sums, 12 words per lane per wave (the controller's table reuses it).
constexpr size_t SCAN_XCHG_BYTES = (size_t)(CT / WAVE) * 12 * WAVE * sizeof(int64_t);

// Scan launch: SCAN_FEATS features per block and, for a split round, block y
// scans both children of the round's split y (wave w: feature w % SCAN_FEATS,
// child w / SCAN_FEATS).  Each block publishes its best record per child;
// the last block to take a ticket is the controller.
template <bool ROOT>
__global__ void __launch_bounds__(ROOT ? SCAN_FEATS * WAVE : CT) k_scan(Args A) {
    constexpr int NT = ROOT ? SCAN_FEATS * WAVE : CT;
    constexpr int NC = ROOT ? 1 : 2;
    State* st = A.st;
    const Quant* q = A.q;
    const int y = ROOT ? 0 : blockIdx.y;
    // the words of State this block needs, loaded before the exit test (y <
    // KMAX indexes them all): the split's Pend index and its gather pieces'
    // range do not wait for the test
    const int32_t done = st->done, nr = ROOT ? 1 : st->n_round;
    const int pidx = ROOT ? 0 : st->round_pend[y];
    const int u0 = ROOT ? 0 : st->unit_off[y], u1 = ROOT ? 0 : st->unit_off[y + 1];
    // one test over all of them (none is negative in a live round), so that
    // they are loaded together rather than after the branch
    if ((done != 0) | (y >= nr) | ((pidx | u0 | u1) < 0)) return;
    // the start of the controller's table, loaded by every block together
    // with its bins (whichever block finishes last is the controller and
    // holds it in registers by then): leaf t and computed split t (a
    // controller loads the entries past the block size itself)
    // Unconditional loads at clamped indices: a load inside a branch is
    // waited for inside it, these stay in flight through the scan.
    int32_t pf_src = 0, pf_node = 0;   // origin and node id of leaf t
    PendSum pf_ps = {};
    if (!ROOT) {
        const int nl_now = st->n_leaves, np_now = st->n_pend;
        const int tl = min((int)threadIdx.x, max(nl_now - 1, 0)), tp = min((int)threadIdx.x, max(np_now - 1, 0));
        pf_src = A.leaf_src[tl];
        pf_node = A.leaf_node[tl];
        pf_ps = A.psum[tp];
    }
    const bool derive = q->const_h != 0;
    const int64_t hqc = q->hq_const;
    const Pend* P = ROOT ? nullptr : A.pend + pidx;
    const int bl = ROOT ? 1 : P->build_left;
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    const int f = blockIdx.x * SCAN_FEATS + (w % SCAN_FEATS);
    const int c = w / SCAN_FEATS;
    const bool fok = f < A.F;
    const int fc = min(f, A.F - 1);
    const int nb_f = A.nbins[fc];
    const uint8_t use_f = A.fmask[fc];
    const int d_f = A.dflt ? A.dflt[fc] : -1;
    const int nb = fok ? max(0, min(NB, nb_f)) : 0;
    const bool use = fok && use_f != 0;
    const int d = fok ? d_f : -1;
    const ScanParams sp = {(double)A.lam, (double)A.gamma, (double)A.mcw, A.msl};
    const bool has_h = !derive;
    const bool built = ROOT || (c == 0) == (bl != 0);
    int64_t* hp = A.hist + (size_t)(ROOT ? 0 : P->parent_slot) * slot_elems(A.F);
    int64_t* hn = A.hist + (size_t)(ROOT ? 0 : P->new_slot) * slot_elems(A.F);
    __shared__ ScanRec s_rec[NT / WAVE];
    __shared__ int s_last;
    extern __shared__ __align__(16) char s_table[];
    int64_t g4[4], h4[4], c4[4];
    int64_t pg[4], ph[4], pc[4];   // the sibling's wave: the parent's bins
    if (ROOT) {
        if (fok) load_bins(hn, A.F, f, lane, g4, h4, c4, has_h);
    } else {
        // the built child: the sum of its gather pieces, the two waves of a
        // feature adding alternate pieces and exchanging their sums in LDS;
        // the sibling's wave loads the parent's bins meanwhile.  A wave's
        // first two pieces go out before the Pend entry is read (their range
        // needs only State), the parent's bins once it is.
        const size_t se = slot_elems(A.F);
        const int r0 = u0 + c;
        const bool la = fok && r0 < u1, lb = fok && r0 + 2 < u1;
        int64_t ag[4], ah[4], ac[4], bg[4], bh[4], bc[4];
        if (la) load_bins(A.pieces + (size_t)r0 * se, A.F, f, lane, ag, ah, ac, has_h);
        if (lb) load_bins(A.pieces + (size_t)(r0 + 2) * se, A.F, f, lane, bg, bh, bc, has_h);
        if (fok && !built) load_bins(hp, A.F, f, lane, pg, ph, pc, has_h);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            g4[i] = (la ? ag[i] : 0) + (lb ? bg[i] : 0);
            h4[i] = (la ? ah[i] : 0) + (lb ? bh[i] : 0);
            c4[i] = (la ? ac[i] : 0) + (lb ? bc[i] : 0);
        }
        if (fok) add_slots(A.pieces, A.F, f, lane, r0 + 4, u1 - 1, 2, g4, h4, c4, has_h);
        YABT_LDS int64_t* xs = (YABT_LDS int64_t*)s_table;   // [wave][12][lane]
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            xs[(w * 12 + i) * WAVE + lane] = g4[i];
            xs[(w * 12 + 4 + i) * WAVE + lane] = h4[i];
            xs[(w * 12 + 8 + i) * WAVE + lane] = c4[i];
        }
        __syncthreads();
        const int wp = (w + SCAN_FEATS) % (2 * SCAN_FEATS);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            g4[i] += xs[(wp * 12 + i) * WAVE + lane];
            h4[i] += xs[(wp * 12 + 4 + i) * WAVE + lane];
            c4[i] += xs[(wp * 12 + 8 + i) * WAVE + lane];
        }
    }
    if (fok) {
        int64_t tot[3];
        if (ROOT) {
            tot[0] = q->tot_g;
            tot[1] = derive ? A.n * hqc : q->tot_h;
            tot[2] = A.n;
        } else {
            for (int i = 0; i < 3; ++i) tot[i] = bl ? P->left[i] : P->tot[i] - P->left[i];
        }
        fill_default(g4, h4, c4, d, tot, has_h, lane);
        if (!built) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                g4[i] = pg[i] - g4[i];
                h4[i] = ph[i] - h4[i];
                c4[i] = pc[i] - c4[i];
            }
        }
        int64_t hs[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) hs[i] = derive ? c4[i] * hqc : h4[i];
        const float bo = (!ROOT && A.use_imat && use)
                             ? path_boost(A.pend_path + (size_t)pidx * A.F, A.imat, A.ib, A.F, f, lane)
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
            publish_record(&A.rec[((size_t)y * 2 + cc) * gridDim.x + blockIdx.x], s_rec[bi]);
        }
        record_published();
        // two levels of tickets, so no one address takes every block's
        // atomic: the last block of split y takes the launch's ticket
        const bool sl = atomicAdd(&st->split_ticket[y], 1u) == gridDim.x - 1;
        if (sl) st->split_ticket[y] = 0;
        s_last = sl;   // for now: the last of split y
    }
    __syncthreads();
    if (!ROOT) {
        // the last block of split y reduces the split's records: wave c the
        // best over the launch's blocks for child c, into the Pend entry and
        // its table gain (depth cap applied), published for the controller
        // before this block takes the launch's ticket
        const bool sl = s_last != 0;
        if (sl && w < 2) {
            const ScanRec r = wave_best_record_agent(A.rec + ((size_t)y * 2 + w) * gridDim.x, gridDim.x, lane);
            if (lane == 0) {
                Pend* Pw = A.pend + pidx;
                publish_record(&Pw->child[w], r);
                __hip_atomic_store(&A.psum[pidx].gain[w], rec_gain(r, P->depth >= A.max_depth), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
                record_published();
            }
        }
        __syncthreads();
        if (threadIdx.x == 0) s_last = sl && atomicAdd(&st->scan_ticket, 1u) == (uint32_t)nr - 1;
        __syncthreads();
    } else if (threadIdx.x == 0) {
        s_last = s_last && atomicAdd(&st->scan_ticket, 1u) == 0u;
    }
    if (ROOT) __syncthreads();
    const bool last = s_last != 0;
    if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    // every wave of the block has loaded its bins (barriers above): store
    if (fok) {
        if (ROOT) {
            if (d >= 0 && (d >> 2) == lane) store_bins(hn, A.F, f, lane, g4, h4, c4, has_h);
        } else if (built) {
            store_bins(hn, A.F, f, lane, g4, h4, c4, has_h);
        } else {
            store_bins(hp, A.F, f, lane, g4, h4, c4, has_h);
        }
    }
    if (!last) return;
    if (threadIdx.x == 0) st->scan_ticket = 0;

    // ---- controller ----
    Table T;
    table_carve(s_table, A.max_leaves, A.pend_cap, &T);
    if (ROOT) {
        __shared__ ScanRec s_root;
        if (w != 0) return;
        const ScanRec r = wave_best_record(A.rec, gridDim.x, lane);
        if (lane == 0) {
            s_root = r;
            int64_t tot[3] = {q->tot_g, derive ? A.n * hqc : q->tot_h, A.n};
            A.value[0] = node_value(tot, q, A.lr, A.lam);
            T.gain[0] = rec_gain(r, 0 >= A.max_depth);
            T.pend[0] = -1;
            T.src[0] = -1;
            T.node[0] = 0;
            *T.root_gain = T.gain[0];
            *T.root_pend = -1;
            st->root_gain = T.gain[0];
        }
        wave_sync();
        control(A, T, 1, 1, 0, &s_root, lane);
    } else {
        // the round's children: their records and table gains, reduced and
        // published by each split's last scan block
        const int nn = st->n_nodes, na = st->n_leaves, np = st->n_pend;
        const int p0 = np - nr;                   // this round's splits: p0 .. np - 1
        if (threadIdx.x < 2 * nr) {
            const int p = p0 + threadIdx.x / 2, c = threadIdx.x & 1;
            T.cgain[p][c] = __hip_atomic_load(&A.psum[p].gain[c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        auto put = [&](int p, const PendSum& S) {
            if (p < p0) {
                T.cgain[p][0] = S.gain[0];
                T.cgain[p][1] = S.gain[1];
            }
            T.cpend[p][0] = S.child_pend[0];
            T.cpend[p][1] = S.child_pend[1];
            T.corigin[p] = S.origin;
            T.ccommit[p] = (uint8_t)S.committed;
        };
        if (threadIdx.x < na) {
            T.src[threadIdx.x] = (int16_t)pf_src;
            T.node[threadIdx.x] = (int16_t)pf_node;
        }
        if (threadIdx.x < np) put(threadIdx.x, pf_ps);
        for (int a = threadIdx.x + NT; a < na; a += NT) {
            T.src[a] = (int16_t)A.leaf_src[a];
            T.node[a] = (int16_t)A.leaf_node[a];
        }
        for (int p = threadIdx.x + NT; p < np; p += NT) put(p, A.psum[p]);
        if (threadIdx.x == 0) {
            *T.root_gain = st->root_gain;
            *T.root_pend = st->root_pend;
        }
        __syncthreads();
        // the committed leaves' gains and computed splits, from their origins
        for (int a = threadIdx.x; a < na; a += NT) {
            T.gain[a] = gain_of(T, T.src[a]);
            T.pend[a] = (int16_t)pend_of(T, T.src[a]);
        }
        __syncthreads();
        if (w != 0) return;
        control(A, T, nn, na, np, nullptr, lane);
    }
}

// Leaf-id planning, one block: run 2 p + c is child c of computed split p --
// empty when that child has a computed split of its own, else labelled with
// the child's node id when the split is committed, or with the node id of
// the final leaf above the split (found by walking up the uncommitted splits
// to the committed node they hang from); with the root alone, one run of the
// identity.  Each run is numbered with its first chunk of LEAF_CHUNK rows.
// The run and chunk counts follow the max_runs = 2 pend_cap + 1 entries of
// leaf_chunk0.
__global__ void __launch_bounds__(LEAF_PLAN) k_leaf_plan(Args A, int64_t n) {
    __shared__ int32_t s_cnt[LEAF_PLAN / WAVE + 1];
    LeafRun* runs = A.leaf_runs;
    int32_t* chunk0 = A.leaf_chunk0;
    int32_t* counts = chunk0 + 2 * A.pend_cap + 1;
    const int np = A.st->n_pend;
    const int st0 = A.out_status[0];
    if (st0 < 1 || st0 == 1 || np == 0) {
        if (threadIdx.x == 0) {
            const bool root = st0 >= 1;
            LeafRun r;
            r.rows = nullptr;
            r.lo = 0;
            r.hi = root ? n : 0;
            r.label = 0;
            runs[0] = r;
            chunk0[0] = 0;
            counts[0] = root ? 1 : 0;
            counts[1] = root ? (int32_t)((n + LEAF_CHUNK - 1) / LEAF_CHUNK) : 0;
        }
        return;
    }
    // thread t owns the runs of splits [t per, (t + 1) per): chunk offsets in
    // thread order are then in run order
    const int per = (np + LEAF_PLAN - 1) / LEAF_PLAN;
    const int p_lo = (int)threadIdx.x * per, p_hi = min(np, p_lo + per);
    int mine = 0;
    for (int p = p_lo; p < p_hi; ++p) {
        const Pend& P = A.pend[p];
        const int32_t cp0 = P.child_pend[0], cp1 = P.child_pend[1];
        const int64_t ps = P.s, pm = P.mid, pe = P.e;
        if (cp0 < 0) mine += (int)((pm - ps + LEAF_CHUNK - 1) / LEAF_CHUNK);
        if (cp1 < 0) mine += (int)((pe - pm + LEAF_CHUNK - 1) / LEAF_CHUNK);
    }
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    const int incl = wave_incl_scan<int>(mine, lane);
    if (lane == WAVE - 1) s_cnt[w] = incl;
    __syncthreads();
    if (threadIdx.x == 0) {
        int acc = 0;
        for (int t = 0; t < LEAF_PLAN / WAVE; ++t) {
            const int v = s_cnt[t];
            s_cnt[t] = acc;
            acc += v;
        }
        s_cnt[LEAF_PLAN / WAVE] = acc;
    }
    __syncthreads();
    int at = s_cnt[w] + incl - mine;
    for (int p = p_lo; p < p_hi; ++p) {
        const Pend& P = A.pend[p];
        const int32_t cn0 = P.child_node[0], cn1 = P.child_node[1];
        const int32_t cp0 = P.child_pend[0], cp1 = P.child_pend[1];
        const int64_t ps = P.s, pm = P.mid, pe = P.e;
        const uint32_t* const dst = P.dst;
        const bool committed = cn0 >= 0;
        int64_t owner = -1;
        if (!committed && (cp0 < 0 || cp1 < 0)) {
            int src = P.origin;
            for (;;) {
                if (src < 0) {
                    owner = 0;
                    break;
                }
                const Pend& Q = A.pend[src >> 1];
                if (Q.child_node[0] >= 0) {
                    owner = Q.child_node[src & 1];
                    break;
                }
                src = Q.origin;
            }
        }
        for (int c = 0; c < 2; ++c) {
            const bool run = (c ? cp1 : cp0) < 0;
            LeafRun r;
            r.rows = dst;
            r.lo = c ? pm : ps;
            r.hi = run ? (c ? pe : pm) : r.lo;
            r.label = committed ? (c ? cn1 : cn0) : owner;
            runs[2 * p + c] = r;
            chunk0[2 * p + c] = at;
            at += (int)((r.hi - r.lo + LEAF_CHUNK - 1) / LEAF_CHUNK);
        }
    }
    if (threadIdx.x == 0) {
        counts[0] = 2 * np;
        counts[1] = min(s_cnt[LEAF_PLAN / WAVE], A.leaf_chunk_cap);
    }
}

// out[row] = leaf node id, one chunk per block (blocks past the chunk count
// exit): the block's run is the last with chunk0 <= its chunk (binary
// search); each thread loads its rows' ids eight at a time before storing.
__global__ void __launch_bounds__(SB) k_leaf_ids(const LeafRun* runs, const int32_t* chunk0, int max_runs,
                                                 int64_t* out) {
    const int nruns = chunk0[max_runs], total = chunk0[max_runs + 1];
    const int b = (int)blockIdx.x;
    if (b >= total || nruns < 1 || nruns > max_runs) return;
    int lo = 0, hi = nruns - 1;   // last run with chunk0 <= b
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (chunk0[mid] <= b) lo = mid;
        else hi = mid - 1;
    }
    const LeafRun r = runs[lo];
    const int64_t c_lo = r.lo + (int64_t)(b - chunk0[lo]) * LEAF_CHUNK;
    const int64_t c_hi = min(r.hi, c_lo + LEAF_CHUNK);
    constexpr int U = 8;
    for (int64_t i0 = c_lo + threadIdx.x; i0 < c_hi; i0 += (int64_t)SB * U) {
        uint32_t rw[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t i = i0 + (int64_t)u * SB;
            rw[u] = i < c_hi ? (r.rows ? r.rows[i] : (uint32_t)i) : 0u;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t i = i0 + (int64_t)u * SB;
            if (i < c_hi) out[rw[u]] = r.label;
        }
    }
}

size_t carve(char* base, int64_t n, int F, int max_leaves, Args* A) {
    Carve c{base, 0};
    const size_t N = (size_t)(2 * max_leaves + 1);
    const int pend_cap = PEND_PER_LEAF * max_leaves + KMAX;
    Args tmp;
    Args& a = A ? *A : tmp;
    a.pend_cap = pend_cap;
    a.rows_ld = ((n > 0 ? n : 1) + 63) / 64 * 64;
    a.st = c.take<State>(1);
    a.q = c.take<Quant>(1);
    a.rows = c.take<uint32_t>((size_t)2 * (size_t)a.rows_ld);
    a.gh = c.take<float2>((size_t)(n > 0 ? n : 1));
    a.hist = c.take<int64_t>((size_t)(pend_cap + 1) * 3 * (size_t)F * NB);
    a.pieces = c.take<int64_t>((size_t)gather_units((F + HFL - 1) / HFL) * 3 * (size_t)F * NB);
    a.pend_path = c.take<uint8_t>((size_t)pend_cap * (size_t)F);
    a.leaf_src = c.take<int32_t>(N);
    a.leaf_node = c.take<int32_t>(N);
    a.pend = c.take<Pend>((size_t)pend_cap);
    a.psum = c.take<PendSum>((size_t)pend_cap);
    a.rec = c.take<ScanRec>((size_t)KMAX * 2 * ((F + SCAN_FEATS - 1) / SCAN_FEATS));
    // chunks: every run is at most one chunk longer than its rows need
    a.leaf_chunk_cap = (int)((n + LEAF_CHUNK - 1) / LEAF_CHUNK + 2 * (int64_t)pend_cap + 2);
    a.leaf_runs = c.take<LeafRun>((size_t)2 * pend_cap + 1);
    a.leaf_chunk0 = c.take<int32_t>((size_t)2 * pend_cap + 3);
    return align_up(c.off, 256);
}

}  // namespace rnd
}  // namespace yabt

using namespace yabt;
using namespace yabt::rnd;

extern "C" {

size_t yabt_grow_batched_workspace_bytes(int64_t n, int F, int max_leaves) {
    if (n < 0 || n > 0xFFFFFFFFll || F < 1 || max_leaves < 1 || max_leaves > MAX_LEAVES) return 0;
    return carve(nullptr, n, F, max_leaves, nullptr);
}

int yabt_grow_batched(const uint8_t* bins_fm, int64_t ld_fm, const uint8_t* bins_rm, int64_t ld_rm,
                      const float* grad, const float* hess, const uint8_t* fmask, const float* imat, float ib,
                      int use_imat, const int32_t* nbins, const int32_t* default_bin, const uint32_t* bin_counts,
                      int64_t n, int F, float lam, float gamma, float mcw, int msl, float lr, int max_leaves,
                      int max_depth, void* workspace,
                      size_t workspace_bytes, int64_t* out_feature, int64_t* out_thr_bin, int64_t* out_left,
                      int64_t* out_right, float* out_value, int64_t* out_depth, int64_t* out_leaf_of_row,
                      int32_t* out_status, hipStream_t stream) {
    if (F < 1 || n < 0 || n > 0xFFFFFFFFll || max_leaves < 1 || max_leaves > MAX_LEAVES)
        return fail(-2, "yabt_grow_batched: bad sizes (need F >= 1, 0 <= n < 2^32, 1 <= max_leaves <= 1024)");
    if (ld_fm < n || ld_fm % 16 || ld_rm < F || ld_rm % 16)
        return fail(-2, "yabt_grow_batched: leading dimensions must be multiples of 16 covering n (bins_fm) and F "
                        "(bins_rm)");
    if (!bins_fm || !bins_rm || !grad || !hess || !fmask || !nbins || (use_imat && !imat) || !workspace ||
        !out_feature || !out_thr_bin || !out_left || !out_right || !out_value || !out_depth || !out_status)
        return fail(-2, "yabt_grow_batched: null pointer argument");
    if (!aligned16(bins_fm) || !aligned16(bins_rm) || !aligned16(grad) || !aligned16(hess))
        return fail(-2, "yabt_grow_batched: bins, grad and hess must be 16-byte aligned");
    Args A;
    memset(&A, 0, sizeof A);
    const size_t need = carve((char*)workspace, n, F, max_leaves, &A);
    if (workspace_bytes < need) return fail(-2, "yabt_grow_batched: workspace too small");
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

    // the mapped flags come from the library's pinned pool; every return waits
    // for the stream before the buffer goes back: enqueued controllers write
    // the flags until the last of them has run
    struct Held {
        PinnedHold hold;
        hipStream_t s;
        ~Held() {
            if (hold.p) (void)hipStreamSynchronize(s);
        }
    } held;
    held.s = stream;
    if (int prc = held.hold.take(sizeof(Flags), hipHostMallocMapped | hipHostMallocCoherent)) return prc;
    Flags* h_flags = static_cast<Flags*>(held.hold.p);
    h_flags->word = 0;
    const hipError_t he = hipHostGetDevicePointer((void**)&A.flags, h_flags, 0);
    if (he != hipSuccess) return hip_fail(he, "yabt_grow_batched: mapped flags");

    const int tiles = (F + HFL - 1) / HFL;
    k_quant_clear<<<1, 1, 0, stream>>>(A.q);
    k_setup<<<launch_grid(n, SB * 16, 1024), SB, 0, stream>>>(A);
    launch_quant_resid(stream, grad, hess, n, A.q);
    k_setup_finish<<<1, 1, 0, stream>>>(A);
    launch_hist_root(stream, bins_fm, ld_fm, grad, hess, n, F, A.q, 0.0, 0.0, 0, A.dflt, A.counts, A.q, A.hist, 1,
                     &A.st->done);
    const int scan_grid = (F + SCAN_FEATS - 1) / SCAN_FEATS;
    const size_t table_lds = table_carve(nullptr, max_leaves, A.pend_cap, nullptr);
    k_scan<true><<<scan_grid, SCAN_FEATS * WAVE, table_lds, stream>>>(A);
    const size_t scan_lds = table_lds > SCAN_XCHG_BYTES ? table_lds : SCAN_XCHG_BYTES;
    int lrc = launch_status("yabt_grow_batched launch");
    if (lrc) return lrc;
    // rounds: at most max_leaves - 1 (one split each); the controller of round
    // r stamps r + 1 into the flags word, so round r may be enqueued once
    // round r - LOOKAHEAD has finished
    volatile Flags* fl = h_flags;
    auto ready = [&](int r) {   // done, or round r - LOOKAHEAD finished
        const int32_t w = fl->word;
        return (w & 1) || (w >> 1) - 1 >= r - LOOKAHEAD;
    };
    for (int r = 1; r < max_leaves; ++r) {
        for (SpinWait sw;;) {
            if (ready(r)) break;
            if (sw.stream_check()) {
                const hipError_t e = hipStreamQuery(stream);
                if (e == hipSuccess) {
                    if (ready(r)) break;
                    return fail(-4, "yabt_grow_batched: stream finished without the round's result");
                }
                if (e != hipErrorNotReady) return hip_fail(e, "yabt_grow_batched: round");
            }
        }
        if (fl->word & 1) break;
        k_part<<<PART_BLOCKS, SB, 0, stream>>>(bins_fm, ld_fm, n, A.st, A.pend);
        k_gather<<<tiles * gather_units(tiles), HBLOCK, 0, stream>>>(bins_rm, ld_rm, grad, hess, A.gh, F, A.q, A.dflt,
                                                                         A.st, A.pend, A.pieces);
        k_scan<false><<<dim3(scan_grid, KMAX), CT, scan_lds, stream>>>(A);
        if ((lrc = launch_status("yabt_grow_batched launch"))) return lrc;
    }
    if (out_leaf_of_row && n > 0) {
        k_leaf_plan<<<1, LEAF_PLAN, 0, stream>>>(A, n);
        k_leaf_ids<<<A.leaf_chunk_cap, SB, 0, stream>>>(A.leaf_runs, A.leaf_chunk0, 2 * A.pend_cap + 1,
                                                        out_leaf_of_row);
    }
    if ((lrc = launch_status("yabt_grow_batched launch"))) return lrc;
    const hipError_t e = hipStreamSynchronize(stream);
    if (e != hipSuccess) return hip_fail(e, "yabt_grow_batched: synchronisation");
    // every round commits at least one split, so max_leaves - 1 rounds finish
    // any tree
    if (!(fl->word & 1)) return fail(-4, "yabt_grow_batched: tree not finished after max_leaves - 1 rounds");
    return 0;
}

}  // extern "C"
