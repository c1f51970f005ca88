// Level-batched growth with best-first results on gfx950.
//
// cgrow (yabt/_cgrow/grow.c:321-408) splits, best leaf first, until no leaf
// has a positive fp32 gain or the leaf budget is reached.  When the budget
// cannot bind -- max_leaves >= 2^max_depth, the depth-wise workloads -- every
// node above the depth cap with a positive gain is split whatever the order,
// and a node's best split depends only on its rows and on the features of its
// ancestors (the interaction boost).  So all nodes of one depth are grown
// together: one routing pass over the rows, one histogram pass for the smaller
// child of every split (counting sort of the rows by child, then per-child
// runs), in-place sibling subtraction, one scan launch for every node of the
// new depth.  The tree is then numbered as cgrow numbers it -- by replaying its
// leaf table (left child replaces the split slot, right child appended,
// first maximum of the fp32 gains above 0) over the computed gains, on the
// host -- so the node arrays, values and leaf ids are those of yabt_grow bit
// for bit (same fixed-point sums, same scan).
//
// Per depth the host reads the new nodes' records (one small copy and one
// stream synchronisation) and writes the next depth's routing table.

#include "common.h"
#include "hist.h"
#include "host.h"
#include "scan.h"
#include "yabt_hip.h"

#include <math.h>
#include <string.h>

#include <vector>

namespace yabt {
namespace lvl {

constexpr int LB = 256;             // threads of the row / scan kernels
constexpr int LROWS = 4096;         // rows per counting / scatter block
constexpr int LCHUNK = 8192;        // sorted rows per histogram block
constexpr int LSCAN = 4;            // features per scan block (one wave each)
constexpr int LDS_SLOTS = 4096;     // child counters kept in LDS up to this many
constexpr int MAX_DEPTH = 16;

struct LNode {                      // a node in breadth-first (provisional) order
    double gain;                    // true gain of its best split, -inf if none
    int32_t f, b;                   // best split, b = -1: none
    int64_t tot[3];                 // totals: sum q(g), sum q(h), rows
    int64_t left[3];                // totals of bins <= b of f
    float value;
    int32_t depth;
};

struct Route {                      // what a node's rows do at the current depth
    int32_t f, b;                   // f = -1: the node is not split
    int32_t left, right;            // children (provisional ids)
    int32_t built_left, built_right;  // index of the child among the built ones, -1: not built
};

struct Ws {
    Quant* q;
    int32_t* row_node;              // (n) provisional node of each row
    int32_t* row_built;             // (n) built-child index of each row's new node, -1: none
    uint32_t* sorted;               // (n) rows sorted by built child
    uint32_t* count;                // (P) rows per built child
    int64_t* off;                   // (P + 1)
    unsigned long long* cursor;     // (P)
    LNode* nodes;                   // (NP)
    Route* route;                   // (NP)
    uint8_t* path;                  // (NP, F)
    int32_t* built_slot;            // (P) slot of each built child
    int32_t* scan_list;             // (2P) nodes scanned at this depth, then their slots
    int32_t* pairs;                 // (2P) (parent slot, built slot) for the subtraction
    int32_t* remap;                 // (NP) final node id
    ScanRec* rec;                   // (P, scan blocks)
    int64_t* hist;                  // (P, 3, F, 256)
    size_t bytes;
};

inline int pool_slots(int max_depth) { return 1 << (max_depth > 0 ? max_depth - 1 : 0); }

Ws carve(char* base, int64_t n, int F, int max_leaves, int max_depth) {
    Carve c{base, 0};
    Ws w;
    const int64_t nn = n > 0 ? n : 1;
    const size_t NP = 2 * (size_t)max_leaves + 1;
    const size_t P = (size_t)pool_slots(max_depth);
    const size_t sblk = (size_t)(F + LSCAN - 1) / LSCAN;
    w.q = c.take<Quant>(1);
    w.row_node = c.take<int32_t>(nn);
    w.row_built = c.take<int32_t>(nn);
    w.sorted = c.take<uint32_t>(nn);
    w.count = c.take<uint32_t>(P);
    w.off = c.take<int64_t>(P + 1);
    w.cursor = c.take<unsigned long long>(P);
    w.nodes = c.take<LNode>(NP);
    w.route = c.take<Route>(NP);
    w.path = c.take<uint8_t>(NP * (size_t)F);
    w.built_slot = c.take<int32_t>(P);
    w.scan_list = c.take<int32_t>(2 * P);
    w.pairs = c.take<int32_t>(2 * P);
    w.remap = c.take<int32_t>(NP);
    w.rec = c.take<ScanRec>(P * sblk);
    w.hist = c.take<int64_t>(P * 3 * (size_t)F * NB);
    w.bytes = align_up(c.off, 256);
    return w;
}

// ---------------------------------------------------------------------------
// setup
// ---------------------------------------------------------------------------

__global__ void __launch_bounds__(LB) k_setup(const float* grad, const float* hess, int64_t n, Quant* q,
                                              int32_t* row_node, Route* route, int NP, uint8_t* path, int64_t path_n,
                                              int64_t* slot0, int64_t slot_n) {
    quant_reduce<LB>(grad, hess, n, q);
    const int64_t tid = (int64_t)blockIdx.x * LB + threadIdx.x, stride = (int64_t)gridDim.x * LB;
    for (int64_t i = tid; i < n; i += stride) row_node[i] = 0;
    for (int64_t i = tid; i < NP; i += stride) {
        route[i].f = -1;
        route[i].built_left = route[i].built_right = -1;
    }
    for (int64_t i = tid; i < path_n; i += stride) path[i] = 0;
    for (int64_t i = tid; i < slot_n; i += stride) slot0[i] = 0;
}

__global__ void k_setup_finish(Quant* q, int64_t n, LNode* nodes, int32_t* scan_list, int32_t* status) {
    LNode& r = nodes[0];
    r.tot[0] = q->tot_g;
    r.tot[1] = 0;
    r.tot[2] = n;
    r.depth = 0;
    r.f = -1;
    r.b = -1;
    r.gain = -INFINITY;
    scan_list[0] = 0;      // the root, slot 0
    scan_list[1] = 0;
    status[0] = q->nonfinite ? -1 : 0;
}

// The root's h total once the histogram pass has added it.
__global__ void k_root_tot(const Quant* q, int64_t n, LNode* nodes) {
    nodes[0].tot[0] = q->tot_g;
    nodes[0].tot[1] = q->const_h ? n * q->hq_const : q->tot_h;
}

// ---------------------------------------------------------------------------
// one depth: children, routing, histograms of the built children, siblings
// ---------------------------------------------------------------------------

// Children totals and paths of the split nodes [id0, id0 + m) (one block each).
__global__ void __launch_bounds__(LB) k_children(LNode* nodes, const Route* route, uint8_t* path, int F, int id0) {
    const int k = id0 + blockIdx.x;
    const Route R = route[k];
    if (R.f < 0) return;
    const LNode& p = nodes[k];
    if (threadIdx.x == 0) {
        LNode& l = nodes[R.left];
        LNode& r = nodes[R.right];
        for (int i = 0; i < 3; ++i) {
            l.tot[i] = p.left[i];
            r.tot[i] = p.tot[i] - p.left[i];
        }
        l.depth = r.depth = p.depth + 1;
        l.f = r.f = -1;
        l.b = r.b = -1;
        l.gain = r.gain = -INFINITY;
    }
    for (int j = threadIdx.x; j < F; j += LB) {
        const uint8_t v = (uint8_t)(path[(size_t)k * F + j] | (j == R.f ? 1 : 0));
        path[(size_t)R.left * F + j] = v;
        path[(size_t)R.right * F + j] = v;
    }
}

// Each row follows its node's split; rows of a built child record its index.
__global__ void __launch_bounds__(LB) k_route(const uint8_t* __restrict__ bins_fm, int64_t ld, int64_t n,
                                              int32_t* __restrict__ row_node, int32_t* __restrict__ row_built,
                                              const Route* __restrict__ route) {
    for (int64_t i = (int64_t)blockIdx.x * LB + threadIdx.x; i < n; i += (int64_t)gridDim.x * LB) {
        const int32_t k = row_node[i];
        const Route R = route[k];
        int32_t bi = -1;
        if (R.f >= 0) {
            const bool gl = (int)bins_fm[(size_t)R.f * ld + i] <= R.b;
            row_node[i] = gl ? R.left : R.right;
            bi = gl ? R.built_left : R.built_right;
        }
        row_built[i] = bi;
    }
}

template <bool LDS>
__global__ void __launch_bounds__(LB) k_count(const int32_t* __restrict__ row_built, int64_t n, int K,
                                              uint32_t* __restrict__ count) {
    __shared__ uint32_t s_cnt[LDS ? LDS_SLOTS : 1];
    if (LDS)
        for (int i = threadIdx.x; i < K; i += LB) s_cnt[i] = 0;
    __syncthreads();
    const int64_t lo = (int64_t)blockIdx.x * LROWS, hi = min(n, lo + LROWS);
    for (int64_t i = lo + threadIdx.x; i < hi; i += LB) {
        const int32_t s = row_built[i];
        if (s < 0) continue;
        if (LDS) atomicAdd(&s_cnt[s], 1u);
        else atomicAdd(&count[s], 1u);
    }
    if (LDS) {
        __syncthreads();
        for (int i = threadIdx.x; i < K; i += LB)
            if (s_cnt[i]) atomicAdd(&count[i], s_cnt[i]);
    }
}

__global__ void __launch_bounds__(1024) k_offsets(const uint32_t* count, int K, int64_t* off,
                                                  unsigned long long* cursor) {
    __shared__ int64_t s_wave[1024 / WAVE];
    int64_t carry = 0;
    for (int base = 0; base < K; base += 1024) {
        const int i = base + threadIdx.x;
        const int64_t c = i < K ? (int64_t)count[i] : 0;
        int64_t tot;
        const int64_t ex = block_excl_scan<1024, int64_t>(c, s_wave, &tot);
        if (i < K) {
            off[i] = carry + ex;
            cursor[i] = (unsigned long long)(carry + ex);
        }
        carry += tot;
    }
    if (threadIdx.x == 0) off[K] = carry;
}

template <bool LDS>
__global__ void __launch_bounds__(LB) k_scatter(const int32_t* __restrict__ row_built, int64_t n, int K,
                                                unsigned long long* __restrict__ cursor, uint32_t* __restrict__ sorted) {
    __shared__ uint32_t s_cnt[LDS ? LDS_SLOTS : 1];
    __shared__ unsigned long long s_base[LDS ? LDS_SLOTS : 1];
    const int64_t lo = (int64_t)blockIdx.x * LROWS, hi = min(n, lo + LROWS);
    if (!LDS) {
        for (int64_t i = lo + threadIdx.x; i < hi; i += LB) {
            const int32_t s = row_built[i];
            if (s >= 0) sorted[atomicAdd(&cursor[s], 1ull)] = (uint32_t)i;
        }
        return;
    }
    for (int i = threadIdx.x; i < K; i += LB) s_cnt[i] = 0;
    __syncthreads();
    for (int64_t i = lo + threadIdx.x; i < hi; i += LB) {
        const int32_t s = row_built[i];
        if (s >= 0) atomicAdd(&s_cnt[s], 1u);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < K; i += LB) {
        s_base[i] = s_cnt[i] ? atomicAdd(&cursor[i], (unsigned long long)s_cnt[i]) : 0ull;
        s_cnt[i] = 0;
    }
    __syncthreads();
    for (int64_t i = lo + threadIdx.x; i < hi; i += LB) {
        const int32_t s = row_built[i];
        if (s < 0) continue;
        const uint32_t r = atomicAdd(&s_cnt[s], 1u);
        sorted[s_base[s] + r] = (uint32_t)i;
    }
}

__global__ void __launch_bounds__(LB) k_zero_slots(int64_t* hist, size_t slot_n, const int32_t* built_slot, int K) {
    const int k = blockIdx.y;
    if (k >= K) return;
    int64_t* h = hist + (size_t)built_slot[k] * slot_n;
    for (size_t i = (size_t)blockIdx.x * LB + threadIdx.x; i < slot_n; i += (size_t)gridDim.x * LB) h[i] = 0;
}

struct LvlLds {
    unsigned long long g[NB * HFL];
    unsigned long long h[NB * HFL];
    uint32_t c[NB * HFL];
};

// Block (tile, chunk): the sorted rows [chunk * LCHUNK, +LCHUNK), one built
// child's run at a time, in the lane = feature layout of hist.h (row ids and
// g/h handed to a row group with DPP), flushed into that child's slot.
// HCH false: no h channel (constant hessian; sum q(h) = count * q(h)).
template <bool HCH>
__global__ void __launch_bounds__(HBLOCK) k_hist(const uint8_t* __restrict__ bins_rm, int64_t ldb,
                                                 const float* __restrict__ grad, const float* __restrict__ hess,
                                                 int F, int K, const int64_t* __restrict__ off,
                                                 const uint32_t* __restrict__ sorted, const Quant* q,
                                                 const int32_t* __restrict__ built_slot, int64_t* hist, int chunks) {
    __shared__ LvlLds L;
    const int tile = blockIdx.x / chunks, chunk = blockIdx.x % chunks;
    const int f0 = tile * HFL;
    const int64_t total = off[K];
    const int64_t c0 = (int64_t)chunk * LCHUNK, c1 = min(total, c0 + LCHUNK);
    if (f0 >= F || c0 >= c1) return;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int fl = lane & (HFL - 1), rg = lane / HFL;
    const bool fok = f0 + fl < F;
    const double scg = q->scg, sch = q->sch;
    // lanes of features >= F read feature f0 and add into their own LDS
    // columns, which the flush skips
    const uint8_t* fb = bins_rm + f0 + (fok ? fl : 0);
    int lo = 0, hi = K - 1;                 // child holding position c0: last s with off[s] <= c0
    while (lo < hi) {
        const int mid = (lo + hi + 1) / 2;
        if (off[mid] <= c0) lo = mid;
        else hi = mid - 1;
    }
    const size_t slot_n = (size_t)3 * F * NB, plane = (size_t)F * NB;
    for (int s = lo; s < K && off[s] < c1; ++s) {
        const int64_t a = max(c0, off[s]), b = min(c1, off[s + 1]);
        if (a >= b) continue;                           // uniform across the block
        for (int i = threadIdx.x; i < NB * HFL; i += HBLOCK) {
            L.g[i] = 0;
            if (HCH) L.h[i] = 0;
            L.c[i] = 0;
        }
        __syncthreads();
        for (int64_t i0 = a + (int64_t)wave * WAVE; i0 < b; i0 += HSTEP) {
            uint32_t r = 0;
            uint64_t qg = 0, qh = 0;
            if (i0 + lane < b) {
                r = sorted[i0 + lane];
                qg = (uint64_t)quantise_wide(grad[r], scg);
                if (HCH) qh = (uint64_t)quantise_wide(hess[r], sch);
            }
            const int nv = (int)min((int64_t)HFL, max((int64_t)0, b - (i0 + HFL * rg)));
            uint32_t bj[HFL];
#define YABT_LVL_LOAD(J)                                                         \
            {                                                                    \
                const uint32_t rj = row_bcast32<J>(r);                           \
                bj[J] = ((J) < nv) ? (uint32_t)fb[(size_t)rj * ldb] : 0u;        \
            }
            YABT_LVL_LOAD(0) YABT_LVL_LOAD(1) YABT_LVL_LOAD(2) YABT_LVL_LOAD(3)
            YABT_LVL_LOAD(4) YABT_LVL_LOAD(5) YABT_LVL_LOAD(6) YABT_LVL_LOAD(7)
            YABT_LVL_LOAD(8) YABT_LVL_LOAD(9) YABT_LVL_LOAD(10) YABT_LVL_LOAD(11)
            YABT_LVL_LOAD(12) YABT_LVL_LOAD(13) YABT_LVL_LOAD(14) YABT_LVL_LOAD(15)
#undef YABT_LVL_LOAD
#define YABT_LVL_ADD(J)                                                          \
            {                                                                    \
                const uint64_t g0 = row_bcast64<J>(qg);                          \
                const uint64_t h0 = HCH ? row_bcast64<J>(qh) : 0ull;             \
                if ((J) < nv) {                                                  \
                    const int at = (int)bj[J] * HFL + fl;                        \
                    atomicAdd(&L.g[at], (unsigned long long)g0);                 \
                    if (HCH) atomicAdd(&L.h[at], (unsigned long long)h0);        \
                    atomicAdd(&L.c[at], 1u);                                     \
                }                                                                \
            }
            YABT_LVL_ADD(0) YABT_LVL_ADD(1) YABT_LVL_ADD(2) YABT_LVL_ADD(3)
            YABT_LVL_ADD(4) YABT_LVL_ADD(5) YABT_LVL_ADD(6) YABT_LVL_ADD(7)
            YABT_LVL_ADD(8) YABT_LVL_ADD(9) YABT_LVL_ADD(10) YABT_LVL_ADD(11)
            YABT_LVL_ADD(12) YABT_LVL_ADD(13) YABT_LVL_ADD(14) YABT_LVL_ADD(15)
#undef YABT_LVL_ADD
        }
        __syncthreads();
        int64_t* out = hist + (size_t)built_slot[s] * slot_n;
        for (int i = threadIdx.x; i < NB * HFL; i += HBLOCK) {
            const int fi = f0 + (i % HFL);
            const uint32_t c = L.c[i];
            if (fi >= F || c == 0) continue;
            const size_t at = (size_t)fi * NB + (size_t)(i / HFL);
            atomicAdd((unsigned long long*)(out + at), L.g[i]);
            if (HCH) atomicAdd((unsigned long long*)(out + plane + at), L.h[i]);
            atomicAdd((unsigned long long*)(out + 2 * plane + at), (unsigned long long)c);
        }
        __syncthreads();
    }
}

// hist[parent] -= hist[built]: the parent's slot becomes the sibling's.
__global__ void __launch_bounds__(LB) k_sub(int64_t* hist, size_t slot_n, const int32_t* pairs, int npairs) {
    const int k = blockIdx.y;
    if (k >= npairs) return;
    int64_t* hp = hist + (size_t)pairs[2 * k] * slot_n;
    const int64_t* hb = hist + (size_t)pairs[2 * k + 1] * slot_n;
    for (size_t i = (size_t)blockIdx.x * LB + threadIdx.x; i < slot_n; i += (size_t)gridDim.x * LB) hp[i] -= hb[i];
}

// ---------------------------------------------------------------------------
// scan: one wave per (node, feature), grid (feature blocks, nodes)
// ---------------------------------------------------------------------------

struct ScanArgs {
    const int32_t* nbins;
    const uint8_t* fmask;
    const float* imat;
    float ib;
    int use_imat;
    ScanParams sp;
    int F;
    float lr, lam;
};

__global__ void __launch_bounds__(LSCAN * WAVE) k_scan(ScanArgs S, const Quant* q, const int64_t* hist,
                                                       const int32_t* scan_list, int nscan, const uint8_t* path,
                                                       ScanRec* rec) {
    const int j = blockIdx.y;
    const int node = scan_list[j], slot = scan_list[nscan + j];
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    const int f = blockIdx.x * LSCAN + w;
    const int F = S.F;
    __shared__ ScanRec s_rec[LSCAN];
    const bool derive = q->const_h != 0;
    const int64_t hqc = q->hq_const;
    if (f < F) {
        const int64_t* hs = hist + (size_t)slot * 3 * F * NB;
        int64_t g4[4], h4[4], c4[4];
        load_bins(hs, F, f, lane, g4, h4, c4, !derive);
        int64_t hh[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) hh[i] = derive ? c4[i] * hqc : h4[i];
        const bool use = S.fmask[f] != 0;
        const int nb = max(0, min(NB, S.nbins[f]));
        const float bo = (S.use_imat && use) ? path_boost(path + (size_t)node * F, S.imat, S.ib, F, f, lane) : 1.0f;
        int64_t t256[3];
        ScanRec r = scan_feature(g4, hh, c4, nb, q->ig, q->ih, S.sp, (double)bo, lane, t256);
        if (!use) no_split(r);
        r.f = f;
        if (lane == 0) s_rec[w] = r;
    } else if (lane == 0) {
        no_split(s_rec[w]);
        s_rec[w].f = -1;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int bi = 0;
        for (int i = 1; i < LSCAN; ++i)
            if (rec_beats(s_rec[i].sel, s_rec[i].f, s_rec[i].b, s_rec[bi].sel, s_rec[bi].f, s_rec[bi].b)) bi = i;
        rec[(size_t)j * gridDim.x + blockIdx.x] = s_rec[bi];
    }
}

// One wave per node of the new depth: its best record (scanned nodes) and
// its value (every node, grow.c:371-379).
__global__ void __launch_bounds__(WAVE) k_pick(const ScanRec* rec, int nblk, const int32_t* scan_list, int nscan,
                                               int id0, int nnew, const Quant* q, float lr, float lam, LNode* nodes) {
    const int j = blockIdx.x, lane = threadIdx.x;
    if (j < nscan) {
        const ScanRec r = wave_best_record(rec + (size_t)j * nblk, nblk, lane);
        if (lane == 0) {
            LNode& L = nodes[scan_list[j]];
            L.f = r.b >= 0 ? r.f : -1;
            L.b = r.b;
            L.gain = r.b >= 0 ? r.gain : -INFINITY;
            for (int i = 0; i < 3; ++i) L.left[i] = r.b >= 0 ? r.left[i] : 0;
        }
    }
    if (lane == 0 && j < nnew) {
        LNode& L = nodes[id0 + j];
        const double G = (double)L.tot[0] * q->ig, H = (double)L.tot[1] * q->ih;
        L.value = (float)(-lr * G / (H + lam));
    }
}

// out[row] = final id of the row's leaf.
__global__ void __launch_bounds__(LB) k_leaf_ids(const int32_t* __restrict__ row_node, int64_t n,
                                                 const int32_t* __restrict__ remap, int64_t* __restrict__ out) {
    for (int64_t i = (int64_t)blockIdx.x * LB + threadIdx.x; i < n; i += (int64_t)gridDim.x * LB)
        out[i] = remap[row_node[i]];
}

}  // namespace lvl
}  // namespace yabt

using namespace yabt;
using namespace yabt::lvl;

extern "C" {

size_t yabt_grow_levelwise_workspace_bytes(int64_t n, int F, int max_leaves, int max_depth) {
    if (n < 0 || n > 0x7FFFFFFFll || F < 1 || max_depth < 0 || max_depth > MAX_DEPTH ||
        max_leaves < (1 << max_depth) || max_leaves > 65535)
        return 0;
    return carve(nullptr, n, F, max_leaves, max_depth).bytes;
}

int yabt_grow_levelwise(const uint8_t* bins_fm, int64_t ld_fm, const uint8_t* bins_rm, int64_t ld_rm,
                        const float* grad, const float* hess, const uint8_t* fmask, const float* imat, float ib,
                        int use_imat, const int32_t* nbins, const uint32_t* bin_counts, int64_t n, int F,
                        float lam, float gamma, float mcw,
                        int msl, float lr, int max_leaves, int max_depth, void* workspace, size_t workspace_bytes,
                        int64_t* out_feature, int64_t* out_thr_bin, int64_t* out_left, int64_t* out_right,
                        float* out_value, int64_t* out_depth, int64_t* out_leaf_of_row, int32_t* out_status,
                        hipStream_t stream) {
    if (F < 1 || n < 0 || n > 0x7FFFFFFFll || max_depth < 0 || max_depth > MAX_DEPTH || max_leaves > 65535)
        return fail(-2, "yabt_grow_levelwise: bad sizes (F >= 1, 0 <= n < 2^31, 0 <= max_depth <= 16)");
    if (max_leaves < (1 << max_depth))
        return fail(-3, "yabt_grow_levelwise: needs max_leaves >= 2^max_depth (the leaf budget must not bind)");
    if (ld_fm < n || ld_fm % 16 || ld_rm < F || ld_rm % 16)
        return fail(-2, "yabt_grow_levelwise: leading dimensions must be multiples of 16 covering n and F");
    if (!bins_fm || !bins_rm || !grad || !hess || !fmask || !nbins || (use_imat && !imat) || !workspace ||
        !out_feature || !out_thr_bin || !out_left || !out_right || !out_value || !out_depth || !out_status)
        return fail(-2, "yabt_grow_levelwise: null pointer argument");
    if (!aligned16(bins_fm) || !aligned16(bins_rm) || !aligned16(grad) || !aligned16(hess))
        return fail(-2, "yabt_grow_levelwise: bins, grad and hess must be 16-byte aligned");
    const Ws w = carve((char*)workspace, n, F, max_leaves, max_depth);
    if (workspace_bytes < w.bytes) return fail(-2, "yabt_grow_levelwise: workspace too small");
    const int NP = 2 * max_leaves + 1;
    const int P = pool_slots(max_depth);
    const size_t slot_n = (size_t)3 * F * NB;
    const int sblk = (F + LSCAN - 1) / LSCAN;
    const int tiles = (F + HFL - 1) / HFL;

    // pinned staging for the per-depth records and tables, from the library's
    // pinned pool; every return waits for the stream before it goes back
    struct Held {
        PinnedHold hold;
        hipStream_t s;
        ~Held() {
            if (hold.p) (void)hipStreamSynchronize(s);
        }
    } pin;
    pin.s = stream;
    const size_t rec_bytes = (size_t)NP * sizeof(LNode), tab_bytes = (size_t)NP * sizeof(Route);
    const size_t list_bytes = (size_t)4 * P * sizeof(int32_t) + (size_t)P * sizeof(int32_t);
    if (int prc = pin.hold.take(rec_bytes + tab_bytes + list_bytes + (size_t)NP * sizeof(int32_t),
                                hipHostMallocDefault))
        return prc;
    LNode* h_nodes = (LNode*)pin.hold.p;
    Route* h_route = (Route*)((char*)pin.hold.p + rec_bytes);
    int32_t* h_lists = (int32_t*)((char*)pin.hold.p + rec_bytes + tab_bytes);    // scan_list (2P), pairs (2P), built_slot (P)
    int32_t* h_remap = h_lists + 5 * P;
    int32_t* h_scan = h_lists;
    int32_t* h_pairs = h_lists + 2 * P;
    int32_t* h_built = h_lists + 4 * P;

    auto copy_in = [&](void* dst, const void* src, size_t bytes) -> int {
        const hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream);
        return e == hipSuccess ? 0 : hip_fail(e, "yabt_grow_levelwise: table copy");
    };
    auto fetch = [&](void* dst, const void* src, size_t bytes) -> int {
        hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, stream);
        if (e == hipSuccess) e = hipStreamSynchronize(stream);
        return e == hipSuccess ? 0 : hip_fail(e, "yabt_grow_levelwise: record copy");
    };

    ScanArgs S;
    S.nbins = nbins;
    S.fmask = fmask;
    S.imat = imat;
    S.ib = ib;
    S.use_imat = use_imat ? 1 : 0;
    S.sp = ScanParams{(double)lam, (double)gamma, (double)mcw, msl};
    S.F = F;
    S.lr = lr;
    S.lam = lam;

    // root
    k_quant_clear<<<1, 1, 0, stream>>>(w.q);
    k_setup<<<launch_grid(max(n, (int64_t)slot_n), LB * 16, 1024), LB, 0, stream>>>(
        grad, hess, n, w.q, w.row_node, w.route, NP, w.path, (int64_t)NP * F, w.hist, (int64_t)slot_n);
    launch_quant_resid(stream, grad, hess, n, w.q);
    k_setup_finish<<<1, 1, 0, stream>>>(w.q, n, w.nodes, w.scan_list, out_status);
    if (n > 0) {
        launch_hist_root(stream, bins_fm, ld_fm, grad, hess, n, F, w.q, 0.0, 0.0, 0, nullptr, bin_counts, w.q, w.hist,
                         1, nullptr);
    }
    k_root_tot<<<1, 1, 0, stream>>>(w.q, n, w.nodes);
    if (max_depth > 0) {
        k_scan<<<dim3(sblk, 1), LSCAN * WAVE, 0, stream>>>(S, w.q, w.hist, w.scan_list, 1, w.path, w.rec);
    }
    k_pick<<<1, WAVE, 0, stream>>>(w.rec, sblk, w.scan_list, max_depth > 0 ? 1 : 0, 0, 1, w.q, lr, lam, w.nodes);
    int rc = launch_status("yabt_grow_levelwise launch");
    if (rc) return rc;
    if ((rc = fetch(h_nodes, w.nodes, sizeof(LNode)))) return rc;
    int32_t const_h = 0;     // constant hessian: the histograms carry no h channel
    {
        int32_t st = 0;
        hipError_t e = hipMemcpy(&st, out_status, sizeof st, hipMemcpyDeviceToHost);
        if (e == hipSuccess) e = hipMemcpy(&const_h, &w.q->const_h, sizeof const_h, hipMemcpyDeviceToHost);
        if (e != hipSuccess) return hip_fail(e, "yabt_grow_levelwise: status");
        if (st < 0) return 0;                      // non-finite g/h: out_status[0] = -1, like yabt_grow
    }

    // host view of the breadth-first tree
    std::vector<int32_t> lch(NP, -1), rch(NP, -1), slot_of(NP, -1);
    slot_of[0] = 0;
    std::vector<int32_t> free_slots;
    for (int s = P - 1; s >= 1; --s) free_slots.push_back(s);
    int level0 = 0, level_n = 1, next_id = 1;     // nodes of the current depth: [level0, level0 + level_n)
    for (int d = 0; d < max_depth; ++d) {
        // split decisions (fp32 gain above 0, as cgrow's leaf table compares them)
        int nsplit = 0;
        for (int k = level0; k < level0 + level_n; ++k) {
            Route& R = h_route[k - level0];
            const LNode& L = h_nodes[k];
            R.f = -1;
            R.b = -1;
            R.left = R.right = -1;
            R.built_left = R.built_right = -1;
            if (L.b >= 0 && (float)L.gain > 0.0f) {
                R.f = L.f;
                R.b = L.b;
                R.left = next_id;
                R.right = next_id + 1;
                lch[k] = next_id;
                rch[k] = next_id + 1;
                next_id += 2;
                ++nsplit;
            } else if (slot_of[k] >= 0) {
                free_slots.push_back(slot_of[k]);
                slot_of[k] = -1;
            }
        }
        if (nsplit == 0) break;
        const bool scan_children = d + 1 < max_depth;
        int nbuilt = 0, npairs = 0, nscan = 0;
        if (scan_children) {
            for (int k = level0; k < level0 + level_n; ++k) {
                Route& R = h_route[k - level0];
                if (R.f < 0) continue;
                const LNode& L = h_nodes[k];
                const int64_t cl = L.left[2], c = L.tot[2];
                const bool bl = cl <= c - cl;              // the smaller child is built, ties left (grow.c:355)
                const int built = bl ? R.left : R.right, other = bl ? R.right : R.left;
                if (free_slots.empty()) return fail(-4, "yabt_grow_levelwise: histogram slot pool exhausted");
                const int bs = free_slots.back();
                free_slots.pop_back();
                slot_of[built] = bs;
                slot_of[other] = slot_of[k];
                slot_of[k] = -1;
                if (bl) R.built_left = nbuilt;
                else R.built_right = nbuilt;
                h_built[nbuilt++] = bs;
                h_pairs[2 * npairs] = slot_of[other];
                h_pairs[2 * npairs + 1] = bs;
                ++npairs;
            }
            for (int k = level0 + level_n; k < next_id; ++k) h_scan[nscan++] = k;
            for (int j = 0; j < nscan; ++j) h_scan[nscan + j] = slot_of[h_scan[j]];
        } else {
            for (int k = level0; k < level0 + level_n; ++k)
                if (slot_of[k] >= 0) {
                    free_slots.push_back(slot_of[k]);
                    slot_of[k] = -1;
                }
        }
        if ((rc = copy_in(w.route + level0, h_route, (size_t)level_n * sizeof(Route)))) return rc;
        k_children<<<level_n, LB, 0, stream>>>(w.nodes, w.route, w.path, F, level0);
        k_route<<<launch_grid(max(n, (int64_t)1), LB * 8, 4096), LB, 0, stream>>>(bins_fm, ld_fm, n, w.row_node,
                                                                                   w.row_built, w.route);
        if (scan_children) {
            if ((rc = copy_in(w.built_slot, h_built, (size_t)nbuilt * sizeof(int32_t)))) return rc;
            if ((rc = copy_in(w.pairs, h_pairs, (size_t)2 * npairs * sizeof(int32_t)))) return rc;
            if ((rc = copy_in(w.scan_list, h_scan, (size_t)2 * nscan * sizeof(int32_t)))) return rc;
            const hipError_t e = hipMemsetAsync(w.count, 0, (size_t)nbuilt * sizeof(uint32_t), stream);
            if (e != hipSuccess) return hip_fail(e, "yabt_grow_levelwise: clear");
            k_zero_slots<<<dim3((unsigned)launch_grid((int64_t)slot_n, LB * 4, 256), (unsigned)nbuilt), LB, 0,
                           stream>>>(w.hist, slot_n, w.built_slot, nbuilt);
            const int rb = (int)((n + LROWS - 1) / LROWS);
            const bool lds = nbuilt <= LDS_SLOTS;
            if (rb > 0) {
                if (lds) k_count<true><<<rb, LB, 0, stream>>>(w.row_built, n, nbuilt, w.count);
                else k_count<false><<<rb, LB, 0, stream>>>(w.row_built, n, nbuilt, w.count);
            }
            k_offsets<<<1, 1024, 0, stream>>>(w.count, nbuilt, w.off, w.cursor);
            if (rb > 0) {
                if (lds) k_scatter<true><<<rb, LB, 0, stream>>>(w.row_built, n, nbuilt, w.cursor, w.sorted);
                else k_scatter<false><<<rb, LB, 0, stream>>>(w.row_built, n, nbuilt, w.cursor, w.sorted);
                // the built children together hold at most half of the rows
                const int chunks = (int)max((int64_t)1, (n / 2 + LCHUNK - 1) / LCHUNK);
                if (const_h)
                    k_hist<false><<<tiles * chunks, HBLOCK, 0, stream>>>(bins_rm, ld_rm, grad, hess, F, nbuilt, w.off,
                                                                         w.sorted, w.q, w.built_slot, w.hist, chunks);
                else
                    k_hist<true><<<tiles * chunks, HBLOCK, 0, stream>>>(bins_rm, ld_rm, grad, hess, F, nbuilt, w.off,
                                                                        w.sorted, w.q, w.built_slot, w.hist, chunks);
            }
            k_sub<<<dim3((unsigned)launch_grid((int64_t)slot_n, LB * 4, 256), (unsigned)npairs), LB, 0, stream>>>(
                w.hist, slot_n, w.pairs, npairs);
            k_scan<<<dim3(sblk, nscan), LSCAN * WAVE, 0, stream>>>(S, w.q, w.hist, w.scan_list, nscan, w.path,
                                                                    w.rec);
        }
        const int id0 = level0 + level_n, nnew = next_id - id0;
        k_pick<<<nnew, WAVE, 0, stream>>>(w.rec, sblk, w.scan_list, scan_children ? nscan : 0, id0, nnew, w.q, lr,
                                          lam, w.nodes);
        if ((rc = launch_status("yabt_grow_levelwise launch"))) return rc;
        if ((rc = fetch(h_nodes + id0, w.nodes + id0, (size_t)nnew * sizeof(LNode)))) return rc;
        level0 = id0;
        level_n = nnew;
    }
    const int n_prov = next_id;

    // cgrow's numbering (grow.c:321-408) replayed over the computed gains;
    // a node at the depth cap carries gain -inf (grow.c:316,392,402)
    auto leaf_gain = [&](int k) -> float {
        const LNode& L = h_nodes[k];
        if (L.depth >= max_depth || L.b < 0) return -INFINITY;
        return (float)L.gain;
    };
    std::vector<int32_t> fid(n_prov, -1), table(max_leaves + 1);
    std::vector<float> tgain(max_leaves + 1);
    fid[0] = 0;
    table[0] = 0;
    tgain[0] = leaf_gain(0);
    int n_active = 1, n_leaves = 1, n_nodes = 1;
    while (n_leaves < max_leaves) {
        int best_k = -1;
        float best_g = 0.0f;
        for (int k = 0; k < n_active; ++k)
            if (tgain[k] > best_g) {
                best_g = tgain[k];
                best_k = k;
            }
        if (best_k < 0) break;
        const int p = table[best_k];
        if (lch[p] < 0) return fail(-4, "yabt_grow_levelwise: replay reached a node the batched pass did not split");
        fid[lch[p]] = n_nodes;
        fid[rch[p]] = n_nodes + 1;
        n_nodes += 2;
        table[best_k] = lch[p];
        tgain[best_k] = leaf_gain(lch[p]);
        table[n_active] = rch[p];
        tgain[n_active] = leaf_gain(rch[p]);
        ++n_active;
        ++n_leaves;
    }
    // outputs in cgrow's numbering (full 2L+1 arrays, unused entries as cgrow initialises them)
    std::vector<int64_t> o_feat(NP, LEAF), o_thr(NP, 0), o_left(NP, -1), o_right(NP, -1), o_depth(NP, 0);
    std::vector<float> o_val(NP, 0.0f);
    for (int k = 0; k < n_prov; ++k) {
        const int i = fid[k];
        if (i < 0) continue;
        const bool split = lch[k] >= 0 && fid[lch[k]] >= 0;
        o_depth[i] = h_nodes[k].depth;
        o_val[i] = split ? 0.0f : h_nodes[k].value;
        if (split) {
            o_feat[i] = h_nodes[k].f;
            o_thr[i] = h_nodes[k].b;
            o_left[i] = fid[lch[k]];
            o_right[i] = fid[rch[k]];
        }
    }
    for (int k = 0; k < n_prov; ++k) h_remap[k] = fid[k];
    const hipError_t e = hipStreamSynchronize(stream);
    if (e != hipSuccess) return hip_fail(e, "yabt_grow_levelwise: synchronisation");
    struct Out {
        void* d;
        const void* h;
        size_t b;
    } outs[] = {{out_feature, o_feat.data(), NP * sizeof(int64_t)}, {out_thr_bin, o_thr.data(), NP * sizeof(int64_t)},
                {out_left, o_left.data(), NP * sizeof(int64_t)},    {out_right, o_right.data(), NP * sizeof(int64_t)},
                {out_value, o_val.data(), NP * sizeof(float)},      {out_depth, o_depth.data(), NP * sizeof(int64_t)},
                {out_status, &n_nodes, sizeof(int32_t)},            {w.remap, h_remap, (size_t)n_prov * sizeof(int32_t)}};
    for (const Out& o : outs)
        if ((rc = copy_in(o.d, o.h, o.b))) return rc;
    if (out_leaf_of_row && n > 0)
        k_leaf_ids<<<launch_grid(n, LB * 8, 4096), LB, 0, stream>>>(w.row_node, n, w.remap, out_leaf_of_row);
    if ((rc = launch_status("yabt_grow_levelwise launch"))) return rc;
    const hipError_t e3 = hipStreamSynchronize(stream);    // the host vectors above are read by the copies
    return e3 == hipSuccess ? 0 : hip_fail(e3, "yabt_grow_levelwise: final synchronisation");
}

}  // extern "C"
