// Per-leaf linear models ("neural leaves", linear form) on gfx950.
//
// Replaces the Gram assembly and batched solve of yabt/neural_leaves.py
// `_fit_linear` (neural_leaves.py:42-90) plus the per-leaf row counts and
// input envelopes of `fit_leaf_networks` (neural_leaves.py:157-176):
//
//   x1 = [(x - mu) / sd (fp32), 1]           (neural_leaves.py:152-155, 67)
//   M[l] = sum_{i in l} x1_i (x1_i h_i)^T    (fp64 products, :68-83)
//   b[l] = -sum_{i in l} g_i x1_i
//   theta[l] = solve(M[l] + diag(lam, .., lam, 1e-8), b[l])   (:85-87)
//
// for every leaf with at least min_samples rows.  Each fp64 product is
// formed exactly as the reference forms it, then rounded once to int64 fixed
// point with one power-of-two scale per call (as the histograms are), so the
// per-leaf sums are exact, order-free and deterministic; the scale keeps every
// sum below 2^62.  Rows are first counting-sorted by leaf (the order inside a
// leaf is free), so each block accumulates one leaf at a time in registers.
//
// Launch sequence (caller's stream), node tables in LDS (n_nodes <= LDS_NODES):
//   k_leaf_init          clear counters, sums, envelopes
//   k_leaf_count         rows per node, per row block and in all (leaf ids only)
//   k_leaf_offsets       node offsets of the sorted rows
//   k_leaf_scatter_stats rows -> sorted by node; envelopes min/max of raw x, max |g|, |h|
//   k_leaf_shifts        max |x1|, fixed-point shifts
// more nodes: k_leaf_stats<K> (counts, envelopes, magnitudes), k_leaf_offsets,
// k_leaf_shifts, k_leaf_scatter (rows -> sorted by node); then
//   k_leaf_gram<K>     fixed-point sums of M and b per (chunk, leaf) segment, added
//                      into the leaf's sums (k_leaf_gram_mfma and k_leaf_reduce<K>
//                      for the fp64 MFMA sums: per-segment partials, then per leaf)
//   k_leaf_solve<K>    fp64 LU with partial pivoting per eligible leaf

#include "common.h"
#include "host.h"
#include "yabt_hip.h"

#include <string.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <tuple>

namespace yabt {

constexpr int LKMAX = 8;                       // model inputs per leaf, at most
constexpr int LB = 256;                        // threads per block
constexpr int LSB = 1024;                      // threads per stats/scatter block
constexpr int LROWS = 4096;                    // rows per stats/scatter block, at least
constexpr int LROW_BLOCKS = 512;               // stats/scatter blocks, at most: each flushes its
                                               // node tables once, so fewer blocks flush less
constexpr int LCHUNK = 4096;                   // sorted positions per gram block
constexpr int LDS_NODES = 640;                 // node tables kept in LDS up to this many nodes

__host__ __device__ constexpr int gram_entries(int K) { return (K + 1) * (K + 2) / 2 + (K + 1); }

struct LeafStats {
    uint32_t max_x1_bits;      // max |x1| (float bits, >= 1 via the bias column)
    uint32_t max_g_bits, max_h_bits;
    int32_t sM, sb;            // fixed-point shifts of M and b
    int32_t status;            // 0 ok; -1 a leaf id outside [0, n_nodes) or a non-finite input; -2 singular system
    int32_t n_fit;             // leaves fitted
};

struct LeafArgs {
    int x_kind;                // 0: fp32 row-major (n, ldx); 1: uint8 feature-major (F, ldx);
                               // 2: fp32 feature-major (F, ldx)
    const void* X;
    int64_t ldx;
    int64_t n;
    const int32_t* feats;
    const float* mu;
    const float* sd;
    const float* grad;
    const float* hess;
    const int64_t* leaf;       // node id per row
    const int64_t* feature;    // node table: leaves have feature == -1
    int n_nodes;
    int min_samples;
    double lam;
    int gram_f64;              // 1: M and b summed in fp64 by MFMA (parts and sums hold double bits)
    int64_t rows_per_block;    // stats/scatter rows per block (a multiple of 4)
    int64_t gram_chunk;        // sorted positions per exact-Gram block (a multiple of LB / 2)
    int vec4;                  // leaf ids, g, h and feature-major inputs aligned for 4-row vector
                               // loads: 1 uint8 inputs, 2 fp32 inputs; 0 none
    // workspace
    LeafStats* st;
    uint32_t* count;           // (n_nodes)
    uint32_t* bcnt;            // (row blocks, n_nodes) rows per row block and node (node tables in LDS)
    int64_t* off;              // (n_nodes + 1)
    unsigned long long* cursor;   // (n_nodes)
    uint8_t* sorted_x;         // rows' inputs in sorted order: 8 bytes (uint8) or K floats per row
    float2* sorted_gh;         // (n) g, h in sorted order
    int64_t* sums;             // (n_nodes, gram_entries(LKMAX))
    int64_t* parts;            // (chunks + n_nodes, gram_entries(LKMAX)) per-segment partial sums
    uint32_t* lo_key;          // (n_nodes, K) order-preserving float keys
    uint32_t* hi_key;
};

__device__ __forceinline__ float key_float(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Raw input j of row i.
template <int K>
__device__ __forceinline__ void load_x(const LeafArgs& A, int64_t i, const int32_t* fs, float x[K]) {
    if (A.x_kind == 0) {
        const float* row = reinterpret_cast<const float*>(A.X) + (size_t)i * (size_t)A.ldx;
#pragma unroll
        for (int j = 0; j < K; ++j) x[j] = row[fs[j]];
    } else if (A.x_kind == 2) {
        const float* Xf = reinterpret_cast<const float*>(A.X);
#pragma unroll
        for (int j = 0; j < K; ++j) x[j] = Xf[(size_t)fs[j] * (size_t)A.ldx + (size_t)i];
    } else {
        const uint8_t* B = reinterpret_cast<const uint8_t*>(A.X);
#pragma unroll
        for (int j = 0; j < K; ++j) x[j] = (float)B[(size_t)fs[j] * (size_t)A.ldx + (size_t)i];
    }
}

__global__ void __launch_bounds__(LB) k_leaf_init(LeafArgs A, int K) {
    const int64_t tid = (int64_t)blockIdx.x * LB + threadIdx.x, stride = (int64_t)gridDim.x * LB;
    const int64_t ne = (int64_t)A.n_nodes * gram_entries(LKMAX);
    for (int64_t i = tid; i < ne; i += stride) A.sums[i] = 0;
    for (int64_t i = tid; i < A.n_nodes; i += stride) {
        A.count[i] = 0;
        A.cursor[i] = 0;
    }
    for (int64_t i = tid; i < (int64_t)A.n_nodes * K; i += stride) {
        A.lo_key[i] = float_key(INFINITY);
        A.hi_key[i] = float_key(-INFINITY);
    }
    if (tid == 0) {
        A.st->max_x1_bits = __float_as_uint(1.0f);
        A.st->max_g_bits = 0;
        A.st->max_h_bits = 0;
        A.st->status = 0;
        A.st->n_fit = 0;
    }
}

// Four consecutive rows i .. i + 3 (i % 4 == 0, A.vec4): their leaf ids, g
// and h, and per input j one word holding the four rows' uint8 inputs (row
// i + r in byte r) -- two 16-byte, two float4 and K 4-byte loads.
template <int K>
struct Rows4 {
    int64_t node[4];
    float g[4], h[4];
    uint32_t xw[K];
};
template <int K>
__device__ __forceinline__ void load_rows4(const LeafArgs& A, const int32_t* fs, int64_t i, Rows4<K>& R) {
    const longlong2 la = *reinterpret_cast<const longlong2*>(A.leaf + i);
    const longlong2 lb = *reinterpret_cast<const longlong2*>(A.leaf + i + 2);
    const float4 g4 = *reinterpret_cast<const float4*>(A.grad + i);
    const float4 h4 = *reinterpret_cast<const float4*>(A.hess + i);
    const uint8_t* B = reinterpret_cast<const uint8_t*>(A.X);
#pragma unroll
    for (int j = 0; j < K; ++j) R.xw[j] = *reinterpret_cast<const uint32_t*>(B + (size_t)fs[j] * (size_t)A.ldx + (size_t)i);
    R.node[0] = la.x;
    R.node[1] = la.y;
    R.node[2] = lb.x;
    R.node[3] = lb.y;
    R.g[0] = g4.x;
    R.g[1] = g4.y;
    R.g[2] = g4.z;
    R.g[3] = g4.w;
    R.h[0] = h4.x;
    R.h[1] = h4.y;
    R.h[2] = h4.z;
    R.h[3] = h4.w;
}

// The same four rows with fp32 feature-major inputs (A.vec4 == 2): one float4
// per input column.
template <int K>
struct Rows4F {
    int64_t node[4];
    float g[4], h[4];
    float4 x[K];
};
template <int K>
__device__ __forceinline__ void load_rows4f(const LeafArgs& A, const int32_t* fs, int64_t i, Rows4F<K>& R) {
    const longlong2 la = *reinterpret_cast<const longlong2*>(A.leaf + i);
    const longlong2 lb = *reinterpret_cast<const longlong2*>(A.leaf + i + 2);
    const float4 g4 = *reinterpret_cast<const float4*>(A.grad + i);
    const float4 h4 = *reinterpret_cast<const float4*>(A.hess + i);
    const float* Xf = reinterpret_cast<const float*>(A.X);
#pragma unroll
    for (int j = 0; j < K; ++j) R.x[j] = *reinterpret_cast<const float4*>(Xf + (size_t)fs[j] * (size_t)A.ldx + (size_t)i);
    R.node[0] = la.x;
    R.node[1] = la.y;
    R.node[2] = lb.x;
    R.node[3] = lb.y;
    R.g[0] = g4.x;
    R.g[1] = g4.y;
    R.g[2] = g4.z;
    R.g[3] = g4.w;
    R.h[0] = h4.x;
    R.h[1] = h4.y;
    R.h[2] = h4.z;
    R.h[3] = h4.w;
}

// Rows [blockIdx.x * rows_per_block, +rows_per_block): counts, envelopes and
// magnitudes, into the global node tables (more nodes than LDS holds).
template <int K>
__global__ void __launch_bounds__(LSB) k_leaf_stats(LeafArgs A) {
    __shared__ float s_red[3][LSB / WAVE];
    __shared__ int s_bad;
    __shared__ int32_t s_fs[LKMAX];
    if (threadIdx.x < K) s_fs[threadIdx.x] = A.feats[threadIdx.x];
    if (threadIdx.x == 0) s_bad = 0;
    __syncthreads();
    const int64_t lo = (int64_t)blockIdx.x * A.rows_per_block, hi = min(A.n, lo + A.rows_per_block);
    float mg = 0.0f, mh = 0.0f;
    int bad = 0;
    for (int64_t i = lo + threadIdx.x; i < hi; i += LSB) {
        const int64_t node = A.leaf[i];
        if (node < 0 || node >= A.n_nodes) {
            bad = 1;
            continue;
        }
        float x[K];
        load_x<K>(A, i, s_fs, x);
        const float gi = A.grad[i], hi_ = A.hess[i];
        if (!isfinite(gi) || !isfinite(hi_)) bad = 1;
        mg = fmaxf(mg, fabsf(gi));
        mh = fmaxf(mh, fabsf(hi_));
        // per-node envelopes; their extremes also bound |x1| (k_leaf_shifts) and
        // expose non-finite inputs (keys beyond those of -inf / +inf)
#pragma unroll
        for (int j = 0; j < K; ++j) {
            // the extremes settle quickly: read first, update only when improving
            const uint32_t kx = float_key(x[j]);
            uint32_t* plo = &A.lo_key[node * K + j];
            uint32_t* phi = &A.hi_key[node * K + j];
            if (kx < *(volatile uint32_t*)plo) atomicMin(plo, kx);
            if (kx > *(volatile uint32_t*)phi) atomicMax(phi, kx);
        }
        atomicAdd(&A.count[node], 1u);
    }
    if (bad) s_bad = 1;
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
#pragma unroll
    for (int d = WAVE / 2; d > 0; d >>= 1) {
        mg = fmaxf(mg, __shfl_xor(mg, d, WAVE));
        mh = fmaxf(mh, __shfl_xor(mh, d, WAVE));
    }
    if (lane == 0) {
        s_red[1][w] = mg;
        s_red[2][w] = mh;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < LSB / WAVE; ++i) {
            mg = fmaxf(mg, s_red[1][i]);
            mh = fmaxf(mh, s_red[2][i]);
        }
        // |x| <= inf as float bits: non-negative floats order like their bits
        atomicMax(&A.st->max_g_bits, __float_as_uint(mg));
        atomicMax(&A.st->max_h_bits, __float_as_uint(mh));
        if (s_bad) atomicMin(&A.st->status, -1);
    }
}

// One block: node offsets of the sorted rows (exclusive scan of the counts)
// and write cursors.
__global__ void __launch_bounds__(1024) k_leaf_offsets(LeafArgs A) {
    __shared__ int64_t s_wave[1024 / WAVE];
    int64_t carry = 0;
    for (int base = 0; base < A.n_nodes; base += 1024) {
        const int i = base + threadIdx.x;
        const int64_t c = i < A.n_nodes ? (int64_t)A.count[i] : 0;
        int64_t tot;
        const int64_t ex = block_excl_scan<1024, int64_t>(c, s_wave, &tot);
        if (i < A.n_nodes) {
            A.off[i] = carry + ex;
            A.cursor[i] = (unsigned long long)(carry + ex);
        }
        carry += tot;
    }
    if (threadIdx.x == 0) A.off[A.n_nodes] = carry;
}

// One block: max |x1| from the envelopes, and the fixed-point shifts.
__global__ void __launch_bounds__(1024) k_leaf_shifts(LeafArgs A, int K) {
    __shared__ uint32_t s_xlo[LKMAX], s_xhi[LKMAX];
    if (threadIdx.x < K) {
        s_xlo[threadIdx.x] = float_key(INFINITY);
        s_xhi[threadIdx.x] = float_key(-INFINITY);
    }
    __syncthreads();
    // thread t takes input t % K of nodes t / K, t / K + 1024 / K, ... in
    // registers, then one LDS atomic each
    if (threadIdx.x < (1024 / K) * K) {
        const int j = threadIdx.x % K, step = 1024 / K;
        uint32_t lo = float_key(INFINITY), hi = float_key(-INFINITY);
        for (int nd = threadIdx.x / K; nd < A.n_nodes; nd += step) {
            lo = min(lo, A.lo_key[nd * K + j]);
            hi = max(hi, A.hi_key[nd * K + j]);
        }
        atomicMin(&s_xlo[j], lo);
        atomicMax(&s_xhi[j], hi);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        // max |x1| <= max(1, max_j max(|xmax_j - mu_j|, |xmin_j - mu_j|) / sd_j),
        // taken 2^-20 above for the fp32 rounding of (x - mu) / sd
        double mx = 1.0;
        for (int j = 0; j < K; ++j) {
            if (s_xlo[j] == float_key(INFINITY)) continue;                 // no rows at all
            if (s_xlo[j] < float_key(-INFINITY) || s_xhi[j] > float_key(INFINITY) ||
                !isfinite(key_float(s_xlo[j])) || !isfinite(key_float(s_xhi[j]))) {
                atomicMin(&A.st->status, -1);                               // a non-finite input
                continue;
            }
            const double m = (double)A.mu[j], d = (double)A.sd[j];
            const double b = fmax(fabs((double)key_float(s_xhi[j]) - m), fabs((double)key_float(s_xlo[j]) - m)) / d;
            mx = fmax(mx, b * (1.0 + 0x1p-20));
        }
        if (!isfinite(mx)) atomicMin(&A.st->status, -1);
        A.st->max_x1_bits = __float_as_uint((float)mx);
        // |p| <= max|x1|^2 max|h| for M and max|x1| max|g| for b; the bounds
        // are taken 2^-20 above to cover the rounding of the fp64 products
        const double bm = mx * mx * (double)__uint_as_float(A.st->max_h_bits) * (1.0 + 0x1p-20);
        const double bb = mx * (double)__uint_as_float(A.st->max_g_bits) * (1.0 + 0x1p-20);
        const float fm = (float)bm, fb = (float)bb;
        A.st->sM = quant_shift((double)fm >= bm ? fm : nextafterf(fm, INFINITY), A.n);
        A.st->sb = quant_shift((double)fb >= bb ? fb : nextafterf(fb, INFINITY), A.n);
    }
}

// Rows [blockIdx.x * rows_per_block, +rows_per_block): rows per node, into
// the block's row of bcnt and the totals (node tables in LDS).  Reads only
// the leaf ids.
__global__ void __launch_bounds__(LSB) k_leaf_count(LeafArgs A) {
    __shared__ uint32_t s_cnt[LDS_NODES];
    __shared__ int s_bad;
    if (threadIdx.x == 0) s_bad = 0;
    for (int i = threadIdx.x; i < A.n_nodes; i += LSB) s_cnt[i] = 0;
    __syncthreads();
    const int64_t lo = (int64_t)blockIdx.x * A.rows_per_block, hi = min(A.n, lo + A.rows_per_block);
    int bad = 0;
    auto count = [&](int64_t node) {
        if (node < 0 || node >= A.n_nodes) bad = 1;
        else atomicAdd(&s_cnt[node], 1u);
    };
    const int64_t ng = A.vec4 ? (hi - lo) / 4 : 0, first = lo + 4 * ng;
    for (int64_t q = threadIdx.x; q < ng; q += LSB) {
        const longlong2 la = *reinterpret_cast<const longlong2*>(A.leaf + lo + 4 * q);
        const longlong2 lb = *reinterpret_cast<const longlong2*>(A.leaf + lo + 4 * q + 2);
        count(la.x);
        count(la.y);
        count(lb.x);
        count(lb.y);
    }
    for (int64_t i = first + threadIdx.x; i < hi; i += LSB) count(A.leaf[i]);
    if (bad) s_bad = 1;
    __syncthreads();
    for (int i = threadIdx.x; i < A.n_nodes; i += LSB) {
        const uint32_t c = s_cnt[i];
        A.bcnt[(size_t)blockIdx.x * (size_t)A.n_nodes + i] = c;
        if (c) atomicAdd(&A.count[i], c);
    }
    if (threadIdx.x == 0 && s_bad) atomicMin(&A.st->status, -1);
}

// Rows [blockIdx.x * rows_per_block, +rows_per_block) to their node's range
// of the sorted arrays (one range per node and block, reserved with one
// atomic add from the block's counts), with the per-node envelopes and the
// magnitudes of g and h taken on the way (node tables in LDS).
template <int K>
__global__ void __launch_bounds__(LSB) k_leaf_scatter_stats(LeafArgs A) {
    __shared__ int32_t s_fs[LKMAX];
    __shared__ uint32_t s_cnt[LDS_NODES];
    __shared__ unsigned long long s_base[LDS_NODES];
    __shared__ uint32_t s_lo[LDS_NODES * K], s_hi[LDS_NODES * K];
    __shared__ float s_red[2][LSB / WAVE];
    __shared__ int s_bad;
    if (threadIdx.x < K) s_fs[threadIdx.x] = A.feats[threadIdx.x];
    if (threadIdx.x == 0) s_bad = 0;
    for (int i = threadIdx.x; i < A.n_nodes; i += LSB) {
        const uint32_t c = A.bcnt[(size_t)blockIdx.x * (size_t)A.n_nodes + i];
        s_base[i] = c ? atomicAdd(&A.cursor[i], (unsigned long long)c) : 0ull;
        s_cnt[i] = 0;
    }
    for (int i = threadIdx.x; i < A.n_nodes * K; i += LSB) {
        s_lo[i] = float_key(INFINITY);
        s_hi[i] = float_key(-INFINITY);
    }
    __syncthreads();
    const int64_t lo = (int64_t)blockIdx.x * A.rows_per_block, hi = min(A.n, lo + A.rows_per_block);
    float mg = 0.0f, mh = 0.0f;
    int bad = 0;
    // a row of a valid node: its envelope and magnitude updates and its
    // place; xw packs its uint8 inputs (K <= 8 bytes), or xf holds fp32 ones
    auto put = [&](int64_t node, const float (&x)[K], float gi, float hi_, uint2 xw) {
        if (!isfinite(gi) || !isfinite(hi_)) bad = 1;
        mg = fmaxf(mg, fabsf(gi));
        mh = fmaxf(mh, fabsf(hi_));
#pragma unroll
        for (int j = 0; j < K; ++j) {
            const uint32_t kx = float_key(x[j]);
            uint32_t* plo = &s_lo[node * K + j];
            uint32_t* phi = &s_hi[node * K + j];
            if (kx < *(volatile uint32_t*)plo) atomicMin(plo, kx);
            if (kx > *(volatile uint32_t*)phi) atomicMax(phi, kx);
        }
        const uint64_t pos = s_base[node] + atomicAdd(&s_cnt[node], 1u);
        A.sorted_gh[pos] = make_float2(gi, hi_);
        if (A.x_kind == 1) {
            reinterpret_cast<uint2*>(A.sorted_x)[pos] = xw;
        } else {
            float* dst = reinterpret_cast<float*>(A.sorted_x) + pos * K;
#pragma unroll
            for (int j = 0; j < K; ++j) dst[j] = x[j];
        }
    };
    const int64_t ng = A.vec4 ? (hi - lo) / 4 : 0, first = lo + 4 * ng;
    if (A.vec4 == 2) {
        for (int64_t q = threadIdx.x; q < ng; q += LSB) {
            Rows4F<K> R;
            load_rows4f<K>(A, s_fs, lo + 4 * q, R);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t node = R.node[r];
                if (node < 0 || node >= A.n_nodes) continue;
                float x[K];
#pragma unroll
                for (int j = 0; j < K; ++j) x[j] = r == 0 ? R.x[j].x : r == 1 ? R.x[j].y : r == 2 ? R.x[j].z : R.x[j].w;
                put(node, x, R.g[r], R.h[r], make_uint2(0, 0));
            }
        }
    }
    for (int64_t q = threadIdx.x; A.vec4 == 1 && q < ng; q += LSB) {
        Rows4<K> R;
        load_rows4<K>(A, s_fs, lo + 4 * q, R);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t node = R.node[r];
            if (node < 0 || node >= A.n_nodes) continue;
            float x[K];
            uint32_t w0 = 0, w1 = 0;
#pragma unroll
            for (int j = 0; j < K; ++j) {
                const uint32_t b = (R.xw[j] >> (8 * r)) & 0xffu;
                x[j] = (float)b;
                if (j < 4) w0 |= b << (8 * j);
                else w1 |= b << (8 * (j - 4));
            }
            put(node, x, R.g[r], R.h[r], make_uint2(w0, w1));
        }
    }
    for (int64_t i = first + threadIdx.x; i < hi; i += LSB) {
        const int64_t node = A.leaf[i];
        if (node < 0 || node >= A.n_nodes) continue;
        float x[K];
        load_x<K>(A, i, s_fs, x);
        uint32_t w0 = 0, w1 = 0;
        if (A.x_kind == 1) {
#pragma unroll
            for (int j = 0; j < K; ++j) {
                const uint32_t b = (uint32_t)x[j];
                if (j < 4) w0 |= b << (8 * j);
                else w1 |= b << (8 * (j - 4));
            }
        }
        put(node, x, A.grad[i], A.hess[i], make_uint2(w0, w1));
    }
    if (bad) s_bad = 1;
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
#pragma unroll
    for (int d = WAVE / 2; d > 0; d >>= 1) {
        mg = fmaxf(mg, __shfl_xor(mg, d, WAVE));
        mh = fmaxf(mh, __shfl_xor(mh, d, WAVE));
    }
    if (lane == 0) {
        s_red[0][w] = mg;
        s_red[1][w] = mh;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < LSB / WAVE; ++i) {
            mg = fmaxf(mg, s_red[0][i]);
            mh = fmaxf(mh, s_red[1][i]);
        }
        // |x| <= inf as float bits: non-negative floats order like their bits
        atomicMax(&A.st->max_g_bits, __float_as_uint(mg));
        atomicMax(&A.st->max_h_bits, __float_as_uint(mh));
        if (s_bad) atomicMin(&A.st->status, -1);
    }
    for (int i = threadIdx.x; i < A.n_nodes * K; i += LSB) {
        if (s_lo[i] != float_key(INFINITY)) atomicMin(&A.lo_key[i], s_lo[i]);
        if (s_hi[i] != float_key(-INFINITY)) atomicMax(&A.hi_key[i], s_hi[i]);
    }
}

// The inputs, g and h of row i go to position pos of the sorted arrays.
template <int K>
__device__ __forceinline__ void put_sorted(const LeafArgs& A, const int32_t* fs, int64_t i, uint64_t pos) {
    A.sorted_gh[pos] = make_float2(A.grad[i], A.hess[i]);
    if (A.x_kind == 1) {
        const uint8_t* B = reinterpret_cast<const uint8_t*>(A.X);
        uint32_t w0 = 0, w1 = 0;
#pragma unroll
        for (int j = 0; j < K; ++j) {
            const uint32_t b = B[(size_t)fs[j] * (size_t)A.ldx + (size_t)i];
            if (j < 4) w0 |= b << (8 * j);
            else w1 |= b << (8 * (j - 4));
        }
        reinterpret_cast<uint2*>(A.sorted_x)[pos] = make_uint2(w0, w1);
    } else {
        float x[K];
        load_x<K>(A, i, fs, x);
        float* dst = reinterpret_cast<float*>(A.sorted_x) + pos * K;
#pragma unroll
        for (int j = 0; j < K; ++j) dst[j] = x[j];
    }
}

// Rows [blockIdx.x * rows_per_block, +rows_per_block) to their node's range
// of the sorted arrays, one cursor atomic per row (more nodes than LDS holds).
template <int K>
__global__ void __launch_bounds__(LSB) k_leaf_scatter(LeafArgs A) {
    __shared__ int32_t s_fs[LKMAX];
    if (threadIdx.x < K) s_fs[threadIdx.x] = A.feats[threadIdx.x];
    __syncthreads();
    const int64_t lo = (int64_t)blockIdx.x * A.rows_per_block, hi = min(A.n, lo + A.rows_per_block);
    for (int64_t i = lo + threadIdx.x; i < hi; i += LSB) {
        const int64_t node = A.leaf[i];
        if (node < 0 || node >= A.n_nodes) continue;
        put_sorted<K>(A, s_fs, i, atomicAdd(&A.cursor[node], 1ull));
    }
}

__device__ __forceinline__ bool leaf_eligible(const LeafArgs& A, int node) {
    return A.feature[node] == LEAF && (int64_t)A.count[node] >= (int64_t)A.min_samples;
}

// Standardised uint8 inputs take 256 values per input: s_x1[j * 256 + b] =
// (double)((float(b) - mu[j]) / sd[j]), x1 formed in fp32 as the reference
// forms it (neural_leaves.py:152-155), one table per block in LDS.
template <int K, int NT, typename T>
__device__ __forceinline__ void x1_table(T* s_x1, const float* mu, const float* sd) {
    for (int i = threadIdx.x; i < K * 256; i += NT) {
        const int j = i / 256, b = i % 256;
        s_x1[i] = (T)(((float)b - mu[j]) / sd[j]);
    }
}

// The node holding sorted position c0: the last l with off[l] <= c0.
__device__ __forceinline__ int node_at(const LeafArgs& A, int64_t c0) {
    int lo = 0, hi = A.n_nodes - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) / 2;
        if (A.off[mid] <= c0) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// How each fixed-point product is rounded and summed (every form is exact
// and independent of the order of the rows):
//   GRAM_RINT  n <= 1024: rint of the fp64 product, summed as int64;
//   GRAM_MAGIC n <= 2^15: the same rounding through the bits of
//              v + 1.5 * 2^52 (round to nearest even; the constant's bits
//              come off once per row later);
//   GRAM_ACC   n > 2^15: one fma per product into a double accumulator that
//              stays in [2^52, 2^53), where the ulp is 1, so that
//              fma(x1, y, acc) = acc + (x1 y rounded to an integer) exactly.
// GRAM_ACC's second factor y has its lowest mantissa bit set (a change of at
// most 2^-52 of it), so that no product is ever exactly halfway between two
// integers: with y = m 2^(e - 52), m odd and >= 2^52, and x1's lowest set
// bit 2^f, the product's lowest set bit is 2^(f + e - 52), which is 2^-1
// only if |x1 y| >= 2^(f + e) = 2^51, above every scaled product (|p| <
// 2^(61 - k) <= 2^45 for n > 2^15, k = ceil(log2 n)).  Without a tie the
// rounding does not depend on the accumulator's parity, so the sums do not
// depend on the order of the rows.  A thread adds at most gram_chunk / (LB
// / 2) products per entry and segment, which the host keeps at most
// 2^(k - 11), so |sum| <= 2^(k - 11) 2^(61 - k) = 2^50 and the accumulator
// never leaves the binade.
enum GramMode { GRAM_RINT = 0, GRAM_MAGIC = 1, GRAM_ACC = 2 };
constexpr double GRAM_MAGIC_C = 6755399441055744.0;   // 1.5 * 2^52

__host__ __device__ constexpr int gram_half_entries(int K) { return (gram_entries(K) + 1) / 2; }

__device__ __forceinline__ double sticky_f64(double v) {
    return __longlong_as_double(__double_as_longlong(v) | 1ll);
}

// The fixed-point products of half P of a row's gram_entries (P = 0: entries
// [0, NE/2), 1: [NE/2, NE)), added into acc[t - the half's first entry]
// (integer sums for GRAM_RINT and GRAM_MAGIC, the binade accumulators for
// GRAM_ACC, as double bits).
template <int K, int MODE, int P>
__device__ __forceinline__ void gram_half(const double (&x1)[K + 1], const double (&xhs)[K + 1], double gs,
                                          uint64_t (&acc)[gram_half_entries(K)]) {
    constexpr int NE = gram_entries(K);
    constexpr int T0 = P == 0 ? 0 : (NE + 1) / 2, T1 = P == 0 ? (NE + 1) / 2 : NE;
    auto add = [&](uint64_t& a, double x, double y) {   // a += round(x y)
        if constexpr (MODE == GRAM_ACC) {
            a = (uint64_t)__double_as_longlong(fma(x, y, __longlong_as_double((long long)a)));
        } else {
            const double v = x * y;
            if constexpr (MODE == GRAM_MAGIC) a += (uint64_t)__double_as_longlong(v + GRAM_MAGIC_C);
            else a += (uint64_t)(int64_t)rint(v);
        }
    };
    int t = 0;
#pragma unroll
    for (int a = 0; a <= K; ++a) {
#pragma unroll
        for (int b = a; b <= K; ++b, ++t) {
            if (t < T0 || t >= T1) continue;
            add(acc[t - T0], x1[a], xhs[b]);          // the reference's x1 (x1 h), times 2^sM
        }
    }
#pragma unroll
    for (int a = 0; a <= K; ++a, ++t) {            // rhs = -(X1 * g)
        if (t < T0 || t >= T1) continue;
        add(acc[t - T0], -x1[a], gs);
    }
}

// One half-block's rows p = p0, p0 + LB / 2, ... < e of a segment: x1 and
// x1 h from the row, then half P of its products into acc (integer sums on
// return, whatever the mode).
template <int K, int MODE, int P>
__device__ __forceinline__ void gram_rows(const LeafArgs& A, const float* s_x1, const float* s_mu,
                                          const float* s_sd, double scM, double scb, int64_t p0, int64_t e,
                                          uint64_t (&acc)[gram_half_entries(K)]) {
    constexpr int NH = gram_half_entries(K);
    const uint64_t magic_bits = (uint64_t)__double_as_longlong(GRAM_MAGIC_C);
    if constexpr (MODE == GRAM_ACC) {
#pragma unroll
        for (int t = 0; t < NH; ++t) acc[t] = magic_bits;
    }
    uint64_t nrow = 0;
    // one row: x1 from its inputs, x1 h, then the products
    auto row = [&](const double (&x1)[K + 1], float2 gh) {
        // Xh = X1 * h (neural_leaves.py:72), scaled by 2^sM: a power-of-two
        // scale commutes with the fp64 rounding (no overflow or underflow at
        // these magnitudes), so x1 * (h 2^sM) is (x1 * h) 2^sM exactly
        const double hs = (double)gh.y * scM;
        double gs = (double)gh.x * scb;
        double xhs[K + 1];
#pragma unroll
        for (int b = 0; b <= K; ++b) xhs[b] = x1[b] * hs;
        if constexpr (MODE == GRAM_ACC) {
#pragma unroll
            for (int b = 0; b <= K; ++b) xhs[b] = sticky_f64(xhs[b]);
            gs = sticky_f64(gs);
        }
        ++nrow;
        gram_half<K, MODE, P>(x1, xhs, gs, acc);
    };
    if (A.x_kind == 1) {
        // uint8 inputs: the next row's inputs and g, h are loaded while this
        // row is summed (two named buffers, loads at clamped positions, so
        // that each wait covers only the row about to be used)
        constexpr int64_t ST = LB / 2;
        const uint2* xs = reinterpret_cast<const uint2*>(A.sorted_x);
        auto table = [&](uint2 v, double (&x1)[K + 1]) {
#pragma unroll
            for (int j = 0; j < K; ++j)
                x1[j] = (double)s_x1[j * 256 + (((j < 4 ? v.x : v.y) >> (8 * (j & 3))) & 0xffu)];
            x1[K] = 1.0;
        };
        if (p0 < e) {
            uint2 va = xs[p0], vb;
            float2 ga = A.sorted_gh[p0], gb;
            for (int64_t p = p0;; p += 2 * ST) {
                const int64_t pb = min(p + ST, e - 1);
                vb = xs[pb];
                gb = A.sorted_gh[pb];
                asm volatile("" ::: "memory");        // keeps the loads here (not sunk to their use)
                {
                    double x1[K + 1];
                    table(va, x1);
                    row(x1, ga);
                }
                if (p + ST >= e) break;
                const int64_t pa = min(p + 2 * ST, e - 1);
                va = xs[pa];
                ga = A.sorted_gh[pa];
                asm volatile("" ::: "memory");
                {
                    double x1[K + 1];
                    table(vb, x1);
                    row(x1, gb);
                }
                if (p + 2 * ST >= e) break;
            }
        }
    } else {
        for (int64_t p = p0; p < e; p += LB / 2) {
            const float2 gh = A.sorted_gh[p];
            double x1[K + 1];
            const float* src = reinterpret_cast<const float*>(A.sorted_x) + (size_t)p * K;
#pragma unroll
            for (int j = 0; j < K; ++j) x1[j] = (double)((src[j] - s_mu[j]) / s_sd[j]);
            x1[K] = 1.0;
            row(x1, gh);
        }
    }
    if constexpr (MODE != GRAM_RINT) {
        // GRAM_ACC: bits(acc) - bits(1.5 * 2^52) is the integer sum (one
        // binade, ulp 1); GRAM_MAGIC: the constant's bits once per row
        const uint64_t off = MODE == GRAM_ACC ? magic_bits : nrow * magic_bits;
#pragma unroll
        for (int t = 0; t < NH; ++t) acc[t] -= off;
    }
}

// Block sums of a half's NH integer accumulators: a reduce-scatter over the
// wave -- v_permlane32_swap pairs entry i with entry i + S/2 (one lane half
// keeps the sum of one, the other half of the other), v_permlane16_swap does
// the same between rows, and DPP row rotations add up each row -- so that
// lane 16 r of value i holds the wave's total of entry id[i] in row r.  The
// entry a lane holds is found by passing the entry numbers through the same
// swaps (make_ids), which also makes the layout independent of the direction
// in which each swap moves data: after a swap a lane's two operands hold the
// same entry, its own and its partner's partial sums.
template <int NH>
struct GramScatter {
    static constexpr int S = (NH + 3) / 4 * 4;       // entries padded to a multiple of 4
    static constexpr int V = S / 4;                  // values per lane after the swaps
    int id[V];

    __device__ __forceinline__ void make_ids() {
        uint32_t a[S / 2];
#pragma unroll
        for (int i = 0; i < S / 2; ++i) {
            const auto sw = __builtin_amdgcn_permlane32_swap((uint32_t)i, (uint32_t)(i + S / 2), false, false);
            a[i] = sw[0];
        }
#pragma unroll
        for (int i = 0; i < V; ++i) {
            const auto sw = __builtin_amdgcn_permlane16_swap(a[i], a[i + V], false, false);
            id[i] = (int)sw[0];
        }
    }

    // acc (NH values, every lane of the wave active) -> out[i]: the wave's
    // total of entry id[i] in every lane of row (lane / 16)
    __device__ __forceinline__ void reduce(const uint64_t (&acc)[NH], uint64_t (&out)[V]) const {
        uint64_t a[S / 2];
#pragma unroll
        for (int i = 0; i < S / 2; ++i) {
            const uint64_t x = acc[i], y = i + S / 2 < NH ? acc[i + S / 2] : 0;
            const auto lo = __builtin_amdgcn_permlane32_swap((uint32_t)x, (uint32_t)y, false, false);
            const auto hi = __builtin_amdgcn_permlane32_swap((uint32_t)(x >> 32), (uint32_t)(y >> 32), false, false);
            a[i] = ((((uint64_t)hi[0]) << 32) | lo[0]) + ((((uint64_t)hi[1]) << 32) | lo[1]);
        }
#pragma unroll
        for (int i = 0; i < V; ++i) {
            const uint64_t x = a[i], y = a[i + V];
            const auto lo = __builtin_amdgcn_permlane16_swap((uint32_t)x, (uint32_t)y, false, false);
            const auto hi = __builtin_amdgcn_permlane16_swap((uint32_t)(x >> 32), (uint32_t)(y >> 32), false, false);
            uint64_t u = ((((uint64_t)hi[0]) << 32) | lo[0]) + ((((uint64_t)hi[1]) << 32) | lo[1]);
            u += dpp64<DPP_ROW_ROR + 8>(u);
            u += dpp64<DPP_ROW_ROR + 4>(u);
            u += dpp64<DPP_ROW_ROR + 2>(u);
            u += dpp64<DPP_ROW_ROR + 1>(u);
            out[i] = u;
        }
    }
};

// Sorted positions [blockIdx.x * gram_chunk, +gram_chunk): the block lists
// the chunk's segments (the eligible nodes whose rows meet it); for each, the
// block's two halves (waves 0-1 and 2-3) each sum half of the gram_entries
// over the segment's rows, a thread's rows in registers (half the
// accumulators per thread: twice the resident waves); waves reduce by the
// reduce-scatter above and the block's sums are added into the node's sums.
// MODE: GramMode, by the row count.
template <int K, int MODE>
__global__ void __launch_bounds__(LB) k_leaf_gram(LeafArgs A) {
    constexpr int NE = gram_entries(K);
    constexpr int NH = gram_half_entries(K);      // entries of the first half (the second has NE - NH)
    constexpr int HT = LB / 2;                    // threads per half
    __shared__ float s_mu[LKMAX], s_sd[LKMAX];
    __shared__ int64_t s_part[2][LB / WAVE][NH];  // two, alternating by segment: one barrier each
    __shared__ float s_x1[K * 256];           // x1 is an fp32 value: half the LDS bytes of doubles
    __shared__ int s_nseg;
    extern __shared__ int s_seg[];                // min(n_nodes, gram_chunk) entries (launch's dynamic LDS)
    // the loads the prologue waits for, issued together
    const int64_t total = A.off[A.n_nodes];
    const int32_t sM = A.st->sM, sb = A.st->sb;
    if (threadIdx.x < K) {
        s_mu[threadIdx.x] = A.mu[threadIdx.x];
        s_sd[threadIdx.x] = A.sd[threadIdx.x];
    }
    if (threadIdx.x == 0) s_nseg = 0;
    if (A.x_kind == 1) x1_table<K, LB>(s_x1, A.mu, A.sd);
    const int64_t c0 = (int64_t)blockIdx.x * A.gram_chunk, c1 = min(total, c0 + A.gram_chunk);
    __syncthreads();
    // the chunk's segments, every thread testing its share of the nodes at
    // once: the eligible nodes whose rows meet [c0, c1), listed in LDS in no
    // particular order (the sums are exact).  The node ranges are disjoint,
    // so at most min(n_nodes, c1 - c0) are listed.  A node-by-node walk with
    // its dependent loads had cost ~3 us a segment, and a chunk of many small
    // leaves twice a chunk's time.
    if (c0 < c1) {
        for (int t = threadIdx.x; t < A.n_nodes; t += LB) {
            const int64_t lo = A.off[t], hi = A.off[t + 1];
            if (lo < c1 && hi > c0 && leaf_eligible(A, t)) s_seg[atomicAdd(&s_nseg, 1)] = t;
        }
    }
    __syncthreads();
    if (c0 >= c1) return;
    const double scM = ldexp(1.0, sM), scb = ldexp(1.0, sb);
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    const int half = threadIdx.x / HT, th = threadIdx.x % HT;   // wave-uniform half
    GramScatter<NH> R;
    int buf = 0;
    // the node and count read from LDS are the same in every lane:
    // readfirstlane keeps them (and what is derived from them) scalar
    const int nseg = __builtin_amdgcn_readfirstlane(s_nseg);
    for (int k = 0; k < nseg; ++k) {
        const int node = __builtin_amdgcn_readfirstlane(s_seg[k]);
        const int64_t s = max(c0, A.off[node]), e = min(c1, A.off[node + 1]);
        uint64_t acc[NH];
#pragma unroll
        for (int t = 0; t < NH; ++t) acc[t] = 0;
        if (half == 0) gram_rows<K, MODE, 0>(A, s_x1, s_mu, s_sd, scM, scb, s + th, e, acc);
        else gram_rows<K, MODE, 1>(A, s_x1, s_mu, s_sd, scM, scb, s + th, e, acc);
        // block sum of this (chunk, node) segment, added into the node's sums
        // with 64-bit integer atomics (exact, so the order of the segments
        // does not matter); a node's segments are its chunks, so an address
        // takes at most rows / gram_chunk + 1 adds.  The next segment writes
        // the other s_part, so one barrier separates the writes from the reads.
        const int nh = half == 0 ? NH : NE - NH;
        uint64_t tot[GramScatter<NH>::V];
        R.reduce(acc, tot);
        R.make_ids();                                 // here, not held across the rows (registers)
        if ((lane & 15) == 0) {
#pragma unroll
            for (int i = 0; i < GramScatter<NH>::V; ++i)
                if (R.id[i] < nh) s_part[buf][w][R.id[i]] = (int64_t)tot[i];
        }
        __syncthreads();
        unsigned long long* out = reinterpret_cast<unsigned long long*>(A.sums + (size_t)node * gram_entries(LKMAX));
        constexpr int HW = HT / WAVE;                 // waves per half
        for (int t = threadIdx.x; t < NE; t += LB) {
            const int hh = t < NH ? 0 : 1, tt = t < NH ? t : t - NH;
            int64_t v = 0;
#pragma unroll
            for (int i = 0; i < HW; ++i) v += s_part[buf][hh * HW + i][tt];
            if (v) atomicAdd(&out[t], (unsigned long long)v);
        }
        buf ^= 1;
    }
}

// The Gram on the matrix cores, in fp64: per (chunk, node) segment each wave
// accumulates D = sum over groups of 4 rows of A B with
// v_mfma_f64_16x16x4_f64, A[a][k] = x1_a of row k (a <= K, else 0) and
// B[k][c] = x1_c h of row k (c <= K), -g of row k (c = K + 1), else 0, so
// that D[a][c] = M[a][c] and D[a][K + 1] = b[a].  Lane l supplies A[l % 16]
// [l / 16] and B[l / 16][l % 16] and holds D[4 r + l / 16][l % 16] in its
// accumulator r.  The sums are fp64 (each product and addition rounded as the
// matrix core rounds it, in a fixed order), written as double bits to the
// segment's partial slot in gram_entries order; no fixed-point scaling.
template <int K>
__global__ void __launch_bounds__(LB) k_leaf_gram_mfma(LeafArgs A) {
    typedef double d4 __attribute__((ext_vector_type(4)));
    constexpr int NE = gram_entries(K);
    static_assert(K + 2 <= 16, "the Gram and the rhs fit one 16 x 16 block");
    __shared__ float s_mu[LKMAX], s_sd[LKMAX];
    __shared__ double s_d[LB / WAVE][16 * 16];
    __shared__ double s_x1[K * 256];
    if (threadIdx.x < K) {
        s_mu[threadIdx.x] = A.mu[threadIdx.x];
        s_sd[threadIdx.x] = A.sd[threadIdx.x];
    }
    if (A.x_kind == 1) x1_table<K, LB>(s_x1, A.mu, A.sd);
    __syncthreads();
    const int64_t total = A.off[A.n_nodes];
    const int64_t c0 = (int64_t)blockIdx.x * LCHUNK, c1 = min(total, c0 + LCHUNK);
    if (c0 >= c1) return;
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    const int kr = lane >> 4, col = lane & 15;   // the lane's row of a 4-row group, its matrix index
    for (int node = node_at(A, c0); node < A.n_nodes && A.off[node] < c1; ++node) {
        const int64_t s = max(c0, A.off[node]), e = min(c1, A.off[node + 1]);
        if (s >= e || !leaf_eligible(A, node)) continue;   // uniform across the block
        d4 acc = {0.0, 0.0, 0.0, 0.0};
        for (int64_t base = s + 4 * w; base < e; base += 4 * (LB / WAVE)) {
            const int64_t p = base + kr;
            double av = 0.0, bv = 0.0;
            if (p < e) {
                const float2 gh = A.sorted_gh[p];
                double x1 = 0.0;
                if (col < K) {
                    if (A.x_kind == 1) {
                        const uint2 v = reinterpret_cast<const uint2*>(A.sorted_x)[p];
                        const uint32_t word = col < 4 ? v.x : v.y;
                        x1 = s_x1[col * 256 + ((word >> (8 * (col & 3))) & 0xffu)];
                    } else {
                        const float xv = reinterpret_cast<const float*>(A.sorted_x)[(size_t)p * K + col];
                        x1 = (double)((xv - s_mu[col]) / s_sd[col]);
                    }
                } else if (col == K) {
                    x1 = 1.0;
                }
                av = x1;
                bv = col <= K ? x1 * (double)gh.y : (col == K + 1 ? -(double)gh.x : 0.0);
            }
            acc = __builtin_amdgcn_mfma_f64_16x16x4f64(av, bv, acc, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) s_d[w][(4 * r + kr) * 16 + col] = acc[r];
        __syncthreads();
        // the segment: the waves' sums in order, entries in gram_entries order
        int64_t* out = A.parts + ((size_t)blockIdx.x + (size_t)node) * gram_entries(LKMAX);
        for (int t = threadIdx.x; t < NE; t += LB) {
            int i;
            if (t < (K + 1) * (K + 2) / 2) {   // M[a][b], a <= b, row by row
                int a = 0, r = t;
                while (r >= K + 1 - a) {
                    r -= K + 1 - a;
                    ++a;
                }
                i = a * 16 + a + r;
            } else {                           // b[a] = D[a][K + 1]
                i = (t - (K + 1) * (K + 2) / 2) * 16 + K + 1;
            }
            double v = s_d[0][i];
#pragma unroll
            for (int q = 1; q < LB / WAVE; ++q) v += s_d[q][i];
            out[t] = __double_as_longlong(v);
        }
        __syncthreads();
    }
}

// Per-leaf fp64 sums of the MFMA Gram's segment partials (exact fixed-point
// sums go straight to the node's sums with integer atomics instead).  One
// block per eligible node, in a fixed order: wave w takes segments w,
// w + RW, ... of chunks first_chunk .. last_chunk (lane t: entry t), then the
// waves' sums in order.
constexpr int RB = 1024;
template <int K>
__global__ void __launch_bounds__(RB) k_leaf_reduce(LeafArgs A) {
    constexpr int NE = gram_entries(K);
    constexpr int RW = RB / WAVE;
    static_assert(NE <= WAVE, "one lane per entry");
    __shared__ double s_w[RW][NE];
    const int node = blockIdx.x;
    if (!leaf_eligible(A, node)) return;
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    const int64_t c0 = A.off[node] / LCHUNK, c1 = (A.off[node + 1] - 1) / LCHUNK;
    if (lane < NE) {
        double ad = 0.0;
        for (int64_t c = c0 + w; c <= c1; c += RW)
            ad += __longlong_as_double(A.parts[((size_t)c + (size_t)node) * gram_entries(LKMAX) + lane]);
        s_w[w][lane] = ad;
    }
    __syncthreads();
    if (threadIdx.x < NE) {
        double v = s_w[0][threadIdx.x];
        for (int q = 1; q < RW; ++q) v += s_w[q][threadIdx.x];
        A.sums[(size_t)node * gram_entries(LKMAX) + threadIdx.x] = __double_as_longlong(v);
    }
}

// 16 lanes per node (lane i: row i of the system): assemble, regularise and
// solve the (K+1) system of an eligible leaf with fp64 LU and partial
// pivoting; zeros elsewhere.  The operations, their order and their
// roundings are those of the one-thread elimination: pivot row p = the first
// row from c on with the largest |M[i][c]| (a NaN diagonal keeps row c; NaN
// elsewhere never wins), rows c and p swapped, then each row i > c updated
// from row c (f = M[i][c] / M[c][c], M[i][j] -= f M[c][j] for j >= c), and
// back substitution from the last row, subtracting the terms left to right.
constexpr int SOLVE_LANES = 16;
template <int K>
__global__ void __launch_bounds__(LB) k_leaf_solve(LeafArgs A, float* out_W, float* out_b, float* out_lo,
                                                  float* out_hi, int64_t* out_count) {
    constexpr int N = K + 1;
    static_assert(N <= SOLVE_LANES, "a row per lane");
    const int li = threadIdx.x % SOLVE_LANES;
    const int gbase = (threadIdx.x & (WAVE - 1)) - li;   // the group's first lane in the wave
    const int node = blockIdx.x * (LB / SOLVE_LANES) + threadIdx.x / SOLVE_LANES;
    const bool live = node < A.n_nodes;   // uniform over the group (groups never straddle a node)
    auto bcast = [&](double v, int src) { return __shfl(v, gbase + src, WAVE); };
    if (live) {
        if (li == 0) {
            out_count[node] = A.count[node];
            out_b[node] = 0.0f;
        }
        if (li < K) {
            out_lo[node * K + li] = key_float(A.lo_key[node * K + li]);
            out_hi[node * K + li] = key_float(A.hi_key[node * K + li]);
            out_W[node * K + li] = 0.0f;
        }
    }
    const bool go = live && leaf_eligible(A, node) && A.st->status == 0;
    // the shuffles below take every lane of the wave: groups without a system
    // run them on zeros and store nothing
    const int64_t* q = A.sums + (size_t)(go ? node : 0) * gram_entries(LKMAX);
    const bool f64 = A.gram_f64 != 0;   // fp64 sums (MFMA) or fixed point
    const double iM = ldexp(1.0, -A.st->sM), ib = ldexp(1.0, -A.st->sb);
    auto entry = [&](int t, double sc) { return f64 ? __longlong_as_double(q[t]) : (double)q[t] * sc; };
    // row li: M[li][b] from the upper triangle (entry t of (a, b), a <= b)
    double row[N], r = 0.0;
#pragma unroll
    for (int b = 0; b < N; ++b) row[b] = 0.0;
    if (go && li < N) {
        // entry of (a, b), a <= b: the rows before a, then b - a
        auto tri = [](int a, int b) { return a * N - a * (a - 1) / 2 + (b - a); };
#pragma unroll
        for (int b = 0; b < N; ++b) row[b] = entry(b >= li ? tri(li, b) : tri(b, li), iM);
        r = entry(N * (N + 1) / 2 + li, ib);
        if (li < K) row[li] += A.lam;                // reg = lam * I ...
        else row[K] += 1e-8;                          // ... but the bias (neural_leaves.py:85-86)
    }
    bool singular = false;
#pragma unroll
    for (int c = 0; c < N; ++c) {
        // pivot: key |M[i][c]| for i > c (NaN: never), |M[c][c]| for i = c (NaN: always)
        const double mc = row[c];
        double key = -1.0;
        if (li == c) key = isnan(mc) ? INFINITY : fabs(mc);
        else if (li > c && li < N) key = isnan(mc) ? -1.0 : fabs(mc);
        double mk = key;
        int pk = li;
#pragma unroll
        for (int d = SOLVE_LANES / 2; d > 0; d >>= 1) {
            const double ok = __shfl_xor(mk, d, WAVE);
            const int op = __shfl_xor(pk, d, WAVE);
            if (ok > mk || (ok == mk && op < pk)) {
                mk = ok;
                pk = op;
            }
        }
        const int p = pk;
        const double diag = bcast(row[c], c);
        const double best = isnan(diag) ? diag : mk;
        if (best == 0.0) singular = true;
        // swap rows c and p
        const int src = li == c ? p : (li == p ? c : li);
#pragma unroll
        for (int b = 0; b < N; ++b) row[b] = bcast(row[b], src);
        r = bcast(r, src);
        if (best != 0.0) {
            double pc[N];
#pragma unroll
            for (int b = 0; b < N; ++b) pc[b] = bcast(row[b], c);
            const double rc = bcast(r, c);
            if (li > c && li < N) {
                const double f = row[c] / pc[c];
#pragma unroll
                for (int b = c; b < N; ++b) row[b] -= f * pc[b];
                r -= f * rc;
            }
        }
    }
    if (!go) return;
    if (singular) {
        if (li == 0) atomicMin(&A.st->status, -2);
        return;
    }
    double th[N], mine = 0.0;
#pragma unroll
    for (int i = N - 1; i >= 0; --i) {
        double v = r;
#pragma unroll
        for (int j = i + 1; j < N; ++j) v -= row[j] * th[j];
        const double ti = v / row[i];
        if (li == i) mine = ti;
        th[i] = bcast(ti, i);
    }
    if (li < K) out_W[node * K + li] = (float)mine;
    if (li == K) out_b[node] = (float)mine;
    if (li == 0) atomicAdd(&A.st->n_fit, 1);
}

__global__ void k_leaf_status(const LeafStats* st, int32_t* out) {
    out[0] = st->status;
    out[1] = st->n_fit;
}

// The fold of the linear models into raw space (neural_leaves.py:178-184) in
// the order and fp32 roundings of the reference's torch expressions: per node,
// prod_j = W[j] * (mu[j] / sd[j]), acc = prod_0 + prod_1 + ... left to right,
// value = value_in + lr * (b - acc), linear[j] = (lr * W[j]) / sd[j].  With
// st, the fit's status words go to out_status too (the fit's k_leaf_status,
// folded into this launch when the two run back to back).
__global__ void __launch_bounds__(LB) k_leaf_fold(int n_nodes, int K, const float* W, const float* b,
                                                  const float* mu, const float* sd, float lr,
                                                  const float* value_in, float* out_value, float* out_linear,
                                                  const LeafStats* st, int32_t* out_status) {
    const int node = blockIdx.x * LB + threadIdx.x;
    if (st && node == 0) {
        out_status[0] = st->status;
        out_status[1] = st->n_fit;
    }
    if (node >= n_nodes) return;
    float acc = 0.0f;
    for (int j = 0; j < K; ++j) {
        const float wj = W[(size_t)node * K + j];
        const float prod = wj * (mu[j] / sd[j]);
        acc = j == 0 ? prod : acc + prod;
        out_linear[(size_t)node * K + j] = (lr * wj) / sd[j];
    }
    out_value[node] = value_in[node] + lr * (b[node] - acc);
}



// ---------------------------------------------------------------------------
// input moments: mu = mean, sd = max(unbiased std, 1e-6) per input
// (neural_leaves.py:152-155), from fp64 sums of x and x^2 reduced in a fixed
// order (per-block partials, then one block), so the result is deterministic
// ---------------------------------------------------------------------------

constexpr int MROWS = 16384;                   // rows per moments block

// fp32 inputs: per-block fp64 partials of x and x^2.
template <int K>
__global__ void __launch_bounds__(LB) k_leaf_moments(int x_kind, const void* X, int64_t ldx, int64_t n,
                                                     const int32_t* feats, double* part) {
    __shared__ int32_t s_fs[LKMAX];
    __shared__ double s_red[LB / WAVE][2 * LKMAX];
    if (threadIdx.x < K) s_fs[threadIdx.x] = feats[threadIdx.x];
    __syncthreads();
    LeafArgs A;
    A.x_kind = x_kind;
    A.X = X;
    A.ldx = ldx;
    const int64_t lo = (int64_t)blockIdx.x * MROWS, hi = min(n, lo + MROWS);
    double s1[K], s2[K];
#pragma unroll
    for (int j = 0; j < K; ++j) s1[j] = s2[j] = 0.0;
    for (int64_t i = lo + threadIdx.x; i < hi; i += LB) {
        float x[K];
        load_x<K>(A, i, s_fs, x);
#pragma unroll
        for (int j = 0; j < K; ++j) {
            const double v = (double)x[j];
            s1[j] += v;
            s2[j] += v * v;
        }
    }
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
#pragma unroll
    for (int j = 0; j < K; ++j) {
#pragma unroll
        for (int d = WAVE / 2; d > 0; d >>= 1) {
            s1[j] += __shfl_xor(s1[j], d, WAVE);
            s2[j] += __shfl_xor(s2[j], d, WAVE);
        }
        if (lane == 0) {
            s_red[w][j] = s1[j];
            s_red[w][LKMAX + j] = s2[j];
        }
    }
    __syncthreads();
    if (threadIdx.x < 2 * K) {
        const int j = threadIdx.x % K, which = threadIdx.x / K;
        double t = 0.0;
        for (int i = 0; i < LB / WAVE; ++i) t += s_red[i][which * LKMAX + j];
        part[((size_t)blockIdx.x * 2 + which) * LKMAX + j] = t;
    }
}

// One wave per input: lane l sums partials l, l + 64, ..., then a fixed
// butterfly; the same order on every run.
__global__ void k_leaf_moments_final(const double* part, int nblocks, int64_t n, int K, float* mu, float* sd) {
    const int j = blockIdx.x, lane = threadIdx.x;
    if (j >= K) return;
    double s1 = 0.0, s2 = 0.0;
    for (int b = lane; b < nblocks; b += WAVE) {
        s1 += part[((size_t)b * 2 + 0) * LKMAX + j];
        s2 += part[((size_t)b * 2 + 1) * LKMAX + j];
    }
#pragma unroll
    for (int d = WAVE / 2; d > 0; d >>= 1) {
        s1 += __shfl_xor(s1, d, WAVE);
        s2 += __shfl_xor(s2, d, WAVE);
    }
    if (lane != 0) return;
    const double m = n > 0 ? s1 / (double)n : NAN;
    const double var = n > 1 ? fmax(s2 - s1 * m, 0.0) / (double)(n - 1) : NAN;
    mu[j] = (float)m;
    sd[j] = fmaxf((float)sqrt(var), 1e-6f);
}

// uint8 inputs: exact integer sums of x and x^2, 16 rows per 16-byte load;
// grid (MU8_BLOCKS, K), one partial pair per block (no atomics).
constexpr int MU8_BLOCKS = 256;

__global__ void __launch_bounds__(LB) k_leaf_moments_u8(const uint8_t* X, int64_t ldx, int64_t n,
                                                        const int32_t* feats, uint64_t* part) {
    __shared__ uint64_t s_red[2][LB / WAVE];
    const int j = blockIdx.y;
    const uint8_t* col = X + (size_t)feats[j] * (size_t)ldx;
    uint64_t s1 = 0, s2 = 0;
    const int64_t n16 = n / 16 * 16;
    const bool vec = ((uintptr_t)col & 15u) == 0;
    const int64_t stride = (int64_t)gridDim.x * LB;
    if (vec) {
        for (int64_t i = ((int64_t)blockIdx.x * LB + threadIdx.x) * 16; i < n16; i += stride * 16) {
            const uint4 v = *reinterpret_cast<const uint4*>(col + i);
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
            uint32_t a1 = 0, a2 = 0;                  // 16 bytes: sums fit 32 bits
#pragma unroll
            for (int k = 0; k < 4; ++k)
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const uint32_t b = (w[k] >> (8 * t)) & 0xffu;
                    a1 += b;
                    a2 += b * b;
                }
            s1 += a1;
            s2 += a2;
        }
    }
    for (int64_t i = (vec ? n16 : 0) + (int64_t)blockIdx.x * LB + threadIdx.x; i < n; i += stride) {
        const uint32_t b = col[i];
        s1 += b;
        s2 += b * b;
    }
    s1 = (uint64_t)wave_sum_i64((int64_t)s1);
    s2 = (uint64_t)wave_sum_i64((int64_t)s2);
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    if (lane == 0) {
        s_red[0][w] = s1;
        s_red[1][w] = s2;
    }
    __syncthreads();
    if (threadIdx.x < 2) {
        uint64_t t = 0;
        for (int i = 0; i < LB / WAVE; ++i) t += s_red[threadIdx.x][i];
        part[((size_t)j * gridDim.x + blockIdx.x) * 2 + threadIdx.x] = t;
    }
}

// One wave per input: exact sums, then mean and unbiased variance from the
// exact n (n - 1) var = n sum x^2 - (sum x)^2.
__global__ void k_leaf_moments_u8_final(const uint64_t* part, int nblocks, int64_t n, float* mu, float* sd) {
    const int j = blockIdx.x, lane = threadIdx.x;
    uint64_t s1 = 0, s2 = 0;
    for (int b = lane; b < nblocks; b += WAVE) {
        s1 += part[((size_t)j * nblocks + b) * 2];
        s2 += part[((size_t)j * nblocks + b) * 2 + 1];
    }
    s1 = (uint64_t)wave_sum_i64((int64_t)s1);
    s2 = (uint64_t)wave_sum_i64((int64_t)s2);
    if (lane != 0) return;
    const double m = (double)s1 / (double)n;
    const __int128 num = (__int128)n * (__int128)s2 - (__int128)s1 * (__int128)s1;
    const double var = n > 1 ? (double)num / ((double)n * (double)(n - 1)) : NAN;
    mu[j] = (float)m;
    sd[j] = fmaxf((float)sqrt(var), 1e-6f);
}

size_t carve_leaf(char* base, int64_t n, int n_nodes, int K, LeafArgs* A) {
    Carve c{base, 0};
    LeafArgs tmp;
    LeafArgs& a = A ? *A : tmp;
    a.st = c.take<LeafStats>(1);
    a.count = c.take<uint32_t>((size_t)n_nodes);
    a.bcnt = c.take<uint32_t>(n_nodes <= LDS_NODES ? (size_t)LROW_BLOCKS * (size_t)n_nodes : 1);
    a.off = c.take<int64_t>((size_t)n_nodes + 1);
    a.cursor = c.take<unsigned long long>((size_t)n_nodes);
    a.sorted_x = c.take<uint8_t>((size_t)(n > 0 ? n : 1) * 4 * LKMAX);
    a.sorted_gh = c.take<float2>((size_t)(n > 0 ? n : 1));
    a.sums = c.take<int64_t>((size_t)n_nodes * gram_entries(LKMAX));
    a.parts = c.take<int64_t>(((size_t)((n + LCHUNK - 1) / LCHUNK) + (size_t)n_nodes) * gram_entries(LKMAX));
    a.lo_key = c.take<uint32_t>((size_t)n_nodes * K);
    a.hi_key = c.take<uint32_t>((size_t)n_nodes * K);
    return align_up(c.off, 256);
}

// Blocks of a Gram kernel resident on the current device at once (its
// occupancy with `lds` bytes of dynamic LDS, times the CU count), per device
// and LDS size, made on first use.
template <typename Kern>
int64_t gram_slots(Kern kern, size_t lds) {
    static std::mutex mu;
    static std::map<std::tuple<int, const void*, size_t>, int64_t> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 1024;
    const auto key = std::make_tuple(dev, reinterpret_cast<const void*>(kern), lds);
    std::lock_guard<std::mutex> g(mu);
    const auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int per_cu = 0, cus = 0;
    int64_t slots = 1024;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, LB, lds) == hipSuccess &&
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && per_cu > 0 &&
        cus > 0)
        slots = (int64_t)per_cu * cus;
    cache[key] = slots;
    return slots;
}

// GRAM_ACC's chunk: LCHUNK positions, or, when that makes more than one full
// wave of resident blocks, the size that makes the chunk count a whole
// multiple of them (a last, partial wave of blocks had left most of the
// device idle for a block's lifetime: 2442 chunks of 4096 at 10M rows on
// 1024 slots), rounded up to whole rows per thread and kept at most
// (LB / 2) 2^(k - 11) so that a thread adds at most 2^(k - 11) products per
// entry and segment (k = ceil(log2 n) >= 16 here).
inline int64_t gram_chunk(int64_t n, int64_t slots) {
    int64_t chunk = LCHUNK;
    const int64_t waves = n / (slots * LCHUNK);
    if (waves >= 1) {
        chunk = (n + slots * waves - 1) / (slots * waves);
        chunk = (chunk + LB / 2 - 1) / (LB / 2) * (LB / 2);
    }
    int k = 0;
    while (k < 62 && ((int64_t)1 << k) < n) ++k;
    const int64_t cap = (int64_t)(LB / 2) << (k > 11 ? k - 11 : 0);
    return chunk < cap ? chunk : cap;
}

template <int K>
void launch_leaf_fit(LeafArgs& A, float* out_W, float* out_b, float* out_lo, float* out_hi, int64_t* out_count,
                     hipStream_t stream) {
    const bool lds = A.n_nodes <= LDS_NODES;
    int64_t per = (A.n + LROW_BLOCKS - 1) / LROW_BLOCKS;
    per = per < LROWS ? LROWS : (per + LSB - 1) / LSB * LSB;
    A.rows_per_block = per;
    const auto al = [](const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; };
    const bool rows_al = lds && al(A.leaf, 16) && al(A.grad, 16) && al(A.hess, 16) && A.ldx % 4 == 0 && per % 4 == 0;
    A.vec4 = (rows_al && A.x_kind == 1 && al(A.X, 4)) ? 1 : (rows_al && A.x_kind == 2 && al(A.X, 16)) ? 2 : 0;
    const int row_blocks = (int)((A.n + per - 1) / per);
    k_leaf_init<<<launch_grid((int64_t)A.n_nodes * gram_entries(LKMAX), LB, 1024), LB, 0, stream>>>(A, K);
    if (lds) {
        if (row_blocks > 0) k_leaf_count<<<row_blocks, LSB, 0, stream>>>(A);
        k_leaf_offsets<<<1, 1024, 0, stream>>>(A);
        if (row_blocks > 0) k_leaf_scatter_stats<K><<<row_blocks, LSB, 0, stream>>>(A);
        k_leaf_shifts<<<1, 1024, 0, stream>>>(A, K);
    } else {
        if (row_blocks > 0) k_leaf_stats<K><<<row_blocks, LSB, 0, stream>>>(A);
        k_leaf_offsets<<<1, 1024, 0, stream>>>(A);
        k_leaf_shifts<<<1, 1024, 0, stream>>>(A, K);
        if (row_blocks > 0) k_leaf_scatter<K><<<row_blocks, LSB, 0, stream>>>(A);
    }
    if (row_blocks > 0) {
        const int chunks = (int)((A.n + LCHUNK - 1) / LCHUNK);
        if (A.gram_f64) {
            k_leaf_gram_mfma<K><<<chunks, LB, 0, stream>>>(A);
            k_leaf_reduce<K><<<A.n_nodes, RB, 0, stream>>>(A);
        } else {
            // dynamic LDS: the chunk's segment list
            A.gram_chunk = LCHUNK;
            if (A.n > 32768) A.gram_chunk = gram_chunk(A.n, gram_slots(k_leaf_gram<K, GRAM_ACC>, 0));
            const size_t seg_lds = sizeof(int) * (size_t)std::min<int64_t>(A.n_nodes, A.gram_chunk);
            const int gc = (int)((A.n + A.gram_chunk - 1) / A.gram_chunk);
            if (A.n > 32768) k_leaf_gram<K, GRAM_ACC><<<gc, LB, seg_lds, stream>>>(A);
            else if (A.n > 1024) k_leaf_gram<K, GRAM_MAGIC><<<gc, LB, seg_lds, stream>>>(A);
            else k_leaf_gram<K, GRAM_RINT><<<gc, LB, seg_lds, stream>>>(A);
        }
    }
    constexpr int per_block = LB / SOLVE_LANES;   // nodes per solve block
    k_leaf_solve<K><<<(A.n_nodes + per_block - 1) / per_block, LB, 0, stream>>>(A, out_W, out_b, out_lo, out_hi,
                                                                               out_count);
}

// ---------------------------------------------------------------------------
// the leaf models' inputs: the tree's split features, most used first
// (neural_leaves.py:27-31), ranked on the device
// ---------------------------------------------------------------------------
//
// The reference takes torch.unique of the internal nodes' features (ascending
// features, their counts), then argsort of the counts, descending, on the
// CPU.  That argsort is libstdc++'s std::sort over (count, position) pairs
// compared by count alone, so its order of equal counts is the introsort's:
// median-of-three partitions (pivot moved to the front, unguarded Hoare
// scans) until 16 elements or 2 floor(log2 m) levels, a heap sort of a range
// past that depth, then one insertion sort of the whole list (the first 16
// guarded, the rest unguarded).  The ranking below runs those steps in one
// lane over an LDS list; a range's steps depend only on the range, so a stack
// of ranges replaces the recursion without changing the order.

constexpr int RANK_T = 256;
constexpr int RANK_MAX_F = 4096;               // features the device ranking takes, at most

struct RankEl {
    int32_t c, f;                              // count, feature
};

namespace rank {

__device__ __forceinline__ bool gt(const RankEl& a, const RankEl& b) { return a.c > b.c; }
__device__ __forceinline__ void swap_at(RankEl* v, int a, int b) {
    const RankEl t = v[a];
    v[a] = v[b];
    v[b] = t;
}

// Sift a hole at `hole` down to a leaf of the heap v[0, len), then `value`
// up from there (the heap's parent is never smaller under gt).
__device__ __forceinline__ void adjust_heap(RankEl* v, int hole, int len, RankEl value) {
    const int top = hole;
    int child = hole;
    while (child < (len - 1) / 2) {
        child = 2 * (child + 1);
        if (gt(v[child], v[child - 1])) --child;
        v[hole] = v[child];
        hole = child;
    }
    if ((len & 1) == 0 && child == (len - 2) / 2) {
        child = 2 * (child + 1);
        v[hole] = v[child - 1];
        hole = child - 1;
    }
    int parent = (hole - 1) / 2;
    while (hole > top && gt(v[parent], value)) {
        v[hole] = v[parent];
        hole = parent;
        parent = (hole - 1) / 2;
    }
    v[hole] = value;
}

// Heap sort of v[0, len): build the heap, then pop its top to the back.
__device__ __forceinline__ void heap_sort(RankEl* v, int len) {
    if (len < 2) return;
    for (int parent = (len - 2) / 2;; --parent) {
        adjust_heap(v, parent, len, v[parent]);
        if (parent == 0) break;
    }
    for (int last = len - 1; last > 0; --last) {
        const RankEl value = v[last];
        v[last] = v[0];
        adjust_heap(v, 0, last, value);
    }
}

// The median of v[a], v[b], v[c] swapped into v[r].
__device__ __forceinline__ void median_to(RankEl* v, int r, int a, int b, int c) {
    if (gt(v[a], v[b])) {
        if (gt(v[b], v[c])) swap_at(v, r, b);
        else if (gt(v[a], v[c])) swap_at(v, r, c);
        else swap_at(v, r, a);
    } else if (gt(v[a], v[c])) {
        swap_at(v, r, a);
    } else if (gt(v[b], v[c])) {
        swap_at(v, r, c);
    } else {
        swap_at(v, r, b);
    }
}

// Hoare partition of v[lo, hi) around v[p] (p < lo), without bounds tests.
__device__ __forceinline__ int partition(RankEl* v, int lo, int hi, int p) {
    for (;;) {
        while (gt(v[lo], v[p])) ++lo;
        --hi;
        while (gt(v[p], v[hi])) --hi;
        if (!(lo < hi)) return lo;
        swap_at(v, lo, hi);
        ++lo;
    }
}

// Insert v[i] into the sorted run before it, without a bounds test.
__device__ __forceinline__ void linear_insert(RankEl* v, int i) {
    const RankEl val = v[i];
    int j = i - 1;
    while (gt(val, v[j])) {
        v[i] = v[j];
        i = j;
        --j;
    }
    v[i] = val;
}

// The first k positions of std::sort over v[0, m).  Every element of a
// partitioned range is >= every element of the ranges after it (the pivot
// stays at the front of the left range), and the final insertion sort never
// moves an element past one that is not smaller, so a range that starts at k
// or later never reaches the first k: it is left unsorted, and the insertion
// sort stops at the end E of the ranges holding positions below k.
__device__ __forceinline__ void sort(RankEl* v, int m, int k, int* stk) {
    if (m < 2) return;
    int top = 0, E = 0;
    int first = 0, last = m, depth = 2 * (31 - __clz(m));
    for (;;) {
        while (last - first > 16) {
            if (depth == 0) {
                heap_sort(v + first, last - first);
                break;
            }
            --depth;
            const int mid = first + (last - first) / 2;
            median_to(v, first, first + 1, mid, last - 1);
            const int cut = partition(v, first + 1, last, first);
            if (cut < k) {   // [cut, last) at this depth, later
                stk[3 * top] = cut;
                stk[3 * top + 1] = last;
                stk[3 * top + 2] = depth;
                ++top;
            }
            last = cut;
        }
        E = last > E ? last : E;   // [first, last), first < k, is final
        if (top == 0) break;
        --top;
        first = stk[3 * top];
        last = stk[3 * top + 1];
        depth = stk[3 * top + 2];
    }
    // the final insertion sort, over [0, E)
    const int g = E > 16 ? 16 : E;
    for (int i = 1; i < g; ++i) {
        if (gt(v[i], v[0])) {
            const RankEl val = v[i];
            for (int j = i; j > 0; --j) v[j] = v[j - 1];
            v[0] = val;
        } else {
            linear_insert(v, i);
        }
    }
    for (int i = g; i < E; ++i) linear_insert(v, i);
}

}  // namespace rank

// One block: counts per feature in LDS, the used features listed in
// ascending order by wave 0, the list sorted by lane 0, the first k written
// (positions past the list get feature 0, so that launches made before the
// host reads *out_m stay in bounds).  *out_m: the number of used features,
// -1 if a node names a feature outside [0, F).
__global__ void __launch_bounds__(RANK_T) k_rank_features(const int64_t* __restrict__ feature, int n_nodes, int F,
                                                          int k, int64_t* __restrict__ out64,
                                                          int32_t* __restrict__ out32, int32_t* __restrict__ out_m) {
    __shared__ uint32_t s_cnt[RANK_MAX_F];
    __shared__ RankEl s_el[RANK_MAX_F];
    __shared__ int s_stk[3 * 64];
    __shared__ int s_m, s_bad;
    for (int f = threadIdx.x; f < F; f += RANK_T) s_cnt[f] = 0u;
    if (threadIdx.x == 0) s_bad = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < n_nodes; i += RANK_T) {
        const int64_t f = feature[i];
        if (f >= F) s_bad = 1;
        else if (f >= 0) atomicAdd(&s_cnt[f], 1u);
    }
    __syncthreads();
    if (threadIdx.x < WAVE) {
        const int lane = threadIdx.x;
        int m = 0;
        for (int f0 = 0; f0 < F; f0 += WAVE) {
            const int f = f0 + lane;
            const uint32_t c = f < F ? s_cnt[f] : 0u;
            const uint64_t bal = __ballot(c > 0u);
            if (c > 0u) {
                const int pos = m + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                                   __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
                s_el[pos].c = (int32_t)c;
                s_el[pos].f = f;
            }
            m += __popcll(bal);
        }
        if (lane == 0) {
            s_m = m;
            rank::sort(s_el, m, k, s_stk);
        }
    }
    __syncthreads();
    const int m = s_m;
    if ((int)threadIdx.x < k) {
        const int f = (int)threadIdx.x < m ? s_el[threadIdx.x].f : 0;
        out64[threadIdx.x] = f;
        out32[threadIdx.x] = f;
    }
    if (threadIdx.x == 0) out_m[0] = s_bad ? -1 : m;
}

}  // namespace yabt

using namespace yabt;

extern "C" {

size_t yabt_leaf_fit_workspace_bytes(int64_t n, int n_nodes, int K) {
    if (n < 0 || n_nodes < 1 || K < 1 || K > LKMAX) return 0;
    return carve_leaf(nullptr, n, n_nodes, K, nullptr);
}

}  // extern "C"

// yabt_leaf_fit's launches; the status words by k_leaf_status unless the
// caller takes the fit's LeafStats (*st_out) to copy them itself.
static int leaf_fit_launch(int x_kind, const void* X, int64_t ldx, int64_t n, const int32_t* feats, int K,
                           const float* mu, const float* sd, const float* grad, const float* hess,
                           const int64_t* leaf_of_row, const int64_t* feature, int n_nodes, int min_samples,
                           double lam, int gram_mode, void* workspace, size_t workspace_bytes, float* out_W,
                           float* out_b, float* out_lo, float* out_hi, int64_t* out_count, int32_t* out_status,
                           hipStream_t stream, const LeafStats** st_out) {
    if (n < 0 || n > 0xFFFFFFFFll || n_nodes < 1 || K < 1 || K > LKMAX || x_kind < 0 || x_kind > 2)
        return fail(-2, "yabt_leaf_fit: bad sizes (need 0 <= n < 2^32, n_nodes >= 1, 1 <= K <= 8, x_kind 0, 1 or 2)");
    if (gram_mode != 0 && gram_mode != 1) return fail(-2, "yabt_leaf_fit: gram_mode must be 0 or 1");
    if (!X || !feats || !mu || !sd || !grad || !hess || !leaf_of_row || !feature || !workspace || !out_W || !out_b ||
        !out_lo || !out_hi || !out_count || !out_status)
        return fail(-2, "yabt_leaf_fit: null pointer argument");
    if (x_kind != 0 ? ldx < n : ldx < 1) return fail(-2, "yabt_leaf_fit: leading dimension too small");
    LeafArgs A;
    memset(&A, 0, sizeof A);
    const size_t need = carve_leaf((char*)workspace, n, n_nodes, K, &A);
    if (workspace_bytes < need) return fail(-2, "yabt_leaf_fit: workspace too small");
    A.x_kind = x_kind;
    A.X = X;
    A.ldx = ldx;
    A.n = n;
    A.feats = feats;
    A.mu = mu;
    A.sd = sd;
    A.grad = grad;
    A.hess = hess;
    A.leaf = leaf_of_row;
    A.feature = feature;
    A.n_nodes = n_nodes;
    A.min_samples = min_samples;
    A.lam = lam;
    A.gram_f64 = gram_mode;
    switch (K) {
        case 1: launch_leaf_fit<1>(A, out_W, out_b, out_lo, out_hi, out_count, stream); break;
        case 2: launch_leaf_fit<2>(A, out_W, out_b, out_lo, out_hi, out_count, stream); break;
        case 3: launch_leaf_fit<3>(A, out_W, out_b, out_lo, out_hi, out_count, stream); break;
        case 4: launch_leaf_fit<4>(A, out_W, out_b, out_lo, out_hi, out_count, stream); break;
        case 5: launch_leaf_fit<5>(A, out_W, out_b, out_lo, out_hi, out_count, stream); break;
        case 6: launch_leaf_fit<6>(A, out_W, out_b, out_lo, out_hi, out_count, stream); break;
        case 7: launch_leaf_fit<7>(A, out_W, out_b, out_lo, out_hi, out_count, stream); break;
        default: launch_leaf_fit<8>(A, out_W, out_b, out_lo, out_hi, out_count, stream); break;
    }
    if (st_out) *st_out = A.st;
    else k_leaf_status<<<1, 1, 0, stream>>>(A.st, out_status);
    return launch_status("yabt_leaf_fit launch");
}

extern "C" {

int yabt_leaf_fit(int x_kind, const void* X, int64_t ldx, int64_t n, const int32_t* feats, int K, const float* mu,
                  const float* sd, const float* grad, const float* hess, const int64_t* leaf_of_row,
                  const int64_t* feature, int n_nodes, int min_samples, double lam, int gram_mode,
                  void* workspace, size_t workspace_bytes, float* out_W, float* out_b, float* out_lo,
                  float* out_hi, int64_t* out_count, int32_t* out_status, hipStream_t stream) {
    return leaf_fit_launch(x_kind, X, ldx, n, feats, K, mu, sd, grad, hess, leaf_of_row, feature, n_nodes,
                           min_samples, lam, gram_mode, workspace, workspace_bytes, out_W, out_b, out_lo, out_hi,
                           out_count, out_status, stream, nullptr);
}

int yabt_leaf_step(int x_kind, const void* X, int64_t ldx, int64_t n, int F, int K, const float* grad,
                   const float* hess, const int64_t* leaf_of_row, const int64_t* feature, const float* value_in,
                   int n_nodes, int min_samples, double lam, float lr, int gram_mode, void* ws_moments,
                   size_t ws_moments_bytes, void* ws_fit, size_t ws_fit_bytes, int64_t* out_feats,
                   int32_t* out_feats32, float* out_mu, float* out_sd, float* out_W, float* out_b, float* out_lo,
                   float* out_hi, int64_t* out_count, float* out_value, float* out_linear, int32_t* out_status,
                   hipStream_t stream) {
    if (!out_status) return fail(-2, "yabt_leaf_step: null pointer argument");
    int rc = yabt_leaf_rank_features(feature, n_nodes, F, K, out_feats, out_feats32, out_status + 2, stream);
    if (rc) return rc;
    rc = yabt_leaf_moments(x_kind, X, ldx, n, out_feats32, K, ws_moments, ws_moments_bytes, out_mu, out_sd, stream);
    if (rc) return rc;
    const LeafStats* st = nullptr;
    rc = leaf_fit_launch(x_kind, X, ldx, n, out_feats32, K, out_mu, out_sd, grad, hess, leaf_of_row, feature,
                         n_nodes, min_samples, lam, gram_mode, ws_fit, ws_fit_bytes, out_W, out_b, out_lo, out_hi,
                         out_count, out_status, stream, &st);
    if (rc) return rc;
    if (!out_value || !out_linear || !value_in) return fail(-2, "yabt_leaf_step: null pointer argument");
    k_leaf_fold<<<(n_nodes + LB - 1) / LB, LB, 0, stream>>>(n_nodes, K, out_W, out_b, out_mu, out_sd, lr, value_in,
                                                           out_value, out_linear, st, out_status);
    return launch_status("yabt_leaf_step launch");
}

int yabt_leaf_fold(int n_nodes, int K, const float* W, const float* b, const float* mu, const float* sd, float lr,
                   const float* value_in, float* out_value, float* out_linear, hipStream_t stream) {
    if (n_nodes < 1 || K < 1 || K > LKMAX) return fail(-2, "yabt_leaf_fold: bad sizes (n_nodes >= 1, 1 <= K <= 8)");
    if (!W || !b || !mu || !sd || !value_in || !out_value || !out_linear)
        return fail(-2, "yabt_leaf_fold: null pointer argument");
    k_leaf_fold<<<(n_nodes + LB - 1) / LB, LB, 0, stream>>>(n_nodes, K, W, b, mu, sd, lr, value_in, out_value,
                                                           out_linear, nullptr, nullptr);
    return launch_status("yabt_leaf_fold launch");
}

int yabt_leaf_rank_features(const int64_t* feature, int n_nodes, int F, int k, int64_t* out_feats,
                            int32_t* out_feats32, int32_t* out_m, hipStream_t stream) {
    if (n_nodes < 1 || F < 1 || F > RANK_MAX_F || k < 1 || k > LKMAX)
        return fail(-2, "yabt_leaf_rank_features: bad sizes (n_nodes >= 1, 1 <= F <= 4096, 1 <= k <= 8)");
    if (!feature || !out_feats || !out_feats32 || !out_m)
        return fail(-2, "yabt_leaf_rank_features: null pointer argument");
    k_rank_features<<<1, RANK_T, 0, stream>>>(feature, n_nodes, F, k, out_feats, out_feats32, out_m);
    return launch_status("yabt_leaf_rank_features launch");
}

size_t yabt_leaf_moments_workspace_bytes(int64_t n) {
    if (n < 0) return 0;
    const int64_t nb = n > 0 ? (n + MROWS - 1) / MROWS : 1;
    const size_t f = (size_t)nb * 2 * LKMAX * sizeof(double), u = (size_t)MU8_BLOCKS * LKMAX * 2 * sizeof(uint64_t);
    return align_up(f > u ? f : u, 256);
}

int yabt_leaf_moments(int x_kind, const void* X, int64_t ldx, int64_t n, const int32_t* feats, int K,
                      void* workspace, size_t workspace_bytes, float* out_mu, float* out_sd, hipStream_t stream) {
    if (n < 1 || K < 1 || K > LKMAX || x_kind < 0 || x_kind > 2)
        return fail(-2, "yabt_leaf_moments: bad sizes (need n >= 1, 1 <= K <= 8, x_kind 0, 1 or 2)");
    if (!X || !feats || !workspace || !out_mu || !out_sd) return fail(-2, "yabt_leaf_moments: null pointer argument");
    if (x_kind != 0 ? ldx < n : ldx < 1) return fail(-2, "yabt_leaf_moments: leading dimension too small");
    if (workspace_bytes < yabt_leaf_moments_workspace_bytes(n)) return fail(-2, "yabt_leaf_moments: workspace too small");
    const int nb = (int)((n + MROWS - 1) / MROWS);
    double* part = (double*)workspace;
    if (x_kind == 1) {
        const int gb = launch_grid((n + 15) / 16, LB, MU8_BLOCKS);
        k_leaf_moments_u8<<<dim3(gb, K), LB, 0, stream>>>((const uint8_t*)X, ldx, n, feats, (uint64_t*)workspace);
        k_leaf_moments_u8_final<<<K, WAVE, 0, stream>>>((const uint64_t*)workspace, gb, n, out_mu, out_sd);
        return launch_status("yabt_leaf_moments launch");
    }
    switch (K) {
        case 1: k_leaf_moments<1><<<nb, LB, 0, stream>>>(x_kind, X, ldx, n, feats, part); break;
        case 2: k_leaf_moments<2><<<nb, LB, 0, stream>>>(x_kind, X, ldx, n, feats, part); break;
        case 3: k_leaf_moments<3><<<nb, LB, 0, stream>>>(x_kind, X, ldx, n, feats, part); break;
        case 4: k_leaf_moments<4><<<nb, LB, 0, stream>>>(x_kind, X, ldx, n, feats, part); break;
        case 5: k_leaf_moments<5><<<nb, LB, 0, stream>>>(x_kind, X, ldx, n, feats, part); break;
        case 6: k_leaf_moments<6><<<nb, LB, 0, stream>>>(x_kind, X, ldx, n, feats, part); break;
        case 7: k_leaf_moments<7><<<nb, LB, 0, stream>>>(x_kind, X, ldx, n, feats, part); break;
        default: k_leaf_moments<8><<<nb, LB, 0, stream>>>(x_kind, X, ldx, n, feats, part); break;
    }
    k_leaf_moments_final<<<K, WAVE, 0, stream>>>(part, nb, n, K, out_mu, out_sd);
    return launch_status("yabt_leaf_moments launch");
}

}  // extern "C"
