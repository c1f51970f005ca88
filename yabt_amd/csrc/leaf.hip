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
// Launch sequence (caller's stream):
//   k_leaf_init        clear counters, sums, envelopes
//   k_leaf_stats<K>    rows per node, envelopes min/max of raw x, max |x1|, |g|, |h|
//   k_leaf_offsets     node offsets of the sorted rows, fixed-point shifts
//   k_leaf_scatter     rows -> sorted by node
//   k_leaf_gram<K>     fixed-point sums of M and b per (chunk, leaf) segment
//   k_leaf_reduce<K>   per-leaf sums of the segments
//   k_leaf_solve<K>    fp64 LU with partial pivoting per eligible leaf

#include "common.h"
#include "host.h"
#include "yabt_hip.h"

#include <string.h>

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
    int x_kind;                // 0: fp32 row-major (n, ldx); 1: uint8 feature-major (F, ldx)
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
    int vec4;                  // 1: uint8 inputs, leaf ids, g and h aligned for 4-row vector loads
    // workspace
    LeafStats* st;
    uint32_t* count;           // (n_nodes)
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

// Rows [blockIdx.x * rows_per_block, +rows_per_block): counts, envelopes and
// magnitudes.
template <int K, bool LDS>
__global__ void __launch_bounds__(LSB) k_leaf_stats(LeafArgs A) {
    __shared__ uint32_t s_cnt[LDS ? LDS_NODES : 1];
    __shared__ uint32_t s_lo[LDS ? LDS_NODES * K : 1], s_hi[LDS ? LDS_NODES * K : 1];
    __shared__ float s_red[3][LSB / WAVE];
    __shared__ int s_bad;
    __shared__ int32_t s_fs[LKMAX];
    if (threadIdx.x < K) s_fs[threadIdx.x] = A.feats[threadIdx.x];
    if (threadIdx.x == 0) s_bad = 0;
    if (LDS) {
        for (int i = threadIdx.x; i < A.n_nodes; i += LSB) s_cnt[i] = 0;
        for (int i = threadIdx.x; i < A.n_nodes * K; i += LSB) {
            s_lo[i] = float_key(INFINITY);
            s_hi[i] = float_key(-INFINITY);
        }
    }
    __syncthreads();
    const int64_t lo = (int64_t)blockIdx.x * A.rows_per_block, hi = min(A.n, lo + A.rows_per_block);
    float mg = 0.0f, mh = 0.0f;
    int bad = 0;
    auto add_row = [&](int64_t node, const float (&x)[K], float gi, float hi_) {
        if (node < 0 || node >= A.n_nodes) {
            bad = 1;
            return;
        }
        if (!isfinite(gi) || !isfinite(hi_)) bad = 1;
        mg = fmaxf(mg, fabsf(gi));
        mh = fmaxf(mh, fabsf(hi_));
        // per-node envelopes; their extremes also bound |x1| (k_leaf_offsets) and
        // expose non-finite inputs (keys beyond those of -inf / +inf)
#pragma unroll
        for (int j = 0; j < K; ++j) {
            // the extremes settle quickly: read first, update only when improving
            const uint32_t kx = float_key(x[j]);
            uint32_t* plo = LDS ? &s_lo[node * K + j] : &A.lo_key[node * K + j];
            uint32_t* phi = LDS ? &s_hi[node * K + j] : &A.hi_key[node * K + j];
            if (kx < *(volatile uint32_t*)plo) atomicMin(plo, kx);
            if (kx > *(volatile uint32_t*)phi) atomicMax(phi, kx);
        }
        if (LDS) atomicAdd(&s_cnt[node], 1u);
        else atomicAdd(&A.count[node], 1u);
    };
    int64_t first = lo;   // rows from here on take the one-row loop
    if (A.vec4) {
        // four consecutive rows per thread and step, every load a vector
        const int64_t ng = (hi - lo) / 4;
        for (int64_t q = threadIdx.x; q < ng; q += LSB) {
            Rows4<K> R;
            load_rows4<K>(A, s_fs, lo + 4 * q, R);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float x[K];
#pragma unroll
                for (int j = 0; j < K; ++j) x[j] = (float)((R.xw[j] >> (8 * r)) & 0xffu);
                add_row(R.node[r], x, R.g[r], R.h[r]);
            }
        }
        first = lo + 4 * ng;
    }
    for (int64_t i = first + threadIdx.x; i < hi; i += LSB) {
        const int64_t node = A.leaf[i];
        if (node < 0 || node >= A.n_nodes) {
            bad = 1;
            continue;
        }
        float x[K];
        load_x<K>(A, i, s_fs, x);
        add_row(node, x, A.grad[i], A.hess[i]);
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
    if (LDS) {
        for (int i = threadIdx.x; i < A.n_nodes; i += LSB)
            if (s_cnt[i]) atomicAdd(&A.count[i], s_cnt[i]);
        for (int i = threadIdx.x; i < A.n_nodes * K; i += LSB) {
            if (s_lo[i] != float_key(INFINITY)) atomicMin(&A.lo_key[i], s_lo[i]);
            if (s_hi[i] != float_key(-INFINITY)) atomicMax(&A.hi_key[i], s_hi[i]);
        }
    }
}

// One block: node offsets of the sorted rows (exclusive scan of the counts),
// write cursors, and the fixed-point shifts.
__global__ void __launch_bounds__(1024) k_leaf_offsets(LeafArgs A, int K) {
    __shared__ int64_t s_wave[1024 / WAVE];
    __shared__ uint32_t s_xlo[LKMAX], s_xhi[LKMAX];
    if (threadIdx.x < K) {
        s_xlo[threadIdx.x] = float_key(INFINITY);
        s_xhi[threadIdx.x] = float_key(-INFINITY);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < A.n_nodes * K; i += 1024) {
        atomicMin(&s_xlo[i % K], A.lo_key[i]);
        atomicMax(&s_xhi[i % K], A.hi_key[i]);
    }
    __syncthreads();
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
    if (threadIdx.x == 0) {
        A.off[A.n_nodes] = carry;
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

// Rows [blockIdx.x * rows_per_block, +rows_per_block) to their node's range
// of `sorted`; the block reserves one range per node with one atomic add.
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
        const float* row = reinterpret_cast<const float*>(A.X) + (size_t)i * (size_t)A.ldx;
        float* dst = reinterpret_cast<float*>(A.sorted_x) + pos * K;
#pragma unroll
        for (int j = 0; j < K; ++j) dst[j] = row[fs[j]];
    }
}

template <int K, bool LDS>
__global__ void __launch_bounds__(LSB) k_leaf_scatter(LeafArgs A) {
    __shared__ int32_t s_fs[LKMAX];
    if (threadIdx.x < K) s_fs[threadIdx.x] = A.feats[threadIdx.x];
    __shared__ uint32_t s_cnt[LDS ? LDS_NODES : 1];
    __shared__ unsigned long long s_base[LDS ? LDS_NODES : 1];
    if (LDS)
        for (int i = threadIdx.x; i < A.n_nodes; i += LSB) s_cnt[i] = 0;
    __syncthreads();
    const int64_t lo = (int64_t)blockIdx.x * A.rows_per_block, hi = min(A.n, lo + A.rows_per_block);
    if (LDS) {
        // vec4: rows [lo, first) in groups of four per thread, the rest one by one
        const int64_t ng = A.vec4 ? (hi - lo) / 4 : 0, first = lo + 4 * ng;
        for (int64_t q = threadIdx.x; q < ng; q += LSB) {
            const longlong2 la = *reinterpret_cast<const longlong2*>(A.leaf + lo + 4 * q);
            const longlong2 lb = *reinterpret_cast<const longlong2*>(A.leaf + lo + 4 * q + 2);
            const int64_t nd[4] = {la.x, la.y, lb.x, lb.y};
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (nd[r] >= 0 && nd[r] < A.n_nodes) atomicAdd(&s_cnt[nd[r]], 1u);
        }
        for (int64_t i = first + threadIdx.x; i < hi; i += LSB) {
            const int64_t node = A.leaf[i];
            if (node >= 0 && node < A.n_nodes) atomicAdd(&s_cnt[node], 1u);
        }
        __syncthreads();
        for (int i = threadIdx.x; i < A.n_nodes; i += LSB) {
            s_base[i] = s_cnt[i] ? atomicAdd(&A.cursor[i], (unsigned long long)s_cnt[i]) : 0ull;
            s_cnt[i] = 0;
        }
        __syncthreads();
        for (int64_t q = threadIdx.x; q < ng; q += LSB) {
            Rows4<K> R;
            load_rows4<K>(A, s_fs, lo + 4 * q, R);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t node = R.node[r];
                if (node < 0 || node >= A.n_nodes) continue;
                const uint64_t pos = s_base[node] + atomicAdd(&s_cnt[node], 1u);
                A.sorted_gh[pos] = make_float2(R.g[r], R.h[r]);
                uint32_t w0 = 0, w1 = 0;
#pragma unroll
                for (int j = 0; j < K; ++j) {
                    const uint32_t b = (R.xw[j] >> (8 * r)) & 0xffu;
                    if (j < 4) w0 |= b << (8 * j);
                    else w1 |= b << (8 * (j - 4));
                }
                reinterpret_cast<uint2*>(A.sorted_x)[pos] = make_uint2(w0, w1);
            }
        }
        for (int64_t i = first + threadIdx.x; i < hi; i += LSB) {
            const int64_t node = A.leaf[i];
            if (node < 0 || node >= A.n_nodes) continue;
            const uint32_t r = atomicAdd(&s_cnt[node], 1u);
            put_sorted<K>(A, s_fs, i, s_base[node] + r);
        }
    } else {
        for (int64_t i = lo + threadIdx.x; i < hi; i += LSB) {
            const int64_t node = A.leaf[i];
            if (node < 0 || node >= A.n_nodes) continue;
            put_sorted<K>(A, s_fs, i, atomicAdd(&A.cursor[node], 1ull));
        }
    }
}

__device__ __forceinline__ bool leaf_eligible(const LeafArgs& A, int node) {
    return A.feature[node] == LEAF && (int64_t)A.count[node] >= (int64_t)A.min_samples;
}

// Standardised uint8 inputs take 256 values per input: s_x1[j * 256 + b] =
// (double)((float(b) - mu[j]) / sd[j]), x1 formed in fp32 as the reference
// forms it (neural_leaves.py:152-155), one table per block in LDS.
template <int K, int NT>
__device__ __forceinline__ void x1_table(double* s_x1, const float* mu, const float* sd) {
    for (int i = threadIdx.x; i < K * 256; i += NT) {
        const int j = i / 256, b = i % 256;
        s_x1[i] = (double)(((float)b - mu[j]) / sd[j]);
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

// The fixed-point products of half P of a row's gram_entries (P = 0: entries
// [0, NE/2), 1: [NE/2, NE)), added into acc[t - the half's first entry].
// FAST: rounded to integers through the bits of v + 1.5 * 2^52 (round to
// nearest even, as rint; the constant's bits come off once per row later).
template <int K, bool FAST, int P>
__device__ __forceinline__ void gram_half(const double (&x1)[K + 1], const double (&xhs)[K + 1], double gs,
                                          uint64_t (&acc)[(gram_entries(K) + 1) / 2]) {
    constexpr int NE = gram_entries(K);
    constexpr int T0 = P == 0 ? 0 : (NE + 1) / 2, T1 = P == 0 ? (NE + 1) / 2 : NE;
    constexpr double MAGIC = 6755399441055744.0;   // 1.5 * 2^52
    int t = 0;
#pragma unroll
    for (int a = 0; a <= K; ++a) {
#pragma unroll
        for (int b = a; b <= K; ++b, ++t) {
            if (t < T0 || t >= T1) continue;
            const double v = x1[a] * xhs[b];      // the reference's product, times 2^sM exactly
            if (FAST) acc[t - T0] += (uint64_t)__double_as_longlong(v + MAGIC);
            else acc[t - T0] += (uint64_t)(int64_t)rint(v);
        }
    }
#pragma unroll
    for (int a = 0; a <= K; ++a, ++t) {            // rhs = -(X1 * g)
        if (t < T0 || t >= T1) continue;
        const double v = -(x1[a] * gs);
        if (FAST) acc[t - T0] += (uint64_t)__double_as_longlong(v + MAGIC);
        else acc[t - T0] += (uint64_t)(int64_t)rint(v);
    }
}

// One half-block's rows p = p0, p0 + LB / 2, ... < e of a segment: x1 and
// x1 h from the row, then half P of its products into acc.
template <int K, bool FAST, int P>
__device__ __forceinline__ void gram_rows(const LeafArgs& A, const double* s_x1, const float* s_mu,
                                          const float* s_sd, double scM, double scb, int64_t p0, int64_t e,
                                          uint64_t (&acc)[(gram_entries(K) + 1) / 2]) {
    constexpr double MAGIC = 6755399441055744.0;   // 1.5 * 2^52
    uint64_t nrow = 0;
    for (int64_t p = p0; p < e; p += LB / 2) {
        const float2 gh = A.sorted_gh[p];
        double x1[K + 1];
        if (A.x_kind == 1) {
            const uint2 v = reinterpret_cast<const uint2*>(A.sorted_x)[p];
#pragma unroll
            for (int j = 0; j < K; ++j) x1[j] = s_x1[j * 256 + (((j < 4 ? v.x : v.y) >> (8 * (j & 3))) & 0xffu)];
        } else {
            const float* src = reinterpret_cast<const float*>(A.sorted_x) + (size_t)p * K;
#pragma unroll
            for (int j = 0; j < K; ++j) x1[j] = (double)((src[j] - s_mu[j]) / s_sd[j]);
        }
        x1[K] = 1.0;
        const double h = (double)gh.y;
        const double gs = (double)gh.x * scb;           // exact power-of-two scaling
        double xhs[K + 1];
#pragma unroll
        for (int b = 0; b <= K; ++b) xhs[b] = (x1[b] * h) * scM;   // Xh = X1 * h (neural_leaves.py:72), scaled
        ++nrow;
        gram_half<K, FAST, P>(x1, xhs, gs, acc);
    }
    if (FAST) {
        const uint64_t off = nrow * (uint64_t)__double_as_longlong(MAGIC);
#pragma unroll
        for (int t = 0; t < (gram_entries(K) + 1) / 2; ++t) acc[t] -= off;
    }
}

// Sorted positions [blockIdx.x * LCHUNK, +LCHUNK): for each node run inside
// the chunk, the block's two halves (waves 0-1 and 2-3) each sum half of the
// gram_entries over every row of the run, a thread's rows in registers
// (half the accumulators per thread: twice the resident waves); waves reduce
// with DPP and the block's sums go to the segment's own partial slot.
// FAST (n > 1024, so every scaled product is below 2^51 in magnitude): the
// products are rounded by the 1.5 * 2^52 trick; otherwise rint.
template <int K, bool FAST>
__global__ void __launch_bounds__(LB) k_leaf_gram(LeafArgs A) {
    constexpr int NE = gram_entries(K);
    constexpr int NH = (NE + 1) / 2;              // entries of the first half (the second has NE - NH)
    constexpr int HT = LB / 2;                    // threads per half
    __shared__ float s_mu[LKMAX], s_sd[LKMAX];
    __shared__ int64_t s_part[LB / WAVE][NH];
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
    const double scM = ldexp(1.0, A.st->sM), scb = ldexp(1.0, A.st->sb);
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    const int half = threadIdx.x / HT, th = threadIdx.x % HT;   // wave-uniform half
    for (int node = node_at(A, c0); node < A.n_nodes && A.off[node] < c1; ++node) {
        const int64_t s = max(c0, A.off[node]), e = min(c1, A.off[node + 1]);
        if (s >= e || !leaf_eligible(A, node)) continue;   // uniform across the block
        uint64_t acc[NH];
#pragma unroll
        for (int t = 0; t < NH; ++t) acc[t] = 0;
        if (half == 0) gram_rows<K, FAST, 0>(A, s_x1, s_mu, s_sd, scM, scb, s + th, e, acc);
        else gram_rows<K, FAST, 1>(A, s_x1, s_mu, s_sd, scM, scb, s + th, e, acc);
        // block sum of this (chunk, node) segment into its own partial slot,
        // chunk + node: distinct for every segment (nodes and chunks both
        // advance along the sorted rows), so no atomics and no contention
        const int nh = half == 0 ? NH : NE - NH;
#pragma unroll
        for (int t = 0; t < NH; ++t) {
            const int64_t v = wave_sum_i64((int64_t)acc[t]);
            if (lane == 0 && t < nh) s_part[w][t] = v;
        }
        __syncthreads();
        int64_t* out = A.parts + ((size_t)blockIdx.x + (size_t)node) * gram_entries(LKMAX);
        constexpr int HW = HT / WAVE;                 // waves per half
        for (int t = threadIdx.x; t < NE; t += LB) {
            const int hh = t < NH ? 0 : 1, tt = t < NH ? t : t - NH;
            int64_t v = 0;
#pragma unroll
            for (int i = 0; i < HW; ++i) v += s_part[hh * HW + i][tt];
            out[t] = v;
        }
        __syncthreads();
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

// One block per eligible node: the sum of its segments' partials (chunks
// first_chunk .. last_chunk of the sorted rows) in a fixed order -- wave w
// takes segments w, w + RW, ... (lane t: entry t), then the waves' sums in
// order.  F64: the partials are fp64 bits (k_leaf_gram_mfma).
constexpr int RB = 1024;
template <int K, bool F64>
__global__ void __launch_bounds__(RB) k_leaf_reduce(LeafArgs A) {
    constexpr int NE = gram_entries(K);
    constexpr int RW = RB / WAVE;
    static_assert(NE <= WAVE, "one lane per entry");
    __shared__ int64_t s_w[RW][NE];
    const int node = blockIdx.x;
    if (!leaf_eligible(A, node)) return;
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    const int64_t c0 = A.off[node] / LCHUNK, c1 = (A.off[node + 1] - 1) / LCHUNK;
    if (lane < NE) {
        int64_t ai = 0;
        double ad = 0.0;
        for (int64_t c = c0 + w; c <= c1; c += RW) {
            const int64_t v = A.parts[((size_t)c + (size_t)node) * gram_entries(LKMAX) + lane];
            if (F64) ad += __longlong_as_double(v);
            else ai += v;
        }
        s_w[w][lane] = F64 ? __double_as_longlong(ad) : ai;
    }
    __syncthreads();
    if (threadIdx.x < NE) {
        int64_t* out = A.sums + (size_t)node * gram_entries(LKMAX);
        if (F64) {
            double v = __longlong_as_double(s_w[0][threadIdx.x]);
            for (int q = 1; q < RW; ++q) v += __longlong_as_double(s_w[q][threadIdx.x]);
            out[threadIdx.x] = __double_as_longlong(v);
        } else {
            int64_t v = 0;
            for (int q = 0; q < RW; ++q) v += s_w[q][threadIdx.x];
            out[threadIdx.x] = v;
        }
    }
}

// One thread per node: assemble, regularise and solve the (K+1) system of an
// eligible leaf with fp64 LU and partial pivoting (row swaps by selects, so
// the matrix stays in registers); zeros elsewhere.
template <int K>
__global__ void __launch_bounds__(LB) k_leaf_solve(LeafArgs A, float* out_W, float* out_b, float* out_lo,
                                                  float* out_hi, int64_t* out_count) {
    constexpr int N = K + 1;
    const int node = blockIdx.x * LB + threadIdx.x;
    if (node >= A.n_nodes) return;
    out_count[node] = A.count[node];
#pragma unroll
    for (int j = 0; j < K; ++j) {
        out_lo[node * K + j] = key_float(A.lo_key[node * K + j]);
        out_hi[node * K + j] = key_float(A.hi_key[node * K + j]);
        out_W[node * K + j] = 0.0f;
    }
    out_b[node] = 0.0f;
    if (!leaf_eligible(A, node) || A.st->status != 0) return;
    const int64_t* q = A.sums + (size_t)node * gram_entries(LKMAX);
    const bool f64 = A.gram_f64 != 0;   // fp64 sums (MFMA) or fixed point
    const double iM = ldexp(1.0, -A.st->sM), ib = ldexp(1.0, -A.st->sb);
    double M[N][N], r[N];
    int t = 0;
#pragma unroll
    for (int a = 0; a < N; ++a)
#pragma unroll
        for (int b = a; b < N; ++b) {
            M[a][b] = f64 ? __longlong_as_double(q[t]) : (double)q[t] * iM;
            ++t;
            M[b][a] = M[a][b];
        }
#pragma unroll
    for (int a = 0; a < N; ++a) {
        r[a] = f64 ? __longlong_as_double(q[t]) : (double)q[t] * ib;
        ++t;
    }
#pragma unroll
    for (int a = 0; a < K; ++a) M[a][a] += A.lam;    // reg = lam * I ...
    M[K][K] += 1e-8;                                  // ... but the bias (neural_leaves.py:85-86)
    bool singular = false;
#pragma unroll
    for (int c = 0; c < N; ++c) {
        int p = c;
        double best = fabs(M[c][c]);
#pragma unroll
        for (int i = c + 1; i < N; ++i)
            if (fabs(M[i][c]) > best) {
                best = fabs(M[i][c]);
                p = i;
            }
        if (best == 0.0) singular = true;
#pragma unroll
        for (int i = c + 1; i < N; ++i)
            if (i == p) {
#pragma unroll
                for (int j = 0; j < N; ++j) {
                    const double tmp = M[c][j];
                    M[c][j] = M[i][j];
                    M[i][j] = tmp;
                }
                const double tr = r[c];
                r[c] = r[i];
                r[i] = tr;
            }
        if (best != 0.0) {
#pragma unroll
            for (int i = c + 1; i < N; ++i) {
                const double f = M[i][c] / M[c][c];
#pragma unroll
                for (int j = c; j < N; ++j) M[i][j] -= f * M[c][j];
                r[i] -= f * r[c];
            }
        }
    }
    if (singular) {
        atomicMin(&A.st->status, -2);
        return;
    }
    double th[N];
#pragma unroll
    for (int i = N - 1; i >= 0; --i) {
        double v = r[i];
#pragma unroll
        for (int j = i + 1; j < N; ++j) v -= M[i][j] * th[j];
        th[i] = v / M[i][i];
    }
#pragma unroll
    for (int j = 0; j < K; ++j) out_W[node * K + j] = (float)th[j];
    out_b[node] = (float)th[K];
    atomicAdd(&A.st->n_fit, 1);
}

__global__ void k_leaf_status(const LeafStats* st, int32_t* out) {
    out[0] = st->status;
    out[1] = st->n_fit;
}

// The fold of the linear models into raw space (neural_leaves.py:178-184) in
// the order and fp32 roundings of the reference's torch expressions: per node,
// prod_j = W[j] * (mu[j] / sd[j]), acc = prod_0 + prod_1 + ... left to right,
// value = value_in + lr * (b - acc), linear[j] = (lr * W[j]) / sd[j].
__global__ void __launch_bounds__(LB) k_leaf_fold(int n_nodes, int K, const float* W, const float* b,
                                                  const float* mu, const float* sd, float lr,
                                                  const float* value_in, float* out_value, float* out_linear) {
    const int node = blockIdx.x * LB + threadIdx.x;
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

template <int K>
void launch_leaf_fit(LeafArgs& A, float* out_W, float* out_b, float* out_lo, float* out_hi, int64_t* out_count,
                     hipStream_t stream) {
    const bool lds = A.n_nodes <= LDS_NODES;
    int64_t per = (A.n + LROW_BLOCKS - 1) / LROW_BLOCKS;
    per = per < LROWS ? LROWS : (per + LSB - 1) / LSB * LSB;
    A.rows_per_block = per;
    const auto al = [](const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; };
    A.vec4 = (lds && A.x_kind == 1 && al(A.leaf, 16) && al(A.grad, 16) && al(A.hess, 16) && al(A.X, 4) &&
              A.ldx % 4 == 0 && per % 4 == 0)
                 ? 1
                 : 0;
    const int row_blocks = (int)((A.n + per - 1) / per);
    k_leaf_init<<<launch_grid((int64_t)A.n_nodes * gram_entries(LKMAX), LB, 1024), LB, 0, stream>>>(A, K);
    if (row_blocks > 0) {
        if (lds) k_leaf_stats<K, true><<<row_blocks, LSB, 0, stream>>>(A);
        else k_leaf_stats<K, false><<<row_blocks, LSB, 0, stream>>>(A);
    }
    k_leaf_offsets<<<1, 1024, 0, stream>>>(A, K);
    if (row_blocks > 0) {
        if (lds) k_leaf_scatter<K, true><<<row_blocks, LSB, 0, stream>>>(A);
        else k_leaf_scatter<K, false><<<row_blocks, LSB, 0, stream>>>(A);
        const int chunks = (int)((A.n + LCHUNK - 1) / LCHUNK);
        if (A.gram_f64) {
            k_leaf_gram_mfma<K><<<chunks, LB, 0, stream>>>(A);
            k_leaf_reduce<K, true><<<A.n_nodes, RB, 0, stream>>>(A);
        } else {
            if (A.n > 1024) k_leaf_gram<K, true><<<chunks, LB, 0, stream>>>(A);
            else k_leaf_gram<K, false><<<chunks, LB, 0, stream>>>(A);
            k_leaf_reduce<K, false><<<A.n_nodes, RB, 0, stream>>>(A);
        }
    }
    k_leaf_solve<K><<<(A.n_nodes + LB - 1) / LB, LB, 0, stream>>>(A, out_W, out_b, out_lo, out_hi, out_count);
}

}  // namespace yabt

using namespace yabt;

extern "C" {

size_t yabt_leaf_fit_workspace_bytes(int64_t n, int n_nodes, int K) {
    if (n < 0 || n_nodes < 1 || K < 1 || K > LKMAX) return 0;
    return carve_leaf(nullptr, n, n_nodes, K, nullptr);
}

int yabt_leaf_fit(int x_kind, const void* X, int64_t ldx, int64_t n, const int32_t* feats, int K, const float* mu,
                  const float* sd, const float* grad, const float* hess, const int64_t* leaf_of_row,
                  const int64_t* feature, int n_nodes, int min_samples, double lam, int gram_mode,
                  void* workspace, size_t workspace_bytes, float* out_W, float* out_b, float* out_lo,
                  float* out_hi, int64_t* out_count, int32_t* out_status, hipStream_t stream) {
    if (n < 0 || n > 0xFFFFFFFFll || n_nodes < 1 || K < 1 || K > LKMAX || (x_kind != 0 && x_kind != 1))
        return fail(-2, "yabt_leaf_fit: bad sizes (need 0 <= n < 2^32, n_nodes >= 1, 1 <= K <= 8, x_kind 0 or 1)");
    if (gram_mode != 0 && gram_mode != 1) return fail(-2, "yabt_leaf_fit: gram_mode must be 0 or 1");
    if (!X || !feats || !mu || !sd || !grad || !hess || !leaf_of_row || !feature || !workspace || !out_W || !out_b ||
        !out_lo || !out_hi || !out_count || !out_status)
        return fail(-2, "yabt_leaf_fit: null pointer argument");
    if (x_kind == 1 ? ldx < n : ldx < 1) return fail(-2, "yabt_leaf_fit: leading dimension too small");
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
    k_leaf_status<<<1, 1, 0, stream>>>(A.st, out_status);
    return launch_status("yabt_leaf_fit launch");
}

int yabt_leaf_fold(int n_nodes, int K, const float* W, const float* b, const float* mu, const float* sd, float lr,
                   const float* value_in, float* out_value, float* out_linear, hipStream_t stream) {
    if (n_nodes < 1 || K < 1 || K > LKMAX) return fail(-2, "yabt_leaf_fold: bad sizes (n_nodes >= 1, 1 <= K <= 8)");
    if (!W || !b || !mu || !sd || !value_in || !out_value || !out_linear)
        return fail(-2, "yabt_leaf_fold: null pointer argument");
    k_leaf_fold<<<(n_nodes + LB - 1) / LB, LB, 0, stream>>>(n_nodes, K, W, b, mu, sd, lr, value_in, out_value,
                                                           out_linear);
    return launch_status("yabt_leaf_fold launch");
}

size_t yabt_leaf_moments_workspace_bytes(int64_t n) {
    if (n < 0) return 0;
    const int64_t nb = n > 0 ? (n + MROWS - 1) / MROWS : 1;
    const size_t f = (size_t)nb * 2 * LKMAX * sizeof(double), u = (size_t)MU8_BLOCKS * LKMAX * 2 * sizeof(uint64_t);
    return align_up(f > u ? f : u, 256);
}

int yabt_leaf_moments(int x_kind, const void* X, int64_t ldx, int64_t n, const int32_t* feats, int K,
                      void* workspace, size_t workspace_bytes, float* out_mu, float* out_sd, hipStream_t stream) {
    if (n < 1 || K < 1 || K > LKMAX || (x_kind != 0 && x_kind != 1))
        return fail(-2, "yabt_leaf_moments: bad sizes (need n >= 1, 1 <= K <= 8, x_kind 0 or 1)");
    if (!X || !feats || !workspace || !out_mu || !out_sd) return fail(-2, "yabt_leaf_moments: null pointer argument");
    if (x_kind == 1 ? ldx < n : ldx < 1) return fail(-2, "yabt_leaf_moments: leading dimension too small");
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
