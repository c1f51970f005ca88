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
//   k_leaf_gram<K>     per-leaf fixed-point sums of M and b
//   k_leaf_solve<K>    fp64 LU with partial pivoting per eligible leaf

#include "common.h"
#include "host.h"
#include "yabt_hip.h"

#include <string.h>

namespace yabt {

constexpr int LKMAX = 8;                       // model inputs per leaf, at most
constexpr int LB = 256;                        // threads per block
constexpr int LROWS = 4096;                    // rows per stats/scatter block
constexpr int LCHUNK = 4096;                   // sorted positions per gram block
constexpr int LDS_NODES = 640;                 // node tables kept in LDS up to this many nodes

__host__ __device__ constexpr int gram_entries(int K) { return (K + 1) * (K + 2) / 2 + (K + 1); }

struct LeafStats {
    uint32_t max_x1_bits;      // max |x1| (float bits, >= 1 via the bias column)
    uint32_t max_g_bits, max_h_bits;
    int32_t sM, sb;            // fixed-point shifts of M and b
    int32_t status;            // 0 ok; -1 a leaf id outside [0, n_nodes) or a non-finite input; -2 singular system
    int32_t pad;
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
    // workspace
    LeafStats* st;
    uint32_t* count;           // (n_nodes)
    int64_t* off;              // (n_nodes + 1)
    unsigned long long* cursor;   // (n_nodes)
    uint32_t* sorted;          // (n)
    int64_t* sums;             // (n_nodes, gram_entries(LKMAX))
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
    }
}

// Rows [blockIdx.x * LROWS, +LROWS): counts, envelopes and magnitudes.
template <int K, bool LDS>
__global__ void __launch_bounds__(LB) k_leaf_stats(LeafArgs A) {
    __shared__ uint32_t s_cnt[LDS ? LDS_NODES : 1];
    __shared__ uint32_t s_lo[LDS ? LDS_NODES * K : 1], s_hi[LDS ? LDS_NODES * K : 1];
    __shared__ float s_red[3][LB / WAVE];
    __shared__ int s_bad;
    __shared__ int32_t s_fs[LKMAX];
    __shared__ float s_mu[LKMAX], s_sd[LKMAX];
    if (threadIdx.x < K) {
        s_fs[threadIdx.x] = A.feats[threadIdx.x];
        s_mu[threadIdx.x] = A.mu[threadIdx.x];
        s_sd[threadIdx.x] = A.sd[threadIdx.x];
    }
    if (threadIdx.x == 0) s_bad = 0;
    if (LDS) {
        for (int i = threadIdx.x; i < A.n_nodes; i += LB) s_cnt[i] = 0;
        for (int i = threadIdx.x; i < A.n_nodes * K; i += LB) {
            s_lo[i] = float_key(INFINITY);
            s_hi[i] = float_key(-INFINITY);
        }
    }
    __syncthreads();
    const int64_t lo = (int64_t)blockIdx.x * LROWS, hi = min(A.n, lo + LROWS);
    float mx = 1.0f, mg = 0.0f, mh = 0.0f;
    int bad = 0;
    for (int64_t i = lo + threadIdx.x; i < hi; i += LB) {
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
#pragma unroll
        for (int j = 0; j < K; ++j) {
            const float xn = (x[j] - s_mu[j]) / s_sd[j];
            if (!isfinite(xn)) bad = 1;
            mx = fmaxf(mx, fabsf(xn));
            // the extremes settle quickly: read first, update only when improving
            const uint32_t kx = float_key(x[j]);
            uint32_t* plo = LDS ? &s_lo[node * K + j] : &A.lo_key[node * K + j];
            uint32_t* phi = LDS ? &s_hi[node * K + j] : &A.hi_key[node * K + j];
            if (kx < *(volatile uint32_t*)plo) atomicMin(plo, kx);
            if (kx > *(volatile uint32_t*)phi) atomicMax(phi, kx);
        }
        if (LDS) atomicAdd(&s_cnt[node], 1u);
        else atomicAdd(&A.count[node], 1u);
    }
    if (bad) s_bad = 1;
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
#pragma unroll
    for (int d = WAVE / 2; d > 0; d >>= 1) {
        mx = fmaxf(mx, __shfl_xor(mx, d, WAVE));
        mg = fmaxf(mg, __shfl_xor(mg, d, WAVE));
        mh = fmaxf(mh, __shfl_xor(mh, d, WAVE));
    }
    if (lane == 0) {
        s_red[0][w] = mx;
        s_red[1][w] = mg;
        s_red[2][w] = mh;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < LB / WAVE; ++i) {
            mx = fmaxf(mx, s_red[0][i]);
            mg = fmaxf(mg, s_red[1][i]);
            mh = fmaxf(mh, s_red[2][i]);
        }
        // |x| <= inf as float bits: non-negative floats order like their bits
        atomicMax(&A.st->max_x1_bits, __float_as_uint(mx));
        atomicMax(&A.st->max_g_bits, __float_as_uint(mg));
        atomicMax(&A.st->max_h_bits, __float_as_uint(mh));
        if (s_bad) atomicMin(&A.st->status, -1);
    }
    if (LDS) {
        for (int i = threadIdx.x; i < A.n_nodes; i += LB)
            if (s_cnt[i]) atomicAdd(&A.count[i], s_cnt[i]);
        for (int i = threadIdx.x; i < A.n_nodes * K; i += LB) {
            if (s_lo[i] != float_key(INFINITY)) atomicMin(&A.lo_key[i], s_lo[i]);
            if (s_hi[i] != float_key(-INFINITY)) atomicMax(&A.hi_key[i], s_hi[i]);
        }
    }
}

// One block: node offsets of the sorted rows (exclusive scan of the counts),
// write cursors, and the fixed-point shifts.
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
    if (threadIdx.x == 0) {
        A.off[A.n_nodes] = carry;
        // |p| <= max|x1|^2 max|h| for M and max|x1| max|g| for b; the bounds
        // are taken 2^-20 above to cover the rounding of the fp64 products
        const double mx = (double)__uint_as_float(A.st->max_x1_bits);
        const double bm = mx * mx * (double)__uint_as_float(A.st->max_h_bits) * (1.0 + 0x1p-20);
        const double bb = mx * (double)__uint_as_float(A.st->max_g_bits) * (1.0 + 0x1p-20);
        const float fm = (float)bm, fb = (float)bb;
        A.st->sM = quant_shift((double)fm >= bm ? fm : nextafterf(fm, INFINITY), A.n);
        A.st->sb = quant_shift((double)fb >= bb ? fb : nextafterf(fb, INFINITY), A.n);
    }
}

// Rows [blockIdx.x * LROWS, +LROWS) to their node's range of `sorted`; the
// block reserves one range per node with one atomic add.
template <bool LDS>
__global__ void __launch_bounds__(LB) k_leaf_scatter(LeafArgs A) {
    __shared__ uint32_t s_cnt[LDS ? LDS_NODES : 1];
    __shared__ unsigned long long s_base[LDS ? LDS_NODES : 1];
    if (LDS)
        for (int i = threadIdx.x; i < A.n_nodes; i += LB) s_cnt[i] = 0;
    __syncthreads();
    const int64_t lo = (int64_t)blockIdx.x * LROWS, hi = min(A.n, lo + LROWS);
    if (LDS) {
        for (int64_t i = lo + threadIdx.x; i < hi; i += LB) {
            const int64_t node = A.leaf[i];
            if (node >= 0 && node < A.n_nodes) atomicAdd(&s_cnt[node], 1u);
        }
        __syncthreads();
        for (int i = threadIdx.x; i < A.n_nodes; i += LB) {
            s_base[i] = s_cnt[i] ? atomicAdd(&A.cursor[i], (unsigned long long)s_cnt[i]) : 0ull;
            s_cnt[i] = 0;
        }
        __syncthreads();
        for (int64_t i = lo + threadIdx.x; i < hi; i += LB) {
            const int64_t node = A.leaf[i];
            if (node < 0 || node >= A.n_nodes) continue;
            const uint32_t r = atomicAdd(&s_cnt[node], 1u);
            A.sorted[s_base[node] + r] = (uint32_t)i;
        }
    } else {
        for (int64_t i = lo + threadIdx.x; i < hi; i += LB) {
            const int64_t node = A.leaf[i];
            if (node < 0 || node >= A.n_nodes) continue;
            A.sorted[atomicAdd(&A.cursor[node], 1ull)] = (uint32_t)i;
        }
    }
}

__device__ __forceinline__ bool leaf_eligible(const LeafArgs& A, int node) {
    return A.feature[node] == LEAF && (int64_t)A.count[node] >= (int64_t)A.min_samples;
}

// Sorted positions [blockIdx.x * LCHUNK, +LCHUNK): for each node run inside
// the chunk, every thread sums the fixed-point products of its rows in
// registers; waves reduce with DPP and add into the node's sums.
template <int K>
__global__ void __launch_bounds__(LB) k_leaf_gram(LeafArgs A) {
    constexpr int NE = gram_entries(K);
    __shared__ int32_t s_fs[LKMAX];
    __shared__ float s_mu[LKMAX], s_sd[LKMAX];
    if (threadIdx.x < K) {
        s_fs[threadIdx.x] = A.feats[threadIdx.x];
        s_mu[threadIdx.x] = A.mu[threadIdx.x];
        s_sd[threadIdx.x] = A.sd[threadIdx.x];
    }
    __syncthreads();
    const int64_t total = A.off[A.n_nodes];
    const int64_t c0 = (int64_t)blockIdx.x * LCHUNK, c1 = min(total, c0 + LCHUNK);
    if (c0 >= c1) return;
    const double scM = ldexp(1.0, A.st->sM), scb = ldexp(1.0, A.st->sb);
    // the node holding position c0: last l with off[l] <= c0
    int lo = 0, hi = A.n_nodes - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) / 2;
        if (A.off[mid] <= c0) lo = mid;
        else hi = mid - 1;
    }
    const int lane = threadIdx.x & (WAVE - 1);
    for (int node = lo; node < A.n_nodes && A.off[node] < c1; ++node) {
        const int64_t s = max(c0, A.off[node]), e = min(c1, A.off[node + 1]);
        if (s >= e || !leaf_eligible(A, node)) continue;   // uniform across the block
        int64_t acc[NE];
#pragma unroll
        for (int t = 0; t < NE; ++t) acc[t] = 0;
        for (int64_t p = s + threadIdx.x; p < e; p += LB) {
            const int64_t i = A.sorted[p];
            float x[K];
            load_x<K>(A, i, s_fs, x);
            const double g = (double)A.grad[i], h = (double)A.hess[i];
            double x1[K + 1];
#pragma unroll
            for (int j = 0; j < K; ++j) x1[j] = (double)((x[j] - s_mu[j]) / s_sd[j]);
            x1[K] = 1.0;
            int t = 0;
#pragma unroll
            for (int a = 0; a <= K; ++a) {
#pragma unroll
                for (int b = a; b <= K; ++b) {
                    const double xh = x1[b] * h;             // Xh = X1 * h    (neural_leaves.py:72)
                    acc[t++] += (int64_t)rint(x1[a] * xh * scM);
                }
            }
#pragma unroll
            for (int a = 0; a <= K; ++a) acc[t++] += (int64_t)rint(-(x1[a] * g) * scb);   // rhs = -(X1 * g)
        }
        int64_t* out = A.sums + (size_t)node * gram_entries(LKMAX);
#pragma unroll
        for (int t = 0; t < NE; ++t) {
            const int64_t v = wave_sum_i64(acc[t]);
            if (lane == 0 && v != 0) atomicAdd((unsigned long long*)&out[t], (unsigned long long)v);
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
    const double iM = ldexp(1.0, -A.st->sM), ib = ldexp(1.0, -A.st->sb);
    double M[N][N], r[N];
    int t = 0;
#pragma unroll
    for (int a = 0; a < N; ++a)
#pragma unroll
        for (int b = a; b < N; ++b) {
            M[a][b] = (double)q[t++] * iM;
            M[b][a] = M[a][b];
        }
#pragma unroll
    for (int a = 0; a < N; ++a) r[a] = (double)q[t++] * ib;
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
}

__global__ void k_leaf_status(const LeafStats* st, int32_t* out) { out[0] = st->status; }

// ---------------------------------------------------------------------------
// input moments: mu = mean, sd = max(unbiased std, 1e-6) per input
// (neural_leaves.py:152-155), from fp64 sums of x and x^2 reduced in a fixed
// order (per-block partials, then one block), so the result is deterministic
// ---------------------------------------------------------------------------

constexpr int MROWS = 16384;                   // rows per moments block

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

__global__ void k_leaf_moments_final(const double* part, int nblocks, int64_t n, int K, float* mu, float* sd) {
    const int j = threadIdx.x;
    if (j >= K) return;
    double s1 = 0.0, s2 = 0.0;
    for (int b = 0; b < nblocks; ++b) {
        s1 += part[((size_t)b * 2 + 0) * LKMAX + j];
        s2 += part[((size_t)b * 2 + 1) * LKMAX + j];
    }
    const double m = n > 0 ? s1 / (double)n : NAN;
    const double var = n > 1 ? fmax(s2 - s1 * m, 0.0) / (double)(n - 1) : NAN;
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
    a.sorted = c.take<uint32_t>((size_t)(n > 0 ? n : 1));
    a.sums = c.take<int64_t>((size_t)n_nodes * gram_entries(LKMAX));
    a.lo_key = c.take<uint32_t>((size_t)n_nodes * K);
    a.hi_key = c.take<uint32_t>((size_t)n_nodes * K);
    return align_up(c.off, 256);
}

template <int K>
void launch_leaf_fit(LeafArgs& A, float* out_W, float* out_b, float* out_lo, float* out_hi, int64_t* out_count,
                     hipStream_t stream) {
    const bool lds = A.n_nodes <= LDS_NODES;
    const int row_blocks = (int)((A.n + LROWS - 1) / LROWS);
    k_leaf_init<<<launch_grid((int64_t)A.n_nodes * gram_entries(LKMAX), LB, 1024), LB, 0, stream>>>(A, K);
    if (row_blocks > 0) {
        if (lds) k_leaf_stats<K, true><<<row_blocks, LB, 0, stream>>>(A);
        else k_leaf_stats<K, false><<<row_blocks, LB, 0, stream>>>(A);
    }
    k_leaf_offsets<<<1, 1024, 0, stream>>>(A);
    if (row_blocks > 0) {
        if (lds) k_leaf_scatter<true><<<row_blocks, LB, 0, stream>>>(A);
        else k_leaf_scatter<false><<<row_blocks, LB, 0, stream>>>(A);
        k_leaf_gram<K><<<(int)((A.n + LCHUNK - 1) / LCHUNK), LB, 0, stream>>>(A);
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
                  const int64_t* feature, int n_nodes, int min_samples, double lam, void* workspace,
                  size_t workspace_bytes, float* out_W, float* out_b, float* out_lo, float* out_hi,
                  int64_t* out_count, int32_t* out_status, hipStream_t stream) {
    if (n < 0 || n > 0xFFFFFFFFll || n_nodes < 1 || K < 1 || K > LKMAX || (x_kind != 0 && x_kind != 1))
        return fail(-2, "yabt_leaf_fit: bad sizes (need 0 <= n < 2^32, n_nodes >= 1, 1 <= K <= 8, x_kind 0 or 1)");
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

size_t yabt_leaf_moments_workspace_bytes(int64_t n) {
    if (n < 0) return 0;
    const int64_t nb = n > 0 ? (n + MROWS - 1) / MROWS : 1;
    return align_up((size_t)nb * 2 * LKMAX * sizeof(double), 256);
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
    k_leaf_moments_final<<<1, WAVE, 0, stream>>>(part, nb, n, K, out_mu, out_sd);
    return launch_status("yabt_leaf_moments launch");
}

}  // extern "C"
