// Quantile binner on gfx950 (yabt/binning.py:29-129, the numpy path).
//
//   yabt_bin_fit        per feature: the quantile edges of a row sample
//                       (numpy's linear quantiles at linspace(0, 1, B+1)[1:-1],
//                       rounded to fp32, de-duplicated), the inter-quartile
//                       scale (numpy's fp32 std when it is zero) and the median
//                       of all rows (NaNs ignored, 0 if none)
//   yabt_bin_transform  bin = #{edges < x} after median imputation, written
//                       straight into the grower's feature-major and row-major
//                       layouts, plus the imputed fp32 matrix
//
// Fit, per feature: the sample column is gathered as order-preserving uint32
// keys (NaN last), sorted by a stable 4 x 8-bit radix sort (one block per
// feature), and the quantiles are read off the sorted keys with numpy's
// arithmetic: virtual index (c - 1) * q in double, d = fp32(b - a), value
// a + d * t (t < 1/2) or b - d * (1 - t) in double (numpy _lerp), rounded to
// fp32; the edges are those values sorted and de-duplicated (np.unique).
// Medians: a 4-pass radix select of the two middle order statistics over all
// rows, combined as numpy's float32 mean of two values.

#include "common.h"
#include "host.h"
#include "yabt_hip.h"

#include <math.h>

namespace yabt {
namespace bin {

constexpr int SB = 1024;            // sort block
constexpr int HT = 16;              // features per histogram / transform tile
constexpr int TB = 256;             // threads per transform / select block
constexpr int MAXE = 255;           // edges per feature (max_bins - 1 <= 255)

__device__ __forceinline__ uint32_t fkey(float v) {
    if (isnan(v)) return 0xFFFFFFFFu;
    const uint32_t b = __float_as_uint(v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float kval(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

struct FitWs {
    uint32_t* orig;        // (F, m) sample keys in sample order
    uint32_t* ka;          // (F, m) sorted keys
    uint32_t* kb;          // (F, m) radix ping-pong, then the std fallback's scratch
    uint32_t* cnt;         // (F) non-NaN rows over all n
    uint32_t* sel_hist;    // (F, 2, 256)
    uint32_t* sel_state;   // (F, 2, 2): prefix, rank
    size_t bytes;
};

FitWs carve_fit(char* base, int64_t m, int F) {
    Carve c{base, 0};
    FitWs w;
    const size_t fm = (size_t)F * (size_t)(m > 0 ? m : 1);
    w.orig = c.take<uint32_t>(fm);
    w.ka = c.take<uint32_t>(fm);
    w.kb = c.take<uint32_t>(fm);
    w.cnt = c.take<uint32_t>(F);
    w.sel_hist = c.take<uint32_t>((size_t)F * 2 * NB);
    w.sel_state = c.take<uint32_t>((size_t)F * 4);
    w.bytes = c.off;
    return w;
}

// keys[f][i] = key of X[rows[i]][f] (rows == null: row i).
__global__ void __launch_bounds__(TB) k_gather_keys(const float* __restrict__ X, int64_t ldx, int F,
                                                    const int64_t* __restrict__ rows, int64_t m,
                                                    uint32_t* __restrict__ keys) {
    const int64_t total = m * F;
    for (int64_t t = (int64_t)blockIdx.x * TB + threadIdx.x; t < total; t += (int64_t)gridDim.x * TB) {
        const int64_t i = t / F;
        const int f = (int)(t - i * F);
        const int64_t r = rows ? rows[i] : i;
        keys[(size_t)f * m + i] = fkey(X[(size_t)r * ldx + f]);
    }
}

// Stable LSD radix sort of each feature's m keys, one block per feature.
// Result in a (4 passes: a -> b -> a -> b -> a).
__global__ void __launch_bounds__(SB) k_sort(uint32_t* __restrict__ ka, uint32_t* __restrict__ kb, int64_t m) {
    __shared__ uint32_t s_base[NB];
    __shared__ uint32_t s_tot[NB];
    __shared__ uint32_t s_wc[SB / WAVE][NB];
    const int f = blockIdx.x, tid = threadIdx.x, w = tid / WAVE;
    uint32_t* a = ka + (size_t)f * m;
    uint32_t* b = kb + (size_t)f * m;
    for (int pass = 0; pass < 4; ++pass) {
        const int shift = 8 * pass;
        const uint32_t* src = (pass & 1) ? b : a;
        uint32_t* dst = (pass & 1) ? a : b;
        if (tid < NB) s_tot[tid] = 0;
        __syncthreads();
        for (int64_t i = tid; i < m; i += SB) atomicAdd(&s_tot[(src[i] >> shift) & 255u], 1u);
        __syncthreads();
        if (tid == 0) {                  // digit starts: exclusive prefix of the counts
            uint32_t run = 0;
            for (int d = 0; d < NB; ++d) {
                const uint32_t c = s_tot[d];
                s_base[d] = run;
                run += c;
            }
        }
        __syncthreads();
        for (int64_t t0 = 0; t0 < m; t0 += SB) {
            for (int j = tid; j < (SB / WAVE) * NB; j += SB) (&s_wc[0][0])[j] = 0;
            __syncthreads();
            const int64_t i = t0 + tid;
            const bool v = i < m;
            const uint32_t key = v ? src[i] : 0u;
            const uint32_t d = (key >> shift) & 255u;
            uint64_t peers = __ballot(v);
#pragma unroll
            for (int bit = 0; bit < 8; ++bit) {
                const bool on = (d >> bit) & 1u;
                const uint64_t bal = __ballot(on);
                peers &= on ? bal : ~bal;
            }
            const uint32_t rk = lane_prefix(peers);
            if (v && rk == 0) s_wc[w][d] = (uint32_t)__popcll(peers);
            __syncthreads();
            if (tid < NB) {
                uint32_t run = 0;
                for (int k = 0; k < SB / WAVE; ++k) {
                    const uint32_t c = s_wc[k][tid];
                    s_wc[k][tid] = run;
                    run += c;
                }
                s_tot[tid] = run;
            }
            __syncthreads();
            if (v) dst[s_base[d] + s_wc[w][d] + rk] = key;
            __syncthreads();
            if (tid < NB) s_base[tid] += s_tot[tid];
            __syncthreads();
        }
    }
}

// numpy's float32 pairwise sum of one buffer, iteratively: blocks of <= 128
// summed with eight accumulators, halves split at multiples of 8.
__device__ float np_pairwise_sum(const float* a, int64_t n) {
    struct Fr {
        int64_t off, n;
        int stage;
        float left;
    };
    Fr st[40];
    int sp = 0;
    st[0] = Fr{0, n, 0, 0.0f};
    float ret = 0.0f;
    while (true) {
        Fr& fr = st[sp];
        if (fr.stage == 0 && fr.n > 128) {
            int64_t n2 = fr.n / 2;
            n2 -= n2 % 8;
            fr.stage = 1;
            st[sp + 1] = Fr{fr.off, n2, 0, 0.0f};
            ++sp;
            continue;
        }
        if (fr.stage == 1) {               // left half done: ret holds it
            fr.left = ret;
            fr.stage = 2;
            int64_t n2 = fr.n / 2;
            n2 -= n2 % 8;
            st[sp + 1] = Fr{fr.off + n2, fr.n - n2, 0, 0.0f};
            ++sp;
            continue;
        }
        float res;
        if (fr.stage == 2) {
            res = fr.left + ret;
        } else if (fr.n < 8) {
            res = 0.0f;
            for (int64_t i = 0; i < fr.n; ++i) res += a[fr.off + i];
        } else {
            float r[8];
            for (int j = 0; j < 8; ++j) r[j] = a[fr.off + j];
            int64_t i = 8;
            for (; i < fr.n - (fr.n % 8); i += 8)
                for (int j = 0; j < 8; ++j) r[j] += a[fr.off + i + j];
            res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
            for (; i < fr.n; ++i) res += a[fr.off + i];
        }
        ret = res;
        if (sp == 0) return ret;
        --sp;
    }
}

// numpy's float32 sum of a contiguous array: 8192-element buffers, each
// summed pairwise, added in order to an accumulator that starts at 0.
__device__ float np_sum(const float* a, int64_t n) {
    float acc = 0.0f;
    for (int64_t i = 0; i < n; i += 8192) acc += np_pairwise_sum(a + i, min((int64_t)8192, n - i));
    return acc;
}

// numpy's linear quantile of the c sorted keys at q (numpy _quantile/_lerp),
// in double.
__device__ double np_quantile(const uint32_t* sk, int64_t c, double q) {
    const double virt = (double)(c - 1) * q;
    int64_t lo, hi;
    double prev;
    if (virt >= (double)(c - 1)) {
        lo = hi = c - 1;
        prev = -1.0;
    } else {
        prev = floor(virt);
        lo = (int64_t)prev;
        hi = lo + 1;
    }
    const double t = virt - prev;
    const float a = kval(sk[lo]), b = kval(sk[hi]);
    const float d = b - a;
    return t >= 0.5 ? (double)b - (double)d * (1.0 - t) : (double)a + (double)d * t;
}

// One block per feature: edges, edge count, scale.
__global__ void __launch_bounds__(TB) k_quantiles(const uint32_t* __restrict__ sorted, const uint32_t* __restrict__ orig,
                                                  float* __restrict__ scratch, int64_t m, int max_bins,
                                                  float* __restrict__ out_edges, int64_t ld_edges,
                                                  int32_t* __restrict__ out_nedges, float* __restrict__ out_scales) {
    __shared__ float s_q[MAXE];
    __shared__ uint32_t s_c;
    const int f = blockIdx.x, tid = threadIdx.x;
    const uint32_t* sk = sorted + (size_t)f * m;
    if (tid == 0) {                         // non-NaN keys sort below 0xFFFFFFFF
        int64_t lo = 0, hi = m;
        while (lo < hi) {
            const int64_t mid = (lo + hi) / 2;
            if (sk[mid] != 0xFFFFFFFFu) lo = mid + 1;
            else hi = mid;
        }
        s_c = (uint32_t)lo;
    }
    __syncthreads();
    const int64_t c = s_c;
    const uint32_t zero_key = 0x80000000u;  // an all-NaN (or empty) column is [0.0] (binning.py:57-59)
    const uint32_t* keys = c > 0 ? sk : &zero_key;
    const int64_t cc = c > 0 ? c : 1;
    const int ne = max_bins - 1;
    const double step = 1.0 / (double)max_bins;   // np.linspace(0, 1, max_bins + 1)
    for (int j = tid; j < ne; j += TB) {
        const double q = (double)(j + 1) * step + 0.0;
        s_q[j] = (float)np_quantile(keys, cc, q);
    }
    __syncthreads();
    if (tid == 0) {
        // np.unique: sort (insertion; the values are already nearly sorted;
        // NaN last) and drop repeats (NaNs count as equal)
        for (int i = 1; i < ne; ++i) {
            const float v = s_q[i];
            int k = i - 1;
            while (k >= 0 && (isnan(v) ? false : (isnan(s_q[k]) || s_q[k] > v))) {
                s_q[k + 1] = s_q[k];
                --k;
            }
            s_q[k + 1] = v;
        }
        int u = 0;
        for (int i = 0; i < ne; ++i)
            if (i == 0 || !(s_q[i] == s_q[u - 1] || (isnan(s_q[i]) && isnan(s_q[u - 1])))) s_q[u++] = s_q[i];
        out_nedges[f] = u;
        for (int i = 0; i < u; ++i) out_edges[(size_t)f * ld_edges + i] = s_q[i];
        // scale: q75 - q25 in double, else numpy's float32 std of the column, else 1
        double s = np_quantile(keys, cc, 0.75) - np_quantile(keys, cc, 0.25);
        if (s == 0.0) {
            float* col = scratch + (size_t)f * m;
            int64_t k = 0;
            const uint32_t* ok = orig + (size_t)f * m;
            for (int64_t i = 0; i < m; ++i)
                if (ok[i] != 0xFFFFFFFFu) col[k++] = kval(ok[i]);
            if (k == 0) col[k++] = 0.0f;
            const float mean = np_sum(col, k) / (float)k;
            for (int64_t i = 0; i < k; ++i) {
                const float x = col[i] - mean;
                col[i] = x * x;
            }
            const float var = np_sum(col, k) / (float)k;
            s = (double)sqrtf(var);
            if (s == 0.0) s = 1.0;
        }
        out_scales[f] = (float)s;
    }
}

// ---------------------------------------------------------------------------
// medians over all rows: radix select of the two middle order statistics
// ---------------------------------------------------------------------------

// Non-NaN count per feature.
__global__ void __launch_bounds__(TB) k_count_valid(const float* __restrict__ X, int64_t ldx, int64_t n, int F,
                                                    uint32_t* __restrict__ cnt) {
    __shared__ uint32_t s_c[HT];
    const int f0 = blockIdx.y * HT;
    if (threadIdx.x < HT) s_c[threadIdx.x] = 0;
    __syncthreads();
    const int j = threadIdx.x % HT;
    const int f = f0 + j;
    uint32_t c = 0;
    if (f < F)
        for (int64_t r = (int64_t)blockIdx.x * (TB / HT) + threadIdx.x / HT; r < n; r += (int64_t)gridDim.x * (TB / HT))
            c += isnan(X[(size_t)r * ldx + f]) ? 0u : 1u;
    atomicAdd(&s_c[j], c);
    __syncthreads();
    if (threadIdx.x < HT && f0 + threadIdx.x < F && s_c[threadIdx.x]) atomicAdd(&cnt[f0 + threadIdx.x], s_c[threadIdx.x]);
}

// state[f][t] = {prefix, rank}: the ranks of the two middle order statistics.
__global__ void k_select_init(const uint32_t* __restrict__ cnt, int F, uint32_t* __restrict__ state,
                              uint32_t* __restrict__ hist) {
    const int f = blockIdx.x * blockDim.x + threadIdx.x;
    if (f >= F) return;
    const uint32_t c = cnt[f];
    const uint32_t k1 = c == 0 ? 0 : (c % 2 ? (c - 1) / 2 : c / 2 - 1);
    const uint32_t k2 = c == 0 ? 0 : c / 2;
    state[(size_t)f * 4 + 0] = 0;
    state[(size_t)f * 4 + 1] = k1;
    state[(size_t)f * 4 + 2] = 0;
    state[(size_t)f * 4 + 3] = k2;
    for (int i = 0; i < 2 * NB; ++i) hist[(size_t)f * 2 * NB + i] = 0;
}

// Histogram of digit `shift` among keys whose higher bits equal each target's prefix.
__global__ void __launch_bounds__(TB) k_select_hist(const float* __restrict__ X, int64_t ldx, int64_t n, int F,
                                                    int shift, const uint32_t* __restrict__ state,
                                                    uint32_t* __restrict__ hist) {
    __shared__ uint32_t s_h[HT][2][NB];
    const int f0 = blockIdx.y * HT;
    for (int i = threadIdx.x; i < HT * 2 * NB; i += TB) (&s_h[0][0][0])[i] = 0;
    __syncthreads();
    const int j = threadIdx.x % HT;
    const int f = f0 + j;
    if (f < F) {
        const uint32_t p1 = state[(size_t)f * 4 + 0], p2 = state[(size_t)f * 4 + 2];
        for (int64_t r = (int64_t)blockIdx.x * (TB / HT) + threadIdx.x / HT; r < n; r += (int64_t)gridDim.x * (TB / HT)) {
            const float v = X[(size_t)r * ldx + f];
            if (isnan(v)) continue;
            const uint32_t k = fkey(v);
            const uint32_t hi = shift == 24 ? 0u : (k >> (shift + 8));
            const uint32_t d = (k >> shift) & 255u;
            if (hi == p1) atomicAdd(&s_h[j][0][d], 1u);
            if (hi == p2) atomicAdd(&s_h[j][1][d], 1u);
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < HT * 2 * NB; i += TB) {
        const int jj = i / (2 * NB), rest = i % (2 * NB);
        const uint32_t v = (&s_h[0][0][0])[i];
        if (f0 + jj < F && v) atomicAdd(&hist[(size_t)(f0 + jj) * 2 * NB + rest], v);
    }
}

// Choose each target's digit; clear the histogram for the next pass.
__global__ void k_select_step(int F, uint32_t* __restrict__ state, uint32_t* __restrict__ hist) {
    const int f = blockIdx.x * blockDim.x + threadIdx.x;
    if (f >= F) return;
    for (int t = 0; t < 2; ++t) {
        uint32_t* h = hist + (size_t)f * 2 * NB + (size_t)t * NB;
        uint32_t k = state[(size_t)f * 4 + 2 * t + 1];
        uint32_t d = 0;
        for (; d < NB - 1; ++d) {
            if (k < h[d]) break;
            k -= h[d];
        }
        state[(size_t)f * 4 + 2 * t + 0] = (state[(size_t)f * 4 + 2 * t + 0] << 8) | d;
        state[(size_t)f * 4 + 2 * t + 1] = k;
        for (int i = 0; i < NB; ++i) h[i] = 0;
    }
}

// median = x_k (odd count) or float32 (x_k1 + x_k2) / 2 (even), 0 if no value
// (np.nanmedian then np.where(isnan, 0, .), binning.py:32-33).
__global__ void k_select_finish(const uint32_t* __restrict__ cnt, int F, const uint32_t* __restrict__ state,
                                float* __restrict__ out_medians) {
    const int f = blockIdx.x * blockDim.x + threadIdx.x;
    if (f >= F) return;
    const uint32_t c = cnt[f];
    float med = 0.0f;
    if (c > 0) {
        const float a = kval(state[(size_t)f * 4 + 0]), b = kval(state[(size_t)f * 4 + 2]);
        med = (c % 2) ? a : (a + b) / 2.0f;
        if (isnan(med)) med = 0.0f;
    }
    out_medians[f] = med;
}

// ---------------------------------------------------------------------------
// transform
// ---------------------------------------------------------------------------

// One thread per (row, 16-feature tile): impute, count edges below x (binary
// search in LDS), write the row's 16 bins to the row-major layout with one
// 16-byte store, each bin to the feature-major layout, and the imputed value.
__global__ void __launch_bounds__(TB) k_transform(const float* __restrict__ X, int64_t ldx, int64_t n, int F,
                                                  const float* __restrict__ edges, int64_t ld_edges,
                                                  const int32_t* __restrict__ nedges, const float* __restrict__ medians,
                                                  uint8_t* __restrict__ out_fm, int64_t ld_fm,
                                                  uint8_t* __restrict__ out_rm, int64_t ld_rm,
                                                  float* __restrict__ out_imp, int64_t ld_imp, int rm_vec) {
    __shared__ float s_e[HT][MAXE + 1];
    __shared__ int s_n[HT];
    __shared__ float s_med[HT];
    const int f0 = blockIdx.y * HT;
    for (int i = threadIdx.x; i < HT * (MAXE + 1); i += TB) {
        const int j = i / (MAXE + 1), k = i % (MAXE + 1);
        s_e[j][k] = (f0 + j < F && k < MAXE) ? edges[(size_t)(f0 + j) * ld_edges + k] : 0.0f;
    }
    if (threadIdx.x < HT) {
        const int f = f0 + threadIdx.x;
        s_n[threadIdx.x] = f < F ? min(max(nedges[f], 0), MAXE) : 0;
        s_med[threadIdx.x] = f < F ? medians[f] : 0.0f;
    }
    __syncthreads();
    for (int64_t r = (int64_t)blockIdx.x * TB + threadIdx.x; r < n; r += (int64_t)gridDim.x * TB) {
        uint32_t w4[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int j = 0; j < HT; ++j) {
            const int f = f0 + j;
            if (f >= F) break;
            float x = X[(size_t)r * ldx + f];
            if (isnan(x)) x = s_med[j];
            int lo = 0, hi = s_n[j];
            while (lo < hi) {
                const int mid = (lo + hi) >> 1;
                if (s_e[j][mid] < x) lo = mid + 1;
                else hi = mid;
            }
            const uint32_t bv = (uint32_t)lo;
            w4[j >> 2] |= bv << (8 * (j & 3));
            if (out_fm) out_fm[(size_t)f * ld_fm + r] = (uint8_t)bv;
            if (out_imp) out_imp[(size_t)r * ld_imp + f] = x;
        }
        if (out_rm) {
            uint8_t* dst = out_rm + (size_t)r * ld_rm + f0;
            if (rm_vec) {
                *reinterpret_cast<uint4*>(dst) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
            } else {
                for (int j = 0; j < HT && f0 + j < F; ++j) dst[j] = (uint8_t)(w4[j >> 2] >> (8 * (j & 3)));
            }
        }
    }
}

}  // namespace bin
}  // namespace yabt

using namespace yabt;
using namespace yabt::bin;

extern "C" {

size_t yabt_bin_fit_workspace_bytes(int64_t m, int F) {
    if (m < 0 || m > 0x7FFFFFFFll || F < 1) return 0;
    return carve_fit(nullptr, m, F).bytes;
}

int yabt_bin_fit(const float* X, int64_t ldx, int64_t n, int F, const int64_t* sample_rows, int64_t m, int max_bins,
                 void* workspace, size_t workspace_bytes, float* out_edges, int64_t ld_edges, int32_t* out_nedges,
                 float* out_scales, float* out_medians, hipStream_t stream) {
    if (n < 0 || F < 1 || ldx < F || m < 0 || m > 0x7FFFFFFFll || max_bins < 2 || max_bins > 256 ||
        ld_edges < max_bins - 1)
        return fail(-2, "yabt_bin_fit: bad sizes (ldx >= F >= 1, 2 <= max_bins <= 256, ld_edges >= max_bins - 1)");
    if (!sample_rows && m != n) return fail(-2, "yabt_bin_fit: without sample_rows the sample is all n rows (m == n)");
    if (!X || !workspace || !out_edges || !out_nedges || !out_scales || !out_medians)
        return fail(-2, "yabt_bin_fit: null pointer argument");
    const FitWs w = carve_fit((char*)workspace, m, F);
    if (workspace_bytes < w.bytes) return fail(-2, "yabt_bin_fit: workspace too small");
    // quantiles and scales of the sample (an empty sample is the column [0.0])
    k_gather_keys<<<launch_grid(max(m, (int64_t)1) * F, TB, 8192), TB, 0, stream>>>(X, ldx, F, sample_rows, m,
                                                                                     w.orig);
    if (m > 0) {
        const hipError_t e =
            hipMemcpyAsync(w.ka, w.orig, (size_t)F * m * sizeof(uint32_t), hipMemcpyDeviceToDevice, stream);
        if (e != hipSuccess) return hip_fail(e, "yabt_bin_fit: key copy");
        k_sort<<<F, SB, 0, stream>>>(w.ka, w.kb, m);
    }
    k_quantiles<<<F, TB, 0, stream>>>(w.ka, w.orig, reinterpret_cast<float*>(w.kb), m, max_bins, out_edges, ld_edges,
                                      out_nedges, out_scales);
    // medians over all n rows
    const hipError_t e = hipMemsetAsync(w.cnt, 0, (size_t)F * sizeof(uint32_t), stream);
    if (e != hipSuccess) return hip_fail(e, "yabt_bin_fit: clear");
    const dim3 grid((unsigned)launch_grid(max(n, (int64_t)1), TB / HT * 8, 1024), (unsigned)((F + HT - 1) / HT));
    k_count_valid<<<grid, TB, 0, stream>>>(X, ldx, n, F, w.cnt);
    k_select_init<<<(F + 63) / 64, 64, 0, stream>>>(w.cnt, F, w.sel_state, w.sel_hist);
    for (int shift = 24; shift >= 0; shift -= 8) {
        k_select_hist<<<grid, TB, 0, stream>>>(X, ldx, n, F, shift, w.sel_state, w.sel_hist);
        k_select_step<<<(F + 63) / 64, 64, 0, stream>>>(F, w.sel_state, w.sel_hist);
    }
    k_select_finish<<<(F + 63) / 64, 64, 0, stream>>>(w.cnt, F, w.sel_state, out_medians);
    return launch_status("yabt_bin_fit launch");
}

int yabt_bin_transform(const float* X, int64_t ldx, int64_t n, int F, const float* edges, int64_t ld_edges,
                       const int32_t* nedges, const float* medians, uint8_t* out_fm, int64_t ld_fm, uint8_t* out_rm,
                       int64_t ld_rm, float* out_imputed, int64_t ld_imputed, hipStream_t stream) {
    if (n < 0 || F < 1 || ldx < F || ld_edges < 1 || (out_fm && ld_fm < n) || (out_imputed && ld_imputed < F))
        return fail(-2, "yabt_bin_transform: bad sizes");
    if (out_rm && ld_rm < F) return fail(-2, "yabt_bin_transform: row-major output needs ld_rm >= F");
    // 16-byte row stores when every 16-feature tile of every row is 16-byte aligned
    const int rm_vec = out_rm && ld_rm % 16 == 0 && aligned16(out_rm) ? 1 : 0;
    if (!X || !edges || !nedges || !medians || !(out_fm || out_rm || out_imputed))
        return fail(-2, "yabt_bin_transform: null pointer argument");
    if (n == 0) return 0;
    const dim3 grid((unsigned)launch_grid(n, TB, 4096), (unsigned)((F + HT - 1) / HT));
    k_transform<<<grid, TB, 0, stream>>>(X, ldx, n, F, edges, ld_edges, nedges, medians, out_fm, ld_fm, out_rm, ld_rm,
                                         out_imputed, ld_imputed, rm_vec);
    return launch_status("yabt_bin_transform launch");
}

}  // extern "C"
