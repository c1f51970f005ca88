// The boosting step around the grower on gfx950: gradients/hessians of the
// losses and the margin update, so consecutive trees need no host copies.
//
//   yabt_grad_hess      LogLoss / MSELoss grad_hess (yabt/boosting.py:35-38, 52-54), at the
//                       margin or at margin + value[leaf] (yabt/neural_leaves.py:147)
//   yabt_margin_update  margin += value[leaf] + sum_j linear[leaf][j] * clamp(x_j, lo, hi)
//                       (yabt/boosting.py:508-511 with Tree.net_contribution,
//                       yabt/tree.py:118-128)
//   yabt_predict        out = base + sum over trees of Tree.predict (yabt/boosting.py:536-545,
//                       yabt/tree.py:82-135), all trees of a forest in one launch

#include "common.h"
#include "host.h"
#include "yabt_hip.h"

namespace yabt {

constexpr int BB = 256;

// loss 0: squared error, g = m - y, h = 1; loss 1: logistic, p = 1 / (1 + e^-m),
// g = p - y, h = max(p (1 - p), 1e-6), in fp32 as the reference's torch code.
template <bool AT_LEAF>
__global__ void __launch_bounds__(BB) k_grad_hess(int loss, const float* __restrict__ margin,
                                                  const int64_t* __restrict__ leaf, const float* __restrict__ value,
                                                  int64_t n_nodes, const float* __restrict__ y, int64_t n,
                                                  float* __restrict__ g, float* __restrict__ h) {
    for (int64_t i = (int64_t)blockIdx.x * BB + threadIdx.x; i < n; i += (int64_t)gridDim.x * BB) {
        float m = margin[i];
        if (AT_LEAF) {
            const int64_t l = leaf[i];
            if (l >= 0 && l < n_nodes) m = m + value[l];
        }
        const float t = y[i];
        if (loss == 0) {
            g[i] = m - t;
            h[i] = 1.0f;
        } else {
            const float p = 1.0f / (1.0f + expf(-m));
            g[i] = p - t;
            h[i] = fmaxf(p * (1.0f - p), 1e-6f);
        }
    }
}

// One row per thread; the leaf's linear model over K inputs with the inputs
// clamped to the leaf's envelope (the reference adds the terms in input order).
template <int K>
__global__ void __launch_bounds__(BB) k_margin_update(float* __restrict__ margin, int64_t n,
                                                      const int64_t* __restrict__ leaf, int64_t n_nodes,
                                                      const float* __restrict__ value,
                                                      const int32_t* __restrict__ feats, const float* __restrict__ lin,
                                                      const float* __restrict__ lo, const float* __restrict__ hi,
                                                      int x_kind, const void* __restrict__ X, int64_t ldx) {
    __shared__ int32_t s_fs[K > 0 ? K : 1];
    if (K > 0 && threadIdx.x < K) s_fs[threadIdx.x] = feats[threadIdx.x];
    __syncthreads();
    for (int64_t i = (int64_t)blockIdx.x * BB + threadIdx.x; i < n; i += (int64_t)gridDim.x * BB) {
        const int64_t node = leaf[i];
        if (node < 0 || node >= n_nodes) continue;
        float c = value[node];
        if (K > 0) {
            float net = 0.0f;
#pragma unroll
            for (int j = 0; j < K; ++j) {
                float x = x_kind == 0   ? reinterpret_cast<const float*>(X)[(size_t)i * (size_t)ldx + s_fs[j]]
                          : x_kind == 2 ? reinterpret_cast<const float*>(X)[(size_t)s_fs[j] * (size_t)ldx + i]
                                        : (float)reinterpret_cast<const uint8_t*>(X)[(size_t)s_fs[j] * (size_t)ldx + i];
                x = fminf(fmaxf(x, lo[node * K + j]), hi[node * K + j]);
                net += lin[node * K + j] * x;
            }
            c += net;
        }
        margin[i] += c;
    }
}

template <int K>
void launch_margin(float* margin, int64_t n, const int64_t* leaf, int64_t n_nodes, const float* value,
                   const int32_t* feats, const float* lin, const float* lo, const float* hi, int x_kind, const void* X,
                   int64_t ldx, hipStream_t stream) {
    k_margin_update<K><<<launch_grid(n, BB * 8, 4096), BB, 0, stream>>>(margin, n, leaf, n_nodes, value, feats, lin,
                                                                       lo, hi, x_kind, X, ldx);
}

// One row per thread, trees in order, each walked from its root as capply
// does (yabt/_cgrow/grow.c:223-239; a walk stops at a leaf, at an out-of-range
// feature or child, or after as many steps as the tree has nodes), then
// value[node] plus the node's clamped linear contribution.
__global__ void __launch_bounds__(BB) k_predict(const float* __restrict__ X, int64_t ldx, int F, int64_t n, int T,
                                                const int64_t* __restrict__ node_off, int64_t n_total,
                                                const int64_t* __restrict__ feature,
                                                const float* __restrict__ threshold, const int64_t* __restrict__ left,
                                                const int64_t* __restrict__ right, const float* __restrict__ value,
                                                int K, const int32_t* __restrict__ net_k,
                                                const int32_t* __restrict__ net_feats, const float* __restrict__ lin,
                                                const float* __restrict__ lo, const float* __restrict__ hi, float base,
                                                int accumulate, float* __restrict__ out) {
    for (int64_t i = (int64_t)blockIdx.x * BB + threadIdx.x; i < n; i += (int64_t)gridDim.x * BB) {
        const float* x = X + (size_t)i * (size_t)ldx;
        float acc = accumulate ? out[i] : base;
        for (int t = 0; t < T; ++t) {
            const int64_t off = node_off[t];
            const int64_t nt = node_off[t + 1] - off;
            if (off < 0 || nt < 1 || off + nt > n_total) continue;
            int64_t node = 0;
            for (int64_t s = 0; s < nt; ++s) {
                const int64_t f = feature[off + node];
                if (f < 0 || f >= F) break;
                const int64_t nxt = (x[f] <= threshold[off + node]) ? left[off + node] : right[off + node];
                if (nxt < 0 || nxt >= nt) break;
                node = nxt;
            }
            const int64_t g = off + node;
            float c = value[g];
            const int kt = net_k ? min(net_k[t], K) : 0;
            if (kt > 0) {
                float net = 0.0f;
                for (int j = 0; j < kt; ++j) {
                    const int fj = net_feats[t * K + j];
                    float xv = (fj >= 0 && fj < F) ? x[fj] : 0.0f;
                    if (lo) xv = fminf(fmaxf(xv, lo[g * K + j]), hi[g * K + j]);
                    net += lin[g * K + j] * xv;
                }
                c += net;
            }
            acc += c;
        }
        out[i] = acc;
    }
}

}  // namespace yabt

using namespace yabt;

extern "C" {

int yabt_grad_hess(int loss, const float* margin, const int64_t* leaf_of_row, const float* value, int64_t n_nodes,
                   const float* y, int64_t n, float* out_g, float* out_h, hipStream_t stream) {
    if ((loss != 0 && loss != 1) || n < 0) return fail(-2, "yabt_grad_hess: loss must be 0 (MSE) or 1 (LogLoss)");
    if (n == 0) return 0;
    if (!margin || !y || !out_g || !out_h) return fail(-2, "yabt_grad_hess: null pointer argument");
    if ((leaf_of_row == nullptr) != (value == nullptr) || (leaf_of_row && n_nodes < 1))
        return fail(-2, "yabt_grad_hess: leaf_of_row and value (n_nodes >= 1) go together");
    const int grid = launch_grid(n, BB * 8, 4096);
    if (leaf_of_row)
        k_grad_hess<true><<<grid, BB, 0, stream>>>(loss, margin, leaf_of_row, value, n_nodes, y, n, out_g, out_h);
    else
        k_grad_hess<false><<<grid, BB, 0, stream>>>(loss, margin, nullptr, nullptr, 0, y, n, out_g, out_h);
    return launch_status("yabt_grad_hess launch");
}

int yabt_margin_update(float* margin, int64_t n, const int64_t* leaf_of_row, const float* value, int64_t n_nodes,
                       int K, const int32_t* feats, const float* linear, const float* lo, const float* hi, int x_kind,
                       const void* X, int64_t ldx, hipStream_t stream) {
    if (n < 0 || n_nodes < 1 || K < 0 || K > 8 || (K > 0 && (x_kind < 0 || x_kind > 2)))
        return fail(-2, "yabt_margin_update: bad sizes (n_nodes >= 1, 0 <= K <= 8, x_kind 0, 1 or 2)");
    if (n == 0) return 0;
    if (!margin || !leaf_of_row || !value || (K > 0 && (!feats || !linear || !lo || !hi || !X)))
        return fail(-2, "yabt_margin_update: null pointer argument");
    switch (K) {
        case 0: launch_margin<0>(margin, n, leaf_of_row, n_nodes, value, feats, linear, lo, hi, x_kind, X, ldx, stream); break;
        case 1: launch_margin<1>(margin, n, leaf_of_row, n_nodes, value, feats, linear, lo, hi, x_kind, X, ldx, stream); break;
        case 2: launch_margin<2>(margin, n, leaf_of_row, n_nodes, value, feats, linear, lo, hi, x_kind, X, ldx, stream); break;
        case 3: launch_margin<3>(margin, n, leaf_of_row, n_nodes, value, feats, linear, lo, hi, x_kind, X, ldx, stream); break;
        case 4: launch_margin<4>(margin, n, leaf_of_row, n_nodes, value, feats, linear, lo, hi, x_kind, X, ldx, stream); break;
        case 5: launch_margin<5>(margin, n, leaf_of_row, n_nodes, value, feats, linear, lo, hi, x_kind, X, ldx, stream); break;
        case 6: launch_margin<6>(margin, n, leaf_of_row, n_nodes, value, feats, linear, lo, hi, x_kind, X, ldx, stream); break;
        case 7: launch_margin<7>(margin, n, leaf_of_row, n_nodes, value, feats, linear, lo, hi, x_kind, X, ldx, stream); break;
        default: launch_margin<8>(margin, n, leaf_of_row, n_nodes, value, feats, linear, lo, hi, x_kind, X, ldx, stream); break;
    }
    return launch_status("yabt_margin_update launch");
}

int yabt_predict(const float* X, int64_t ldx, int64_t n, int F, int T, const int64_t* node_off, int64_t n_total,
                 const int64_t* feature, const float* threshold, const int64_t* left, const int64_t* right,
                 const float* value, int K, const int32_t* net_k, const int32_t* net_feats, const float* linear,
                 const float* lo, const float* hi, float base, int accumulate, float* out, hipStream_t stream) {
    if (n < 0 || F < 1 || ldx < F || T < 0 || n_total < 0 || K < 0 || K > 8)
        return fail(-2, "yabt_predict: bad sizes (ldx >= F >= 1, 0 <= K <= 8)");
    if (n == 0) return 0;
    if (!X || !out || (T > 0 && (!node_off || !feature || !threshold || !left || !right || !value)))
        return fail(-2, "yabt_predict: null pointer argument");
    if (net_k && (K < 1 || !net_feats || !linear || (lo == nullptr) != (hi == nullptr)))
        return fail(-2, "yabt_predict: linear leaves need K >= 1, net_feats and linear (lo and hi together)");
    k_predict<<<launch_grid(n, BB, 8192), BB, 0, stream>>>(X, ldx, F, n, T, node_off, n_total, feature, threshold,
                                                          left, right, value, K, net_k, net_feats, linear, lo, hi,
                                                          base, accumulate, out);
    return launch_status("yabt_predict launch");
}

}  // extern "C"
