// Split scan of exact histograms: grow.c's double-precision Newton gain
// (grow.c:151-176) evaluated on int64 prefix sums, with grow.c's tie-breaks
// (first bin within a feature, grow.c:170; first feature across, grow.c:181-192).
#pragma once

#include "common.h"

namespace yabt {

struct ScanParams {
    double lam, gamma, mcw;   // float-rounded, widened to double as grow.c receives them
    int msl;
};

struct ScanRec {
    double sel;               // gain * boost[f]; what the argmax ranks
    double gain;              // true gain at the chosen bin
    int32_t b;                // chosen bin, -1: no valid split on this feature
    int32_t pad;
    int64_t left[3];          // (sum q(g), sum q(h), count) of bins <= b
};

// Bins 4*lane .. 4*lane+3 of one feature of a histogram slot [3][F][256].
__device__ __forceinline__ void load_bins(const int64_t* slot, int F, int f, int lane, int64_t g4[4], int64_t h4[4],
                                          int64_t c4[4]) {
    const size_t plane = (size_t)F * NB, at = (size_t)f * NB + 4 * lane;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        g4[j] = slot[at + j];
        h4[j] = slot[plane + at + j];
        c4[j] = slot[2 * plane + at + j];
    }
}

__device__ __forceinline__ void store_bins(int64_t* slot, int F, int f, int lane, const int64_t g4[4],
                                           const int64_t h4[4], const int64_t c4[4]) {
    const size_t plane = (size_t)F * NB, at = (size_t)f * NB + 4 * lane;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        slot[at + j] = g4[j];
        slot[plane + at + j] = h4[j];
        slot[2 * plane + at + j] = c4[j];
    }
}

// Restore the skipped default bin d of one feature: bin d += node total minus
// the sum over all 256 bins (exact; a no-op when nothing was skipped).
__device__ __forceinline__ void fill_default(int64_t g4[4], int64_t h4[4], int64_t c4[4], int d, const int64_t tot[3],
                                             bool counts, int lane) {
    int64_t sg = g4[0] + g4[1] + g4[2] + g4[3];
    int64_t sh = h4[0] + h4[1] + h4[2] + h4[3];
    int64_t sc = c4[0] + c4[1] + c4[2] + c4[3];
    sg = wave_sum<int64_t>(sg);
    sh = wave_sum<int64_t>(sh);
    sc = wave_sum<int64_t>(sc);
    if (d >= 0 && (d >> 2) == lane) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if ((d & 3) == j) {
                g4[j] += tot[0] - sg;
                h4[j] += tot[1] - sh;
                if (counts) c4[j] += tot[2] - sc;
            }
    }
}

// One wave scans one feature; lane l holds bins 4l..4l+3 (g, h, count).
// Every lane returns the feature's record; t256 receives the totals over all
// 256 bins (the node totals, used for node values).
__device__ inline ScanRec scan_feature(const int64_t g4[4], const int64_t h4[4], const int64_t c4[4], int nb,
                                       double ig, double ih, const ScanParams& sp, double bo, int lane,
                                       int64_t t256[3]) {
    int64_t pg[4], ph[4], pc[4];
    pg[0] = g4[0];
    ph[0] = h4[0];
    pc[0] = c4[0];
#pragma unroll
    for (int j = 1; j < 4; ++j) {
        pg[j] = pg[j - 1] + g4[j];
        ph[j] = ph[j - 1] + h4[j];
        pc[j] = pc[j - 1] + c4[j];
    }
    const int64_t og = wave_excl_scan<int64_t>(pg[3], lane);
    const int64_t oh = wave_excl_scan<int64_t>(ph[3], lane);
    const int64_t oc = wave_excl_scan<int64_t>(pc[3], lane);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        pg[j] += og;
        ph[j] += oh;
        pc[j] += oc;
    }
    t256[0] = __shfl(pg[3], WAVE - 1, WAVE);
    t256[1] = __shfl(ph[3], WAVE - 1, WAVE);
    t256[2] = __shfl(pc[3], WAVE - 1, WAVE);
    // totals over the feature's used bins b < nb (grow.c:151-156)
    int64_t Gt = 0, Ht = 0, Ct = 0;
    if (nb > 0) {
        const int jj = (nb - 1) & 3, src = (nb - 1) >> 2;
        int64_t vg = pg[0], vh = ph[0], vc = pc[0];
#pragma unroll
        for (int j = 1; j < 4; ++j)
            if (jj == j) {
                vg = pg[j];
                vh = ph[j];
                vc = pc[j];
            }
        Gt = __shfl(vg, src, WAVE);
        Ht = __shfl(vh, src, WAVE);
        Ct = __shfl(vc, src, WAVE);
    }
    const double G = (double)Gt * ig, H = (double)Ht * ih;
    const double parent = G * G / (H + sp.lam);
    double best_sel = -INFINITY, best_gain = -INFINITY;
    int best_j = -1;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int b = 4 * lane + j;
        if (b + 1 < nb) {
            const int64_t cl = pc[j], cr = Ct - pc[j];
            const double GL = (double)pg[j] * ig, GR = (double)(Gt - pg[j]) * ig;
            const double HL = (double)ph[j] * ih, HR = (double)(Ht - ph[j]) * ih;
            if (cl >= sp.msl && cr >= sp.msl && HL >= sp.mcw && HR >= sp.mcw) {
                const double gain = 0.5 * (GL * GL / (HL + sp.lam) + GR * GR / (HR + sp.lam) - parent) - sp.gamma;
                const double sel = gain * bo;
                if (sel > best_sel) {
                    best_sel = sel;
                    best_gain = gain;
                    best_j = j;
                }
            }
        }
    }
    ScanRec r;
    r.sel = best_sel;
    r.gain = best_gain;
    r.b = best_j < 0 ? -1 : 4 * lane + best_j;
    r.pad = 0;
    r.left[0] = r.left[1] = r.left[2] = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (best_j == j) {
            r.left[0] = pg[j];
            r.left[1] = ph[j];
            r.left[2] = pc[j];
        }
    // wave argmax: larger sel, then lower bin; lanes without a valid bin lose
#pragma unroll
    for (int dd = WAVE / 2; dd > 0; dd >>= 1) {
        const double os = __shfl_xor(r.sel, dd, WAVE);
        const double ogn = __shfl_xor(r.gain, dd, WAVE);
        const int ob = __shfl_xor(r.b, dd, WAVE);
        const int64_t l0 = __shfl_xor(r.left[0], dd, WAVE);
        const int64_t l1 = __shfl_xor(r.left[1], dd, WAVE);
        const int64_t l2 = __shfl_xor(r.left[2], dd, WAVE);
        const bool take = ob >= 0 && (r.b < 0 || os > r.sel || (os == r.sel && ob < r.b));
        if (take) {
            r.sel = os;
            r.gain = ogn;
            r.b = ob;
            r.left[0] = l0;
            r.left[1] = l1;
            r.left[2] = l2;
        }
    }
    return r;
}

__device__ __forceinline__ void no_split(ScanRec& r) {
    r.sel = -INFINITY;
    r.gain = -INFINITY;
    r.b = -1;
}

// boost[f] = 1 + ib * max(0, max_{p on path} imat[p][f]) in fp32 (grow.c:111-122);
// the running max ignores NaN like grow.c's `row[j] > boost[j]`.
__device__ inline float path_boost(const uint8_t* path, const float* imat, float ib, int F, int f, int lane) {
    float m = 0.0f;
    for (int p = lane; p < F; p += WAVE)
        if (path[p]) {
            const float v = imat[(size_t)p * F + f];
            if (v > m) m = v;
        }
#pragma unroll
    for (int dd = WAVE / 2; dd > 0; dd >>= 1) {
        const float o = __shfl_xor(m, dd, WAVE);
        if (o > m) m = o;
    }
    return 1.0f + ib * m;
}

// Feature-major reduction of one node's records (grow.c:181-192), NT threads;
// returns the winning feature (-1 if none) in every thread.
template <int NT>
__device__ int reduce_records(const ScanRec* rec, int F) {
    __shared__ double s_key[NT / WAVE];
    __shared__ int s_idx[NT / WAVE];
    double key = -INFINITY;
    int idx = INT_MAX;
    for (int f = threadIdx.x; f < F; f += NT) {
        const ScanRec& r = rec[f];
        if (r.b >= 0 && better(r.sel, f, key, idx)) {
            key = r.sel;
            idx = f;
        }
    }
    block_argmax<NT>(key, idx, s_key, s_idx);
    return idx == INT_MAX ? -1 : idx;
}

}  // namespace yabt
