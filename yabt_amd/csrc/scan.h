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
    int32_t f;                // feature (set by the caller)
    int64_t left[3];          // (sum q(g), sum q(h), count) of bins <= b
};

// Bins 4*lane .. 4*lane+3 of one feature of a histogram slot [3][F][256];
// has_h false: the h plane is not read (h4 is set to zero).
__device__ __forceinline__ void load_bins(const int64_t* slot, int F, int f, int lane, int64_t g4[4], int64_t h4[4],
                                          int64_t c4[4], bool has_h) {
    const size_t plane = (size_t)F * NB, at = (size_t)f * NB + 4 * lane;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        g4[j] = slot[at + j];
        h4[j] = has_h ? slot[plane + at + j] : 0;
        c4[j] = slot[2 * plane + at + j];
    }
}

__device__ __forceinline__ void store_bins(int64_t* slot, int F, int f, int lane, const int64_t g4[4],
                                           const int64_t h4[4], const int64_t c4[4], bool has_h) {
    const size_t plane = (size_t)F * NB, at = (size_t)f * NB + 4 * lane;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        slot[at + j] = g4[j];
        if (has_h) slot[plane + at + j] = h4[j];
        slot[2 * plane + at + j] = c4[j];
    }
}

// Restore the skipped default bin d of one feature: bin d += node total minus
// the sum over all 256 bins (exact; a no-op when nothing was skipped).  has_h
// false: the h channel is not kept (derived from the counts afterwards).
__device__ __forceinline__ void fill_default(int64_t g4[4], int64_t h4[4], int64_t c4[4], int d, const int64_t tot[3],
                                             bool has_h, int lane) {
    if (d < 0) return;
    const int64_t sg = wave_sum_i64(g4[0] + g4[1] + g4[2] + g4[3]);
    const int64_t sh = has_h ? wave_sum_i64(h4[0] + h4[1] + h4[2] + h4[3]) : 0;
    const int64_t sc = wave_sum_i64(c4[0] + c4[1] + c4[2] + c4[3]);
    if ((d >> 2) == lane) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if ((d & 3) == j) {
                g4[j] += tot[0] - sg;
                if (has_h) h4[j] += tot[1] - sh;
                c4[j] += tot[2] - sc;
            }
    }
}

// (sel, b) of `other` beats mine: larger sel, then lower bin; b < 0 never wins.
__device__ __forceinline__ bool split_beats(double os, int ob, double s, int b) {
    return ob >= 0 && (b < 0 || os > s || (os == s && ob < b));
}

// One wave scans one feature; lane l holds bins 4l..4l+3 (g, h, count).
// Every lane returns the feature's record; t256 receives the totals over all
// 256 bins (the node totals).  Prefix sums use DPP row shifts plus scalar row
// totals, the argmax DPP row rotations (every lane of a row ends with the
// row's winner) plus the four row winners.
__device__ __forceinline__ ScanRec scan_feature(const int64_t g4[4], const int64_t h4[4], const int64_t c4[4], int nb,
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
    const int64_t og = wave_incl_scan_i64(pg[3], lane) - pg[3];
    const int64_t oh = wave_incl_scan_i64(ph[3], lane) - ph[3];
    const int64_t oc = wave_incl_scan_i64(pc[3], lane) - pc[3];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        pg[j] += og;
        ph[j] += oh;
        pc[j] += oc;
    }
    t256[0] = readlane64(pg[3], WAVE - 1);
    t256[1] = readlane64(ph[3], WAVE - 1);
    t256[2] = readlane64(pc[3], WAVE - 1);
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
        Gt = readlane64(vg, src);
        Ht = readlane64(vh, src);
        Ct = readlane64(vc, src);
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
    // lane-best record kept in place; the wave argmax moves only (sel, b)
    int64_t lg = 0, lh = 0, lc = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (best_j == j) {
            lg = pg[j];
            lh = ph[j];
            lc = pc[j];
        }
    double s = best_sel;
    int b = best_j < 0 ? -1 : 4 * lane + best_j;
#define YABT_ARGMAX_STEP(M)                                                    \
    {                                                                          \
        const double os = dpp_f64<DPP_ROW_ROR + (M)>(s);                     \
        const int ob = (int)dpp32<DPP_ROW_ROR + (M)>((uint32_t)b);           \
        if (split_beats(os, ob, s, b)) {                                       \
            s = os;                                                            \
            b = ob;                                                            \
        }                                                                      \
    }
    YABT_ARGMAX_STEP(8) YABT_ARGMAX_STEP(4) YABT_ARGMAX_STEP(2) YABT_ARGMAX_STEP(1)
#undef YABT_ARGMAX_STEP
    // rows 0..3: each row now holds its winner in every lane
    double ws = readlane_f64(s, 0);
    int wb = __builtin_amdgcn_readlane(b, 0);
#pragma unroll
    for (int row = 1; row < 4; ++row) {
        const double os = readlane_f64(s, 16 * row);
        const int ob = __builtin_amdgcn_readlane(b, 16 * row);
        if (split_beats(os, ob, ws, wb)) {
            ws = os;
            wb = ob;
        }
    }
    ScanRec r;
    r.f = -1;
    if (wb < 0) {
        r.sel = -INFINITY;
        r.gain = -INFINITY;
        r.b = -1;
        r.left[0] = r.left[1] = r.left[2] = 0;
        return r;
    }
    const int src = wb >> 2;     // the lane whose lane-best is the winner
    r.sel = ws;
    r.b = wb;
    r.gain = readlane_f64(best_gain, src);
    r.left[0] = readlane64(lg, src);
    r.left[1] = readlane64(lh, src);
    r.left[2] = readlane64(lc, src);
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
#define YABT_MAX_STEP(M)                                                       \
    {                                                                          \
        const float o = __uint_as_float(dpp32<DPP_ROW_ROR + (M)>(__float_as_uint(m))); \
        if (o > m) m = o;                                                      \
    }
    YABT_MAX_STEP(8) YABT_MAX_STEP(4) YABT_MAX_STEP(2) YABT_MAX_STEP(1)
#undef YABT_MAX_STEP
    float r = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(m), 0));
#pragma unroll
    for (int row = 1; row < 4; ++row) {
        const float o = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(m), 16 * row));
        if (o > r) r = o;
    }
    return 1.0f + ib * r;
}

// Record a beats record b in grow.c's feature order (grow.c:181-192): a valid
// split beats none, then larger sel, then the lower feature.
__device__ __forceinline__ bool rec_beats(double sa, int fa, int ba, double sb, int fb, int bb) {
    return ba >= 0 && (bb < 0 || sa > sb || (sa == sb && fa < fb));
}

// One wave (all 64 lanes active): the best of the lanes' records `mine` (the
// lane's index my_idx, -1: none) in every lane (b = -1: none valid).
__device__ inline ScanRec wave_reduce_record(const ScanRec& mine, int my_idx) {
    // rotations inside each 16-lane row leave the row's best in all of its
    // lanes (valid records have distinct features: the order is total), then
    // the four rows' bests meet
    double s = mine.sel;
    int f = mine.f, b = mine.b, idx = my_idx;
    auto take = [&](double os, int of, int ob, int oi) {
        if (rec_beats(os, of, ob, s, f, b)) {
            s = os;
            f = of;
            b = ob;
            idx = oi;
        }
    };
    take(dpp_f64<DPP_ROW_ROR + 8>(s), (int)dpp32<DPP_ROW_ROR + 8>((uint32_t)f), (int)dpp32<DPP_ROW_ROR + 8>((uint32_t)b),
         (int)dpp32<DPP_ROW_ROR + 8>((uint32_t)idx));
    take(dpp_f64<DPP_ROW_ROR + 4>(s), (int)dpp32<DPP_ROW_ROR + 4>((uint32_t)f), (int)dpp32<DPP_ROW_ROR + 4>((uint32_t)b),
         (int)dpp32<DPP_ROW_ROR + 4>((uint32_t)idx));
    take(dpp_f64<DPP_ROW_ROR + 2>(s), (int)dpp32<DPP_ROW_ROR + 2>((uint32_t)f), (int)dpp32<DPP_ROW_ROR + 2>((uint32_t)b),
         (int)dpp32<DPP_ROW_ROR + 2>((uint32_t)idx));
    take(dpp_f64<DPP_ROW_ROR + 1>(s), (int)dpp32<DPP_ROW_ROR + 1>((uint32_t)f), (int)dpp32<DPP_ROW_ROR + 1>((uint32_t)b),
         (int)dpp32<DPP_ROW_ROR + 1>((uint32_t)idx));
    {
        const double s0 = s;
        const int f0 = f, b0 = b, i0 = idx;
        s = readlane_f64(s0, 0);
        f = __builtin_amdgcn_readlane(f0, 0);
        b = __builtin_amdgcn_readlane(b0, 0);
        idx = __builtin_amdgcn_readlane(i0, 0);
#pragma unroll
        for (int row = 1; row < 4; ++row)
            take(readlane_f64(s0, 16 * row), __builtin_amdgcn_readlane(f0, 16 * row),
                 __builtin_amdgcn_readlane(b0, 16 * row), __builtin_amdgcn_readlane(i0, 16 * row));
    }
    ScanRec r;
    const uint64_t owner = __ballot(idx >= 0 && my_idx == idx);
    if (owner == 0) {
        r = mine;          // no valid record anywhere: every lane's is empty
        r.b = -1;
        r.f = -1;
        return r;
    }
    const int src = __ffsll((unsigned long long)owner) - 1;
    r.sel = readlane_f64(mine.sel, src);
    r.gain = readlane_f64(mine.gain, src);
    r.b = __builtin_amdgcn_readlane(mine.b, src);
    r.f = __builtin_amdgcn_readlane(mine.f, src);
    r.left[0] = readlane64(mine.left[0], src);
    r.left[1] = readlane64(mine.left[1], src);
    r.left[2] = readlane64(mine.left[2], src);
    return r;
}

__device__ __forceinline__ ScanRec empty_record() {
    ScanRec e;
    e.sel = -INFINITY;
    e.gain = -INFINITY;
    e.b = -1;
    e.f = INT_MAX;
    e.left[0] = e.left[1] = e.left[2] = 0;
    return e;
}

// A block's scan record for the block that takes the last ticket of the
// launch (which may run on another XCD, behind another L2).  The record is
// written with agent-scope atomic stores, which write through to the
// device's point of coherence, and record_published() waits for them; the
// ticket that follows can then be a relaxed atomic.  An agent-scope release
// fence here would write back the whole L2's dirty lines instead, and with
// tens of blocks per XCD those writebacks queue behind one another.  The
// reader takes the last ticket, then an agent-scope acquire fence (which
// invalidates its L2) before it loads the records.
static_assert(sizeof(ScanRec) % 8 == 0, "a record is whole 64-bit words");
__device__ __forceinline__ void publish_record(ScanRec* dst, const ScanRec& r) {
    uint64_t w[sizeof(ScanRec) / 8];
    __builtin_memcpy(w, &r, sizeof(ScanRec));
    uint64_t* d = reinterpret_cast<uint64_t*>(dst);
#pragma unroll
    for (int i = 0; i < (int)(sizeof(ScanRec) / 8); ++i)
        __hip_atomic_store(d + i, w[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The calling wave's stores so far have completed (publish_record's are at
// the device's point of coherence).
__device__ __forceinline__ void record_published() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// One wave (all 64 lanes active): the best of rec[0, n) in every lane (b = -1:
// none valid).
__device__ inline ScanRec wave_best_record(const ScanRec* rec, int n, int lane) {
    ScanRec mine = empty_record();
    int my_idx = -1;
    for (int i = lane; i < n; i += WAVE) {
        const ScanRec r = rec[i];
        if (rec_beats(r.sel, r.f, r.b, mine.sel, mine.f, mine.b)) {
            mine = r;
            my_idx = i;
        }
    }
    return wave_reduce_record(mine, my_idx);
}

// wave_best_record over records other blocks of the launch published with
// publish_record: read with agent-scope atomic loads, which no stale line of
// this XCD's L2 can serve.
__device__ inline ScanRec wave_best_record_agent(const ScanRec* rec, int n, int lane) {
    ScanRec mine = empty_record();
    int my_idx = -1;
    for (int i = lane; i < n; i += WAVE) {
        uint64_t w[sizeof(ScanRec) / 8];
        const uint64_t* src = reinterpret_cast<const uint64_t*>(rec + i);
#pragma unroll
        for (int k = 0; k < (int)(sizeof(ScanRec) / 8); ++k)
            w[k] = __hip_atomic_load(src + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ScanRec r;
        __builtin_memcpy(&r, w, sizeof(ScanRec));
        if (rec_beats(r.sel, r.f, r.b, mine.sel, mine.f, mine.b)) {
            mine = r;
            my_idx = i;
        }
    }
    return wave_reduce_record(mine, my_idx);
}

// Several waves' worth of wave_best_record at once: out[k] = the best of
// rec[i n, i n + n) for i = w0 + k stride < nchild (n <= 64: one record per
// lane), all loads issued before any reduction.
template <int K>
__device__ inline void wave_best_records(const ScanRec* rec, int n, int w0, int stride, int nchild, int lane,
                                         ScanRec (&out)[K]) {
    ScanRec mine[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int i = w0 + k * stride;
        mine[k] = (i < nchild && lane < n) ? rec[(size_t)i * n + lane] : empty_record();
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int i = w0 + k * stride;
        if (i >= nchild) break;
        out[k] = wave_reduce_record(mine[k], mine[k].b >= 0 ? lane : -1);
    }
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
