/*
 * grow_oracle.c -- CPU oracle for the YABT leaf-wise tree-growing hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  The product (yabt_amd/) never links, loads or
 * calls this code.  It is used by tests/, by __graft_entry__.smoke() and by the
 * cpu_baseline leg of bench.py, always as the reference the HIP path is
 * compared against (or timed beside), never as something that is shipped.
 *
 * One best-first grower, two arithmetic modes:
 *
 *   OR_MODE_FP32   restates yabt/_cgrow/grow.c `cgrow` (grow.c:243-427):
 *                  fp32 per-bin sums accumulated in row order (grow.c:37-62),
 *                  the sparse builder (grow.c:68-107), the in-place two-pointer
 *                  partition (grow.c:201-217), the double-precision split scan
 *                  with its feature-major tie-break (grow.c:129-197) and the
 *                  fp32 leaf table (grow.c:284-407).  tests/golden/ pins this
 *                  mode bit-for-bit against the compiled reference grow.c.
 *
 *   OR_MODE_FIXED  the arithmetic contract of the HIP path: gradients and
 *                  hessians are quantised to int64 fixed point with one
 *                  power-of-two scale per channel and call (or_hist_contract:
 *                  the narrow or_hist_shift when its residual is small, else
 *                  the wide or_wide_shift), histograms are
 *                  exact integer sums (order-free, so sibling subtraction and
 *                  the default-bin fill are exact), the partition is stable, and
 *                  the split scan evaluates the reference's double-precision
 *                  gain formula on the exact prefix sums.  The HIP path must be
 *                  bit-identical to this mode.
 *
 * Every floating-point expression keeps the reference's operation order; build
 * with -ffp-contract=off (the Makefile does) so no multiply-add is fused.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define OR_B 256      /* histogram width: grow_c.py:417 always passes MAX_BINS=256 */
#define OR_LEAF (-1)  /* grow.c:28 */

enum { OR_MODE_FP32 = 0, OR_MODE_FIXED = 1 };

/* ------------------------------------------------------------------------- */
/* fixed-point quantisation (OR_MODE_FIXED only)                              */
/* ------------------------------------------------------------------------- */

/* Shift s such that q = rint(x * 2^s) keeps every partial sum of n values
 * below 2^62 in magnitude: with max|x| < 2^e and n <= 2^k, |q| <= 2^(61-k),
 * so |sum| <= 2^61 (+ n/2 rounding).  Zero input gets shift 0. */
int or_quant_shift(float maxabs, int64_t n)
{
    if (!(maxabs > 0.0f)) return 0;
    int e = 0;
    (void)frexpf(maxabs, &e);          /* maxabs = m * 2^e, m in [0.5, 1) */
    int k = 0;
    while (k < 62 && ((int64_t)1 << k) < n) ++k;
    return 61 - k - e;
}

/* The node histograms' shift (the contract of the exact grower): with
 * max|x| < 2^e and n <= 2^k, s = 30 - min(k, 11) - e, so |q| <= 2^19 for
 * n > 2048 (2^(30-k) below) and any 2^min(k,11) of them sum below 2^31 in
 * magnitude -- the most the device's packed root histogram adds into one
 * 32-bit half between two unpacks.  Zero input gets shift 0. */
int or_hist_shift(float maxabs, int64_t n)
{
    if (!(maxabs > 0.0f)) return 0;
    int e = 0;
    (void)frexpf(maxabs, &e);
    int k = 0;
    while (k < 11 && ((int64_t)1 << k) < n) ++k;
    return 30 - k - e;
}

/* The wide contract's shift: s = 61 - max(k, 21) - e, so every partial sum
 * of n quantised values stays below 2^61 (+ rounding). */
int or_wide_shift(float maxabs, int64_t n)
{
    if (!(maxabs > 0.0f)) return 0;
    int e = 0;
    (void)frexpf(maxabs, &e);
    int k = 0;
    while (k < 62 && ((int64_t)1 << k) < n) ++k;
    if (k < 21) k = 21;
    return 61 - k - e;
}

static inline int64_t quantise(float x, double scale)
{
    return (int64_t)rint((double)x * scale);
}

/* Residual and mass of one channel at the narrow shift s (the contract of
 * the exact grower, yabt_amd/csrc/common.h hist_shift / quant_resid):
 * R = sum rint(|y - rint(y)| * 2^21) and M = sum rint(|x| * 2^(s+1)) with
 * y = x * 2^s, every step exact in fp32 (power-of-two scalings and the
 * distance of y to its nearest integer), so R and M are exact integers. */
static void resid_mass(const float *x, int64_t n, int s, uint64_t *r, uint64_t *m)
{
    uint64_t rr = 0, mm = 0;
    for (int64_t i = 0; i < n; ++i) {
        const float y = ldexpf(x[i], s);
        const float d = y - rintf(y);
        rr += (uint64_t)rintf(ldexpf(fabsf(d), 21));
        mm += (uint64_t)rintf(ldexpf(fabsf(x[i]), s + 1));
    }
    *r = rr;
    *m = mm;
}

/* max |x| over n values; returns -1 if any value is not finite. */
static int max_abs(const float *x, int64_t n, float *out)
{
    float m = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        if (!isfinite(x[i])) return -1;
        float a = fabsf(x[i]);
        if (a > m) m = a;
    }
    *out = m;
    return 0;
}

/* The per-call contract: the narrow shifts (or_hist_shift) when their
 * quantisation residual is at most 2^-17 of the mass for both channels
 * (R <= 8 M: R counts 2^-21 and M 2^-1 of a quantum), else the wide shifts
 * (or_wide_shift).  out: sg, sh, wide;
 * sums (may be NULL): R_g, R_h, M_g, M_h.  Returns -1 on a non-finite value. */
int or_hist_contract(const float *grad, const float *hess, int64_t n, int *out, uint64_t *sums)
{
    float mg = 0.0f, mh = 0.0f;
    if (max_abs(grad, n, &mg) || max_abs(hess, n, &mh)) return -1;
    const int sgn = or_hist_shift(mg, n), shn = or_hist_shift(mh, n);
    uint64_t rg, rh, mmg, mmh;
    resid_mass(grad, n, sgn, &rg, &mmg);
    resid_mass(hess, n, shn, &rh, &mmh);
    const int narrow = rg <= 8 * mmg && rh <= 8 * mmh;
    out[0] = narrow ? sgn : or_wide_shift(mg, n);
    out[1] = narrow ? shn : or_wide_shift(mh, n);
    out[2] = !narrow;
    if (sums) {
        sums[0] = rg;
        sums[1] = rh;
        sums[2] = mmg;
        sums[3] = mmh;
    }
    return 0;
}

int or_quant_shifts(const float *grad, const float *hess, int64_t n, int *sg, int *sh)
{
    int c[3];
    if (or_hist_contract(grad, hess, n, c, NULL)) return -1;
    *sg = c[0];
    *sh = c[1];
    return 0;
}

/* ------------------------------------------------------------------------- */
/* histograms                                                                 */
/* ------------------------------------------------------------------------- */

/* fp32 dense histogram of rows[lo:hi] into out[3][F][256] (grow.c:37-62).
 * Feature f's codes are bins_fm[f*n : f*n+n]; each feature is summed in row
 * order, so the result does not depend on the thread count. */
void or_hist_f32(const uint8_t *bins_fm, const float *grad, const float *hess,
                 const int64_t *rows, int64_t lo, int64_t hi, int64_t n, int F,
                 float *out)
{
    const size_t plane = (size_t)F * OR_B;
#pragma omp parallel for schedule(static)
    for (int f = 0; f < F; ++f) {
        float *sg = out + (size_t)f * OR_B;
        float *sh = sg + plane;
        float *sc = sh + plane;
        for (int k = 0; k < OR_B; ++k) sg[k] = sh[k] = sc[k] = 0.0f;
        const uint8_t *col = bins_fm + (size_t)f * (size_t)n;
        for (int64_t i = lo; i < hi; ++i) {
            const int64_t r = rows[i];
            const unsigned k = col[r];
            sg[k] += grad[r];
            sh[k] += hess[r];
            sc[k] += 1.0f;
        }
    }
}

/* fp32 sparse histogram (grow.c:68-107): explicit CSR entries are scattered in
 * row order, then every feature's default bin receives node total minus the
 * explicit sum, formed in double and rounded once to fp32. */
void or_hist_sparse_f32(const int64_t *indptr, const int32_t *indices,
                        const int32_t *data, const int32_t *default_bin,
                        const float *grad, const float *hess,
                        const int64_t *rows, int64_t lo, int64_t hi, int F,
                        float *out)
{
    const size_t plane = (size_t)F * OR_B;
    memset(out, 0, 3 * plane * sizeof(float));
    double *ex = (double *)calloc((size_t)3 * (size_t)F, sizeof(double));
    double tg = 0.0, th = 0.0, tc = 0.0;
    for (int64_t i = lo; i < hi; ++i) {
        const int64_t r = rows[i];
        const float gv = grad[r], hv = hess[r];
        tg += gv;
        th += hv;
        tc += 1.0;
        for (int64_t j = indptr[r]; j < indptr[r + 1]; ++j) {
            const int f = indices[j];
            const size_t at = (size_t)f * OR_B + (size_t)data[j];
            out[at] += gv;
            out[plane + at] += hv;
            out[2 * plane + at] += 1.0f;
            ex[3 * f + 0] += gv;
            ex[3 * f + 1] += hv;
            ex[3 * f + 2] += 1.0;
        }
    }
    for (int f = 0; f < F; ++f) {
        const size_t at = (size_t)f * OR_B + (size_t)default_bin[f];
        out[at] += (float)(tg - ex[3 * f + 0]);
        out[plane + at] += (float)(th - ex[3 * f + 1]);
        out[2 * plane + at] += (float)(tc - ex[3 * f + 2]);
    }
    free(ex);
}

/* Exact int64 histogram of rows[lo:hi]: qg/qh/qc are [F][256] each. */
void or_hist_fixed(const uint8_t *bins_fm, const float *grad, const float *hess,
                   const int64_t *rows, int64_t lo, int64_t hi, int64_t n, int F,
                   int sg, int sh, int64_t *qg, int64_t *qh, int64_t *qc)
{
    const double scg = ldexp(1.0, sg), sch = ldexp(1.0, sh);
#pragma omp parallel for schedule(static)
    for (int f = 0; f < F; ++f) {
        int64_t *og = qg + (size_t)f * OR_B;
        int64_t *oh = qh + (size_t)f * OR_B;
        int64_t *oc = qc + (size_t)f * OR_B;
        for (int k = 0; k < OR_B; ++k) og[k] = oh[k] = oc[k] = 0;
        const uint8_t *col = bins_fm + (size_t)f * (size_t)n;
        for (int64_t i = lo; i < hi; ++i) {
            const int64_t r = rows[i];
            const unsigned k = col[r];
            og[k] += quantise(grad[r], scg);
            oh[k] += quantise(hess[r], sch);
            oc[k] += 1;
        }
    }
}

/* ------------------------------------------------------------------------- */
/* split scan (grow.c:129-197)                                                */
/* ------------------------------------------------------------------------- */

typedef struct {
    double sel;   /* gain * boost[f], what the argmax ranks        */
    double gain;  /* true (unboosted) gain at the chosen bin        */
    int b;        /* chosen bin, -1 if the feature has no valid bin  */
} or_feat_best;

static or_feat_best scan_f32(const float *hg, const float *hh, const float *hc,
                             int nb, double lam, double gamma, double mcw, int msl,
                             double bo)
{
    or_feat_best r = {-INFINITY, -INFINITY, -1};
    double Gt = 0.0, Ht = 0.0, Ct = 0.0;
    for (int k = 0; k < nb; ++k) {
        Gt += hg[k];
        Ht += hh[k];
        Ct += hc[k];
    }
    const double parent = Gt * Gt / (Ht + lam);
    double GL = 0.0, HL = 0.0, CL = 0.0;
    for (int k = 0; k + 1 < nb; ++k) {
        GL += hg[k];
        HL += hh[k];
        CL += hc[k];
        const double GR = Gt - GL, HR = Ht - HL, CR = Ct - CL;
        if (!(CL >= msl && CR >= msl && HL >= mcw && HR >= mcw)) continue;
        const double gain = 0.5 * (GL * GL / (HL + lam) + GR * GR / (HR + lam) - parent) - gamma;
        const double sel = gain * bo;
        if (sel > r.sel) {
            r.sel = sel;
            r.gain = gain;
            r.b = k;
        }
    }
    return r;
}

static or_feat_best scan_fixed(const int64_t *qg, const int64_t *qh, const int64_t *qc,
                               int nb, double ig, double ih, double lam, double gamma,
                               double mcw, int msl, double bo)
{
    or_feat_best r = {-INFINITY, -INFINITY, -1};
    int64_t Gt = 0, Ht = 0, Ct = 0;
    for (int k = 0; k < nb; ++k) {
        Gt += qg[k];
        Ht += qh[k];
        Ct += qc[k];
    }
    const double G = (double)Gt * ig, H = (double)Ht * ih;
    const double parent = G * G / (H + lam);
    int64_t gl = 0, hl = 0, cl = 0;
    for (int k = 0; k + 1 < nb; ++k) {
        gl += qg[k];
        hl += qh[k];
        cl += qc[k];
        const int64_t cr = Ct - cl;
        const double GL = (double)gl * ig, GR = (double)(Gt - gl) * ig;
        const double HL = (double)hl * ih, HR = (double)(Ht - hl) * ih;
        if (!(cl >= msl && cr >= msl && HL >= mcw && HR >= mcw)) continue;
        const double gain = 0.5 * (GL * GL / (HL + lam) + GR * GR / (HR + lam) - parent) - gamma;
        const double sel = gain * bo;
        if (sel > r.sel) {
            r.sel = sel;
            r.gain = gain;
            r.b = k;
        }
    }
    return r;
}

/* Feature-major reduction with strict '>' (grow.c:181-192): the lowest
 * feature among equal maxima wins; returns the true gain or -inf. */
static double reduce_features(const or_feat_best *fb, int F, int *of, int *ob)
{
    double best_sel = -INFINITY, best_gain = -INFINITY;
    int bf = -1, bb = -1;
    for (int f = 0; f < F; ++f) {
        if (fb[f].b >= 0 && fb[f].sel > best_sel) {
            best_sel = fb[f].sel;
            best_gain = fb[f].gain;
            bf = f;
            bb = fb[f].b;
        }
    }
    *of = bf;
    *ob = bb;
    return bf < 0 ? -INFINITY : best_gain;
}

static int clamp_nb(int nb) { return nb < 0 ? 0 : (nb > OR_B ? OR_B : nb); }

double or_best_split_f32(const float *hist, const int32_t *nbins, double lam,
                         double gamma, double mcw, int msl, const uint8_t *fmask,
                         const float *boost, int F, int *of, int *ob)
{
    const size_t plane = (size_t)F * OR_B;
    or_feat_best *fb = (or_feat_best *)malloc((size_t)(F > 0 ? F : 1) * sizeof(or_feat_best));
#pragma omp parallel for schedule(static)
    for (int f = 0; f < F; ++f) {
        or_feat_best r = {-INFINITY, -INFINITY, -1};
        if (fmask[f]) {
            const float *hg = hist + (size_t)f * OR_B;
            r = scan_f32(hg, hg + plane, hg + 2 * plane, clamp_nb(nbins[f]), lam, gamma,
                         mcw, msl, (double)boost[f]);
        }
        fb[f] = r;
    }
    const double g = reduce_features(fb, F, of, ob);
    free(fb);
    return g;
}

double or_best_split_fixed(const int64_t *qg, const int64_t *qh, const int64_t *qc,
                           int sg, int sh, const int32_t *nbins, double lam,
                           double gamma, double mcw, int msl, const uint8_t *fmask,
                           const float *boost, int F, int *of, int *ob)
{
    const double ig = ldexp(1.0, -sg), ih = ldexp(1.0, -sh);
    or_feat_best *fb = (or_feat_best *)malloc((size_t)(F > 0 ? F : 1) * sizeof(or_feat_best));
#pragma omp parallel for schedule(static)
    for (int f = 0; f < F; ++f) {
        or_feat_best r = {-INFINITY, -INFINITY, -1};
        if (fmask[f]) {
            const size_t o = (size_t)f * OR_B;
            r = scan_fixed(qg + o, qh + o, qc + o, clamp_nb(nbins[f]), ig, ih, lam, gamma,
                           mcw, msl, (double)boost[f]);
        }
        fb[f] = r;
    }
    const double g = reduce_features(fb, F, of, ob);
    free(fb);
    return g;
}

/* boost[j] = 1 + ib * max(0, max_{p on path} imat[p][j]) in fp32 (grow.c:111-122). */
void or_compute_boost(const uint8_t *path, const float *imat, float ib, float *boost, int F)
{
    for (int j = 0; j < F; ++j) boost[j] = 0.0f;
    for (int p = 0; p < F; ++p) {
        if (!path[p]) continue;
        const float *row = imat + (size_t)p * F;
        for (int j = 0; j < F; ++j)
            if (row[j] > boost[j]) boost[j] = row[j];
    }
    for (int j = 0; j < F; ++j) boost[j] = 1.0f + ib * boost[j];
}

/* ------------------------------------------------------------------------- */
/* partitions                                                                 */
/* ------------------------------------------------------------------------- */

/* In-place two-pointer partition of rows[lo:hi] by col[r] <= b (grow.c:201-217);
 * returns the first right position.  Row order inside each side is whatever
 * the swap sequence leaves (not stable). */
int64_t or_partition_twoptr(const uint8_t *col, int64_t *rows, int64_t lo, int64_t hi, int b)
{
    int64_t i = lo, j = hi - 1;
    while (i <= j) {
        const int64_t r = rows[i];
        if ((int)col[r] <= b) {
            ++i;
        } else {
            rows[i] = rows[j];
            rows[j] = r;
            --j;
        }
    }
    return i;
}

/* Stable partition (left rows, then right rows, each in input order) -- the
 * order the HIP partition produces; `tmp` holds hi-lo entries. */
int64_t or_partition_stable(const uint8_t *col, int64_t *rows, int64_t lo, int64_t hi,
                            int b, int64_t *tmp)
{
    int64_t nl = 0;
    for (int64_t i = lo; i < hi; ++i)
        if ((int)col[rows[i]] <= b) ++nl;
    int64_t pl = 0, pr = nl;
    for (int64_t i = lo; i < hi; ++i) {
        const int64_t r = rows[i];
        if ((int)col[r] <= b) tmp[pl++] = r;
        else tmp[pr++] = r;
    }
    memcpy(rows + lo, tmp, (size_t)(hi - lo) * sizeof(int64_t));
    return lo + nl;
}

/* ------------------------------------------------------------------------- */
/* the grower                                                                 */
/* ------------------------------------------------------------------------- */

/* Exact sparse builder: explicit entries are added, the default bin gets the
 * node total minus the explicit sum (exact in integers, so equal to dense). */
static void hist_sparse_fixed(const int64_t *indptr, const int32_t *indices,
                              const int32_t *data, const int32_t *default_bin,
                              const float *grad, const float *hess,
                              const int64_t *rows, int64_t lo, int64_t hi, int F,
                              double scg, double sch, int64_t *qg, int64_t *qh, int64_t *qc)
{
    const size_t plane = (size_t)F * OR_B;
    memset(qg, 0, plane * sizeof(int64_t));
    memset(qh, 0, plane * sizeof(int64_t));
    memset(qc, 0, plane * sizeof(int64_t));
    int64_t *ex = (int64_t *)calloc((size_t)3 * (size_t)F, sizeof(int64_t));
    int64_t tg = 0, th = 0, tc = 0;
    for (int64_t i = lo; i < hi; ++i) {
        const int64_t r = rows[i];
        const int64_t gq = quantise(grad[r], scg), hq = quantise(hess[r], sch);
        tg += gq;
        th += hq;
        tc += 1;
        for (int64_t j = indptr[r]; j < indptr[r + 1]; ++j) {
            const int f = indices[j];
            const size_t at = (size_t)f * OR_B + (size_t)data[j];
            qg[at] += gq;
            qh[at] += hq;
            qc[at] += 1;
            ex[3 * f + 0] += gq;
            ex[3 * f + 1] += hq;
            ex[3 * f + 2] += 1;
        }
    }
    for (int f = 0; f < F; ++f) {
        const size_t at = (size_t)f * OR_B + (size_t)default_bin[f];
        qg[at] += tg - ex[3 * f + 0];
        qh[at] += th - ex[3 * f + 1];
        qc[at] += tc - ex[3 * f + 2];
    }
    free(ex);
}

typedef struct {
    int mode, F, use_sparse;
    int64_t n;
    const uint8_t *bins;
    const float *grad, *hess;
    const int64_t *indptr;
    const int32_t *indices, *data, *default_bin;
    const int32_t *nbins;
    const uint8_t *fmask;
    double lam, gamma, mcw;
    int msl;
    int sg, sh;
    double scg, sch, ig, ih;
    size_t slot;        /* elements per node histogram: 3*F*256 */
    float *hf;          /* OR_MODE_FP32 store  [nodes][3][F][256] */
    int64_t *hq;        /* OR_MODE_FIXED store [nodes][3][F][256] */
    int64_t *rows;
    int64_t *tmp;
} grower;

static void g_build(grower *G, int node, int64_t lo, int64_t hi)
{
    const size_t plane = (size_t)G->F * OR_B;
    if (G->mode == OR_MODE_FP32) {
        float *o = G->hf + (size_t)node * G->slot;
        if (G->use_sparse)
            or_hist_sparse_f32(G->indptr, G->indices, G->data, G->default_bin, G->grad,
                               G->hess, G->rows, lo, hi, G->F, o);
        else
            or_hist_f32(G->bins, G->grad, G->hess, G->rows, lo, hi, G->n, G->F, o);
    } else {
        int64_t *o = G->hq + (size_t)node * G->slot;
        if (G->use_sparse)
            hist_sparse_fixed(G->indptr, G->indices, G->data, G->default_bin, G->grad,
                              G->hess, G->rows, lo, hi, G->F, G->scg, G->sch, o, o + plane,
                              o + 2 * plane);
        else
            or_hist_fixed(G->bins, G->grad, G->hess, G->rows, lo, hi, G->n, G->F, G->sg,
                          G->sh, o, o + plane, o + 2 * plane);
    }
}

/* dst = a - b over one node histogram (grow.c:361,368) */
static void g_subtract(grower *G, int dst, int a, int b)
{
    if (G->mode == OR_MODE_FP32) {
        float *d = G->hf + (size_t)dst * G->slot;
        const float *x = G->hf + (size_t)a * G->slot, *y = G->hf + (size_t)b * G->slot;
        for (size_t i = 0; i < G->slot; ++i) d[i] = x[i] - y[i];
    } else {
        int64_t *d = G->hq + (size_t)dst * G->slot;
        const int64_t *x = G->hq + (size_t)a * G->slot, *y = G->hq + (size_t)b * G->slot;
        for (size_t i = 0; i < G->slot; ++i) d[i] = x[i] - y[i];
    }
}

/* Leaf value from feature 0's 256 bins (grow.c:302-308, 371-379). */
static float g_value(grower *G, int node, float lr, float lam)
{
    const size_t plane = (size_t)G->F * OR_B;
    double gs = 0.0, hs = 0.0;
    if (G->mode == OR_MODE_FP32) {
        const float *o = G->hf + (size_t)node * G->slot;
        for (int k = 0; k < OR_B; ++k) {
            gs += o[k];
            hs += o[plane + k];
        }
    } else {
        const int64_t *o = G->hq + (size_t)node * G->slot;
        int64_t tg = 0, th = 0;
        for (int k = 0; k < OR_B; ++k) {
            tg += o[k];
            th += o[plane + k];
        }
        gs = (double)tg * G->ig;
        hs = (double)th * G->ih;
    }
    return (float)(-lr * gs / (hs + lam));
}

static double g_best(grower *G, int node, const float *boost, int *of, int *ob)
{
    const size_t plane = (size_t)G->F * OR_B;
    if (G->mode == OR_MODE_FP32)
        return or_best_split_f32(G->hf + (size_t)node * G->slot, G->nbins, G->lam, G->gamma,
                                 G->mcw, G->msl, G->fmask, boost, G->F, of, ob);
    const int64_t *o = G->hq + (size_t)node * G->slot;
    return or_best_split_fixed(o, o + plane, o + 2 * plane, G->sg, G->sh, G->nbins, G->lam,
                               G->gamma, G->mcw, G->msl, G->fmask, boost, G->F, of, ob);
}

/* Best-first leaf-wise growth.  Outputs match cgrow (grow.c:243-250, arrays of
 * 2*max_leaves+1); returns the node count, or -1 for non-finite gradients or
 * hessians in OR_MODE_FIXED, -2 for bad sizes, -3 for allocation failure.
 * Optional traces (NULL to skip): rows_out[n] final row order, seg_lo/seg_hi
 * each node's [lo,hi) in rows_out, split_gain the true gain of each split,
 * quant[2] the (grad, hess) shifts of OR_MODE_FIXED. */
int or_grow(int mode, const uint8_t *bins_fm, const float *grad, const float *hess,
            const uint8_t *fmask, const float *imat, float ib, int use_imat,
            const int64_t *indptr, const int32_t *indices, const int32_t *data,
            const int32_t *default_bin, int use_sparse, const int32_t *nbins,
            int64_t n, int F, float lam, float gamma, float mcw, int msl, float lr,
            int max_leaves, int max_depth, int n_threads,
            int64_t *o_feature, int64_t *o_thr, int64_t *o_left, int64_t *o_right,
            float *o_value, int64_t *o_depth,
            int64_t *rows_out, int64_t *seg_lo, int64_t *seg_hi, double *split_gain,
            int *quant, void *hist_out)
{
#ifdef _OPENMP
    if (n_threads > 0) omp_set_num_threads(n_threads);
#else
    (void)n_threads;
#endif
    if (F < 1 || n < 0 || max_leaves < 1) return -2;
    const int nodes = 2 * max_leaves + 1;
    for (int i = 0; i < nodes; ++i) {
        o_feature[i] = OR_LEAF;
        o_thr[i] = 0;
        o_left[i] = -1;
        o_right[i] = -1;
        o_value[i] = 0.0f;
        o_depth[i] = 0;
        if (seg_lo) seg_lo[i] = 0;
        if (seg_hi) seg_hi[i] = 0;
        if (split_gain) split_gain[i] = 0.0;
    }

    grower G;
    memset(&G, 0, sizeof G);
    G.mode = mode;
    G.F = F;
    G.n = n;
    G.use_sparse = use_sparse;
    G.bins = bins_fm;
    G.grad = grad;
    G.hess = hess;
    G.indptr = indptr;
    G.indices = indices;
    G.data = data;
    G.default_bin = default_bin;
    G.nbins = nbins;
    G.fmask = fmask;
    G.lam = lam;
    G.gamma = gamma;
    G.mcw = mcw;
    G.msl = msl;
    G.slot = (size_t)3 * (size_t)F * OR_B;
    if (mode == OR_MODE_FIXED) {
        if (or_quant_shifts(grad, hess, n, &G.sg, &G.sh)) return -1;
        G.scg = ldexp(1.0, G.sg);
        G.sch = ldexp(1.0, G.sh);
        G.ig = ldexp(1.0, -G.sg);
        G.ih = ldexp(1.0, -G.sh);
        if (quant) {
            quant[0] = G.sg;
            quant[1] = G.sh;
        }
    }

    int64_t *lo = (int64_t *)calloc((size_t)nodes, sizeof(int64_t));
    int64_t *hi = (int64_t *)calloc((size_t)nodes, sizeof(int64_t));
    uint8_t *path = (uint8_t *)calloc((size_t)nodes * (size_t)F, 1);
    float *boost = (float *)malloc((size_t)F * sizeof(float));
    int64_t *leaf_node = (int64_t *)malloc((size_t)nodes * sizeof(int64_t));
    float *leaf_gain = (float *)malloc((size_t)nodes * sizeof(float));
    int *leaf_f = (int *)malloc((size_t)nodes * sizeof(int));
    int *leaf_b = (int *)malloc((size_t)nodes * sizeof(int));
    G.rows = (int64_t *)malloc((size_t)(n > 0 ? n : 1) * sizeof(int64_t));
    G.tmp = (int64_t *)malloc((size_t)(n > 0 ? n : 1) * sizeof(int64_t));
    if (mode == OR_MODE_FP32)
        G.hf = (float *)malloc((size_t)nodes * G.slot * sizeof(float));
    else
        G.hq = (int64_t *)malloc((size_t)nodes * G.slot * sizeof(int64_t));
    int status = 0;
    if (!lo || !hi || !path || !boost || !leaf_node || !leaf_gain || !leaf_f || !leaf_b ||
        !G.rows || !G.tmp || (!G.hf && !G.hq)) {
        status = -3;
        goto done;
    }

    for (int64_t i = 0; i < n; ++i) G.rows[i] = i;
    for (int j = 0; j < F; ++j) boost[j] = 1.0f;

    lo[0] = 0;
    hi[0] = n;
    g_build(&G, 0, 0, n);
    o_value[0] = g_value(&G, 0, lr, lam);
    int n_nodes = 1;
    {
        int f0 = -1, b0 = -1;
        double g0 = g_best(&G, 0, boost, &f0, &b0);
        if (0 >= max_depth) g0 = -INFINITY;
        leaf_node[0] = 0;
        leaf_gain[0] = (float)g0;
        leaf_f[0] = f0;
        leaf_b[0] = b0;
        if (split_gain) split_gain[0] = g0;
    }
    int n_active = 1, n_leaves = 1;

    while (n_leaves < max_leaves) {
        /* active leaf with the largest fp32 gain, strict '>' from 0 (grow.c:322-330) */
        int k = -1;
        float kg = 0.0f;
        for (int a = 0; a < n_active; ++a)
            if (leaf_gain[a] > kg) {
                kg = leaf_gain[a];
                k = a;
            }
        if (k < 0) break;

        const int nid = (int)leaf_node[k];
        const int f = leaf_f[k], b = leaf_b[k];
        const int64_t s = lo[nid], e = hi[nid];
        const uint8_t *col = bins_fm + (size_t)f * (size_t)n;
        const int64_t mid = (mode == OR_MODE_FP32)
                                ? or_partition_twoptr(col, G.rows, s, e, b)
                                : or_partition_stable(col, G.rows, s, e, b, G.tmp);

        const int nl = n_nodes, nr = n_nodes + 1;
        n_nodes += 2;
        const int64_t d = o_depth[nid] + 1;
        lo[nl] = s;
        hi[nl] = mid;
        lo[nr] = mid;
        hi[nr] = e;
        o_depth[nl] = d;
        o_depth[nr] = d;
        memcpy(path + (size_t)nl * F, path + (size_t)nid * F, (size_t)F);
        memcpy(path + (size_t)nr * F, path + (size_t)nid * F, (size_t)F);
        path[(size_t)nl * F + f] = 1;
        path[(size_t)nr * F + f] = 1;

        /* smaller child built, ties to the left; sibling = parent - child */
        if (mid - s <= e - mid) {
            g_build(&G, nl, s, mid);
            g_subtract(&G, nr, nid, nl);
        } else {
            g_build(&G, nr, mid, e);
            g_subtract(&G, nl, nid, nr);
        }
        o_value[nl] = g_value(&G, nl, lr, lam);
        o_value[nr] = g_value(&G, nr, lr, lam);

        o_feature[nid] = f;
        o_thr[nid] = b;
        o_left[nid] = nl;
        o_right[nid] = nr;
        o_value[nid] = 0.0f;
        n_leaves += 1;

        int cf = -1, cb = -1;
        if (use_imat) or_compute_boost(path + (size_t)nl * F, imat, ib, boost, F);
        double cg = g_best(&G, nl, boost, &cf, &cb);
        if (d >= max_depth) cg = -INFINITY;
        leaf_node[k] = nl;
        leaf_gain[k] = (float)cg;
        leaf_f[k] = cf;
        leaf_b[k] = cb;
        if (split_gain) split_gain[nl] = cg;

        if (use_imat) or_compute_boost(path + (size_t)nr * F, imat, ib, boost, F);
        cg = g_best(&G, nr, boost, &cf, &cb);
        if (d >= max_depth) cg = -INFINITY;
        leaf_node[n_active] = nr;
        leaf_gain[n_active] = (float)cg;
        leaf_f[n_active] = cf;
        leaf_b[n_active] = cb;
        if (split_gain) split_gain[nr] = cg;
        n_active += 1;
    }
    status = n_nodes;
    if (rows_out && n > 0) memcpy(rows_out, G.rows, (size_t)n * sizeof(int64_t));
    if (seg_lo)
        for (int i = 0; i < n_nodes; ++i) seg_lo[i] = lo[i];
    if (seg_hi)
        for (int i = 0; i < n_nodes; ++i) seg_hi[i] = hi[i];
    /* every node's histogram as the grower held it when it scanned the node
     * (fp32 or fixed point by mode; a split node's slot is not reused) */
    if (hist_out)
        memcpy(hist_out, mode == OR_MODE_FP32 ? (void *)G.hf : (void *)G.hq,
               (size_t)n_nodes * G.slot * (mode == OR_MODE_FP32 ? sizeof(float) : sizeof(int64_t)));

done:
    free(lo);
    free(hi);
    free(path);
    free(boost);
    free(leaf_node);
    free(leaf_gain);
    free(leaf_f);
    free(leaf_b);
    free(G.rows);
    free(G.tmp);
    free(G.hf);
    free(G.hq);
    return status;
}

/* Row routing on raw X (n,F) row-major: x[f] <= threshold goes left
 * (grow.c:223-239). */
void or_apply(const float *X, const int64_t *feature, const float *threshold,
              const int64_t *left, const int64_t *right, int64_t n, int F, int n_threads,
              int64_t *out_node)
{
#ifdef _OPENMP
    if (n_threads > 0) omp_set_num_threads(n_threads);
#else
    (void)n_threads;
#endif
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < n; ++r) {
        const float *x = X + (size_t)r * (size_t)F;
        int64_t node = 0;
        for (int64_t f = feature[0]; f != OR_LEAF; f = feature[node])
            node = (x[f] <= threshold[node]) ? left[node] : right[node];
        out_node[r] = node;
    }
}
