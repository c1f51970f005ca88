"""Oracle pieces pinned by closed forms and brute force (no reference run).

Each check is chosen so a plausible mistake fails it: a histogram summing the
wrong channel or skipping a row, a prefix off by one bin, a reversed
tie-break, a fused or reordered gain expression, a quantisation shift that
can overflow, a partition that loses or duplicates rows.
"""

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import WIDE_KINDS, grad_hess, uniform_bins


def _brute_hist(bins_nf, g, h, rows):
    n, F = bins_nf.shape
    out = np.zeros((3, F, 256), np.float64)
    for f in range(F):
        b = bins_nf[rows, f]
        np.add.at(out[0, f], b, g[rows].astype(np.float64))
        np.add.at(out[1, f], b, h[rows].astype(np.float64))
        np.add.at(out[2, f], b, 1.0)
    return out


def test_hist_f32_against_fp64_brute_force():
    rng = np.random.default_rng(0)
    n, F = 20_000, 6
    bins = uniform_bins(rng, n, F)
    g, h = grad_hess(rng, n)
    rows = np.sort(rng.choice(n, 9000, replace=False))
    got = O.hist_f32(bins.T, g, h, rows=rows)
    ref = _brute_hist(bins, g, h, rows)
    assert np.array_equal(got[2], ref[2])
    for c in (0, 1):
        assert np.abs(got[c] - ref[c]).max() / np.abs(ref[c]).max() < 1e-6


def test_hist_fixed_is_exact_integer_sum():
    """Independent restatement: numpy rint of x * 2^s, summed in int64."""
    rng = np.random.default_rng(1)
    n, F = 7000, 5
    bins = uniform_bins(rng, n, F, 40)
    g, h = grad_hess(rng, n, "laplace")
    sg, sh = O.quant_shifts(g, h)
    qg = np.rint(g.astype(np.float64) * 2.0 ** sg).astype(np.int64)
    qh = np.rint(h.astype(np.float64) * 2.0 ** sh).astype(np.int64)
    rows = rng.permutation(n)[:5000]
    got = O.hist_fixed(bins.T, g, h, sg, sh, rows=rows)
    for f in range(F):
        b = bins[rows, f]
        for c, q in ((0, qg), (1, qh)):
            ref = np.zeros(256, np.int64)
            np.add.at(ref, b, q[rows])
            assert np.array_equal(got[c, f], ref)
        assert np.array_equal(got[2, f], np.bincount(b, minlength=256))


@pytest.mark.parametrize("maxabs,n", [(1.0, 1), (0.75, 1000), (5.5, 10_000_000), (1e-30, 3),
                                      (3e38, 2), (0.0, 10)])
def test_quant_shift_bounds(maxabs, n):
    s = O.quant_shift(maxabs, n)
    if maxabs == 0.0:
        assert s == 0
        return
    k = int(np.ceil(np.log2(n))) if n > 1 else 0
    q = np.rint(np.float64(np.float32(maxabs)) * 2.0 ** s)
    assert q <= 2.0 ** (61 - k)               # every |q| fits the bound
    assert n * q < 2.0 ** 62                 # so every partial sum does
    assert 2 * q > 2.0 ** (61 - k - 1)       # and the scale is not wastefully small


def test_quant_shift_closed_form():
    assert O.quant_shift(1.0, 1) == 60        # 1.0 = 0.5 * 2^1, n <= 2^0
    assert O.quant_shift(1.0, 2) == 59
    assert O.quant_shift(0.5, 1024) == 51     # 0.5 = 0.5 * 2^0, n = 2^10
    with pytest.raises(ValueError):
        O.quant_shifts(np.array([1.0, np.inf], np.float32), np.ones(2, np.float32))


@pytest.mark.parametrize("maxabs,n", [(1.0, 1), (0.75, 1000), (1.9999999, 2048), (1.9999999, 2049),
                                      (5.5, 10_000_000), (1e-30, 3), (3e38, 2), (0.0, 10), (0.25, 4_000_000)])
def test_hist_shift_bounds(maxabs, n):
    """The node histograms' shift: any min(n, 2048) quantised values sum
    below 2^31 in magnitude (one 32-bit half of the packed root word between
    two unpacks), all n below 2^62, and the scale is the largest power of two
    that does so (one more bit would break the 2048-row bound)."""
    s = O.hist_shift(maxabs, n)
    if maxabs == 0.0:
        assert s == 0
        return
    w = min(int(np.ceil(np.log2(n))) if n > 1 else 0, 11)
    q = np.rint(np.float64(np.float32(maxabs)) * 2.0 ** s)
    assert q <= 2.0 ** (30 - w)
    assert min(n, 2048) * q < 2.0 ** 31
    assert n * q < 2.0 ** 62
    # maximal: with s + 1, values just below 2^e (e: maxabs = m 2^e, m in [0.5, 1))
    # would round to 2^(31 - w), and 2^w of them would reach 2^31
    e = int(np.frexp(np.float32(maxabs))[1])
    assert 2.0 ** (s + 1 + e) * 2 ** w >= 2.0 ** 31


def test_hist_shift_closed_form():
    assert O.hist_shift(1.0, 1) == 29          # 1.0 = 0.5 * 2^1, n <= 2^0: 30 - 0 - 1
    assert O.hist_shift(1.0, 2048) == 18       # 30 - 11 - 1
    assert O.hist_shift(1.0, 10_000_000) == 18  # the window caps k at 11
    assert O.hist_shift(0.5, 1024) == 20       # 0.5 = 0.5 * 2^0: 30 - 10 - 0
    # n = 2 (k = 1): max|g| = 1.5 = 0.75 * 2^1, max|h| = 0.5 = 0.5 * 2^0
    assert O.quant_shifts(np.array([1.0, -1.5], np.float32), np.array([0.25, 0.5], np.float32)) == (28, 29)


@pytest.mark.parametrize("maxabs,n", [(1.0, 1), (0.75, 1000), (1.9999999, 1 << 21), (1.9999999, (1 << 21) + 1),
                                      (5.5, 10_000_000), (1e-30, 3), (3e38, 2), (0.0, 10)])
def test_wide_shift_bounds(maxabs, n):
    """The wide contract's shift: every |q| <= 2^(61 - K) with K = max(k, 21),
    so all n sum below 2^62 and a packing window of 2^(K // 2) rows, shifted
    by its count bits K // 2 + 1, stays below 2^63; maximal (one more bit
    would break the 2^(61 - K) bound)."""
    s = O.wide_shift(maxabs, n)
    if maxabs == 0.0:
        assert s == 0
        return
    k = int(np.ceil(np.log2(n))) if n > 1 else 0
    K = max(k, 21)
    q = np.rint(np.float64(np.float32(maxabs)) * 2.0 ** s)
    assert q <= 2.0 ** (61 - K)
    assert n * q < 2.0 ** 62
    w = K // 2
    assert 2 ** w * q * 2.0 ** (w + 1) < 2.0 ** 63
    e = int(np.frexp(np.float32(maxabs))[1])
    assert 2.0 ** (s + 1 + e) > 2.0 ** (61 - K)


def test_wide_shift_closed_form():
    assert O.wide_shift(1.0, 1) == 39            # 61 - 21 - 1: small n count as 2^21 rows
    assert O.wide_shift(1.0, 1 << 21) == 39
    assert O.wide_shift(1.0, (1 << 21) + 1) == 38
    assert O.wide_shift(5.5, 10_000_000) == 34   # 5.5 = 0.6875 * 2^3, k = 24


def _resid_mass_np(x, s):
    """The contract's residual and mass of one channel, restated in float64
    (every step below is exact in float64 for float32 inputs)."""
    y = x.astype(np.float64) * 2.0 ** s
    r = np.rint(np.abs(y - np.rint(y)) * 2.0 ** 21)
    m = np.rint(np.abs(x.astype(np.float64)) * 2.0 ** (s + 1))
    return int(r.sum()), int(m.sum())


@pytest.mark.parametrize("kind,n", [("normal", 1000), ("normal", 300_000), ("laplace", 50_000), ("logistic", 4096),
                                    *[(k, 20_000) for k in WIDE_KINDS]])
def test_hist_contract_against_numpy(kind, n):
    """or_hist_contract's residuals and masses equal an independent float64
    restatement, its decision is R <= 8 M on both channels, and its shifts
    are the narrow or the wide ones accordingly; the outlier and heavy-tailed
    kinds select wide, the well-scaled ones narrow."""
    rng = np.random.default_rng(n)
    g, h = grad_hess(rng, n, kind)
    sg, sh, wide, sums = O.hist_contract(g, h)
    sgn = O.hist_shift(float(np.abs(g).max()), n)
    shn = O.hist_shift(float(np.abs(h).max()), n)
    rg, mg = _resid_mass_np(g, sgn)
    rh, mh = _resid_mass_np(h, shn)
    assert sums == (rg, rh, mg, mh)
    assert wide == int(not (rg <= 8 * mg and rh <= 8 * mh))
    assert wide == int(kind in WIDE_KINDS)
    if wide:
        assert (sg, sh) == (O.wide_shift(float(np.abs(g).max()), n), O.wide_shift(float(np.abs(h).max()), n))
    else:
        assert (sg, sh) == (sgn, shn)
    assert O.quant_shifts(g, h) == (sg, sh)


def test_hist_contract_closed_form():
    """Values on the narrow grid have no residual (narrow); a value of half a
    narrow quantum rounds to 0 (ties to even) with residual 2^20 and mass 1
    in the contract's units, so enough of them select wide; all zeros keep
    shift 0 and narrow."""
    n = 4096
    grid = np.array([1.0, -0.5, 0.25, 1.5], np.float32)   # max 1.5: e = 1, s = 30 - 11 - 1 = 18
    g = np.tile(grid, n // 4)
    h = np.ones(n, np.float32)
    sg, sh, wide, sums = O.hist_contract(g, h)
    assert (sg, sh, wide) == (18, 18, 0) and sums[0] == sums[1] == 0
    m_grid = int((np.abs(grid.astype(np.float64)) * 2.0 ** 19).sum()) * (n // 4)
    assert sums[2] == m_grid and sums[3] == n * 2 ** 19
    for k, want_wide in ((200, 0), (3500, 1)):
        g2 = g.copy()
        g2[:k] = np.float32(2.0 ** -19)
        _, _, wide2, (rg, _, mg, _) = O.hist_contract(g2, h)
        assert rg == k * 2 ** 20
        assert mg == m_grid - int((np.abs(g[:k].astype(np.float64)) * 2.0 ** 19).sum()) + k
        assert wide2 == want_wide == int(rg > 8 * mg)
    assert O.hist_contract(np.zeros(8, np.float32), np.zeros(8, np.float32))[:3] == (0, 0, 0)


def _brute_split(bins_nf, g, h, lam, gamma, mcw, msl, nbins, fmask, boost):
    """Enumerate every (f, b), summing the rows on each side directly."""
    n, F = bins_nf.shape
    g = g.astype(np.float64)
    h = h.astype(np.float64)
    best = (-np.inf, -np.inf, -1, -1)  # sel, gain, f, b
    for f in range(F):
        if not fmask[f]:
            continue
        used = bins_nf[:, f] < nbins[f]
        G, H, C = g[used].sum(), h[used].sum(), used.sum()
        parent = G * G / (H + lam)
        for b in range(nbins[f] - 1):
            left = used & (bins_nf[:, f] <= b)
            GL, HL, CL = g[left].sum(), h[left].sum(), left.sum()
            GR, HR, CR = G - GL, H - HL, C - CL
            if CL >= msl and CR >= msl and HL >= mcw and HR >= mcw:
                gain = 0.5 * (GL * GL / (HL + lam) + GR * GR / (HR + lam) - parent) - gamma
                sel = gain * boost[f]
                # direct sums can differ from prefix sums in the last ulp: a tie
                # within 1e-9 keeps the earlier (lower f, then lower b) candidate
                if not np.isfinite(best[0]) or sel > best[0] + 1e-9 * abs(best[0]):
                    best = (sel, gain, f, b)
    return best


@pytest.mark.parametrize("kind", ["normal", "outlier"])
@pytest.mark.parametrize("seed", range(4))
def test_best_split_against_brute_force(seed, kind):
    rng = np.random.default_rng(seed)
    n, F = 600, 5
    nb = 20
    bins = uniform_bins(rng, n, F, nb)
    g, h = grad_hess(rng, n, kind)
    lam, gamma, mcw, msl = 1.0, 0.0, 1e-3, [1, 10, 30, 50][seed]
    nbins = np.full(F, nb, np.int32)
    fmask = np.array([1, 1, seed % 2, 1, 1], np.uint8)
    boost = np.float32(1) + np.float32(0.3) * rng.random(F).astype(np.float32)
    ref = _brute_split(bins, g, h, lam, gamma, mcw, msl, nbins, fmask, boost)
    g32, f32, b32 = O.best_split_f32(O.hist_f32(bins.T, g, h), nbins, lam, gamma, mcw, msl,
                                     fmask, boost)
    sg, sh = O.quant_shifts(g, h)
    gfx, ffx, bfx = O.best_split_fixed(O.hist_fixed(bins.T, g, h, sg, sh), sg, sh, nbins, lam,
                                       gamma, mcw, msl, fmask, boost)
    assert (f32, b32) == (ref[2], ref[3]) == (ffx, bfx)
    wide = O.hist_contract(g, h)[2]
    assert wide == int(kind == "outlier")
    # narrow: q keeps 20 bits of max|g| here (n = 600), node sums carry ~1e-6
    # relative error; wide: 40 bits of max|g| = 50, the gain is the fp64 one
    assert g32 == pytest.approx(ref[1], rel=1e-6)
    assert gfx == pytest.approx(ref[1], rel=1e-9 if wide else 1e-5)
    # on the quantised values themselves (q 2^-s, exact in fp64) the fixed-point
    # scan is the brute force up to the fp64 rounding of the gain expression
    gq = np.rint(g.astype(np.float64) * 2.0 ** sg) * 2.0 ** -sg
    hq = np.rint(h.astype(np.float64) * 2.0 ** sh) * 2.0 ** -sh
    refq = _brute_split(bins, gq, hq, lam, gamma, mcw, msl, nbins, fmask, boost)
    assert (refq[2], refq[3]) == (ffx, bfx) and gfx == pytest.approx(refq[1], rel=1e-12)


def test_best_split_tie_breaks():
    """Equal gains: lowest bin within a feature, lowest feature across."""
    n = 400
    col = np.repeat(np.arange(4), 100).astype(np.uint8)     # bins 0..3, 100 rows each
    bins = np.stack([col, col], 1)                           # two identical features
    g = np.where(col < 2, -1.0, 1.0).astype(np.float32)      # best cut: bin <= 1
    h = np.ones(n, np.float32)
    nbins = np.full(2, 6, np.int32)                          # bins 4, 5 exist but are empty
    for mode_hist, split in ((O.hist_f32, O.best_split_f32),):
        gain, f, b = split(mode_hist(bins.T, g, h), nbins, 1.0, 0.0, 1e-3, 1)
        assert (f, b) == (0, 1)
    sg, sh = O.quant_shifts(g, h)
    gain, f, b = O.best_split_fixed(O.hist_fixed(bins.T, g, h, sg, sh), sg, sh, nbins, 1.0, 0.0,
                                    1e-3, 1)
    assert (f, b) == (0, 1)
    # closed form: GL=-200, HL=200, GR=200, HR=200, parent 0
    assert gain == pytest.approx(0.5 * (200 ** 2 / 201 + 200 ** 2 / 201))


def test_boost_closed_form():
    rng = np.random.default_rng(3)
    F = 9
    imat = rng.normal(size=(F, F)).astype(np.float32)
    path = np.zeros(F, np.uint8)
    path[[1, 4, 6]] = 1
    got = O.compute_boost(path, imat, 0.5)
    m = np.maximum(imat[[1, 4, 6]].max(axis=0), 0).astype(np.float32)
    assert np.array_equal(got, np.float32(1) + np.float32(0.5) * m)
    assert np.array_equal(O.compute_boost(np.zeros(F, np.uint8), imat, 0.5), np.ones(F, np.float32))


@pytest.mark.parametrize("stable", [False, True])
def test_partition_membership(stable):
    rng = np.random.default_rng(4)
    n = 5000
    col = rng.integers(0, 256, n).astype(np.uint8)
    rows = rng.permutation(n)[:3111]
    out, mid = O.partition(col, rows, 99, stable=stable)
    assert sorted(out.tolist()) == sorted(rows.tolist())
    assert mid == int((col[rows] <= 99).sum())
    assert (col[out[:mid]] <= 99).all() and (col[out[mid:]] > 99).all()
    if stable:
        keep = col[rows] <= 99
        assert np.array_equal(out, np.concatenate([rows[keep], rows[~keep]]))


def test_apply_against_numpy_routing():
    rng = np.random.default_rng(5)
    n, F = 3000, 4
    bins = uniform_bins(rng, n, F, 30)
    g, h = grad_hess(rng, n)
    t = O.grow(bins.T, g, h, mode=O.MODE_FIXED, max_leaves=20, msl=5)
    thr = np.where(t["feature"] >= 0, t["thr_bin"], 0).astype(np.float32)
    X = bins.astype(np.float32)
    got = O.apply(X, t["feature"], thr, t["left"], t["right"])
    ref = np.zeros(n, np.int64)
    for r in range(n):
        node = 0
        while t["feature"][node] >= 0:
            f = t["feature"][node]
            node = t["left"][node] if X[r, f] <= thr[node] else t["right"][node]
        ref[r] = node
    assert np.array_equal(got, ref)
    assert np.array_equal(got, O.leaf_of_rows(t, n))


def test_fixed_tree_splits_are_node_optimal():
    """Every split of a fixed-point tree is the brute-force best of its node's
    rows, and every leaf value is -lr*G/(H+lam) of its rows."""
    rng = np.random.default_rng(6)
    n, F, nb = 1500, 4, 16
    bins = uniform_bins(rng, n, F, nb)
    g, h = grad_hess(rng, n)
    t = O.grow(bins.T, g, h, mode=O.MODE_FIXED, max_leaves=12, msl=15,
               nbins=np.full(F, nb, np.int32))
    nbins = np.full(F, nb, np.int32)
    for nid in range(t["n_nodes"]):
        rows = t["rows"][t["seg_lo"][nid]:t["seg_hi"][nid]]
        if t["feature"][nid] >= 0:
            best = _brute_split(bins[rows], g[rows], h[rows], 1.0, 0.0, np.float32(1e-3), 15,
                                nbins, np.ones(F, np.uint8), np.ones(F, np.float32))
            assert (t["feature"][nid], t["thr_bin"][nid]) == (best[2], best[3])
        else:
            G, H = g[rows].astype(np.float64).sum(), h[rows].astype(np.float64).sum()
            assert t["value"][nid] == pytest.approx(-0.1 * G / (H + 1.0), abs=1e-6)
