"""Per-stage parity of the HIP kernels against the CPU oracle, through the C ABI.

Histograms: bit-exact against the oracle's fixed-point histogram (same shifts
and contract), counts bit-exact against the reference-order fp32 histogram,
g/h sums within 1e-5 normwise of it, and within 1e-9 normwise of fp64 sums
under the wide contract.  Split scan: identical (gain bits, feature, bin) to the
oracle's fixed-point scan.  Partition: identical row order to the oracle's
stable partition and the same membership as the reference two-pointer one.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import WIDE_KINDS, grad_hess, normwise_rel, skewed_bins, uniform_bins
from yabt_amd import grow_hip as G

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0) if torch.cuda.is_available() else None


def _layouts(bins):
    return G.make_layouts(torch.from_numpy(bins), DEV)


def _hist_f64(bins, g, h):
    n, F = bins.shape
    out = np.zeros((2, F, 256))
    for f in range(F):
        np.add.at(out[0, f], bins[:, f], g.astype(np.float64))
        np.add.at(out[1, f], bins[:, f], h.astype(np.float64))
    return out


@pytest.mark.parametrize("n,F,kind,skew", [
    (1, 1, "normal", False), (17, 3, "normal", False), (1000, 16, "normal", False),
    (4099, 17, "laplace", False), (50_000, 33, "normal", False), (20_000, 24, "normal", True),
    (65_536, 100, "logistic", False),
    # more rows per block than the 2048 a packed (q(g) << 32) + q(h) cell may take between unpacks
    (300_001, 20, "normal", False), (600_000, 7, "laplace", True), (1_048_577, 3, "logistic", False),
    # tail tiles (F % 16 in 1..4: the last tile's features replicated over its columns), odd and even n
    (2, 1, "normal", False), (3, 2, "normal", False), (2_500_001, 36, "normal", True), (777_777, 50, "laplace", False),
    # the wide contract: two 64-bit cells per update (h varies) or one (h = 1),
    # full and tail tiles, skewed bins
    (3, 2, "cauchy_h", False), (65_536, 100, "outlier1e5", False), (300_001, 20, "cauchy_h", False),
    (777_777, 50, "studentt_h", False), (1_048_577, 3, "outlier1e3", False), (2_500_001, 36, "lognormal3", True),
    (400_000, 17, "cauchy", False),
])
def test_root_hist_exact(n, F, kind, skew):
    print(f"root n={n} F={F} kind={kind} skew={skew}", flush=True)
    rng = np.random.default_rng(n + F)
    bins = skewed_bins(rng, n, F) if skew else uniform_bins(rng, n, F)
    g, h = grad_hess(rng, n, kind)
    lay = _layouts(bins)
    got, (sg, sh, wide) = G.hist(lay, torch.from_numpy(g), torch.from_numpy(h))
    got = got.cpu().numpy()
    assert (sg, sh, wide) == O.hist_contract(g, h)[:3]
    if kind in WIDE_KINDS and n > 3 or kind in ("normal", "logistic"):   # laplace sits near the threshold
        assert wide == int(kind in WIDE_KINDS and n > 3)
    ref = O.hist_fixed(bins.T, g, h, sg, sh)
    assert np.array_equal(got, ref)
    f32 = O.hist_f32(bins.T, g, h)
    assert np.array_equal(got[2], f32[2].astype(np.int64))
    # exact sums of the quantised values against fp64 sums of the inputs: each
    # value is rounded once to a multiple of 2^-s, so a bin of c rows is off
    # by at most c * 2^-(s+1) (plus the fp64 sums' own rounding)
    f64 = _hist_f64(bins, g, h)
    for c, s in ((0, sg), (1, sh)):
        slack = got[2] * 2.0 ** (-s - 1) + 1e-12 * np.abs(f64[c]).max()
        assert (np.abs(got[c] * 2.0 ** -s - f64[c]) <= slack).all()
        if wide:  # 37-40 bits of the largest |x|: the fp64 sums, normwise
            assert normwise_rel(got[c] * 2.0 ** -s, f64[c]) < 1e-9
    if n <= 100_000 and not wide:  # the reference's fp32 sums drift past 1e-5 on their own beyond that,
        # and with an outlier or heavy tails (fp32 adds at the outlier's ulp)
        assert normwise_rel(got[0] * 2.0 ** -sg, f32[0]) < 1e-5
        assert normwise_rel(got[1] * 2.0 ** -sh, f32[1]) < 1e-5


def _count_table(bins, seg=65536):
    """The per-fit count table on the CPU: (F, 256) counts, then per feature
    and 65536-row segment the largest count of any bin."""
    n, F = bins.shape
    nseg = (n + seg - 1) // seg
    counts = np.zeros((F, 256), np.int64)
    segmax = np.zeros((F, nseg), np.int64)
    for f in range(F):
        counts[f] = np.bincount(bins[:, f], minlength=256)
        for s in range(nseg):
            segmax[f, s] = np.bincount(bins[s * seg:(s + 1) * seg, f], minlength=256).max()
    return counts, segmax


@pytest.mark.parametrize("n,F,kind,hot", [
    (300_001, 20, "normal", None), (1_000_003, 17, "normal", None), (4_000_000, 36, "normal", None),
    (2_500_001, 36, "normal", "skew"), (600_000, 7, "laplace", "skew"), (65_536, 100, "logistic", None),
    # one feature holds 70 000 rows of one bin in one place: the chunks that
    # contain them need the packed cells' epochs, the others do not
    (1_200_000, 100, "normal", "hot"), (1_200_000, 100, "cauchy_h", "hot"), (1_200_000, 100, "laplace", "hot"),
])
def test_root_hist_count_table(n, F, kind, hot):
    """yabt_bin_counts' table (counts and per-segment maxima) against numpy,
    and the root histogram that reads it (packed cells without epochs where
    the table allows) against the oracle's exact sums."""
    print(f"root table n={n} F={F} kind={kind} hot={hot}", flush=True)
    rng = np.random.default_rng(n + 3 * F)
    bins = skewed_bins(rng, n, F) if hot == "skew" else uniform_bins(rng, n, F)
    if hot == "hot":
        bins[400_000:470_000, 5] = 77
    g, h = grad_hess(rng, n, kind)
    lay = _layouts(bins)
    lib = G._lib.load()
    table = lay.counts()
    assert table.numel() == int(lib.yabt_bin_counts_words(n, F))
    counts, segmax = _count_table(bins)
    tab = table.cpu().numpy().view(np.uint32).astype(np.int64)
    assert np.array_equal(tab[:F * 256].reshape(F, 256), counts)
    assert np.array_equal(tab[F * 256:].reshape(F, -1), segmax)
    sg, sh, wide = O.hist_contract(g, h)[:3]
    gd, hd = G._dev_f32(torch.from_numpy(g), DEV), G._dev_f32(torch.from_numpy(h), DEV)
    out = torch.zeros((3, F, 256), dtype=torch.int64, device=DEV)
    G._lib.check(lib.yabt_hist_root(G._ptr(lay.fm), lay.ld_fm, G._ptr(gd), G._ptr(hd), n, F, G._ptr(table),
                                    sg, sh, wide, G._ptr(out), G._stream(DEV)), "yabt_hist_root")
    got = out.cpu().numpy()
    ref = O.hist_fixed(bins.T, g, h, sg, sh)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("n,F,m,kind", [(5000, 16, 1, "normal"), (5000, 16, 777, "normal"), (40_000, 21, 19_999, "normal"),
                                        (40_000, 100, 40_000, "normal"), (10, 3, 0, "normal"),
                                        # n > 2^18: packed words, pipelined gather
                                        (300_000, 20, 5, "normal"), (300_000, 17, 150_001, "normal"),
                                        (600_000, 9, 600_000, "normal"),
                                        # the wide contract: windows of 2^10 .. 2^11 rows
                                        (5000, 16, 777, "lognormal3"), (300_000, 17, 150_001, "cauchy_h"),
                                        (600_000, 9, 600_000, "outlier1e5"), (3_000_000, 5, 2_500_000, "studentt_h")])
def test_gather_hist_exact(n, F, m, kind):
    print(f"gather n={n} F={F} m={m} kind={kind}", flush=True)
    rng = np.random.default_rng(m + 7)
    bins = uniform_bins(rng, n, F)
    g, h = grad_hess(rng, n, kind)
    rows = np.sort(rng.choice(n, size=m, replace=False)).astype(np.int64)
    lay = _layouts(bins)
    got, (sg, sh, wide) = G.hist(lay, torch.from_numpy(g), torch.from_numpy(h),
                                 torch.from_numpy(rows.astype(np.int32)))
    assert (sg, sh, wide) == O.hist_contract(g, h)[:3]
    assert wide == int(kind in WIDE_KINDS)
    ref = O.hist_fixed(bins.T, g, h, sg, sh, rows=rows)
    assert np.array_equal(got.cpu().numpy(), ref)


def test_hist_large_count_exact():
    """Counts and sums exact with 100 000 rows in one bin (test_fixes.py:22-32)."""
    n = 100_000
    bins = np.zeros((n, 2), np.uint8)
    g = np.ones(n, np.float32)
    h = np.full(n, 0.5, np.float32)
    got, (sg, sh, _) = G.hist(_layouts(bins), torch.from_numpy(g), torch.from_numpy(h))
    got = got.cpu().numpy()
    assert got[2, 0, 0] == n
    assert got[0, 0, 0] * 2.0 ** -sg == n
    assert got[1, 0, 0] * 2.0 ** -sh == 0.5 * n


@pytest.mark.parametrize("n", [2048, 3072, 3073, (1 << 19) + 3, 1 << 22])
def test_hist_packed_window_extreme(n):
    """Every row in one bin with the largest |g| and h the shift allows (they
    round to |q| = 2^19, or 2^(30 - 11) at n = 2048): each half of the packed
    root cell takes an epoch of 3072 such rows, 1.5 * 2^30, between two
    unpacks, and the sums must stay exact."""
    bins = np.zeros((n, 1), np.uint8)
    g = np.full(n, -1.9999999, np.float32)
    h = np.full(n, 1.9999999, np.float32)
    got, (sg, sh, _) = G.hist(_layouts(bins), torch.from_numpy(g), torch.from_numpy(h))
    got = got.cpu().numpy()
    qg = int(np.rint(np.float64(g[0]) * 2.0 ** sg))
    qh = int(np.rint(np.float64(h[0]) * 2.0 ** sh))
    assert -qg == qh == 2 ** 19          # the largest |q| the shift allows
    assert got[2, 0, 0] == n
    assert int(got[0, 0, 0]) == n * qg
    assert int(got[1, 0, 0]) == n * qh
    assert (got[:, 0, 1:] == 0).all()


@pytest.mark.parametrize("n", [(1 << 21) + 5, (1 << 22) + 3])
def test_hist_wide_window_extreme(n):
    """The wide contract's packed gather word at its bound: every h equal to
    the largest value below 2^e (|q(h)| within 2^-23 of 2^(61 - K)), all rows in
    one bin, so each window of 2^(K // 2) rows adds 2^(61 - K + K // 2) << cb
    into one cell; g (N(0,1) with one 1e5 outlier) selects the wide contract."""
    rng = np.random.default_rng(n)
    bins = np.zeros((n, 2), np.uint8)
    bins[:, 1] = rng.integers(0, 256, n)
    g = rng.normal(size=n).astype(np.float32)
    g[7] = 1e5
    h = np.full(n, 1.9999999, np.float32)
    rows = np.arange(n, dtype=np.int32)
    got, (sg, sh, wide) = G.hist(_layouts(bins), torch.from_numpy(g), torch.from_numpy(h), torch.from_numpy(rows))
    got = got.cpu().numpy()
    assert wide == 1 and (sg, sh, wide) == O.hist_contract(g, h)[:3]
    K = max(int(np.ceil(np.log2(n))), 21)
    qh = int(np.rint(np.float64(h[0]) * 2.0 ** sh))
    # 1.9999999 = 2 - 2^-23 is exactly (2^24 - 1) 2^-23: q(h) = 2^(61-K) - 2^(61-K-24+1), a hair below the bound
    assert 2 ** (61 - K) - 2 ** (61 - K - 23) <= qh <= 2 ** (61 - K)
    assert got[2, 0, 0] == n and int(got[1, 0, 0]) == n * qh
    qg = np.rint(g.astype(np.float64) * 2.0 ** sg).astype(np.int64)
    assert int(got[0, 0, 0]) == int(qg.sum())
    assert np.array_equal(got, O.hist_fixed(bins.T, g, h, sg, sh, rows=rows.astype(np.int64)))


def _random_qhist(rng, F, n=3000, nb=256):
    bins = uniform_bins(rng, n, F, nb)
    g, h = grad_hess(rng, n)
    sg, sh = O.quant_shifts(g, h)
    return O.hist_fixed(bins.T, g, h, sg, sh), sg, sh


@pytest.mark.parametrize("seed", range(6))
def test_best_split_identical(seed):
    rng = np.random.default_rng(seed)
    F = int(rng.integers(1, 70))
    q, sg, sh = _random_qhist(rng, F, nb=int(rng.choice([4, 30, 256])))
    kw = dict(nbins=rng.integers(1, 257, size=F).astype(np.int32),
              lam=float(rng.choice([0.0, 1.0, 2.5])), gamma=float(rng.choice([0.0, 0.3])),
              mcw=1e-3, msl=int(rng.choice([0, 1, 20])),
              fmask=(rng.random(F) < 0.8).astype(np.uint8),
              boost=(1 + 0.5 * rng.random(F)).astype(np.float32))
    ref = O.best_split_fixed(q, sg, sh, **kw)
    got = G.best_split(torch.from_numpy(q).to(DEV), sg, sh, **kw)
    assert got[1:] == ref[1:]
    assert np.float64(got[0]).tobytes() == np.float64(ref[0]).tobytes()


def test_best_split_ties_and_no_split():
    # duplicated features tie exactly: the lowest feature wins (grow.c:181-192)
    rng = np.random.default_rng(3)
    q, sg, sh = _random_qhist(rng, 1)
    q3 = np.concatenate([q, q, q], axis=1)
    got = G.best_split(torch.from_numpy(q3).to(DEV), sg, sh, msl=1)
    ref = O.best_split_fixed(q3, sg, sh, msl=1)
    assert got[1:] == ref[1:] and got[1] == 0
    # msl above the node size: no valid split anywhere
    got = G.best_split(torch.from_numpy(q3).to(DEV), sg, sh, msl=10**6)
    assert got[1] == -1 and got[0] == float("-inf")


@pytest.mark.parametrize("n,m,b", [(1, 1, 0), (5000, 5000, 127), (70_000, 33_333, 3),
                                   (70_000, 70_000, 255), (300_000, 250_001, 100)])
def test_partition_identical(n, m, b):
    rng = np.random.default_rng(m)
    F = 5
    bins = uniform_bins(rng, n, F)
    lay = _layouts(bins)
    f = int(rng.integers(F))
    if m == n:
        rows = np.arange(n, dtype=np.int64)
        got, mid = G.partition(lay, f, b)
    else:
        rows = rng.permutation(n)[:m].astype(np.int64)
        got, mid = G.partition(lay, f, b, torch.from_numpy(rows.astype(np.int32)))
    ref, rmid = O.partition(bins[:, f], rows, b, stable=True)
    assert mid == rmid
    assert np.array_equal(got.cpu().numpy().astype(np.int64), ref)
    two, tmid = O.partition(bins[:, f], rows, b, stable=False)
    assert tmid == mid
    assert set(two[:tmid].tolist()) == set(ref[:mid].tolist())


def test_apply_matches_oracle():
    rng = np.random.default_rng(11)
    n, F = 20_000, 7
    bins = uniform_bins(rng, n, F, 50)
    g, h = grad_hess(rng, n)
    tree = O.grow(bins.T, g, h, mode=O.MODE_FIXED, max_leaves=40, msl=5)
    X = rng.normal(size=(n, F)).astype(np.float32) * 20
    thr = np.where(tree["feature"] >= 0, tree["thr_bin"], 0).astype(np.float32)
    ref = O.apply(X, tree["feature"], thr, tree["left"], tree["right"])
    got = G.apply_hip(torch.from_numpy(X).to(DEV), torch.from_numpy(tree["feature"]),
                      torch.from_numpy(thr), torch.from_numpy(tree["left"]),
                      torch.from_numpy(tree["right"]))
    assert np.array_equal(got.cpu().numpy(), ref)
