"""Where two trees grown on the same inputs part, and whether the arithmetic
explains it.

The exact grower sums g and h in exact fixed point; the reference's cgrow
sums them in fp32 in row order and subtracts sibling histograms in fp32
(grow.c:37-62, 355-369).  When the two pick different splits, this module
finds the first decision in cgrow's best-first order where they differ and
measures it on the node's rows in float64:

* ``first_difference(a, b)``: the first split event (cgrow numbers the
  children of its i-th split 2i + 1, 2i + 2, grow.c:338-339) whose parent
  node, feature or bin differs, or where one tree stops splitting;
* ``decision_gap(...)``: the float64 gains of the two choices from the node's
  rows, and rigorous bounds on how far each arithmetic's gains can be from
  them -- fp32 row-order sums (recursive summation, |error| <= (c - 1) u
  sum |x| per bin of c rows, u = 2^-24; a subtracted node adds its parent's
  and the built sibling's bounds plus the subtraction's rounding) and exact
  fixed-point sums (c 2^-(s+1) per bin of c rows) -- propagated through the
  gain expression (grow.c:151-176) with interval arithmetic.

A departure is explained when the float64 gain gap is at most the sum of
the bounds of both choices under both arithmetics.  Tensors may live on any
device; the sums are float64 bincounts over the node's rows.
"""

from __future__ import annotations

import numpy as np
import torch

U32 = 2.0 ** -24          # unit roundoff of float32


def split_events(feature, left) -> list[tuple[int, int]]:
    """(parent node, split feature) of each split in the order cgrow made
    them: the i-th split's left child is node 2i + 1."""
    feature = np.asarray(feature)
    left = np.asarray(left)
    parent_of = {int(left[p]): p for p in np.nonzero(feature >= 0)[0]}
    out = []
    i = 0
    while 2 * i + 1 in parent_of:
        p = parent_of[2 * i + 1]
        out.append((int(p), int(feature[p])))
        i += 1
    return out


def first_difference(a: dict, b: dict):
    """The first split event where trees a and b (node arrays: feature,
    thr_bin, left) differ: None if every split is the same, else a dict with
    the event index and each tree's (parent, feature, bin), None for a tree
    that made no such split."""
    ea, eb = split_events(a["feature"], a["left"]), split_events(b["feature"], b["left"])
    for i in range(max(len(ea), len(eb))):
        da = (ea[i][0], ea[i][1], int(np.asarray(a["thr_bin"])[ea[i][0]])) if i < len(ea) else None
        db = (eb[i][0], eb[i][1], int(np.asarray(b["thr_bin"])[eb[i][0]])) if i < len(eb) else None
        if da != db:
            return {"event": i, "a": da, "b": db}
    return None


def canonical_first_difference(a: dict, b: dict):
    """The first node, in pre-order from the root, where trees a and b
    split differently (another feature or bin, or one splits and the other
    does not), comparing nodes by their path rather than their best-first
    number; None if the trees are the same split by split.  When the leaf
    budget cannot bind (max_leaves >= 2^max_depth) cgrow splits every node
    with a positive gain above the depth cap, whatever the order, so this is
    the comparison that matters there.  Returns the node ids in a and b and
    each tree's (feature, bin) there, None for a leaf."""
    fa, ta, la, ra = (np.asarray(a[k]) for k in ("feature", "thr_bin", "left", "right"))
    fb, tb, lb, rb = (np.asarray(b[k]) for k in ("feature", "thr_bin", "left", "right"))
    stack = [(0, 0)]
    while stack:
        na, nb = stack.pop()
        sa = (int(fa[na]), int(ta[na])) if fa[na] >= 0 else None
        sb = (int(fb[nb]), int(tb[nb])) if fb[nb] >= 0 else None
        if sa != sb:
            return {"node_a": int(na), "node_b": int(nb), "a": sa, "b": sb}
        if sa is not None:
            stack.append((int(ra[na]), int(rb[nb])))
            stack.append((int(la[na]), int(lb[nb])))
    return None


def path_features(feature, left, right, node: int) -> list[int]:
    """Split features of the node's ancestors (the path mask, grow.c:340-350)."""
    feature, left, right = np.asarray(feature), np.asarray(left), np.asarray(right)
    parent = {}
    for p in np.nonzero(feature >= 0)[0]:
        parent[int(left[p])] = int(p)
        parent[int(right[p])] = int(p)
    out = []
    k = node
    while k in parent:
        k = parent[k]
        out.append(int(feature[k]))
    return out


def path_boost(tree: dict, node: int, imat, ib: float) -> np.ndarray:
    """compute_boost at `node` (grow.c:111-122): 1 + ib max over the path's
    features of imat[p, j], clamped at 0, in float32; ones off any path."""
    imat = np.asarray(imat, np.float32)
    F = imat.shape[0]
    path = sorted(set(path_features(tree["feature"], tree["left"], tree["right"], node)))
    if not path:
        return np.ones(F, np.float32)
    m = np.maximum(imat[path].max(axis=0), np.float32(0))
    return (np.float32(1) + np.float32(ib) * m).astype(np.float32)


def node_rows(feature, thr_bin, left, right, bins_fm: torch.Tensor, node: int) -> torch.Tensor:
    """Row ids of `node`: the rows whose path of bins <= thr_bin tests leads
    through it (the partition membership, grow.c:201-217)."""
    feature, thr_bin = np.asarray(feature), np.asarray(thr_bin)
    left, right = np.asarray(left), np.asarray(right)
    parent = {}
    for p in np.nonzero(feature >= 0)[0]:
        parent[int(left[p])] = (int(p), True)
        parent[int(right[p])] = (int(p), False)
    path = []
    k = node
    while k in parent:
        p, is_left = parent[k]
        path.append((p, is_left))
        k = p
    n = bins_fm.shape[1]
    keep = torch.ones(n, dtype=torch.bool, device=bins_fm.device)
    for p, is_left in path:
        go_left = bins_fm[int(feature[p])] <= int(thr_bin[p])
        keep &= go_left if is_left else ~go_left
    return torch.nonzero(keep).flatten()


def _bin_stats(bins_fm, grad, hess, rows, F):
    """(4, F, 256) float64: sum g, sum h, sum |g|, sum |h| and (F, 256) counts
    of the rows, per (feature, bin)."""
    g = grad[rows].double()
    h = hess[rows].double()
    out = torch.zeros((4, F, 256), dtype=torch.float64, device=bins_fm.device)
    cnt = torch.zeros((F, 256), dtype=torch.float64, device=bins_fm.device)
    for f in range(F):
        b = bins_fm[f, rows].long()
        for c, w in enumerate((g, h, g.abs(), h.abs())):
            out[c, f] = torch.bincount(b, weights=w, minlength=256)
        cnt[f] = torch.bincount(b, minlength=256).double()
    return out, cnt


def fp32_bin_error_bounds(tree: dict, bins_fm, grad, hess, node: int, F: int):
    """Per (feature, bin) bounds (2, F, 256) on |fp32 sum - exact sum| of g
    and h in the histogram cgrow scans at `node`: a built node's bins are
    row-order fp32 sums (at most c - 1 roundings of partial sums bounded by
    sum |x|), a subtracted node's are parent - built sibling in fp32 (both
    bounds plus u (|parent| + |sibling|))."""
    feature, left, right = (np.asarray(tree[k]) for k in ("feature", "left", "right"))
    parent = {}
    for p in np.nonzero(feature >= 0)[0]:
        parent[int(left[p])] = int(p)
        parent[int(right[p])] = int(p)
    cache = {}

    def stats(k):
        if k not in cache:
            rows = node_rows(tree["feature"], tree["thr_bin"], left, right, bins_fm, k)
            cache[k] = (_bin_stats(bins_fm, grad, hess, rows, F), int(rows.numel()))
        return cache[k]

    def bound(k):
        (s, cnt), m = stats(k)
        if k not in parent:                     # the root: built from all rows
            return (torch.clamp(cnt - 1, min=0) * U32 * s[2:4] / (1 - m * U32))
        p = parent[k]
        sib = int(right[p]) if int(left[p]) == k else int(left[p])
        (ss, _), ms = stats(sib)
        built_left = m <= ms if int(left[p]) == k else ms <= m   # cgrow builds the smaller child, ties left
        built = (k == int(left[p])) == built_left
        if built:
            return torch.clamp(cnt - 1, min=0) * U32 * s[2:4] / (1 - m * U32)
        (sp, _), _ = stats(p)
        (sb, cb), mb = stats(sib)
        direct_sib = torch.clamp(cb - 1, min=0) * U32 * sb[2:4] / (1 - mb * U32)
        return bound(p) + direct_sib + U32 * (sp[2:4] + sb[2:4])

    return bound(node), stats(node)[0][0]


def _gain_interval(GL, HL, GR, HR, Gt, Ht, eGL, eHL, eGR, eHR, eGt, eHt, lam, gamma):
    """Bounds of grow.c's gain 0.5 (GL^2/(HL+lam) + GR^2/(HR+lam) - Gt^2/(Ht+lam)) - gamma
    over every G, H within the given distances of the float64 sums."""
    def term(G, H, eG, eH):
        lo_g = max(0.0, abs(G) - eG)
        hi_g = abs(G) + eG
        den_lo, den_hi = H + lam - eH, H + lam + eH
        if den_lo <= 0:
            return -np.inf, np.inf
        return lo_g * lo_g / den_hi, hi_g * hi_g / den_lo
    l = term(GL, HL, eGL, eHL)
    r = term(GR, HR, eGR, eHR)
    t = term(Gt, Ht, eGt, eHt)
    return 0.5 * (l[0] + r[0] - t[1]) - gamma, 0.5 * (l[1] + r[1] - t[0]) - gamma


def gain_and_bound(stats, err, f: int, b: int, nb: int, lam: float, gamma: float):
    """float64 gain of splitting feature f at bin b (bins >= nb unused,
    grow.c:151-156) and the largest distance of any gain computed from sums
    within `err` (2, F, 256) of the float64 ones."""
    G = stats[0, f, :nb].cpu().numpy()
    H = stats[1, f, :nb].cpu().numpy()
    eg = err[0, f, :nb].cpu().numpy()
    eh = err[1, f, :nb].cpu().numpy()
    GL, HL = G[:b + 1].sum(), H[:b + 1].sum()
    Gt, Ht = G.sum(), H.sum()
    GR, HR = Gt - GL, Ht - HL
    eGL, eHL = eg[:b + 1].sum(), eh[:b + 1].sum()
    eGR, eHR = eg[b + 1:].sum(), eh[b + 1:].sum()
    eGt, eHt = eg.sum(), eh.sum()
    gain = 0.5 * (GL * GL / (HL + lam) + GR * GR / (HR + lam) - Gt * Gt / (Ht + lam)) - gamma
    lo, hi = _gain_interval(GL, HL, GR, HR, Gt, Ht, eGL, eHL, eGR, eHR, eGt, eHt, lam, gamma)
    return float(gain), float(max(gain - lo, hi - gain))


def decision_gap(ref_tree: dict, diff: dict, bins_fm: torch.Tensor, grad: torch.Tensor, hess: torch.Tensor,
                 nbins, shifts: tuple[int, int], lam: float = 1.0, gamma: float = 0.0,
                 boost_of=None) -> dict:
    """Measure a first difference between the reference-arithmetic tree
    `ref_tree` (side "b" of `diff`) and the exact-arithmetic tree (side "a")
    at a node where both chose a split: the float64 gains of both choices on
    the node's rows, and each arithmetic's bound for each choice (fp32 bins
    from fp32_bin_error_bounds, exact bins within count * 2^-(s+1) of the
    float64 sums with the exact grower's shifts).  ``boost_of(node)`` gives
    the node's per-feature boost (grow.c:111-122) when an interaction
    matrix steers the scan; the compared quantity is then gain * boost.
    Returns the gap, the summed bounds and whether the gap is within them."""
    a, b = diff["a"], diff["b"]
    if a is None or b is None or a[0] != b[0]:
        raise ValueError("decision_gap measures two splits of one node")
    node = a[0]
    F = bins_fm.shape[0]
    err32, stats = fp32_bin_error_bounds(ref_tree, bins_fm, grad, hess, node, F)
    _, cnt = _bin_stats(bins_fm, grad, hess,
                        node_rows(ref_tree["feature"], ref_tree["thr_bin"], ref_tree["left"], ref_tree["right"],
                                  bins_fm, node), F)
    sg, sh = shifts
    errx = torch.stack([cnt * 2.0 ** (-sg - 1), cnt * 2.0 ** (-sh - 1)])
    boost = None if boost_of is None else np.asarray(boost_of(node), np.float64)
    out = {"node": node, "rows": int(cnt[0].sum().item())}
    total = 0.0
    for side, (_, f, bb) in (("exact", a), ("reference", b)):
        nb = int(np.asarray(nbins)[f])
        g, e32 = gain_and_bound(stats, err32, f, bb, nb, lam, gamma)
        _, ex = gain_and_bound(stats, errx, f, bb, nb, lam, gamma)
        w = 1.0 if boost is None else float(boost[f])
        out[side] = {"feature": f, "bin": bb, "gain": g * w, "bound_fp32": e32 * w, "bound_exact": ex * w}
        total += (e32 + ex) * w
    out["gap"] = abs(out["exact"]["gain"] - out["reference"]["gain"])
    out["bound"] = total
    out["explained"] = out["gap"] <= total
    return out
