"""Linear leaf models on the GPU (mirror of yabt/neural_leaves.py:21-184).

``fit_leaf_networks`` keeps the reference's signature and result: after a tree
is grown, every leaf with at least ``leaf_net_min_samples`` rows gets a ridge
model over up to ``leaf_net_features`` inputs, fitted to the Newton objective
at ``margin + value[leaf]``, folded into raw space and shrunk by the learning
rate, with per-leaf input envelopes.  The per-leaf Gram matrices, envelopes,
counts, solves and the input moments run in the HIP kernels of
``csrc/leaf.hip`` (``yabt_leaf_moments``, ``yabt_leaf_fit``, ``yabt_leaf_fold``,
and for binned inputs the split-feature ranking, ``yabt_leaf_rank_features``),
the targets g, h at margin + value[leaf] in ``yabt_grad_hess``
(``csrc/boost.hip``); the padding of the features by correlation is the
reference's own torch expressions.  Only the linear form
(``leaf_net_hidden == 0``) is provided.
"""

from __future__ import annotations

from dataclasses import replace

import torch

from . import _lib, boost_ops
from .tree import Tree


def _stream(dev: torch.device):
    return torch.cuda.current_stream(dev).cuda_stream


def _used_features(feature: torch.Tensor, k: int) -> torch.Tensor:
    """The tree's split features, most used first (neural_leaves.py:27-31).
    Evaluated on the host with the reference's own torch calls: the node
    array is tiny, and torch's CPU argsort fixes the order of equal counts
    (insertion order up to 16 distinct features, introsort order above)."""
    f = feature.cpu()
    f = f[f >= 0]
    if f.numel() == 0:
        return torch.empty(0, dtype=torch.long)
    vals, counts = f.unique(return_counts=True)
    return vals[counts.argsort(descending=True)][:k]


def _select_features(tree: Tree, Xraw: torch.Tensor, grad: torch.Tensor, k: int) -> torch.Tensor:
    """The tree's split features, most used first, padded by |corr(x, g)|
    (neural_leaves.py:21-39)."""
    k = min(k, Xraw.shape[1])
    used = _used_features(tree.feature, k).to(Xraw.device)
    if used.numel() >= k:
        return used
    score = (Xraw.T @ grad - Xraw.mean(dim=0) * grad.sum()).abs()
    score = score / Xraw.std(dim=0).clamp_min(1e-6)
    score[used] = float("-inf")
    extra = score.argsort(descending=True)[: k - used.numel()]
    return torch.cat([used, extra])


# Gram sums of yabt_leaf_fit: "exact" (the fp64 products rounded to int64
# fixed point and summed exactly) or "mfma" (fp64 sums on the matrix cores).
GRAM_MODES = {"exact": 0, "mfma": 1}
# features up to which yabt_leaf_rank_features ranks the split features on the device
RANK_MAX_FEATURES = 4096
GRAM = "exact"


def _leaf_fit(X: torch.Tensor, x_kind: int, feats: torch.Tensor, mu: torch.Tensor, sd: torch.Tensor,
              grad: torch.Tensor, hess: torch.Tensor, leaf_idx: torch.Tensor, feature: torch.Tensor,
              min_samples: int, lam: float, gram: str | None = None):
    """Enqueue one ``yabt_leaf_fit`` call; returns (W, b, lo, hi, count,
    status) on X's device without waiting: status = [0 / -1 / -2, leaves
    fitted] (see _check_status)."""
    lib = _lib.load()
    dev = X.device
    if dev.type != "cuda":
        raise RuntimeError("yabt_leaf_fit needs device tensors")
    mode = GRAM_MODES[GRAM if gram is None else gram]
    n = int(grad.shape[0])
    K = int(feats.numel())
    N = int(feature.shape[0])
    if x_kind == 0:
        if X.dtype != torch.float32 or X.dim() != 2 or X.shape[0] != n or X.stride(1) != 1:
            raise ValueError("X must be fp32 (n, F) with unit column stride")
        ldx = X.stride(0)
    else:
        dt = torch.uint8 if x_kind == 1 else torch.float32
        if X.dtype != dt or X.dim() != 2 or X.shape[1] < n or X.stride(1) != 1:
            raise ValueError(f"X must be {'uint8' if x_kind == 1 else 'fp32'} (F, ld >= n)")
        ldx = X.stride(0)
    fi = feats.to(dev, torch.int32).contiguous()
    m = mu.to(dev, torch.float32).contiguous()
    s = sd.to(dev, torch.float32).contiguous()
    g = grad.to(dev, torch.float32).contiguous()
    h = hess.to(dev, torch.float32).contiguous()
    li = leaf_idx.to(dev, torch.int64).contiguous()
    ft = feature.to(dev, torch.int64).contiguous()
    nbytes = int(lib.yabt_leaf_fit_workspace_bytes(n, N, K))
    if nbytes == 0:
        raise ValueError("yabt_leaf_fit: invalid sizes (1 <= K <= 8 inputs)")
    # per call, from torch's caching allocator on the current stream: calls
    # from several host threads on their own streams never share it
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    W = torch.empty((N, K), dtype=torch.float32, device=dev)
    b = torch.empty(N, dtype=torch.float32, device=dev)
    lo = torch.empty((N, K), dtype=torch.float32, device=dev)
    hi = torch.empty((N, K), dtype=torch.float32, device=dev)
    cnt = torch.empty(N, dtype=torch.int64, device=dev)
    status = torch.empty(2, dtype=torch.int32, device=dev)
    _lib.check(lib.yabt_leaf_fit(x_kind, X.data_ptr(), ldx, n, fi.data_ptr(), K, m.data_ptr(), s.data_ptr(),
                                 g.data_ptr(), h.data_ptr(), li.data_ptr(), ft.data_ptr(), N, int(min_samples),
                                 float(lam), mode, ws.data_ptr(), nbytes, W.data_ptr(), b.data_ptr(), lo.data_ptr(),
                                 hi.data_ptr(), cnt.data_ptr(), status.data_ptr(), _stream(dev)),
               "yabt_leaf_fit")
    return W, b, lo, hi, cnt, status


def _check_status(st: int) -> None:
    if st == -1:
        raise ValueError("yabt_leaf_fit: a leaf id is out of range or an input is not finite")
    if st == -2:
        raise RuntimeError("yabt_leaf_fit: singular leaf system (torch.linalg.solve would raise)")


def leaf_fit(X: torch.Tensor, x_kind: int, feats: torch.Tensor, mu: torch.Tensor, sd: torch.Tensor,
             grad: torch.Tensor, hess: torch.Tensor, leaf_idx: torch.Tensor, feature: torch.Tensor,
             min_samples: int, lam: float, gram: str | None = None):
    """One ``yabt_leaf_fit`` call.  X: fp32 (n, F) row-major (x_kind 0),
    uint8 feature-major (F, ld >= n) (x_kind 1) or fp32 feature-major (F, ld
    >= n) (x_kind 2).  Returns (W (N, K), b (N),
    lo (N, K), hi (N, K), count (N)) on X's device; W, b act on the
    standardised inputs.  gram: "exact" or "mfma" (default GRAM)."""
    W, b, lo, hi, cnt, status = _leaf_fit(X, x_kind, feats, mu, sd, grad, hess, leaf_idx, feature, min_samples,
                                          lam, gram)
    _check_status(int(status[0].item()))
    return W, b, lo, hi, cnt


def leaf_moments(X: torch.Tensor, x_kind: int, feats: torch.Tensor, n: int):
    """(mu, sd) of the selected inputs over n rows: mean and unbiased std
    clamped at 1e-6 (neural_leaves.py:152-154), from ``yabt_leaf_moments``."""
    lib = _lib.load()
    dev = X.device
    K = int(feats.numel())
    if x_kind == 0 and (X.dtype != torch.float32 or X.shape[0] != n or X.stride(1) != 1):
        raise ValueError("X must be fp32 (n, F) with unit column stride")
    if x_kind == 1 and (X.dtype != torch.uint8 or X.shape[1] < n or X.stride(1) != 1):
        raise ValueError("X must be uint8 (F, ld >= n)")
    if x_kind == 2 and (X.dtype != torch.float32 or X.shape[1] < n or X.stride(1) != 1):
        raise ValueError("X must be fp32 (F, ld >= n)")
    fi = feats.to(dev, torch.int32).contiguous()
    nbytes = int(lib.yabt_leaf_moments_workspace_bytes(n))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    mu = torch.empty(K, dtype=torch.float32, device=dev)
    sd = torch.empty(K, dtype=torch.float32, device=dev)
    _lib.check(lib.yabt_leaf_moments(x_kind, X.data_ptr(), X.stride(0), n, fi.data_ptr(), K, ws.data_ptr(),
                                     nbytes, mu.data_ptr(), sd.data_ptr(), _stream(dev)),
               "yabt_leaf_moments")
    return mu, sd


def fold(tree: Tree, W, db, mu, sd, lr, feats, lo, hi) -> Tree:
    """Normalisation and shrinkage folded into raw space (neural_leaves.py:178-184)
    by ``yabt_leaf_fold``: the reference's torch expressions in their fp32
    order, the K products added left to right as torch's CPU reduction adds
    the reference's K = 8 inputs."""
    lib = _lib.load()
    dev = W.device
    N, K = int(W.shape[0]), int(W.shape[1])
    value_in = tree.value.to(dev, torch.float32).contiguous()
    value = torch.empty_like(value_in)
    linear = torch.empty((N, K), dtype=torch.float32, device=dev)
    Wc, bc = W.contiguous(), db.contiguous()
    m, s = mu.to(dev, torch.float32).contiguous(), sd.to(dev, torch.float32).contiguous()
    _lib.check(lib.yabt_leaf_fold(N, K, Wc.data_ptr(), bc.data_ptr(), m.data_ptr(), s.data_ptr(), float(lr),
                                  value_in.data_ptr(), value.data_ptr(), linear.data_ptr(), _stream(dev)),
               "yabt_leaf_fold")
    return replace(tree, value=value, leaf_net_feats=feats, leaf_net_linear=linear, leaf_net_lo=lo,
                   leaf_net_hi=hi)


def _leaf_step(tree: Tree, X: torch.Tensor, x_kind: int, n: int, feats: torch.Tensor | None, grad: torch.Tensor,
               hess: torch.Tensor, leaf_idx: torch.Tensor, params, rank_k: int = 0) -> Tree | None:
    """Moments, fit and fold of one tree's leaf models: every tensor and
    workspace is prepared first, then the launches go out back to back (the
    device runs them without waiting on the host), then the one wait for the
    status.  tree's node arrays are on X's device.  With rank_k > 0 (feats
    None) the split features are ranked on the device first and the fit
    takes the first rank_k; None if the tree uses fewer than rank_k features
    (the caller then pads them on the host)."""
    lib = _lib.load()
    dev = X.device
    K, N = (rank_k if rank_k else int(feats.numel())), int(tree.feature.shape[0])
    mode = GRAM_MODES[GRAM]
    if x_kind == 0 and (X.dtype != torch.float32 or X.dim() != 2 or X.shape[0] != n or X.stride(1) != 1):
        raise ValueError("X must be fp32 (n, F) with unit column stride")
    if x_kind == 1 and (X.dtype != torch.uint8 or X.dim() != 2 or X.shape[1] < n or X.stride(1) != 1):
        raise ValueError("X must be uint8 (F, ld >= n)")
    if x_kind == 2 and (X.dtype != torch.float32 or X.dim() != 2 or X.shape[1] < n or X.stride(1) != 1):
        raise ValueError("X must be fp32 (F, ld >= n)")
    fi = None if rank_k else feats.to(dev, torch.int32).contiguous()
    g = grad.to(dev, torch.float32).contiguous()
    h = hess.to(dev, torch.float32).contiguous()
    li = leaf_idx.to(dev, torch.int64).contiguous()
    ft = tree.feature.to(dev, torch.int64).contiguous()
    value_in = tree.value.to(dev, torch.float32).contiguous()
    mbytes = int(lib.yabt_leaf_moments_workspace_bytes(n))
    fbytes = int(lib.yabt_leaf_fit_workspace_bytes(n, N, K))
    if fbytes == 0:
        raise ValueError("yabt_leaf_fit: invalid sizes (1 <= K <= 8 inputs)")
    # two allocations per call from torch's caching allocator on the current
    # stream, cut into 256-byte aligned pieces: the workspaces and the
    # outputs used only here, and the outputs the tree keeps (a view keeps
    # its whole allocation alive)
    def carve(sizes):
        up = [(v + 255) // 256 * 256 for v in sizes]
        base = torch.empty(sum(up), dtype=torch.uint8, device=dev)
        offs, o = [], 0
        for u in up:
            offs.append(o)
            o += u
        return base, offs
    # the transient pieces go to the C ABI as addresses (no tensor views:
    # each view costs host time while the device waits); the status and the
    # outputs the tree keeps are views
    tb, to = carve([max(mbytes, 1), fbytes, 4 * K, 4 * K, 4 * N * K, 4 * N, 8 * N, 12, 4 * K])
    a0 = tb.data_ptr()
    a_mws, a_fws, a_mu, a_sd, a_W, a_b, a_cnt, _, a_fi = (a0 + o for o in to)
    status = tb[to[7]:to[7] + 12].view(torch.int32)
    kb, ko = carve([4 * N * K, 4 * N * K, 4 * N, 4 * N * K, 8 * K])
    lo, hi, linear = (kb[o:o + 4 * N * K].view(torch.float32).view(N, K) for o in (ko[0], ko[1], ko[3]))
    value = kb[ko[2]:ko[2] + 4 * N].view(torch.float32)
    ldx, st = X.stride(0), _stream(dev)
    min_samples = int(getattr(params, "leaf_net_min_samples", 50))
    lam = float(getattr(params, "leaf_net_l2", 1.0))
    lr = float(params.learning_rate)
    if rank_k:
        # ranking, moments, fit and fold in one call: the launches go out
        # without a return to Python between them
        feats = kb[ko[4]:ko[4] + 8 * K].view(torch.int64)
        _lib.check(lib.yabt_leaf_step(x_kind, X.data_ptr(), ldx, n, int(X.shape[0]), K, g.data_ptr(),
                                      h.data_ptr(), li.data_ptr(), ft.data_ptr(), value_in.data_ptr(), N,
                                      min_samples, lam, lr, mode, a_mws, mbytes, a_fws, fbytes, feats.data_ptr(),
                                      a_fi, a_mu, a_sd, a_W, a_b, lo.data_ptr(), hi.data_ptr(), a_cnt,
                                      value.data_ptr(), linear.data_ptr(), status.data_ptr(), st),
                   "yabt_leaf_step")
    else:
        a_fi = fi.data_ptr()
        _lib.check(lib.yabt_leaf_moments(x_kind, X.data_ptr(), ldx, n, a_fi, K, a_mws, mbytes, a_mu, a_sd, st),
                   "yabt_leaf_moments")
        _lib.check(lib.yabt_leaf_fit(x_kind, X.data_ptr(), ldx, n, a_fi, K, a_mu, a_sd,
                                     g.data_ptr(), h.data_ptr(), li.data_ptr(), ft.data_ptr(), N, min_samples,
                                     lam, mode, a_fws, fbytes, a_W, a_b, lo.data_ptr(), hi.data_ptr(), a_cnt,
                                     status.data_ptr(), st), "yabt_leaf_fit")
        _lib.check(lib.yabt_leaf_fold(N, K, a_W, a_b, a_mu, a_sd, lr, value_in.data_ptr(), value.data_ptr(),
                                      linear.data_ptr(), st), "yabt_leaf_fold")
    st_, n_fit, n_used = status.tolist()   # the one wait for the device
    if rank_k and n_used < K:
        return None
    _check_status(st_)
    # no eligible leaf: the tree is returned unchanged (neural_leaves.py:156-158)
    if n_fit == 0:
        return tree
    return replace(tree, value=value, leaf_net_feats=feats, leaf_net_linear=linear, leaf_net_lo=lo,
                   leaf_net_hi=hi)


def feature_major(Xraw: torch.Tensor) -> torch.Tensor:
    """A feature-major fp32 copy (F, ld) of the raw inputs (n, F), ld the
    row count rounded up to a multiple of 4, so that every column starts
    16-byte aligned: the leaf models' row passes then read four rows of an
    input with one vector load (yabt_leaf_fit's x_kind 2).  Made once per fit
    (n F 4 bytes: 400 MB at 2M x 50)."""
    n, F = Xraw.shape
    ld = (n + 3) // 4 * 4
    out = torch.zeros((F, ld), dtype=torch.float32, device=Xraw.device)
    out[:, :n] = Xraw.t()
    return out


def fit_leaf_networks(tree: Tree, Xraw: torch.Tensor, y: torch.Tensor, margin: torch.Tensor, loss_fn,
                      params, gen: torch.Generator | None = None, leaf_idx: torch.Tensor | None = None,
                      X_fmajor: torch.Tensor | None = None) -> Tree:
    """Drop-in for yabt.neural_leaves.fit_leaf_networks (neural_leaves.py:131-184),
    linear leaves; Xraw (n, F) fp32 on a HIP device.  ``X_fmajor``: the same
    inputs feature-major (``feature_major(Xraw)``), kept by a caller that
    fits many trees on them; the models are the same either way."""
    if getattr(params, "leaf_net_hidden", 0) != 0:
        raise NotImplementedError("MLP leaves (leaf_net_hidden > 0) are not provided by this backend")
    dev = Xraw.device
    tree_d = replace(tree, feature=tree.feature.to(dev), threshold=tree.threshold.to(dev),
                     left=tree.left.to(dev), right=tree.right.to(dev), value=tree.value.to(dev))
    if leaf_idx is None:
        leaf_idx = tree_d.apply(Xraw)
    grad, hess = boost_ops.grad_hess(loss_fn, margin, y, leaf_idx, tree_d.value)
    n, F = Xraw.shape
    k = min(getattr(params, "leaf_net_features", 8), F)
    if X_fmajor is not None and 1 <= k <= 8 and F <= RANK_MAX_FEATURES:
        # the split features ranked on the device (the reference's order,
        # neural_leaves.py:27-31); None when the tree uses fewer than k, which
        # the host then pads by gradient correlation
        out = _leaf_step(tree_d, X_fmajor, 2, n, None, grad, hess, leaf_idx, params, rank_k=k)
        if out is not None:
            return tree if out is tree_d else out
    feats = _select_features(tree_d, Xraw, grad, getattr(params, "leaf_net_features", 8))
    if feats.numel() == 0:
        return tree
    if X_fmajor is not None:
        out = _leaf_step(tree_d, X_fmajor, 2, Xraw.shape[0], feats, grad, hess, leaf_idx, params)
        return tree if out is tree_d else out
    X = Xraw if Xraw.dtype == torch.float32 and Xraw.stride(1) == 1 else Xraw.float().contiguous()
    out = _leaf_step(tree_d, X, 0, X.shape[0], feats, grad, hess, leaf_idx, params)
    return tree if out is tree_d else out


def fit_leaf_networks_binned(tree: Tree, bins_fm: torch.Tensor, grad: torch.Tensor, hess: torch.Tensor,
                             leaf_idx: torch.Tensor, params, n: int | None = None) -> Tree:
    """The same fit with raw inputs x = float(bin) read straight from the
    feature-major bins (F, ld) (the identity-binner case), and g, h already
    evaluated at margin + value[leaf]."""
    if getattr(params, "leaf_net_hidden", 0) != 0:
        raise NotImplementedError("MLP leaves (leaf_net_hidden > 0) are not provided by this backend")
    dev = bins_fm.device
    n = int(grad.shape[0]) if n is None else n
    feature = tree.feature.to(dev)
    k = min(getattr(params, "leaf_net_features", 8), bins_fm.shape[0])
    if 1 <= k <= 8 and bins_fm.shape[0] <= RANK_MAX_FEATURES:
        tree_d = replace(tree, feature=feature, value=tree.value.to(dev))
        out = _fit_binned_ranked(tree_d, bins_fm, grad, hess, leaf_idx, params, n, k)
        if out is not None:
            return tree if out is tree_d else out
    feats = _used_features(feature, k).to(dev)
    if feats.numel() == 0:
        return tree
    if feats.numel() < k:
        # padding by gradient correlation needs the raw columns: take them as floats
        Xraw = bins_fm[:, :n].t().float()
        feats = _select_features(replace(tree, feature=feature), Xraw, grad, k)
    tree_d = replace(tree, feature=feature, value=tree.value.to(dev))
    out = _leaf_step(tree_d, bins_fm, 1, n, feats, grad, hess, leaf_idx, params)
    return tree if out is tree_d else out


def _fit_binned_ranked(tree_d: Tree, bins_fm: torch.Tensor, grad: torch.Tensor, hess: torch.Tensor,
                       leaf_idx: torch.Tensor, params, n: int, k: int) -> Tree | None:
    """The binned fit with the split features ranked on the device: the
    host never waits for the tree before the launches.  None when the tree
    uses fewer than k features (or names one outside the bins)."""
    return _leaf_step(tree_d, bins_fm, 1, n, None, grad, hess, leaf_idx, params, rank_k=k)
