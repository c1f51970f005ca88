"""Concurrent growers: two host threads, each on its own default-priority
stream, grow different trees at the same time, and every tree equals the
one the same call grows alone.

cgrow takes its scratch per call (yabt/_cgrow/grow.c:271-287), so the
reference grower may be called from several threads at once (ctypes drops
the GIL); the HIP growers take their workspaces per call from torch's
caching allocator on the calling stream and their pinned host buffers from
a locked pool, so they may be too.
"""

import threading

import numpy as np
import pytest
import torch

from yabt_amd import grow_hip as G

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0) if torch.cuda.is_available() else None

CASES = [
    # (n, F, bins, seed, grower kwargs)
    (200_000, 40, 256, 1, dict(max_leaves=63)),                                   # in rounds
    (150_000, 30, 64, 2, dict(max_leaves=32, max_depth=5)),                       # depth by depth
    (90_000, 25, 128, 3, dict(max_leaves=40, growth="sequential")),               # split by split
    (60_000, 20, 256, 4, dict(max_leaves=31, arithmetic="reference")),            # cgrow's arithmetic
]


def _inputs(n, F, nb, seed):
    rng = np.random.default_rng(seed)
    bins = torch.from_numpy(rng.integers(0, nb, size=(n, F)).astype(np.uint8))
    lay = G.make_layouts(bins, DEV)
    g = torch.from_numpy(rng.normal(size=n).astype(np.float32)).to(DEV)
    h = torch.from_numpy(rng.uniform(0.1, 1.0, size=n).astype(np.float32)).to(DEV)
    return lay, g, h, np.full(F, nb, np.int32)


def _grow(case, inputs):
    n, F, _, _, kw = case
    lay, g, h, nbins = inputs
    res = G.grow_device(lay, g, h, nbins, **kw)
    torch.cuda.current_stream().synchronize()
    out = {k: getattr(res, k).cpu().numpy() for k in ("feature", "thr_bin", "left", "right", "depth")}
    out["value"] = res.value.cpu().numpy().view(np.uint32)
    out["leaf"] = G.leaf_ids(res, n, F, kw["max_leaves"]).cpu().numpy()
    return out


def _same(a, b):
    return all(np.array_equal(a[k], b[k]) for k in a)


def test_two_threads_grow_their_own_trees():
    inputs = [_inputs(n, F, nb, s) for n, F, nb, s, _ in CASES]
    alone = [_grow(c, x) for c, x in zip(CASES, inputs)]
    torch.cuda.synchronize()
    errors = []

    def worker(tid):
        try:
            stream = torch.cuda.Stream(device=DEV)   # default priority
            with torch.cuda.stream(stream):
                for rep in range(3):
                    for ci in range(tid, len(CASES), 2):
                        got = _grow(CASES[ci], inputs[ci])
                        if not _same(got, alone[ci]):
                            errors.append(f"thread {tid} rep {rep}: case {ci} differs from its lone run")
        except Exception as e:  # noqa: BLE001 - reported by the main thread
            errors.append(f"thread {tid}: {e!r}")

    print("two threads, two streams, four growers", flush=True)
    threads = [threading.Thread(target=worker, args=(t,)) for t in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=100)
    assert not any(t.is_alive() for t in threads), "a grower thread did not finish"
    assert not errors, errors


def test_first_use_of_a_fresh_layout_on_two_streams():
    """Two threads, each on its own stream, make a fresh layout's lazily built
    tables (bin counts, default bins, the reference root rank table) at the
    same time; every tree equals the one grown alone on another layout of
    the same bins."""
    n, F, nb = 120_000, 36, 256
    rng = np.random.default_rng(11)
    bins_np = rng.integers(0, nb, size=(n, F)).astype(np.uint8)
    bins_np[rng.random((n, F)) < 0.6] = 0      # a modal bin worth skipping
    bins = torch.from_numpy(bins_np)
    g = torch.from_numpy(rng.normal(size=n).astype(np.float32)).to(DEV)
    h = torch.from_numpy(rng.uniform(0.1, 1.0, size=n).astype(np.float32)).to(DEV)
    nbins = np.full(F, nb, np.int32)
    kws = [dict(max_leaves=63), dict(max_leaves=31, arithmetic="reference")]
    lone = G.make_layouts(bins, DEV)
    torch.cuda.synchronize()
    alone = [_grow((n, F, nb, 0, kw), (lone, g, h, nbins)) for kw in kws]
    for rep in range(3):
        fresh = G.make_layouts(bins, DEV)
        torch.cuda.synchronize()
        barrier = threading.Barrier(2)
        errors = []

        def worker(tid):
            try:
                stream = torch.cuda.Stream(device=DEV)   # default priority
                with torch.cuda.stream(stream):
                    barrier.wait(timeout=60)
                    for k in (tid, 1 - tid):
                        got = _grow((n, F, nb, 0, kws[k]), (fresh, g, h, nbins))
                        if not _same(got, alone[k]):
                            errors.append(f"rep {rep} thread {tid}: grower {k} differs from its lone run")
            except Exception as e:  # noqa: BLE001 - reported by the main thread
                errors.append(f"rep {rep} thread {tid}: {e!r}")

        print(f"fresh layout, two streams, rep {rep}", flush=True)
        threads = [threading.Thread(target=worker, args=(t,)) for t in range(2)]
        for t in threads:
            t.start()
        for t in threads:
            t.join(timeout=100)
        assert not any(t.is_alive() for t in threads), "a grower thread did not finish"
        assert not errors, errors
