"""yabt_hist_noalloc (no device allocation, scratch in a static device array)
against yabt_hist through the C ABI: identical histograms and shifts on two
calls in a row, the second on a smaller input, for the streaming root and for
a gathered row list; no allocation after the first call; replays of the call
captured into a HIP graph."""

import numpy as np
import pytest
import torch

from yabt_amd import _lib
from yabt_amd import grow_hip as G

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0) if torch.cuda.is_available() else None


def _noalloc():
    return _lib.load().yabt_hist_noalloc


def _case(n, F, seed, m, outlier=None):
    rng = np.random.default_rng(seed)
    bins = rng.integers(0, 256, size=(n, F)).astype(np.uint8)
    g = rng.normal(size=n).astype(np.float32)
    if outlier is not None:   # selects the wide contract
        g[n // 2] = outlier
    h = rng.uniform(0.1, 1.0, size=n).astype(np.float32)
    lay = G.make_layouts(torch.from_numpy(bins), DEV)
    rows = torch.from_numpy(np.sort(rng.choice(n, size=m, replace=False)).astype(np.int32)).to(DEV)
    return lay, torch.from_numpy(g).to(DEV), torch.from_numpy(h).to(DEV), rows


def _run_noalloc(fn, lay, g, h, rows):
    out = torch.full((3, lay.F, 256), -7, dtype=torch.int64, device=DEV)
    shifts = torch.full((3,), -99, dtype=torch.int32, device=DEV)
    m = 0 if rows is None else rows.shape[0]
    rc = fn(G._ptr(lay.fm), lay.ld_fm, G._ptr(lay.rm), lay.ld_rm, G._ptr(g), G._ptr(h), lay.n, lay.F,
            G._ptr(rows), m, G._ptr(out), G._ptr(shifts), G._stream(DEV))
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    return out.cpu().numpy(), shifts.cpu().tolist()


def test_noalloc_matches_yabt_hist_twice():
    fn = _noalloc()
    for n, F, seed, m, outlier in [(300_001, 37, 1, 120_000, None), (40_000, 20, 2, 9_000, None),
                                   (50_000, 18, 3, 20_000, 1e5)]:
        print(f"yabt_hist_noalloc n={n} F={F} rows={m} outlier={outlier}", flush=True)
        lay, g, h, rows = _case(n, F, seed, m, outlier)
        for r in (None, rows):
            got, got_s = _run_noalloc(fn, lay, g, h, r)
            want, want_s = G.hist(lay, g, h, r)
            assert got_s == list(want_s)
            assert np.array_equal(got, want.cpu().numpy())
            assert int(got[2].sum()) == (n if r is None else m) * F


def test_noalloc_allocates_nothing_and_replays_under_capture():
    """After a first call (which looks up the device's scratch address and
    loads the kernels), further calls change neither torch's allocator
    counters nor the device's free memory; the call captured into a HIP graph
    replays three times, with eager work between the replays, each replay
    equal to yabt_hist's histogram and shifts."""
    fn = _noalloc()
    lay, g, h, rows = _case(60_000, 21, 5, 25_000)
    want, want_s = G.hist(lay, g, h, rows)
    want = want.cpu().numpy()
    out = torch.full((3, lay.F, 256), -7, dtype=torch.int64, device=DEV)
    shifts = torch.full((3,), -99, dtype=torch.int32, device=DEV)

    def call():
        return fn(G._ptr(lay.fm), lay.ld_fm, G._ptr(lay.rm), lay.ld_rm, G._ptr(g), G._ptr(h), lay.n, lay.F,
                  G._ptr(rows), rows.shape[0], G._ptr(out), G._ptr(shifts), G._stream(DEV))

    assert call() == 0, _lib.last_error()
    torch.cuda.synchronize()
    stats0 = torch.cuda.memory_stats(DEV)
    free0 = torch.cuda.mem_get_info(DEV)[0]
    for _ in range(5):
        assert call() == 0, _lib.last_error()
    torch.cuda.synchronize()
    stats1 = torch.cuda.memory_stats(DEV)
    free1 = torch.cuda.mem_get_info(DEV)[0]
    for k in ("allocation.all.allocated", "segment.all.allocated", "reserved_bytes.all.current"):
        assert stats1.get(k, 0) == stats0.get(k, 0), k
    assert free1 >= free0
    assert np.array_equal(out.cpu().numpy(), want) and shifts.cpu().tolist() == list(want_s)

    print("yabt_hist_noalloc under graph capture", flush=True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        assert call() == 0, _lib.last_error()
    for rep in range(3):
        out.fill_(-7)
        shifts.fill_(-99)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), want), f"replay {rep}"
        assert shifts.cpu().tolist() == list(want_s), f"replay {rep}"
        # an eager call between the replays, on the same scratch (other inputs)
        got2, got2_s = _run_noalloc(fn, lay, h, g, None)
        want2, want2_s = G.hist(lay, h, g)
        assert np.array_equal(got2, want2.cpu().numpy()) and got2_s == list(want2_s)
