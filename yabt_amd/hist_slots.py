"""K-slot histogram op (mirror of yabt/cuda_hist.py:71-89).

``build_hist(binned, slot, g, h, w, K, F, B)`` returns the (3, K, F, B) fp32
histogram the level-wise grower builds per level (yabt/tree.py:414-452): row
i adds (g[i], h[i], w[i]) into bin binned[i, f] of node slot[i] for every
feature f.  The HIP kernels (``csrc/slots.hip``, ``yabt_hist_slots``) sum
exact int64 fixed point and round once to fp32, so the result is
deterministic; rows whose slot lies outside [0, K) are skipped.
"""

from __future__ import annotations

import torch

from . import _lib


def is_available() -> bool:
    """True if the HIP library loads and a device is present (cuda_hist.py:71-77)."""
    return _lib.is_available() and torch.cuda.is_available()


def build_hist(binned: torch.Tensor, slot: torch.Tensor, g: torch.Tensor, h: torch.Tensor, w: torch.Tensor,
               K: int, F: int, B: int) -> torch.Tensor:
    """Fused (3, K, F, B) histogram (cuda_hist.py:79-89); B must be 256."""
    if B != 256:
        raise ValueError("build_hist: the histogram width is 256 bins")
    lib = _lib.load()
    dev = binned.device
    if dev.type != "cuda":
        raise RuntimeError("build_hist needs device tensors")
    n = int(slot.shape[0])
    if binned.dtype != torch.uint8 or binned.dim() != 2 or binned.shape[0] != n or binned.shape[1] < F:
        raise ValueError("binned must be uint8 (n, >= F)")
    b = binned if binned.stride(1) == 1 else binned.contiguous()
    s = slot.to(dev, torch.int64).contiguous()
    gg, hh, ww = (x.to(dev, torch.float32).contiguous() for x in (g, h, w))
    nbytes = int(lib.yabt_hist_slots_workspace_bytes(n, F, K))
    if nbytes == 0:
        raise ValueError("build_hist: invalid sizes")
    # per call, from torch's caching allocator on the current stream: calls
    # from several host threads on their own streams never share it
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    out = torch.empty((3, K, F, B), dtype=torch.float32, device=dev)
    status = torch.empty(4, dtype=torch.int32, device=dev)
    _lib.check(lib.yabt_hist_slots(b.data_ptr(), b.stride(0), s.data_ptr(), gg.data_ptr(), hh.data_ptr(),
                                   ww.data_ptr(), n, F, int(K), ws.data_ptr(), nbytes, out.data_ptr(),
                                   status.data_ptr(), torch.cuda.current_stream(dev).cuda_stream),
               "yabt_hist_slots")
    if int(status[0].item()) != 0:
        raise ValueError("build_hist: g, h or w holds a non-finite value")
    build_hist.last_shifts = tuple(int(v) for v in status[1:].cpu())
    return out
