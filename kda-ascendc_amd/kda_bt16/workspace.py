"""Workspace pool for the records stage 1 hands to stage 2.

One grow-only device buffer per (device, stream), for the forward's
records only; the backward's larger workspace is taken per call from torch's
caching allocator (:func:`scratch`), so a training step leaves no
backward-sized lease behind for later forwards.  Work on one stream runs
in order, so the next forward on the same stream may overwrite the records
of the previous one; forwards on different streams never share a buffer.
The buffer is sized exactly by ``kda_bt16_workspace_bytes`` (17 KiB per
(batch, head, 16-token chunk): 272 MiB at B=1 T=8192 H=32, 1.06 GiB at
B=16 T=2048 H=32), rounded up to 2 MiB, and kept until :func:`clear`.

This replaces the reference's per-call ``torch.empty`` intermediates
(``/root/reference/src/kda_bt16/kernels.py:572-579``).  Unlike the
reference's ``reuse_workspace`` cache (kernels.py:525-536), the pooled
buffer is never returned to the caller, so reuse cannot alias user-visible
tensors.
"""

from __future__ import annotations

import threading

import torch

_ALIGN = 2 << 20
_pool: dict[tuple[int, int], torch.Tensor] = {}
_lock = threading.Lock()


def lease(device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    """Return a uint8 device buffer of at least ``nbytes`` for ``stream``."""
    key = (device.index if device.index is not None else torch.cuda.current_device(), int(stream))
    with _lock:
        buf = _pool.get(key)
        if buf is None or buf.numel() < nbytes:
            _pool.pop(key, None)
            size = max(_ALIGN, (nbytes + _ALIGN - 1) // _ALIGN * _ALIGN)
            buf = torch.empty(size, dtype=torch.uint8, device=device)
            _pool[key] = buf
        return buf


def scratch(device: torch.device, nbytes: int) -> torch.Tensor:
    """A uint8 device buffer of ``nbytes`` (rounded up to 256 B) for one
    call, from torch's caching allocator (not pooled here)."""
    return torch.empty(max(256, (nbytes + 255) // 256 * 256), dtype=torch.uint8, device=device)


def clear() -> None:
    """Drop every pooled buffer (they return to torch's caching allocator)."""
    with _lock:
        _pool.clear()


def pooled_bytes() -> int:
    with _lock:
        return sum(b.numel() for b in _pool.values())
