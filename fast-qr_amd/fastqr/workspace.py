"""Output and scratch workspaces.

Mirrors the reference's allocator helpers (submissions/candidate.py:3682-3806):
``allocate_column_major_H``, ``allocate_tau`` and ``allocate_h_tau`` return
column-major H (stride (n*n, 1, n)) and contiguous tau.  With the output cache
on (the default here; ``FASTQR_OUTPUT_WORKSPACE_CACHE=0`` turns it off) the
tensors are cached per input object, keyed by ``id(data)`` and guarded by a
weak reference, exactly like ``_workspace_tensor`` (submissions/candidate.py:3708-3749):
different inputs never share output storage, and a second call on the same
input object reuses (overwrites) the first call's H and tau.

The T-factor scratch of the blocked path is cached per (device, stream): calls
on one stream are serialised by the stream, so they can share it.
"""
from __future__ import annotations

import weakref

import torch

from ._lib import env_flag

_OUTPUT_CACHE: dict[tuple, tuple[weakref.ref, torch.Tensor]] = {}
# (H, tau) pairs already handed out by allocate_h_tau, one dictionary lookup
# per call; the tensors are the per-kind cache entries above
_PAIR_CACHE: dict[tuple, tuple[weakref.ref, torch.Tensor, torch.Tensor]] = {}
_SCRATCH: dict[tuple, torch.Tensor] = {}


def output_cache_enabled() -> bool:
    return env_flag("FASTQR_OUTPUT_WORKSPACE_CACHE", True)


def _key(data: torch.Tensor, kind: str, shape: tuple, stride: tuple) -> tuple:
    dev = data.device
    return (kind, id(data), shape, stride, dev.type, -1 if dev.index is None else dev.index)


def _cached(data: torch.Tensor, kind: str, shape: tuple, stride: tuple, zero: bool,
            cache_enabled: bool | None) -> torch.Tensor:
    if cache_enabled is None:
        cache_enabled = output_cache_enabled()
    if cache_enabled:
        key = _key(data, kind, shape, stride)
        hit = _OUTPUT_CACHE.get(key)
        if hit is not None:
            ref, tensor = hit
            if ref() is data and tuple(tensor.shape) == shape and tuple(tensor.stride()) == stride:
                if zero:
                    tensor.zero_()
                return tensor
            _OUTPUT_CACHE.pop(key, None)
        try:
            ref = weakref.ref(data, lambda _r, k=key: _OUTPUT_CACHE.pop(k, None))
        except TypeError:
            ref = None
        tensor = torch.empty_strided(shape, stride, device=data.device, dtype=torch.float32)
        if zero:
            tensor.zero_()
        if ref is not None:
            _OUTPUT_CACHE[key] = (ref, tensor)
        return tensor
    tensor = torch.empty_strided(shape, stride, device=data.device, dtype=torch.float32)
    if zero:
        tensor.zero_()
    return tensor


def allocate_column_major_H(batch: int, n: int, data: torch.Tensor, *,
                            cache_enabled: bool | None = None) -> torch.Tensor:
    """(batch, n, n) fp32 with stride (n*n, 1, n) on data's device."""
    shape = (batch, n, n)
    return _cached(data, "h_colmajor", shape, (n * n, 1, n), False, cache_enabled)


def allocate_tau(batch: int, n: int, data: torch.Tensor, *, zero: bool = False,
                 cache_enabled: bool | None = None) -> torch.Tensor:
    """(batch, n) contiguous fp32 on data's device."""
    return _cached(data, "tau", (batch, n), (n, 1), zero, cache_enabled)


def allocate_h_tau(batch: int, n: int, data: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    enabled = output_cache_enabled()
    if not enabled:
        return (allocate_column_major_H(batch, n, data, cache_enabled=False),
                allocate_tau(batch, n, data, cache_enabled=False))
    key = (id(data), batch, n, data.get_device())
    hit = _PAIR_CACHE.get(key)
    if hit is not None and hit[0]() is data:
        return hit[1], hit[2]
    h = allocate_column_major_H(batch, n, data, cache_enabled=True)
    tau = allocate_tau(batch, n, data, cache_enabled=True)
    try:
        ref = weakref.ref(data, lambda _r, k=key: _PAIR_CACHE.pop(k, None))
    except TypeError:
        return h, tau
    _PAIR_CACHE[key] = (ref, h, tau)
    return h, tau


def scratch(device: torch.device, stream_ptr: int, nbytes: int) -> torch.Tensor | None:
    """A uint8 device buffer of at least nbytes (256-byte aligned), cached per (device, stream)."""
    if nbytes <= 0:
        return None
    key = (device.type, device.index, stream_ptr)
    buf = _SCRATCH.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
        _SCRATCH[key] = buf
    return buf


def clear() -> None:
    _OUTPUT_CACHE.clear()
    _PAIR_CACHE.clear()
    _SCRATCH.clear()
