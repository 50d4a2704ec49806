"""``custom_kernel(data) -> (H, tau)``: the drop-in entry point.

Same interface as the reference submission (official/submission.py:5-6,
official/task.py:4-5; dispatcher submissions/candidate.py:8383-8415): ``data``
is a (batch, n, n) fp32 CUDA tensor (any strides), the result is
``(H, tau)`` in torch.geqrf's compact-Householder convention with H
column-major.  The work is one call into the gfx950 C ABI
(include/fastqr.h, ``fastqr_geqrf_f32``) on torch's current stream; the
kernel path is picked from n alone (``path_for``).  There is no fallback: a
missing library raises ``FastQRUnavailable`` and a failed call raises
``FastQRError`` (the reference silently fell back to torch.geqrf,
submissions/candidate.py:4445-4457).
"""
from __future__ import annotations

import torch

from . import workspace
from ._lib import FastQRError, ext


def path_for(n: int) -> str:
    """Name of the kernel path for size n: 'wave64' (n <= 64) or 'blocked'."""
    return ext().path_name(int(n))


def _validate(data: torch.Tensor) -> None:
    if not isinstance(data, torch.Tensor):
        raise TypeError("data must be a torch.Tensor")
    if data.dtype != torch.float32:
        raise TypeError(f"data must be float32, got {data.dtype}")
    if data.dim() != 3 or data.shape[1] != data.shape[2]:
        raise ValueError(f"data must have shape (batch, n, n), got {tuple(data.shape)}")
    if not data.is_cuda:
        raise ValueError("data must be a CUDA (HIP) tensor")


# Raw handle of the current stream of a device, without building a Stream
# object (about 0.1 us instead of 2 us per call: at 20 x 32 the whole call
# must stay below the kernel's ~8 us or back-to-back calls become host-bound).
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _current_stream_ptr(device_index: int) -> int:
    if _raw_stream is not None:
        return _raw_stream(device_index)
    return torch.cuda.current_stream(device_index).cuda_stream


def _launch(data: torch.Tensor, h: torch.Tensor, tau: torch.Tensor, b: int, n: int,
            sptr: int) -> tuple[torch.Tensor, torch.Tensor]:
    mod = ext()
    nbytes = mod.workspace_bytes(b, n)
    ws = workspace.scratch(data.device, sptr, nbytes) if nbytes > 0 else None
    ws_ptr = 0 if ws is None else ws.data_ptr()
    ws_len = 0 if ws is None else ws.numel()
    as0, as1, as2 = data.stride()
    hs0, hs1, hs2 = h.stride()
    ts0, ts1 = tau.stride()
    rc = mod.geqrf(data.data_ptr(), b, n, as0, as1, as2, h.data_ptr(), hs0, hs1, hs2,
                   tau.data_ptr(), ts0, ts1, ws_ptr, ws_len, sptr)
    if rc != 0:
        raise FastQRError(rc, mod.last_error())
    return h, tau


def geqrf_into(data: torch.Tensor, h: torch.Tensor, tau: torch.Tensor,
               stream: torch.cuda.Stream | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Factor ``data`` into caller-provided ``h`` (columns contiguous) and ``tau``."""
    _validate(data)
    b, n, _ = data.shape
    if tuple(h.shape) != (b, n, n) or h.dtype != torch.float32 or h.device != data.device:
        raise ValueError("H must be a float32 (batch, n, n) tensor on data's device")
    if tuple(tau.shape) != (b, n) or tau.dtype != torch.float32 or tau.device != data.device:
        raise ValueError("tau must be a float32 (batch, n) tensor on data's device")
    sptr = stream.cuda_stream if stream is not None else _current_stream_ptr(data.get_device())
    return _launch(data, h, tau, b, n, sptr)


def custom_kernel(data: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Batched compact-Householder QR of a (batch, n, n) fp32 CUDA tensor."""
    _validate(data)
    b, n, _ = data.shape
    idx = data.get_device()
    if idx != torch.cuda.current_device():
        with torch.cuda.device(idx):
            return custom_kernel(data)
    # H and tau come from the allocator helpers (right shape, dtype, device):
    # no second validation
    h, tau = workspace.allocate_h_tau(b, n, data)
    return _launch(data, h, tau, b, n, _current_stream_ptr(idx))
