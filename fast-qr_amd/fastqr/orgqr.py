"""``householder_product(h, tau) -> Q``: explicit Q of compact-Householder factors.

Same meaning as ``torch.linalg.householder_product(A, tau)``, the call the
reference's checker makes on ``custom_kernel``'s output
(official/reference.py:199), for square (batch, n, n) fp32 CUDA/HIP tensors
with n reflectors: Q = H_0 H_1 ... H_{n-1}, H_k = I - tau[k] v_k v_k^T.  One
call into the gfx950 C ABI (include/fastqr.h, ``fastqr_orgqr_f32``) on torch's
current stream; no fallback (a missing library raises ``FastQRUnavailable``,
a failed call ``FastQRError``).
"""
from __future__ import annotations

import torch

from . import workspace
from ._lib import FastQRError, ext
from .qr import _current_stream_ptr


def _check(h: torch.Tensor, tau: torch.Tensor) -> tuple[int, int]:
    if not isinstance(h, torch.Tensor) or not isinstance(tau, torch.Tensor):
        raise TypeError("h and tau must be torch.Tensors")
    if h.dtype != torch.float32 or tau.dtype != torch.float32:
        raise TypeError("h and tau must be float32")
    if h.dim() != 3 or h.shape[1] != h.shape[2]:
        raise ValueError(f"h must have shape (batch, n, n), got {tuple(h.shape)}")
    b, n, _ = h.shape
    if tuple(tau.shape) != (b, n):
        raise ValueError(f"tau must have shape {(b, n)}, got {tuple(tau.shape)}")
    if not h.is_cuda or tau.device != h.device:
        raise ValueError("h and tau must be CUDA (HIP) tensors on one device")
    return b, n


def householder_product(h: torch.Tensor, tau: torch.Tensor, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """Q (column-major, like geqrf's H) from the geqrf factors ``(h, tau)``.

    ``out`` may be given with contiguous columns (stride (*, 1, >= n)); it may
    be ``h`` itself with h's layout (Q then replaces the factors in place).
    """
    b, n = _check(h, tau)
    idx = h.get_device()
    if idx != torch.cuda.current_device():
        with torch.cuda.device(idx):
            return householder_product(h, tau, out=out)
    if out is None:
        out = torch.empty_strided((b, n, n), (n * n, 1, n), dtype=torch.float32, device=h.device)
    elif tuple(out.shape) != (b, n, n) or out.dtype != torch.float32 or out.device != h.device:
        raise ValueError("out must be a float32 (batch, n, n) tensor on h's device")
    if b == 0 or n == 0:
        return out
    mod = ext()
    sptr = _current_stream_ptr(idx)
    ws = workspace.scratch(h.device, sptr, mod.orgqr_workspace_bytes(b, n))  # None when none is needed
    hs0, hs1, hs2 = h.stride()
    ts0, ts1 = tau.stride()
    qs0, qs1, qs2 = out.stride()
    rc = mod.orgqr(h.data_ptr(), b, n, hs0, hs1, hs2, tau.data_ptr(), ts0, ts1, out.data_ptr(), qs0, qs1, qs2,
                   0 if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(), sptr)
    if rc != 0:
        raise FastQRError(rc, mod.last_error())
    return out


def apply_q(h: torch.Tensor, tau: torch.Tensor, c: torch.Tensor, *, transpose: bool = False) -> torch.Tensor:
    """Q C (or Q^T C with ``transpose``) for geqrf factors ``(h, tau)``, without forming Q.

    The meaning of ``torch.ormqr(h, tau, c, left=True, transpose=transpose)``
    (the reference's call on geqrf factors, submissions/candidate.py:7231-7237):
    ``h`` is (batch, m, r) with r <= m reflectors below its diagonal, ``tau``
    (batch, r), ``c`` (batch, m, k).  One call into the gfx950 C ABI
    (``fastqr_ormqr_f32``): the compact-WY transforms of every 32-column panel
    applied to a column-major copy of C by the MFMA update kernels.  Returns a
    new tensor (column-major, like geqrf's H); ``c`` is not modified.
    """
    if not isinstance(h, torch.Tensor) or not isinstance(tau, torch.Tensor) or not isinstance(c, torch.Tensor):
        raise TypeError("h, tau and c must be torch.Tensors")
    if h.dtype != torch.float32 or tau.dtype != torch.float32 or c.dtype != torch.float32:
        raise TypeError("h, tau and c must be float32")
    if h.dim() != 3 or h.shape[2] > h.shape[1]:
        raise ValueError(f"h must have shape (batch, m, r) with r <= m, got {tuple(h.shape)}")
    b, m, r = h.shape
    if tuple(tau.shape) != (b, r):
        raise ValueError(f"tau must have shape {(b, r)}, got {tuple(tau.shape)}")
    if c.dim() != 3 or c.shape[0] != b or c.shape[1] != m:
        raise ValueError(f"c must have shape ({b}, {m}, k), got {tuple(c.shape)}")
    if not h.is_cuda or tau.device != h.device or c.device != h.device:
        raise ValueError("h, tau and c must be CUDA (HIP) tensors on one device")
    idx = h.get_device()
    if idx != torch.cuda.current_device():
        with torch.cuda.device(idx):
            return apply_q(h, tau, c, transpose=transpose)
    k = c.shape[2]
    out = torch.empty_strided((b, m, k), (m * k, 1, m), dtype=torch.float32, device=h.device)
    out.copy_(c)
    if b == 0 or m == 0 or k == 0 or r == 0:
        return out
    if h.stride(1) != 1 or h.stride(2) < m:  # the kernels read V in column segments
        h = h.transpose(-1, -2).contiguous().transpose(-1, -2)
    mod = ext()
    sptr = _current_stream_ptr(idx)
    ws = workspace.scratch(h.device, sptr, mod.ormqr_workspace_bytes(b, m, r, k))
    hs0, hs1, hs2 = h.stride()
    ts0, ts1 = tau.stride()
    cs0, cs1, cs2 = out.stride()
    rc = mod.ormqr(h.data_ptr(), b, m, r, hs0, hs1, hs2, tau.data_ptr(), ts0, ts1, out.data_ptr(), k, cs0, cs1, cs2,
                   1 if transpose else 0, 0 if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(), sptr)
    if rc != 0:
        raise FastQRError(rc, mod.last_error())
    return out
