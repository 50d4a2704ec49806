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
    """Q C (or Q^T C with ``transpose``) for the geqrf factors ``(h, tau)``.

    The meaning of ``torch.ormqr(h, tau, c, left=True, transpose=transpose)``
    for square h with n reflectors and C of shape (batch, n, k): Q is formed
    by ``householder_product`` (the HIP kernels) and applied with one batched
    fp32 GEMM (``torch.bmm``, hipBLAS), a plain library product.
    """
    b, n = _check(h, tau)
    if not isinstance(c, torch.Tensor) or c.dtype != torch.float32 or c.device != h.device:
        raise TypeError("c must be a float32 tensor on h's device")
    if c.dim() != 3 or c.shape[0] != b or c.shape[1] != n:
        raise ValueError(f"c must have shape ({b}, {n}, k), got {tuple(c.shape)}")
    q = householder_product(h, tau)
    qm = q.transpose(-1, -2) if transpose else q
    return torch.bmm(qm.contiguous(), c.contiguous())
