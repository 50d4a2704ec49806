"""Blocked QR with a reduced-precision trailing update and fp32 repair.

An experimental variant kept apart from ``custom_kernel`` (whose every
product is fp32).  Same keyword interface as the reference's prototype
``blocked_geqrf_reference`` (tools/blocked_qr_reference.py:193-262):

* ``precision_mode`` rounds the operands of each trailing-update product
  (tools/blocked_qr_reference.py:34-50): ``"fp32"`` (none), ``"tf32-input"``
  (10 stored mantissa bits, nearest-even), ``"fp16-input"``; the gfx950 form
  adds ``"bf16-input"``.  fp16 and bf16 operands go through the matching
  MFMA instructions with fp32 accumulation; tf32 is rounded in registers and
  multiplied by the fp32 MFMA (gfx950 has no xf32 instruction).
* ``r_maintenance_mode="panel-prefix"`` rewrites each panel's finished R rows
  from the input by the reflectors so far, in fp32
  (tools/blocked_qr_reference.py:157-175).
* ``panel_refresh_mode="prefix"`` recomputes each panel from the input by the
  reflectors before it, in fp32, before factoring it
  (tools/blocked_qr_reference.py:178-189).

Only ``update_mode="compact-wy"`` (the block update the GPU kernels
implement) is offered, with panels of 16 or 32 columns, n <= 2048.  One call
into the C ABI (``fastqr_geqrf_mixed_f32``) on torch's current stream; no
fallback.
"""
from __future__ import annotations

import torch

from ._lib import (FASTQR_MIXED_PANEL_REFRESH, FASTQR_MIXED_R_MAINTENANCE, FASTQR_PREC_BF16_INPUT,
                   FASTQR_PREC_FP16_INPUT, FASTQR_PREC_FP32, FASTQR_PREC_TF32_INPUT, FastQRError, ext)
from .qr import _current_stream_ptr, _validate

UPDATE_MODES = ("compact-wy",)
PRECISION_MODES = ("fp32", "tf32-input", "fp16-input", "bf16-input")
R_MAINTENANCE_MODES = ("none", "panel-prefix")
PANEL_REFRESH_MODES = ("none", "prefix")
PANEL_WIDTHS = (16, 32)
MAX_N = 2048

_PREC = {
    "fp32": FASTQR_PREC_FP32,
    "tf32-input": FASTQR_PREC_TF32_INPUT,
    "fp16-input": FASTQR_PREC_FP16_INPUT,
    "bf16-input": FASTQR_PREC_BF16_INPUT,
}


def _flags(r_maintenance_mode: str, panel_refresh_mode: str) -> int:
    flags = 0
    if r_maintenance_mode == "panel-prefix":
        flags |= FASTQR_MIXED_R_MAINTENANCE
    if panel_refresh_mode == "prefix":
        flags |= FASTQR_MIXED_PANEL_REFRESH
    return flags


@torch.no_grad()
def blocked_geqrf_mixed(
    data: torch.Tensor,
    *,
    panel_width: int = 32,
    column_major_h: bool = True,
    update_mode: str = "compact-wy",
    precision_mode: str = "fp32",
    r_maintenance_mode: str = "none",
    panel_refresh_mode: str = "none",
) -> tuple[torch.Tensor, torch.Tensor]:
    """``(H, tau)`` of ``data`` (batch, n, n) fp32 on the GPU, geqrf convention.

    H is column-major (stride (n*n, 1, n)) unless ``column_major_h`` is False.
    """
    if panel_width <= 0:
        raise ValueError("panel_width must be positive")
    if panel_width not in PANEL_WIDTHS:
        raise ValueError(f"panel_width must be one of {PANEL_WIDTHS} on the GPU, got {panel_width}")
    if update_mode not in UPDATE_MODES:
        raise ValueError(f"update_mode must be one of {UPDATE_MODES} on the GPU, got {update_mode!r}")
    if precision_mode not in PRECISION_MODES:
        raise ValueError(f"precision_mode must be one of {PRECISION_MODES}, got {precision_mode!r}")
    if r_maintenance_mode not in R_MAINTENANCE_MODES:
        raise ValueError(
            f"r_maintenance_mode must be one of {R_MAINTENANCE_MODES}, got {r_maintenance_mode!r}"
        )
    if panel_refresh_mode not in PANEL_REFRESH_MODES:
        raise ValueError(f"panel_refresh_mode must be one of {PANEL_REFRESH_MODES}, got {panel_refresh_mode!r}")
    _validate(data)
    b, n, _ = data.shape
    if n > MAX_N:
        raise ValueError(f"n={n} exceeds the mixed-precision variant's maximum {MAX_N}")
    idx = data.get_device()
    if idx != torch.cuda.current_device():
        with torch.cuda.device(idx):
            return blocked_geqrf_mixed(data, panel_width=panel_width, column_major_h=column_major_h,
                                       update_mode=update_mode, precision_mode=precision_mode,
                                       r_maintenance_mode=r_maintenance_mode,
                                       panel_refresh_mode=panel_refresh_mode)
    h = torch.empty_strided((b, n, n), (n * n, 1, n), dtype=torch.float32, device=data.device)
    tau = torch.empty((b, n), dtype=torch.float32, device=data.device)
    if b == 0 or n == 0:
        return (h if column_major_h else h.contiguous()), tau
    flags = _flags(r_maintenance_mode, panel_refresh_mode)
    mod = ext()
    sptr = _current_stream_ptr(idx)
    nbytes = mod.geqrf_mixed_workspace_bytes(b, n, panel_width, flags)
    # per call, not the shared per-stream scratch: with R maintenance it holds
    # a copy of the whole batch, which should not stay cached
    ws = torch.empty(nbytes, dtype=torch.uint8, device=data.device)
    as0, as1, as2 = data.stride()
    rc = mod.geqrf_mixed(data.data_ptr(), b, n, as0, as1, as2, h.data_ptr(), n * n, 1, n, tau.data_ptr(), n, 1,
                         panel_width, _PREC[precision_mode], flags, ws.data_ptr(), ws.numel(), sptr)
    if rc != 0:
        raise FastQRError(rc, mod.last_error())
    return (h if column_major_h else h.contiguous()), tau
