"""CPU oracle of the mixed-precision blocked QR — TEST INFRASTRUCTURE ONLY.

Only tests/ may import this module, as the checker of
``fastqr.blocked_geqrf_mixed`` (the product path never imports it).

Restates the reference's prototype ``blocked_geqrf_reference``
(tools/blocked_qr_reference.py:193-262) in numpy float32:

* operand rounding of the update products (tools/blocked_qr_reference.py:34-50):
  ``tf32-input`` keeps 11 significant bits (frexp mantissa times 2048,
  rounded half to even), ``fp16-input`` a round trip through IEEE half;
  ``bf16-input`` (the gfx950 variant's extra mode) keeps 8 significant bits
  the same way as tf32;
* the three update forms — reflector by reflector
  (tools/blocked_qr_reference.py:55-67), the explicit panel transform
  (:70-84) and compact WY, T^T between V^T X and V (:87-122);
* the fp32 repairs: R rows of each panel rewritten from the input by the
  reflectors so far (:142-175), each panel recomputed from the input by the
  reflectors before it (:178-189).

Each panel is factored by ``torch.geqrf`` on CPU, the reference's own call
(tools/blocked_qr_reference.py:245).  ``mutation`` plants a mistake for the
tests: 1 = compact WY with T in place of T^T, 2 = the panel refresh drops the
last reflector before the panel, 3 = no operand rounding.
"""
from __future__ import annotations

import numpy as np

UPDATE_MODES = ("reflectors", "block-full", "compact-wy")
PRECISION_MODES = ("fp32", "tf32-input", "fp16-input", "bf16-input")
R_MAINTENANCE_MODES = ("none", "panel-prefix")
PANEL_REFRESH_MODES = ("none", "prefix")

_F32 = np.float32


def _keep_significant_bits(x: np.ndarray, scale: float) -> np.ndarray:
    mant, expo = np.frexp(np.asarray(x, dtype=_F32))  # mant in [0.5, 1)
    mant = np.round(mant * _F32(scale)) / _F32(scale)  # half to even
    return np.ldexp(mant, expo).astype(_F32)


def quantize_tf32(x) -> np.ndarray:
    """11 significant bits (10 stored), round half to even."""
    return _keep_significant_bits(x, 2048.0)


def quantize_bf16(x) -> np.ndarray:
    """8 significant bits (7 stored), round half to even."""
    return _keep_significant_bits(x, 256.0)


def round_operand(x, mode: str) -> np.ndarray:
    x = np.asarray(x, dtype=_F32)
    if mode == "fp32":
        return x
    if mode == "tf32-input":
        return quantize_tf32(x)
    if mode == "fp16-input":
        return x.astype(np.float16).astype(_F32)
    if mode == "bf16-input":
        return quantize_bf16(x)
    raise ValueError(f"precision_mode must be one of {PRECISION_MODES}, got {mode!r}")


def _mm(left, right, mode: str) -> np.ndarray:
    return np.matmul(round_operand(left, mode), round_operand(right, mode))


def _reflector(h: np.ndarray, j: int) -> np.ndarray:
    """v_j restricted to rows j.. of the panel: (1, h[j+1:, j]), batched."""
    v = h[:, j:, j].copy()
    v[:, 0] = 1.0
    return v


def panel_v(panel_h: np.ndarray) -> np.ndarray:
    """Unit lower-trapezoidal V of a factored panel (batch, rows, w)."""
    v = np.tril(panel_h, -1).astype(_F32)
    w = panel_h.shape[-1]
    v[:, np.arange(w), np.arange(w)] = 1.0
    return v


def compact_wy_t(v: np.ndarray, tau: np.ndarray) -> np.ndarray:
    """Upper-triangular T with H_0 H_1 ... H_{w-1} = I - V T V^T (forward, columnwise)."""
    b, _, w = v.shape
    t = np.zeros((b, w, w), dtype=_F32)
    for j in range(w):
        t[:, j, j] = tau[:, j]
        if j:
            y = -tau[:, j, None] * np.einsum("bri,br->bi", v[:, :, :j], v[:, :, j])
            t[:, :j, j] = np.einsum("bik,bk->bi", t[:, :j, :j], y)
    return t


def apply_reflectors(x: np.ndarray, panel_h: np.ndarray, panel_tau: np.ndarray, mode: str = "fp32") -> None:
    """x <- H_{w-1} ... H_0 x one reflector at a time (in place)."""
    for j in range(panel_h.shape[-1]):
        v = _reflector(panel_h, j)
        target = x[:, j:, :]
        dot = _mm(v[:, None, :], target, mode)[:, 0, :]
        tj = round_operand(panel_tau[:, j], mode)[:, None, None]
        target -= (tj * round_operand(v, mode)[:, :, None]) * round_operand(dot, mode)[:, None, :]


def apply_block_full(x: np.ndarray, panel_h: np.ndarray, panel_tau: np.ndarray, mode: str = "fp32") -> None:
    b, rows, _ = panel_h.shape
    transform = np.broadcast_to(np.eye(rows, dtype=_F32), (b, rows, rows)).copy()
    apply_reflectors(transform, panel_h, panel_tau)  # fp32
    x[...] = _mm(transform, x, mode)


def apply_compact_wy(x: np.ndarray, panel_h: np.ndarray, panel_tau: np.ndarray, mode: str = "fp32",
                     mutation: int = 0) -> None:
    """x <- x - V (T^T (V^T x)), every product on rounded operands (in place)."""
    v = panel_v(panel_h)
    t = compact_wy_t(v, panel_tau)
    if mutation == 3:
        mode = "fp32"
    vt = np.swapaxes(v, 1, 2)
    proj = _mm(vt, x, mode)
    tt = t if mutation == 1 else np.swapaxes(t, 1, 2)
    mid = _mm(tt, proj, mode)
    x -= _mm(v, mid, mode)


def apply_prefix(target: np.ndarray, h: np.ndarray, tau: np.ndarray, ncols: int) -> None:
    """target <- H_{ncols-1} ... H_0 target in fp32, reflectors from the columns of h (in place)."""
    for j in range(ncols):
        v = _reflector(h, j)
        sub = target[:, j:, :]
        dot = np.einsum("br,brc->bc", v, sub)
        sub -= (tau[:, j, None, None] * v[:, :, None]) * dot[:, None, :]


def refresh_panel(work, tau, original, k: int, w: int, mutation: int = 0) -> None:
    if k == 0:
        return
    fresh = original[:, :, k:k + w].copy()
    apply_prefix(fresh, work, tau, k - 1 if mutation == 2 else k)
    work[:, k:, k:k + w] = fresh[:, k:, :]


def repair_panel_r(work, tau, original, k: int, w: int) -> None:
    n = work.shape[-1]
    proj = original[:, :, k:].copy()
    apply_prefix(proj, work, tau, k + w)
    for lc in range(w):
        c = k + lc
        work[:, k:c + 1, c] = proj[:, k:c + 1, lc]
    if k + w < n:
        work[:, k:k + w, k + w:] = proj[:, k:k + w, w:]


def _geqrf_panel(panel: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    import torch

    h, t = torch.geqrf(torch.from_numpy(np.ascontiguousarray(panel, dtype=_F32)))
    return h.numpy(), t.numpy()


def blocked_geqrf_mixed(a, panel_width: int = 32, update_mode: str = "reflectors", precision_mode: str = "fp32",
                        r_maintenance_mode: str = "none", panel_refresh_mode: str = "none",
                        mutation: int = 0) -> tuple[np.ndarray, np.ndarray]:
    """(H, tau) as numpy float32 arrays (batch, n, n) / (batch, n), geqrf convention."""
    if panel_width <= 0:
        raise ValueError("panel_width must be positive")
    if update_mode not in UPDATE_MODES:
        raise ValueError(f"update_mode must be one of {UPDATE_MODES}, got {update_mode!r}")
    if precision_mode not in PRECISION_MODES:
        raise ValueError(f"precision_mode must be one of {PRECISION_MODES}, got {precision_mode!r}")
    if r_maintenance_mode not in R_MAINTENANCE_MODES:
        raise ValueError(f"r_maintenance_mode must be one of {R_MAINTENANCE_MODES}, got {r_maintenance_mode!r}")
    if panel_refresh_mode not in PANEL_REFRESH_MODES:
        raise ValueError(f"panel_refresh_mode must be one of {PANEL_REFRESH_MODES}, got {panel_refresh_mode!r}")
    try:
        import torch

        if isinstance(a, torch.Tensor):
            a = a.detach().cpu().numpy()
    except ImportError:  # pragma: no cover
        pass
    a = np.array(a, dtype=_F32)
    if a.ndim != 3 or a.shape[1] != a.shape[2]:
        raise ValueError("data must be a float32 array with shape (batch, n, n)")
    b, n, _ = a.shape
    work = a.copy()
    tau = np.zeros((b, n), dtype=_F32)
    for k in range(0, n, panel_width):
        w = min(panel_width, n - k)
        if panel_refresh_mode == "prefix":
            refresh_panel(work, tau, a, k, w, mutation)
        ph, pt = _geqrf_panel(work[:, k:, k:k + w])
        work[:, k:, k:k + w] = ph
        tau[:, k:k + w] = pt
        if k + w < n:
            x = work[:, k:, k + w:]
            if update_mode == "reflectors":
                apply_reflectors(x, ph, pt, "fp32" if mutation == 3 else precision_mode)
            elif update_mode == "block-full":
                apply_block_full(x, ph, pt, "fp32" if mutation == 3 else precision_mode)
            else:
                apply_compact_wy(x, ph, pt, precision_mode, mutation)
        if r_maintenance_mode == "panel-prefix":
            repair_panel_r(work, tau, a, k, w)
    return work, tau
