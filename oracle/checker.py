"""Correctness gates for (H, tau) — TEST INFRASTRUCTURE ONLY.

Two families of gates:

1. ``official_check`` restates the reference evaluator's checker,
   official/reference.py:150-266 (``check_implementation``): Q is materialised
   with householder_product(H, tau), R = triu(H), and in fp64
     * per matrix  ||R - Q^T A||_1 <= 20 * n * eps32 * ||A||_1
       (official/reference.py:213-227)
     * max_b ||Q^T Q - I||_1 <= 100 * n * eps32 * ||I||_1
       (official/reference.py:229-244)
   plus the shape/dtype/finiteness checks (official/reference.py:168-179).
   The diagnostics (lower leakage, reconstruction) follow
   official/reference.py:246-265 and tools/diagnose.py:22-75.

2. ``frobenius_gates`` and ``rdiag_tau_agreement`` implement the stated
   acceptance tolerances for this build:
     ||QR - A||_F / ||A||_F <= 1e-5 * n
     ||Q^T Q - I||_F       <= 1e-5 * n
     |R_ii| and tau agree with CPU geqrf to 1e-4 relative (same sign of R_ii),
     compared on the columns whose |R_ii| lies above the rounding floor
     2 * sqrt(n) * eps32 * ||A||_2 / 1e-4 and whose fp32 reference is itself
     determined (see ``rdiag_tau_agreement``).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch

EPS32 = float(np.finfo(np.float32).eps)
FACTOR_RTOL_FACTOR = 20.0  # official/reference.py:5
ORTH_RTOL_FACTOR = 100.0  # official/reference.py:6


def _t(x) -> torch.Tensor:
    if isinstance(x, torch.Tensor):
        return x.detach().cpu()
    return torch.from_numpy(np.ascontiguousarray(x))


def _l1(x: torch.Tensor) -> torch.Tensor:
    return torch.linalg.matrix_norm(x.double(), ord=1, dim=(-2, -1))


def official_check(a, h, tau) -> tuple[bool, str]:
    """Restatement of official/reference.py:182-266 on CPU tensors."""
    a = _t(a)
    h = _t(h)
    tau = _t(tau)
    if a.ndim != 3:
        return False, "data must be (batch, n, n)"
    batch, n, _ = a.shape
    if tuple(h.shape) != (batch, n, n):
        return False, f"H shape must be {(batch, n, n)}, got {tuple(h.shape)}"
    if tuple(tau.shape) != (batch, n):
        return False, f"tau shape must be {(batch, n)}, got {tuple(tau.shape)}"
    if h.dtype != torch.float32 or tau.dtype != torch.float32:
        return False, "H and tau must be float32"
    if not torch.isfinite(h).all() or not torch.isfinite(tau).all():
        return False, "H or tau contains NaN or Inf"
    factor_rtol = FACTOR_RTOL_FACTOR * max(n, 1) * EPS32
    orth_rtol = ORTH_RTOL_FACTOR * max(n, 1) * EPS32

    q = torch.linalg.householder_product(h, tau)
    r = torch.triu(h)
    if not torch.isfinite(q).all():
        return False, "Q materialized from (H, tau) contains NaN or Inf"
    a64, q64, r64 = a.double(), q.double(), r.double()
    projected = q64.transpose(-1, -2) @ a64
    factor_residual = _l1(r64 - projected)
    factor_scale = _l1(a64)
    factor_allowed = factor_rtol * factor_scale
    factor_scaled = factor_residual / (EPS32 * max(n, 1) * factor_scale.clamp_min(1e-30))
    if bool((factor_residual > factor_allowed).any()):
        worst = int(factor_scaled.argmax())
        return False, (
            f"R - Q.T @ A is too large: matrix={worst}, residual={factor_residual[worst].item():.3g}, "
            f"allowed={factor_allowed[worst].item():.3g}, scaled={factor_scaled[worst].item():.3g}"
        )
    eye = torch.eye(n, dtype=torch.float64).expand(batch, n, n)
    orth_residual = _l1(q64.transpose(-1, -2) @ q64 - eye).amax()
    orth_allowed = orth_rtol * _l1(eye).amax()
    orth_scaled = orth_residual / (EPS32 * max(n, 1))
    if orth_residual.item() > orth_allowed.item():
        return False, (
            f"Q is not orthogonal enough: residual={orth_residual.item():.3g}, "
            f"allowed={orth_allowed.item():.3g}, scaled={orth_scaled.item():.3g}"
        )
    tri_scaled = _l1(torch.tril(projected, -1)).amax() / (EPS32 * max(n, 1) * _l1(a64).amax())
    recon_scaled = _l1(q64 @ r64 - a64).amax() / (EPS32 * max(n, 1) * _l1(a64).amax())
    return True, (
        f"scaled_factor_residual={factor_scaled.amax().item():.3g}; "
        f"scaled_reconstruction_residual={recon_scaled.item():.3g}; "
        f"scaled_triangular_residual={tri_scaled.item():.3g}; "
        f"scaled_orthogonality_residual={orth_scaled.item():.3g}; batch={batch}; n={n}"
    )


def diagnose(a, h, tau) -> dict:
    """Scaled residuals of (H, tau), restating tools/diagnose.py:22-75.

    factor = ||R - Q^T A||_1, tri = ||tril(Q^T A, -1)||_1 and reconstruction
    = ||QR - A||_1, each over eps32 * n * ||A||_1; orth = ||Q^T Q - I||_1 over
    eps32 * n; the maximum over the batch of each.
    """
    a = _t(a)
    h = _t(h)
    tau = _t(tau)
    n = a.shape[-1]
    q64 = torch.linalg.householder_product(h, tau).double()
    r64 = torch.triu(h).double()
    a64 = a.double()
    projected = q64.transpose(-1, -2) @ a64
    scale = _l1(a64).clamp_min(1e-30) * EPS32 * n
    eye = torch.eye(n, dtype=torch.float64).expand_as(projected)
    return {
        "factor_scaled_max": float((_l1(r64 - projected) / scale).max()),
        "tri_scaled_max": float((_l1(torch.tril(projected, -1)) / scale).max()),
        "orth_scaled_max": float((_l1(q64.transpose(-1, -2) @ q64 - eye) / (EPS32 * n)).max()),
        "reconstruction_scaled_max": float((_l1(q64 @ r64 - a64) / scale).max()),
    }


@dataclass
class GateReport:
    ok: bool
    recon_rel_max: float
    orth_max: float
    recon_limit: float
    orth_limit: float
    per_matrix_recon: list = field(default_factory=list)

    def message(self) -> str:
        return (
            f"max ||QR-A||_F/||A||_F={self.recon_rel_max:.3e} (limit {self.recon_limit:.1e}); "
            f"max ||QtQ-I||_F={self.orth_max:.3e} (limit {self.orth_limit:.1e})"
        )


def frobenius_gates(a, h, tau, chunk: int = 8) -> GateReport:
    """||QR-A||_F/||A||_F <= 1e-5 n and ||Q^T Q - I||_F <= 1e-5 n per matrix, in fp64."""
    a = _t(a)
    h = _t(h)
    tau = _t(tau)
    batch, n, _ = a.shape
    limit = 1e-5 * n
    recon, orth = [], []
    for s in range(0, batch, chunk):
        hs, ts, as_ = h[s : s + chunk], tau[s : s + chunk], a[s : s + chunk]
        q = torch.linalg.householder_product(hs.double(), ts.double())
        r = torch.triu(hs.double())
        recon_err = torch.linalg.matrix_norm(q @ r - as_.double(), ord="fro", dim=(-2, -1))
        scale = torch.linalg.matrix_norm(as_.double(), ord="fro", dim=(-2, -1)).clamp_min(1e-300)
        recon.extend((recon_err / scale).tolist())
        eye = torch.eye(n, dtype=torch.float64)
        orth.extend(torch.linalg.matrix_norm(q.transpose(-1, -2) @ q - eye, ord="fro", dim=(-2, -1)).tolist())
    rmax = max(recon) if recon else 0.0
    omax = max(orth) if orth else 0.0
    ok = all(math.isfinite(x) for x in recon + orth) and rmax <= limit and omax <= limit
    return GateReport(ok, rmax, omax, limit, limit, recon)


@dataclass
class AgreementReport:
    ok: bool
    rdiag_rel_max: float
    tau_rel_max: float
    compared: int
    masked: int
    limit: float
    compared_per_matrix: list = field(default_factory=list)
    sign_flips: int = 0  # columns whose undetermined sign (alpha ~ 0) came out the other way
    r_only: int = 0  # compared columns after such a flip (|R_ii| compared, tau not)

    def compared_fraction(self, members=None) -> float:
        """Fraction of columns above the floor, over all matrices or `members`."""
        per = self.compared_per_matrix
        idx = range(len(per)) if members is None else members
        cols = (self.compared + self.masked) // max(len(per), 1)
        tot = sum(per[i] for i in idx)
        return tot / max(cols * len(list(idx)), 1)

    def message(self) -> str:
        flips = (f", {self.sign_flips} undetermined sign(s) taken the other way ({self.r_only} later columns "
                 f"compared by |R_ii| only)" if self.sign_flips else "")
        return (
            f"|R_ii| rel max={self.rdiag_rel_max:.3e}, tau rel max={self.tau_rel_max:.3e} "
            f"(limit {self.limit:.0e}) over {self.compared} columns, {self.masked} below the rounding floor"
            + flips
        )


def norm2_estimate(a: torch.Tensor, iters: int = 30) -> torch.Tensor:
    """Spectral-norm estimate per matrix by power iteration on A^T A (fp64)."""
    a = a.double()
    gen = torch.Generator().manual_seed(0)
    x = torch.randn(a.shape[0], a.shape[-1], 1, generator=gen, dtype=torch.float64)
    x = x / torch.linalg.vector_norm(x, dim=-2, keepdim=True)
    est = torch.zeros(a.shape[0], dtype=torch.float64)
    for _ in range(iters):
        y = a.transpose(-1, -2) @ (a @ x)
        nrm = torch.linalg.vector_norm(y, dim=-2, keepdim=True).clamp_min(1e-300)
        est = nrm.reshape(-1).sqrt()
        x = y / nrm
    return est


# Calibration of the floor (MKL fp32 geqrf against MKL fp64 geqrf, and the HIP
# path against both, on the benchmark inputs -- Gaussian n = 32..4096 and every
# structured family of the 640 x 512 and 60 x 1024 workloads -- and on the
# task's 22 test and 12 benchmark cases).  Above floor_factor = 1 one fp32 code
# stays within 3.0e-5 of fp64 on the benchmark inputs (clustered spectrum;
# Gaussian 1.9e-5), but the last columns of the banded test case reach 6.1e-4
# (MKL) and 1.2e-4 (HIP path, where MKL happens to be within 8e-6): their R_ii
# carry the rounding of every earlier step, about n eps32 ||A|| rather than
# sqrt(n) eps32 ||A||.  Hence floor_factor = 2 (the banded case's worst
# compared column then differs by 4.9e-5), and a column is compared only where
# the fp32 reference is itself determined to a quarter of the tolerance (fp32
# geqrf within DETERMINACY * rtol of fp64 geqrf on the same input).
DEFAULT_FLOOR_FACTOR = 2.0
DETERMINACY = 0.25
# alpha / beta below this many sqrt(n) eps32 has a sign set by rounding
SIGN_TOL_FACTOR = 8.0

# Minimum fraction of columns compared per structure family at these settings
# (observed on the benchmark workloads in brackets): Gaussian [1.000 at n = 32,
# 0.994 at 176, 0.991 at 352, 0.988 at 512, 0.977 at 1024, 0.955 at 2048,
# 0.910 at 4096]; the rank-deficient and clustered spectra compare their
# leading half [0.497], near-rank inputs their leading n - 256 columns [0.748
# at n = 1024].
MIN_COMPARED_FRACTION = {"dense": {32: 0.97, 176: 0.98, 352: 0.98, 512: 0.975, 1024: 0.96, 2048: 0.93, 4096: 0.88},
                         "rankdef": 0.45, "clustered": 0.45, "nearrank": 0.70}


def min_compared_fraction(family: str, n: int):
    """Expected minimum compared fraction for a family at size n, or None."""
    v = MIN_COMPARED_FRACTION.get(family)
    if isinstance(v, dict):
        return v.get(n)
    return v


def rdiag_tau_agreement(a, h, tau, h_ref, tau_ref, rtol: float = 1e-4,
                        floor_factor: float = DEFAULT_FLOOR_FACTOR,
                        determinacy: float | None = DETERMINACY) -> AgreementReport:
    """Compare |R_ii| and tau with a reference factorisation (CPU geqrf).

    Column i of matrix b is compared when
        |R_ii(ref)| > floor_factor * sqrt(n) * eps32 * ||A_b||_2 / rtol,
    i.e. where the rounding spread between two correct fp32 Householder codes
    (about sqrt(n) * eps32 * ||A||_2 in absolute terms) stays below rtol *
    |R_ii| (calibration above), and, with ``determinacy``, where the fp32
    reference agrees with fp64 geqrf of the same input to determinacy * rtol
    (its |R_ii| and tau are then fixed by the input, not by rounding).  Below
    the floor the R_ii of rank-deficient, clustered and near-rank inputs are
    rounding noise and their tau is arbitrary in [1, 2]; those columns are
    counted, not compared.  On compared columns the sign of R_ii must match
    (same LAPACK convention).
    """
    a = _t(a).double()
    h = _t(h).double()
    tau = _t(tau).double()
    h_ref = _t(h_ref).double()
    tau_ref = _t(tau_ref).double()
    batch, n, _ = a.shape
    d = torch.diagonal(h, dim1=-2, dim2=-1)
    dr = torch.diagonal(h_ref, dim1=-2, dim2=-1)
    a2 = norm2_estimate(a).reshape(batch, 1)
    floor = floor_factor * math.sqrt(max(n, 1)) * EPS32 * a2 / rtol
    mask = dr.abs() > floor
    h64, t64 = torch.geqrf(a)
    if determinacy is not None:
        d64 = torch.diagonal(h64, dim1=-2, dim2=-1).abs()
        fixed_r = (dr.abs() - d64).abs() <= determinacy * rtol * d64
        fixed_t = (tau_ref - t64).abs() <= determinacy * rtol * t64.abs()
        mask = mask & fixed_r & fixed_t
    # Undetermined signs: where alpha / beta = 1 - tau is below the rounding
    # level of alpha (SIGN_TOL_FACTOR sqrt(n) eps32, from fp64 geqrf), the
    # sign of alpha -- hence of beta = R_kk -- is decided by rounding, and a
    # correct fp32 code may pick either.  After such a column k picks the other
    # sign the factorisations go different ways: every later |R_jj| is still
    # the same (R is unique up to the signs of its rows), but the later tau and
    # reflectors are not.  Columns from k on keep the |R_jj| comparison only.
    undetermined = (1.0 - t64).abs() <= SIGN_TOL_FACTOR * math.sqrt(max(n, 1)) * EPS32
    flipped = undetermined & (torch.sign(d) != torch.sign(dr))
    after = torch.cumsum(flipped.to(torch.int64), dim=-1) > 0  # from the first flip on
    rel_r = (d.abs() - dr.abs()).abs() / dr.abs().clamp_min(1e-300)
    rel_t = (tau - tau_ref).abs() / tau_ref.abs().clamp_min(1e-300)
    sign_ok = bool(((torch.sign(d) == torch.sign(dr)) | ~mask | after).all())
    tmask = mask & ~after
    rmax = float(torch.where(mask, rel_r, torch.zeros_like(rel_r)).max()) if mask.any() else 0.0
    tmax = float(torch.where(tmask, rel_t, torch.zeros_like(rel_t)).max()) if tmask.any() else 0.0
    ok = sign_ok and rmax <= rtol and tmax <= rtol
    return AgreementReport(ok, rmax, tmax, int(mask.sum()), int((~mask).sum()), rtol, mask.sum(dim=-1).tolist(),
                           int(flipped.sum()), int((mask & after).sum()))
