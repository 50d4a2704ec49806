"""Writes the golden fixtures used by tests/test_oracle.py and the GPU tests.

Inputs are seeded fp32 matrices; expected outputs come from the reference's
own path, torch.geqrf on CPU (official/reference.py:145-147), and from scipy's
LAPACK sgeqrf as a second, independent LAPACK.  Run from the repository root:

    python tests/golden/make_golden.py
"""
from pathlib import Path

import numpy as np
import scipy.linalg.lapack as lapack
import torch

HERE = Path(__file__).resolve().parent


def case(name, a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    h, tau = torch.geqrf(torch.from_numpy(a))
    hs = np.empty_like(a)
    ts = np.empty(a.shape[:2], dtype=np.float32)
    for i in range(a.shape[0]):
        qr, t, _, info = lapack.sgeqrf(a[i])
        assert info == 0
        hs[i] = qr
        ts[i] = t
    np.savez_compressed(HERE / f"{name}.npz", a=a, h=h.numpy(), tau=tau.numpy(), h_scipy=hs, tau_scipy=ts)
    print(f"wrote {name}.npz  a{a.shape}")


def main():
    torch.set_num_threads(1)
    g = torch.Generator().manual_seed(20240601)
    case("gauss_20x32", torch.randn((20, 32, 32), generator=g).numpy())
    for n in (1, 2, 3, 4, 5, 8):
        case(f"gauss_6x{n}", torch.randn((6, n, n), generator=g).numpy())
    # structured 8x8 (rank-deficient: trailing columns copies of leading ones;
    # column-scaled; upper triangular)
    base = torch.randn((4, 8, 8), generator=g)
    rd = base.clone()
    rd[:, :, 6:] = rd[:, :, :2]
    case("rankdef_4x8", rd.numpy())
    scaled = base * torch.logspace(0.0, -4.0, 8)
    case("colscaled_4x8", scaled.numpy())
    case("upper_4x8", (torch.triu(base) + torch.eye(8)).numpy())


if __name__ == "__main__":
    main()
