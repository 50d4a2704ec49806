"""Seeded synthetic workloads for batched QR.

The five benchmark workloads are fixed here with one seed each.  All
matrices are drawn on the CPU from ``torch.Generator('cpu').manual_seed(seed)``;
structured matrices are built in fp64 and rounded to fp32, so the identical
fp32 bytes go to the GPU path and to CPU ``torch.geqrf``.

Structured families:
  * ``rankdef``  A = U diag(s) V^T, s_i = 1 for i < r, 0 otherwise (r = n/2).
  * ``clustered`` half the singular values at 1, half at 1e-6.
  * ``nearrank`` leading n - 256 singular values at 1, trailing 256 at 1e-7.
U and V are Haar-distributed: Q of a Gaussian matrix times diag(sign(diag R)).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class Shape:
    batch: int
    n: int
    mix: str = "dense"  # dense | c3mixed | c4mixed
    seed: int = 0

    @property
    def label(self) -> str:
        return f"{self.batch}x{self.n}" + ("" if self.mix == "dense" else f"-{self.mix}")


# One entry per benchmark workload; C2 and C5 hold two shapes each.
WORKLOADS: dict[str, tuple[Shape, ...]] = {
    "C1": (Shape(20, 32, "dense", 1001),),
    "C2": (Shape(40, 176, "dense", 2001), Shape(40, 352, "dense", 2002)),
    "C3": (Shape(640, 512, "c3mixed", 3001),),
    "C4": (Shape(60, 1024, "c4mixed", 4001),),
    "C5": (Shape(8, 2048, "dense", 5001), Shape(2, 4096, "dense", 5002)),
}


def haar(n: int, gen: torch.Generator, count: int = 1) -> torch.Tensor:
    """`count` Haar-distributed n x n orthogonal matrices in fp64."""
    g = torch.randn((count, n, n), generator=gen, dtype=torch.float64)
    q, r = torch.linalg.qr(g)
    d = torch.sign(torch.diagonal(r, dim1=-2, dim2=-1))
    d = torch.where(d == 0, torch.ones_like(d), d)
    return q * d.unsqueeze(-2)


def svd_structured(n: int, singular: torch.Tensor, gen: torch.Generator, count: int) -> torch.Tensor:
    """`count` matrices U diag(s) V^T with Haar U, V, returned in fp32."""
    out = torch.empty((count, n, n), dtype=torch.float32)
    chunk = 32
    for s0 in range(0, count, chunk):
        k = min(chunk, count - s0)
        u = haar(n, gen, k)
        v = haar(n, gen, k)
        out[s0 : s0 + k] = ((u * singular.reshape(1, 1, n)) @ v.transpose(-1, -2)).to(torch.float32)
    return out


def rankdef_singular(n: int, rank: int) -> torch.Tensor:
    s = torch.zeros(n, dtype=torch.float64)
    s[:rank] = 1.0
    return s


def clustered_singular(n: int, low: float = 1e-6) -> torch.Tensor:
    s = torch.ones(n, dtype=torch.float64)
    s[n // 2 :] = low
    return s


def nearrank_singular(n: int, tail: int = 256, low: float = 1e-7) -> torch.Tensor:
    s = torch.ones(n, dtype=torch.float64)
    s[n - min(tail, n) :] = low
    return s


def generate(shape: Shape, seed: int | None = None) -> torch.Tensor:
    """Row-major contiguous (batch, n, n) fp32 CPU tensor for a workload shape."""
    seed = shape.seed if seed is None else seed
    gen = torch.Generator("cpu").manual_seed(seed)
    b, n = shape.batch, shape.n
    a = torch.randn((b, n, n), generator=gen, dtype=torch.float32)
    if shape.mix == "dense":
        return a.contiguous()
    if shape.mix == "c3mixed":
        # exactly 50% N(0,1), 25% rank-deficient (s_i = 0 for i >= n/2),
        # 25% clustered (half at 1, half at 1e-6), at seeded positions.
        perm = torch.randperm(b, generator=gen)
        n_rd = b // 4
        n_cl = b // 4
        rd_idx = perm[:n_rd]
        cl_idx = perm[n_rd : n_rd + n_cl]
        a[rd_idx] = svd_structured(n, rankdef_singular(n, n // 2), gen, n_rd)
        a[cl_idx] = svd_structured(n, clustered_singular(n), gen, n_cl)
        return a.contiguous()
    if shape.mix == "c4mixed":
        # 75% N(0,1) plus 25% near-rank-deficient (trailing 256 singular values 1e-7).
        perm = torch.randperm(b, generator=gen)
        n_nr = b // 4
        nr_idx = perm[:n_nr]
        a[nr_idx] = svd_structured(n, nearrank_singular(n), gen, n_nr)
        return a.contiguous()
    raise ValueError(f"unknown mix {shape.mix!r}")


def structure_labels(shape: Shape, seed: int | None = None) -> list[str]:
    """Per-matrix family labels for a workload (same draw order as `generate`)."""
    seed = shape.seed if seed is None else seed
    gen = torch.Generator("cpu").manual_seed(seed)
    b, n = shape.batch, shape.n
    torch.randn((b, n, n), generator=gen, dtype=torch.float32)
    labels = ["dense"] * b
    if shape.mix == "c3mixed":
        perm = torch.randperm(b, generator=gen).tolist()
        for i in perm[: b // 4]:
            labels[i] = "rankdef"
        for i in perm[b // 4 : b // 2]:
            labels[i] = "clustered"
    elif shape.mix == "c4mixed":
        perm = torch.randperm(b, generator=gen).tolist()
        for i in perm[: b // 4]:
            labels[i] = "nearrank"
    return labels


def flops(batch: int, n: int) -> float:
    """4 n^3 / 3 per matrix (geqrf flop count for square matrices)."""
    return batch * 4.0 * n**3 / 3.0


def bytes_moved(batch: int, n: int) -> float:
    """Algorithmic HBM bytes: read A once, write H once, write tau."""
    return batch * (8.0 * n * n + 4.0 * n)
