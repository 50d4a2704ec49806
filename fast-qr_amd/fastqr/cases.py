"""The official task's input profiles and case lists.

Restates the evaluator's input generator, official/reference.py:8-142
(``generate_input``, ``_apply_case``, ``_generate_mixed``), for the nine
conditioning profiles the task defines (dense, upper, diagonal, rankdef,
nearrank, clustered, band, nearcollinear, rowscale) and the heterogeneous
``mixed`` batch, plus the 22 test and 12 benchmark specs of
official/task.yml:85-121.

Draw order matters for reproducibility: the base Gaussian batch is drawn first,
then each profile's extra randomness, and for ``mixed`` the per-matrix labels
followed by the profiles in their fixed order -- the order of the reference.
The reference draws on the CUDA device when one is present
(official/reference.py:130-131), so its bytes depend on the device RNG; here
the generator runs on the CPU by default, which makes the bytes identical on
every host (the same fp32 tensor then goes to the GPU path and to CPU
torch.geqrf).  ``device="cuda"`` draws on the GPU as the reference does.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

EPS32 = float(torch.finfo(torch.float32).eps)

# official/reference.py:24-27: profiles of a mixed batch and their weights
# (dense about half of the matrices).
MIXED_PROFILES = ("dense", "rankdef", "nearrank", "clustered", "band", "rowscale", "nearcollinear")
MIXED_WEIGHTS = (6.0, 1.0, 1.0, 1.0, 1.0, 1.0, 1.0)
PROFILES = MIXED_PROFILES + ("upper", "diagonal")


@dataclass(frozen=True)
class Case:
    batch: int
    n: int
    cond: int
    seed: int
    case: str = "dense"

    @property
    def label(self) -> str:
        return f"{self.case}-{self.batch}x{self.n}-c{self.cond}-s{self.seed}"


# official/task.yml:85-107
TESTS: tuple[Case, ...] = (
    Case(20, 32, 1, 53124), Case(40, 176, 1, 3321), Case(40, 352, 1, 1200),
    Case(16, 512, 2, 32523), Case(4, 1024, 2, 4327), Case(1, 4096, 1, 75342),
    Case(16, 512, 4, 32524, "dense"), Case(16, 512, 0, 32525, "rankdef"),
    Case(16, 512, 0, 32526, "clustered"), Case(16, 512, 0, 32527, "band"),
    Case(16, 512, 0, 32528, "rowscale"), Case(16, 512, 0, 32529, "nearcollinear"),
    Case(4, 1024, 4, 4328, "dense"), Case(4, 1024, 0, 4329, "rankdef"),
    Case(4, 1024, 0, 4330, "nearrank"), Case(4, 1024, 0, 4331, "clustered"),
    Case(2, 2048, 2, 224466, "dense"), Case(2, 2048, 0, 224467, "rankdef"),
    Case(1, 4096, 0, 75343, "upper"), Case(16, 512, 2, 32530, "mixed"),
    Case(4, 1024, 2, 4332, "mixed"), Case(2, 2048, 2, 224468, "mixed"),
)

# official/task.yml:109-121
BENCHMARKS: tuple[Case, ...] = (
    Case(20, 32, 1, 43214), Case(40, 176, 1, 423011), Case(40, 352, 1, 123456),
    Case(640, 512, 2, 1029), Case(60, 1024, 2, 75342), Case(8, 2048, 1, 224466),
    Case(2, 4096, 1, 32412), Case(640, 512, 2, 770001, "mixed"),
    Case(60, 1024, 2, 770002, "mixed"), Case(640, 512, 0, 770003, "rankdef"),
    Case(640, 512, 0, 770004, "clustered"), Case(60, 1024, 0, 770005, "nearrank"),
)


def column_scaling(a: torch.Tensor, cond: int) -> torch.Tensor:
    """Columns times logspace(0, -cond, n) (official/reference.py:9-15)."""
    if not cond:
        return a.contiguous()
    n = a.shape[-1]
    return a * torch.logspace(0.0, -float(cond), n, device=a.device, dtype=torch.float32)


def band_mask(n: int, bandwidth: int, device) -> torch.Tensor:
    """|i - j| <= bandwidth (official/reference.py:18-20)."""
    i = torch.arange(n, device=device)
    return (i[:, None] - i[None, :]).abs() <= bandwidth


def apply_profile(a: torch.Tensor, case: str, cond: int, gen: torch.Generator) -> torch.Tensor:
    """One conditioning profile on a drawn base batch (official/reference.py:30-98)."""
    m, n = a.shape[0], a.shape[-1]
    dev = a.device
    f32 = torch.float32
    if case == "dense":
        return column_scaling(a, cond)
    if case == "upper":
        a = torch.triu(a)
        a.diagonal(dim1=-2, dim2=-1).add_(torch.linspace(1.0, 0.25, n, device=dev, dtype=f32))
        return column_scaling(a, cond)
    if case == "diagonal":
        d = torch.randn((m, n), device=dev, dtype=f32, generator=gen)
        signs = d.sign().clamp(min=0.0).mul(2.0).sub(1.0)
        return torch.diag_embed(signs * torch.logspace(0.0, -float(max(cond, 2)), n, device=dev, dtype=f32))
    if case == "rankdef":
        rank = max(1, (3 * n) // 4)
        a[:, :, rank:] = 0.0
        return column_scaling(a, cond)
    if case == "nearrank":
        rank = max(1, (3 * n) // 4)
        tail = n - rank
        if tail > 0:
            noise = torch.randn((m, n, tail), device=dev, dtype=f32, generator=gen)
            a[:, :, rank:] = a[:, :, :tail] + 1.0e-5 * noise
        return column_scaling(a, cond)
    if case == "clustered":
        s = torch.ones((n,), device=dev, dtype=f32)
        s[n // 2:] = 4.0 * EPS32
        if n >= 8:
            s[max(0, n // 2 - 2):min(n, n // 2 + 2)] = torch.sqrt(torch.tensor(EPS32, device=dev))
        return a * s
    if case == "band":
        a = a * band_mask(n, max(2, min(32, n // 32)), dev)
        a.diagonal(dim1=-2, dim2=-1).add_(torch.linspace(1.0, 0.5, n, device=dev, dtype=f32))
        return column_scaling(a, cond)
    if case == "nearcollinear":
        base = torch.randn((m, n, 1), device=dev, dtype=f32, generator=gen)
        noise = torch.randn((m, n, n), device=dev, dtype=f32, generator=gen)
        return column_scaling(base.expand(m, n, n) + 1.0e-4 * noise, cond)
    if case == "rowscale":
        s = torch.logspace(0.0, -float(max(cond, 4)), n, device=dev, dtype=f32)
        return s.reshape(1, n, 1) * a
    raise ValueError(f"unknown QR test case: {case}")


def mixed_labels(m: int, gen: torch.Generator, device) -> torch.Tensor:
    """Per-matrix profile indices of a mixed batch (official/reference.py:112-121)."""
    w = torch.tensor(MIXED_WEIGHTS, dtype=torch.float32, device=device)
    labels = torch.multinomial(w, m, replacement=True, generator=gen)
    if m >= 2:
        dense = labels == 0
        if not bool(dense.any()):
            labels[int(torch.randint(0, m, (1,), device=device, generator=gen))] = 0
        elif bool(dense.all()):
            pos = int(torch.randint(0, m, (1,), device=device, generator=gen))
            labels[pos] = int(torch.randint(1, len(MIXED_PROFILES), (1,), device=device, generator=gen))
    return labels


def generate_mixed(a: torch.Tensor, cond: int, gen: torch.Generator) -> tuple[torch.Tensor, torch.Tensor]:
    """Heterogeneous batch (official/reference.py:101-125); returns (batch, labels)."""
    labels = mixed_labels(a.shape[0], gen, a.device)
    for k, prof in enumerate(MIXED_PROFILES):
        sel = labels == k
        if bool(sel.any()):
            a[sel] = apply_profile(a[sel], prof, cond, gen)
    return a, labels


def generate(c: Case, device: str = "cpu") -> torch.Tensor:
    """Row-major contiguous (batch, n, n) fp32 input of a case
    (official/reference.py:128-142)."""
    if c.batch <= 0 or c.n <= 0 or c.cond < 0:
        raise ValueError(f"invalid case {c}")
    gen = torch.Generator(device=device)
    gen.manual_seed(c.seed)
    case = c.case.lower()
    a = torch.randn((c.batch, c.n, c.n), device=device, dtype=torch.float32, generator=gen)
    if case == "mixed":
        a, _ = generate_mixed(a, c.cond, gen)
    else:
        a = apply_profile(a, case, c.cond, gen)
    return a.contiguous()


def labels_of(c: Case, device: str = "cpu") -> list[str]:
    """Profile name of each matrix of a case (same draws as ``generate``)."""
    if c.case.lower() != "mixed":
        return [c.case.lower()] * c.batch
    gen = torch.Generator(device=device)
    gen.manual_seed(c.seed)
    torch.randn((c.batch, c.n, c.n), device=device, dtype=torch.float32, generator=gen)
    return [MIXED_PROFILES[i] for i in mixed_labels(c.batch, gen, device).tolist()]
