"""CPU tests of the official case generator (fastqr.cases).

Each profile of official/reference.py:30-98 is pinned by the structure it must
produce, checked against the plain Gaussian base batch the same seed draws
first; the mixed batch by its label rules (official/reference.py:101-125).
The exact random stream of the reference (its draw order) is not pinned by
these properties: the reference module cannot be imported on this Python
(official/task.py needs typing.NotRequired, Python 3.11).
"""
import math

import pytest
import torch

from fastqr import cases
from fastqr.cases import Case


def base(c: Case) -> torch.Tensor:
    g = torch.Generator().manual_seed(c.seed)
    return torch.randn((c.batch, c.n, c.n), generator=g, dtype=torch.float32)


def test_case_lists_match_task_yml_counts():
    assert len(cases.TESTS) == 22 and len(cases.BENCHMARKS) == 12
    # the benchmark list holds the five ranked shapes and four structured batches
    shapes = {(c.batch, c.n) for c in cases.BENCHMARKS}
    assert shapes == {(20, 32), (40, 176), (40, 352), (640, 512), (60, 1024), (8, 2048), (2, 4096)}
    assert {c.case for c in cases.TESTS} == set(cases.PROFILES) - {"diagonal"} | {"mixed"}


@pytest.mark.parametrize("cond", [0, 1, 3])
def test_dense_scales_columns_by_logspace(cond):
    c = Case(3, 12, cond, 77)
    a = cases.generate(c)
    s = torch.logspace(0.0, -float(cond), 12) if cond else torch.ones(12)
    torch.testing.assert_close(a, base(c) * s, rtol=0, atol=0)


def test_upper_is_triangular_with_boosted_diagonal():
    c = Case(2, 10, 0, 5, "upper")
    a = cases.generate(c)
    assert torch.equal(a, torch.triu(a))
    expect = torch.triu(base(c))
    expect.diagonal(dim1=-2, dim2=-1).add_(torch.linspace(1.0, 0.25, 10))
    assert torch.equal(a, expect)


def test_diagonal_has_signed_logspace_entries():
    c = Case(3, 9, 1, 8, "diagonal")
    a = cases.generate(c)
    assert torch.equal(a, torch.diag_embed(torch.diagonal(a, dim1=-2, dim2=-1)))
    mag = torch.logspace(0.0, -2.0, 9)  # cond raised to at least 2
    torch.testing.assert_close(torch.diagonal(a, dim1=-2, dim2=-1).abs(), mag.expand(3, 9), rtol=0, atol=0)


@pytest.mark.parametrize("n", [1, 4, 16])
def test_rankdef_zeroes_trailing_quarter(n):
    c = Case(2, n, 0, 9, "rankdef")
    a = cases.generate(c)
    rank = max(1, (3 * n) // 4)
    assert torch.count_nonzero(a[:, :, rank:]) == 0
    assert torch.equal(a[:, :, :rank], base(c)[:, :, :rank])


def test_nearrank_tail_copies_leading_columns_plus_small_noise():
    c = Case(2, 16, 0, 10, "nearrank")
    a = cases.generate(c)
    d = a[:, :, 12:] - a[:, :, :4]
    assert 0 < float(d.abs().max()) < 1e-4
    assert torch.equal(a[:, :, :12], base(c)[:, :, :12])


@pytest.mark.parametrize("n", [6, 16])
def test_clustered_column_scales(n):
    c = Case(2, n, 0, 11, "clustered")
    a = cases.generate(c)
    s = torch.ones(n)
    s[n // 2:] = 4.0 * cases.EPS32
    if n >= 8:
        s[n // 2 - 2:n // 2 + 2] = math.sqrt(cases.EPS32)
    torch.testing.assert_close(a, base(c) * s, rtol=0, atol=0)


def test_band_is_zero_outside_band():
    n = 128
    c = Case(2, n, 1, 12, "band")
    a = cases.generate(c)
    bw = max(2, min(32, n // 32))
    i = torch.arange(n)
    outside = (i[:, None] - i[None, :]).abs() > bw
    assert torch.count_nonzero(a[:, outside]) == 0
    assert torch.count_nonzero(a[:, ~outside]) == a[:, ~outside].numel()


def test_nearcollinear_columns_are_close():
    c = Case(2, 12, 0, 13, "nearcollinear")
    a = cases.generate(c)
    spread = (a - a[:, :, :1]).abs().max()
    assert 0 < float(spread) < 1e-2
    assert float(a[:, :, 0].abs().max()) > 1e-2


def test_rowscale_scales_rows():
    c = Case(2, 10, 0, 14, "rowscale")
    a = cases.generate(c)
    s = torch.logspace(0.0, -4.0, 10).reshape(1, 10, 1)
    torch.testing.assert_close(a, s * base(c), rtol=0, atol=0)


@pytest.mark.parametrize("batch", [1, 2, 7, 40])
def test_mixed_labels_and_profiles(batch):
    c = Case(batch, 16, 2, 1000 + batch, "mixed")
    a = cases.generate(c)
    labels = cases.labels_of(c)
    assert len(labels) == batch
    if batch >= 2:
        assert "dense" in labels and any(x != "dense" for x in labels)
    b0 = base(c)
    s = torch.logspace(0.0, -2.0, 16)
    for i, lab in enumerate(labels):
        if lab == "dense":
            assert torch.equal(a[i], b0[i] * s)
        elif lab == "rankdef":
            assert torch.count_nonzero(a[i, :, 12:]) == 0
        elif lab == "band":
            idx = torch.arange(16)
            assert torch.count_nonzero(a[i][(idx[:, None] - idx[None, :]).abs() > 2]) == 0
    assert cases.generate(c).equal(a)  # deterministic


def test_invalid_case_rejected():
    with pytest.raises(ValueError):
        cases.generate(Case(1, 4, 0, 1, "nosuch"))
    with pytest.raises(ValueError):
        cases.generate(Case(0, 4, 0, 1))
