"""GPU parity of the explicit Q (fastqr.householder_product, C ABI
fastqr_orgqr_f32) against the oracle: CPU torch.linalg.householder_product
in fp64 on the same (H, tau) -- the reference checker's own call
(official/reference.py:199) -- and, at the full benchmark sizes, against the
size-independent properties Q R = A and Q^T Q = I.

Tolerances (the build's stated fp32 gates): ||Q - Q_ref||_F <= 1e-5 n,
||Q^T Q - I||_F <= 1e-5 n, ||Q triu(H) - A||_F / ||A||_F <= 1e-5 n.
"""
import sys

import pytest
import torch

import fastqr
from fastqr import custom_kernel, inputs

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def gaussian(batch, n, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn((batch, n, n), generator=g, dtype=torch.float32)


def check_q(a_cpu, h, tau, q):
    n = a_cpu.shape[-1]
    hd, td, qd = h.cpu().double(), tau.cpu().double(), q.cpu().double()
    q_ref = torch.linalg.householder_product(hd, td)
    err = torch.linalg.matrix_norm(qd - q_ref).max().item()
    assert err <= 1e-5 * n, f"||Q - Q_ref||_F = {err:.3e} > {1e-5 * n:.1e}"
    eye = torch.eye(n, dtype=torch.float64)
    orth = torch.linalg.matrix_norm(qd.transpose(-1, -2) @ qd - eye).max().item()
    assert orth <= 1e-5 * n, f"||Q^T Q - I||_F = {orth:.3e}"
    rec = (torch.linalg.matrix_norm(qd @ torch.triu(hd) - a_cpu.double())
           / torch.linalg.matrix_norm(a_cpu.double()).clamp_min(1e-300)).max().item()
    assert rec <= 1e-5 * n, f"||QR - A||_F/||A||_F = {rec:.3e}"
    return err, orth, rec


# every path of the factorisation and of the Q update: one panel (n <= 32),
# ragged last panels, the strip-resident update, the row-split update (n > 2048)
@pytest.mark.parametrize("batch,n", [(5, 1), (5, 2), (4, 5), (4, 31), (4, 32), (3, 33), (3, 64), (3, 100),
                                     (3, 176), (3, 177), (2, 256), (3, 352), (2, 512), (2, 1000), (1, 2049),
                                     (1, 3000)])
def test_householder_product_matches_oracle(cuda, batch, n):
    _say(f"[orgqr] batch={batch} n={n}")
    a = gaussian(batch, n, 500 + n)
    h, tau = custom_kernel(a.to(cuda))
    q = fastqr.householder_product(h, tau)
    torch.cuda.synchronize()
    err, orth, rec = check_q(a, h, tau, q)
    _say(f"  ||Q-Qref||={err:.2e} ||QtQ-I||={orth:.2e} ||QR-A||/||A||={rec:.2e}")


# batches of 48 and more, and tall matrices in batches of 16 or fewer, share one
# update per four panels: full groups, a
# ragged last group (n not a multiple of 128), a last panel narrower than 32;
# from batch 256 on the group's narrow updates are left-looking (a last
# column block of one column, a ragged last group)
@pytest.mark.parametrize("batch,n", [(48, 300), (50, 97), (64, 33), (48, 129), (49, 520), (16, 1057), (3, 1100),
                                     (256, 97), (300, 200), (260, 300)])
def test_grouped_panels_match_oracle(cuda, batch, n):
    _say(f"[orgqr grouped] batch={batch} n={n}")
    a = gaussian(batch, n, 900 + n)
    h, tau = custom_kernel(a.to(cuda))
    q = fastqr.householder_product(h, tau)
    torch.cuda.synchronize()
    err, orth, rec = check_q(a, h, tau, q)
    _say(f"  ||Q-Qref||={err:.2e} ||QtQ-I||={orth:.2e} ||QR-A||/||A||={rec:.2e}")
    # the same factors one matrix at a time take the ungrouped path: same Q up to rounding
    q1 = fastqr.householder_product(h[:1].contiguous(), tau[:1].contiguous())
    torch.cuda.synchronize()
    assert torch.linalg.matrix_norm((q1 - q[:1]).double()).max().item() <= 1e-5 * n


@pytest.mark.parametrize("n", [24, 100, 200])
def test_in_place_and_strided_factors_give_identical_q(cuda, n):
    a = gaussian(3, n, 7).to(cuda)
    h, tau = custom_kernel(a)
    q = fastqr.householder_product(h, tau)
    hr = h.contiguous()  # row-major copy of the factors: any H strides are read
    q_rm = fastqr.householder_product(hr, tau)
    hi = h.clone()
    q_in = fastqr.householder_product(hi, tau, out=hi)  # formed in place over the factors
    torch.cuda.synchronize()
    assert q_in.data_ptr() == hi.data_ptr()
    assert torch.equal(q, q_rm) and torch.equal(q, q_in)


@pytest.mark.parametrize("n", [20, 90, 300])
def test_zero_tau_gives_identity(cuda, n):
    h = gaussian(2, n, 9).to(cuda).transpose(-1, -2).contiguous().transpose(-1, -2)
    q = fastqr.householder_product(h, torch.zeros((2, n), device=cuda))
    torch.cuda.synchronize()
    assert torch.equal(q.cpu(), torch.eye(n).expand(2, n, n))


@pytest.mark.parametrize("name,idx", [("C3", 0), ("C4", 0), ("C5", 0), ("C5", 1)])
def test_full_workload_q_reconstructs_input(cuda, name, idx):
    shape = inputs.WORKLOADS[name][idx]
    _say(f"[orgqr full] {name} {shape.label}")
    a = inputs.generate(shape).to(cuda)
    h, tau = custom_kernel(a)
    q = fastqr.householder_product(h, tau)
    r = torch.triu(h).contiguous()
    n = shape.n
    rec = torch.linalg.matrix_norm(torch.bmm(q.contiguous(), r) - a) / torch.linalg.matrix_norm(a)
    eye = torch.eye(n, device=cuda)
    orth = torch.linalg.matrix_norm(torch.bmm(q.transpose(-1, -2).contiguous(), q.contiguous()) - eye)
    torch.cuda.synchronize()
    _say(f"  max ||QR-A||/||A||={rec.max().item():.2e} max ||QtQ-I||={orth.max().item():.2e}")
    assert rec.max().item() <= 1e-5 * n
    assert orth.max().item() <= 1e-5 * n


# Q C and Q^T C (torch.ormqr's meaning, fastqr.apply_q over the C ABI
# fastqr_ormqr_f32) against the oracle: CPU torch.ormqr in fp64 on the same
# factors; tolerance ||X - X_ref||_F <= 1e-5 n ||C||_F.  Square factors come
# from custom_kernel; rectangular (m x r) ones, as the reference's call on a
# leading column block (submissions/candidate.py:7231-7237), from CPU geqrf.
# The shapes cover one and several panel groups, r not a multiple of 32 (a
# partial last panel and group), k of 1 and not a multiple of 32, m not a
# multiple of 4 (element loads), and groups taller than 2048 rows (the
# row-split kernels with a group T, also in chunks of 4096 columns of C).
@pytest.mark.parametrize("batch,m,r,k,transpose", [
    (3, 20, 20, 5, False), (3, 100, 100, 100, True), (2, 600, 600, 7, True), (2, 600, 600, 7, False),
    (2, 512, 512, 512, False), (2, 512, 512, 512, True), (4, 300, 77, 45, False), (4, 300, 77, 45, True),
    (3, 333, 333, 1, True), (2, 333, 200, 70, False), (1, 2100, 2100, 33, True), (1, 2100, 2100, 33, False),
    (1, 4096, 4096, 40, False), (1, 4096, 4096, 40, True), (2, 3000, 200, 50, True), (2, 3000, 200, 50, False),
    (1, 2100, 64, 4200, True), (1, 2101, 70, 33, False)])
def test_apply_q_matches_ormqr(cuda, batch, m, r, k, transpose):
    _say(f"[apply_q] batch={batch} m={m} r={r} k={k} transpose={transpose}")
    g = torch.Generator().manual_seed(300 + m + r)
    cm = torch.randn((batch, m, k), generator=g, dtype=torch.float32)
    if r == m:
        h, tau = custom_kernel(gaussian(batch, m, 300 + m).to(cuda))
    else:
        h, tau = torch.geqrf(torch.randn((batch, m, r), generator=g, dtype=torch.float32))
        h, tau = h.to(cuda), tau.to(cuda)
    c_dev = cm.to(cuda)
    x = fastqr.apply_q(h, tau, c_dev, transpose=transpose)
    torch.cuda.synchronize()
    assert torch.equal(c_dev.cpu(), cm)  # C itself is not modified
    x_ref = torch.ormqr(h.cpu().double(), tau.cpu().double(), cm.double(), left=True, transpose=transpose)
    err = (torch.linalg.matrix_norm(x.cpu().double() - x_ref) / torch.linalg.matrix_norm(cm.double())).max().item()
    _say(f"  ||X - X_ref||_F / ||C||_F = {err:.2e}")
    assert err <= 1e-5 * m, f"||X - X_ref||_F / ||C||_F = {err:.3e}"
    # Q^T (Q C) = C and Q (Q^T C) = C
    back = fastqr.apply_q(h, tau, x, transpose=not transpose)
    torch.cuda.synchronize()
    assert (torch.linalg.matrix_norm((back.cpu() - cm).double()) /
            torch.linalg.matrix_norm(cm.double())).max().item() <= 1e-5 * m


def test_apply_q_equals_explicit_q_product(cuda):
    """Q C by the compact-WY path against the explicit Q (householder_product)
    times C in fp64: two different kernel paths over the same factors."""
    a = gaussian(4, 384, 77)
    h, tau = custom_kernel(a.to(cuda))
    c = torch.randn((4, 384, 96), generator=torch.Generator().manual_seed(78))
    x = fastqr.apply_q(h, tau, c.to(cuda))
    q = fastqr.householder_product(h, tau)
    torch.cuda.synchronize()
    ref = q.cpu().double() @ c.double()
    err = (torch.linalg.matrix_norm(x.cpu().double() - ref) / torch.linalg.matrix_norm(c.double())).max().item()
    assert err <= 1e-5 * 384, err


def test_ormqr_c_abi_with_padded_c(cuda):
    """fastqr_ormqr_f32 through ctypes on a C with padded columns (leading
    dimension m + 3: element loads) and a batch stride beyond one matrix;
    the padding is left untouched."""
    import ctypes

    b, m, k = 3, 200, 50
    a = gaussian(b, m, 91)
    h, tau = custom_kernel(a.to(cuda))
    ldc = m + 3
    cbuf = torch.randn((b, k + 1, ldc), generator=torch.Generator().manual_seed(92)).to(cuda)
    cview = cbuf[:, :k, :m].transpose(-1, -2)  # (b, m, k), strides (ldc*(k+1), 1, ldc)
    c_ref = torch.ormqr(h.cpu().double(), tau.cpu().double(), cview.cpu().double(), left=True, transpose=True)
    before = cbuf.cpu()
    lib = fastqr.cdll()
    nbytes = lib.fastqr_ormqr_workspace_bytes(b, m, m, k)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=cuda)
    torch.cuda.synchronize()
    rc = lib.fastqr_ormqr_f32(h.data_ptr(), b, m, m, *h.stride(), tau.data_ptr(), *tau.stride(), cview.data_ptr(), k,
                              *cview.stride(), 1, ws.data_ptr(), nbytes, 0)
    torch.cuda.synchronize()
    assert rc == 0, lib.fastqr_last_error()
    after = cbuf.cpu()
    err = (torch.linalg.matrix_norm(after[:, :k, :m].transpose(-1, -2).double() - c_ref) /
           torch.linalg.matrix_norm(before[:, :k, :m].double())).max().item()
    assert err <= 1e-5 * m, err
    assert torch.equal(after[:, :k, m:], before[:, :k, m:])  # row padding
    assert torch.equal(after[:, k:, :], before[:, k:, :])    # the extra column


def test_forced_error_in_householder_product_surfaces(cuda):
    h = torch.randn((2, 40, 40), device=cuda)
    tau = torch.zeros((2, 40), device=cuda)
    fastqr.cdll().fastqr_debug_force_error(-99)
    with pytest.raises(fastqr.FastQRError) as exc:
        fastqr.householder_product(h, tau)
    assert exc.value.code == -99
