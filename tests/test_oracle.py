"""Pins the CPU oracle (oracle/hhqr.c, oracle/checker.py) before it is trusted.

Checks, each chosen so a plausible mistake (sign, index, transposed operand,
dropped term) fails at least one:
  * golden vectors from torch.geqrf (the reference's own path) and scipy's
    LAPACK sgeqrf, tests/golden/*.npz;
  * closed forms: the slarfg reflector, n = 1, the 2x2 factorisation;
  * known answers: upper-triangular input -> tau == 0 and H == A bit-exact
    (tests/test_qr_smoke.py:8078-8085 of the reference), zero matrix, a column
    already zero below the diagonal;
  * invariants: Q R = A and Q^T Q = I through the official checker
    (official/reference.py:182-266) and its diagnostics bounds
    (tests/test_qr_smoke.py:192-200);
  * compact WY: I - V T V^T equals the product of the reflectors, and the
    blocked factorisation equals the unblocked one within 2e-5
    (the pattern of tests/test_qr_smoke.py:261-276);
  * planted mistakes in the oracle (mutation flags) are caught.
"""
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import checker, oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLDEN / f"{name}.npz") as z:
        return {k: z[k] for k in z.files}


GOLDEN_CASES = ["gauss_20x32", "gauss_6x1", "gauss_6x2", "gauss_6x3", "gauss_6x4", "gauss_6x5", "gauss_6x8",
                "rankdef_4x8", "colscaled_4x8", "upper_4x8"]


@pytest.mark.parametrize("name", GOLDEN_CASES)
def test_golden_lapack_vectors_agree_with_each_other(name):
    g = load(name)
    # torch.geqrf (MKL) and scipy sgeqrf are two LAPACKs: they agree on R diag / tau
    ag = checker.rdiag_tau_agreement(g["a"], g["h_scipy"], g["tau_scipy"], g["h"], g["tau"])
    assert ag.ok, ag.message()


@pytest.mark.parametrize("name", GOLDEN_CASES)
def test_restated_oracle_matches_golden(name):
    g = load(name)
    h, tau = oracle.geqrf_restated(g["a"])
    ok, msg = checker.official_check(g["a"], h, tau)
    assert ok, msg
    ag = checker.rdiag_tau_agreement(g["a"], h, tau, g["h"], g["tau"])
    assert ag.ok, ag.message()
    # well-conditioned columns: the whole compact factor matches LAPACK closely
    if name.startswith("gauss"):
        np.testing.assert_allclose(h, g["h"], rtol=0, atol=2e-4 * np.abs(g["h"]).max())
        np.testing.assert_allclose(tau, g["tau"], rtol=0, atol=2e-5)


def test_reflector_closed_forms():
    # slarfg: beta = -sign(alpha) ||(alpha, x)||, tau = (beta - alpha) / beta
    beta, tau, denom, active = oracle.reflector(3.0, 16.0)
    assert active and beta == -5.0 and tau == pytest.approx(1.6) and denom == 8.0
    beta, tau, denom, active = oracle.reflector(-3.0, 16.0)
    assert active and beta == 5.0 and tau == pytest.approx(1.6) and denom == -8.0
    beta, tau, denom, active = oracle.reflector(0.0, 4.0)  # alpha = +0 takes beta <= 0
    assert active and beta == -2.0 and tau == 1.0 and denom == 2.0
    beta, tau, denom, active = oracle.reflector(-7.0, 0.0)  # sigma == 0: identity, beta = alpha
    assert not active and beta == -7.0 and tau == 0.0


def test_n1_is_identity_factorisation():
    a = np.array([[[2.5]], [[-1.0]], [[0.0]]], dtype=np.float32)
    h, tau = oracle.geqrf_restated(a)
    assert np.array_equal(h, a) and np.array_equal(tau, np.zeros((3, 1), np.float32))


def test_2x2_closed_form():
    a = np.array([[[3.0, 1.0], [4.0, 2.0]]], dtype=np.float32)
    h, tau = oracle.geqrf_restated(a)
    # alpha=3, x=4: beta=-5, tau=1.6, v1=4/8=0.5 ; R01 = 1 - tau*(1 + 0.5*2) = -2.2 ;
    # R11 = 2 - tau*0.5*(1 + 0.5*2) = 0.4 ; the last column has no reflector.
    np.testing.assert_allclose(h[0], [[-5.0, -2.2], [0.5, 0.4]], rtol=1e-6)
    np.testing.assert_allclose(tau[0], [1.6, 0.0], rtol=1e-6)
    ref_h, ref_tau = torch.geqrf(torch.from_numpy(a))
    np.testing.assert_allclose(h, ref_h.numpy(), rtol=1e-6)
    np.testing.assert_allclose(tau, ref_tau.numpy(), rtol=1e-6)


def test_upper_triangular_input_known_answer():
    g = load("upper_4x8")
    h, tau = oracle.geqrf_restated(g["a"])
    assert np.array_equal(tau, np.zeros_like(tau))
    assert np.array_equal(h, g["a"])
    assert np.array_equal(g["tau"], np.zeros_like(g["tau"]))  # LAPACK agrees


def test_zero_matrix_and_zero_subcolumn():
    h, tau = oracle.geqrf_restated(np.zeros((2, 5, 5), np.float32))
    assert not h.any() and not tau.any()
    a = np.random.default_rng(0).standard_normal((1, 5, 5)).astype(np.float32)
    a[0, 1:, 0] = 0.0  # column 0 already reduced
    h, tau = oracle.geqrf_restated(a)
    assert tau[0, 0] == 0.0 and h[0, 0, 0] == a[0, 0, 0]


def test_fp32_restatement_close_to_fp64_restatement():
    g = load("gauss_20x32")
    h32, t32 = oracle.geqrf_restated(g["a"])
    h64, t64 = oracle.geqrf_restated_f64(g["a"])
    ag = checker.rdiag_tau_agreement(g["a"], h32, t32, h64.astype(np.float32), t64.astype(np.float32))
    assert ag.ok, ag.message()


def _reflector_product(v_block, tau):
    m, nb = v_block.shape
    q = np.eye(m)
    for j in range(nb):
        v = np.zeros(m)
        v[j] = 1.0
        v[j + 1 :] = v_block[j + 1 :, j]
        q = q @ (np.eye(m) - tau[j] * np.outer(v, v))
    return q


def test_compact_wy_equals_reflector_product():
    g = load("gauss_6x8")
    h, tau = oracle.geqrf_restated(g["a"])
    for b in range(3):
        v_block = h[b].astype(np.float64)
        t = oracle.larft(h[b], tau[b]).astype(np.float64)
        m, nb = v_block.shape
        v = np.tril(v_block, -1) + np.eye(m, nb)
        wy = np.eye(m) - v @ t @ v.T
        np.testing.assert_allclose(wy, _reflector_product(v_block, tau[b]), atol=2e-6)
        assert np.allclose(np.tril(t, -1), 0.0)  # T is upper triangular
        np.testing.assert_allclose(np.diag(t), tau[b], rtol=1e-6)


@pytest.mark.parametrize("nb", [1, 3, 5, 8, 32])
def test_blocked_restatement_matches_unblocked(nb):
    # tools/blocked_qr_reference.py panel loop; tests/test_qr_smoke.py:203-214, 261-276
    a = torch.randn((3, 40, 40), generator=torch.Generator().manual_seed(nb)).numpy()
    hb, tb = oracle.geqrf_restated_blocked(a, nb)
    hu, tu = oracle.geqrf_restated(a)
    np.testing.assert_allclose(hb, hu, rtol=2e-5, atol=2e-5)
    np.testing.assert_allclose(tb, tu, rtol=2e-5, atol=2e-5)
    ok, msg = checker.official_check(a, hb, tb)
    assert ok, msg


def test_geqrf_passes_checker_with_diagnostic_bounds():
    g = load("gauss_20x32")
    ok, msg = checker.official_check(g["a"], g["h"], g["tau"])
    assert ok, msg
    fields = dict(kv.split("=") for kv in msg.split("; "))
    assert float(fields["scaled_factor_residual"]) < 20.0
    assert float(fields["scaled_orthogonality_residual"]) < 100.0
    assert checker.frobenius_gates(g["a"], g["h"], g["tau"]).ok


@pytest.mark.parametrize("mutation,kind", [(1, "agreement"), (2, "official"), (3, "official")])
def test_planted_mistakes_are_caught(mutation, kind):
    a = torch.randn((4, 24, 24), generator=torch.Generator().manual_seed(7)).numpy()
    if mutation == 1:
        # flipped beta sign: still a valid QR, but not LAPACK's factorisation
        h, tau = oracle.geqrf_restated(a, mutation=1)
        ref_h, ref_tau = torch.geqrf(torch.from_numpy(a))
        assert not checker.rdiag_tau_agreement(a, h, tau, ref_h, ref_tau).ok
    else:
        # T in place of T^T, or a dropped unit diagonal, in the trailing update
        h, tau = oracle.geqrf_restated_blocked(a, 4, mutation=mutation)
        ok, _ = checker.official_check(a, h, tau)
        assert not ok
        assert not checker.frobenius_gates(a, h, tau).ok


def test_checker_rejects_bad_outputs():
    g = load("gauss_6x8")
    a, h, tau = g["a"], g["h"].copy(), g["tau"].copy()
    assert not checker.official_check(a, h[:, :, :7], tau)[0]
    bad = tau.copy()
    bad[0, 0] = np.nan
    assert not checker.official_check(a, h, bad)[0]
    h2 = h.copy()
    h2[1, 3, 2] += 0.5  # corrupt a reflector entry
    assert not checker.official_check(a, h2, tau)[0]


def test_norm2_estimate_is_a_tight_lower_bound():
    # power iteration on A^T A approaches ||A||_2 from below: never above it,
    # within 3% after its 30 steps; exact for a rank-one matrix and for
    # U diag(s) V^T with a clear gap (||A||_2 = s_1)
    from fastqr import inputs

    gen = torch.Generator().manual_seed(11)
    mats = [torch.randn((3, 64, 64), generator=gen, dtype=torch.float64),
            torch.randn((2, 512, 512), generator=gen, dtype=torch.float64)]
    u = torch.randn((2, 40, 1), generator=gen, dtype=torch.float64)
    mats.append(u @ u.transpose(-1, -2))
    s = torch.linspace(1.0, 0.1, 96, dtype=torch.float64)
    s[0] = 7.0
    g32 = torch.Generator().manual_seed(12)
    mats.append(inputs.svd_structured(96, s, g32, 2).double())
    for a in mats:
        est = checker.norm2_estimate(a)
        true = torch.linalg.matrix_norm(a, ord=2)
        assert bool((est <= true * (1 + 1e-9)).all()), (est, true)
        assert bool((est >= 0.97 * true).all()), (est, true)
    assert torch.allclose(checker.norm2_estimate(mats[2]), torch.linalg.matrix_norm(mats[2], ord=2), rtol=1e-12)
    assert torch.allclose(checker.norm2_estimate(mats[3]), torch.full((2,), 7.0, dtype=torch.float64), rtol=1e-5)


def _other_sign_factorisation(a):
    """A valid Householder QR of one fp64 matrix that takes the other sign of
    beta in column 0 (beta = +sign(alpha) ||x||), then LAPACK geqrf on the
    trailing block: what a correct code produces when alpha ~ 0 rounds the
    other way."""
    n = a.shape[-1]
    x = a[:, 0].clone()
    alpha, sigma = x[0].item(), float((x[1:] ** 2).sum())
    beta = math.copysign(math.sqrt(alpha * alpha + sigma), alpha)  # LAPACK: -sign(alpha) ||x||
    tau0 = (beta - alpha) / beta
    v = x / (alpha - beta)
    v[0] = 1.0
    b = a - tau0 * torch.outer(v, v @ a)
    h2, t2 = torch.geqrf(b[1:, 1:])
    h = b.clone()
    h[1:, 0] = v[1:]
    h[0, 0] = beta
    h[1:, 1:] = h2
    tau = torch.cat([torch.tensor([tau0], dtype=a.dtype), t2])
    return h, tau


@pytest.mark.parametrize("ratio,flip_allowed", [(1e-9, True), (0.3, False)])
def test_undetermined_sign_is_accepted_only_where_alpha_vanishes(ratio, flip_allowed):
    # column 0 with alpha / ||x|| = ratio: at 1e-9 its sign is rounding noise
    # and the other-sign factorisation must pass (later columns compared by
    # |R_jj| only); at 0.3 the sign is determined and the same construction
    # is a planted mistake the agreement must catch
    g = torch.Generator().manual_seed(21)
    a = torch.randn((8, 8), generator=g, dtype=torch.float64)
    a[0, 0] = ratio * torch.linalg.vector_norm(a[1:, 0])
    h_alt, t_alt = _other_sign_factorisation(a)
    q = torch.linalg.householder_product(h_alt, t_alt)
    assert torch.allclose(q @ torch.triu(h_alt), a, atol=1e-12)  # a valid QR of A
    a32 = a.float().unsqueeze(0)
    h_ref, t_ref = torch.geqrf(a32)
    rep = checker.rdiag_tau_agreement(a32, h_alt.float().unsqueeze(0), t_alt.float().unsqueeze(0), h_ref, t_ref)
    assert rep.ok == flip_allowed, rep.message()
    if flip_allowed:
        assert rep.sign_flips == 1 and rep.r_only >= 6


def test_agreement_floor_masks_rank_deficient_tail_only():
    g = load("rankdef_4x8")
    rep = checker.rdiag_tau_agreement(g["a"], g["h_scipy"], g["tau_scipy"], g["h"], g["tau"])
    assert rep.ok and rep.masked >= 4 * 2  # the two copied columns per matrix are noise
    assert rep.compared >= 4 * 5
    assert math.isfinite(rep.rdiag_rel_max)


# ---- explicit Q (householder_product) -------------------------------------
def test_orgqr_restated_matches_torch_householder_product():
    # torch.linalg.householder_product is the reference checker's own call
    # (official/reference.py:199); the restatement must agree on golden factors
    for name in ("gauss_20x32", "gauss_6x1", "gauss_6x5", "rankdef_4x8", "upper_4x8"):
        d = load(name)
        q = oracle.orgqr_restated(d["h"], d["tau"])
        q_ref = torch.linalg.householder_product(torch.from_numpy(d["h"]).double(),
                                                 torch.from_numpy(d["tau"]).double()).numpy()
        np.testing.assert_allclose(q, q_ref, rtol=0, atol=1e-12)


def test_orgqr_restated_closed_forms_and_invariants():
    # n = 1: Q = 1 - tau; tau = 0: Q = I
    np.testing.assert_allclose(oracle.orgqr_restated(np.array([[[3.0]]]), np.array([[0.25]])), [[[0.75]]])
    h = np.random.default_rng(3).standard_normal((2, 7, 7))
    np.testing.assert_array_equal(oracle.orgqr_restated(h, np.zeros((2, 7))), np.broadcast_to(np.eye(7), (2, 7, 7)))
    # one reflector: Q = I - tau v v^T exactly
    hh = np.zeros((4, 4))
    hh[1:, 0] = [0.5, -1.0, 2.0]
    tau = np.array([1.2, 0, 0, 0])
    v = np.array([1.0, 0.5, -1.0, 2.0])
    np.testing.assert_allclose(oracle.orgqr_restated(hh, tau), np.eye(4) - 1.2 * np.outer(v, v), atol=1e-15)
    # on geqrf factors: Q orthogonal and Q triu(H) = A
    a = torch.randn((3, 24, 24), generator=torch.Generator().manual_seed(8), dtype=torch.float64)
    hq, tq = torch.geqrf(a)
    q = oracle.orgqr_restated(hq.numpy(), tq.numpy())
    np.testing.assert_allclose(np.einsum("bki,bkj->bij", q, q), np.broadcast_to(np.eye(24), q.shape), atol=1e-12)
    np.testing.assert_allclose(q @ np.triu(hq.numpy()), a.numpy(), atol=1e-12)


def test_orgqr_planted_order_mistake_is_caught():
    a = torch.randn((2, 12, 12), generator=torch.Generator().manual_seed(9), dtype=torch.float64)
    hq, tq = torch.geqrf(a)
    q_bad = oracle.orgqr_restated(hq.numpy(), tq.numpy(), mutation=1)
    assert np.abs(q_bad @ np.triu(hq.numpy()) - a.numpy()).max() > 1e-3
