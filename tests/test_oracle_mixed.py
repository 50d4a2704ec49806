"""Pins the CPU oracle of the mixed-precision blocked QR (oracle/mixed.py).

Checks, each chosen so a plausible mistake fails at least one:
  * operand rounding against closed forms (ties to even, carries into the
    exponent, fixed points, the relative error bound) and, bit for bit over
    a million values including every tie pattern, against the integer
    round-to-nearest-even the gfx950 kernel uses (qr_mixed.hip);
  * the reference's own tests of its prototype (tests/test_qr_smoke.py:
    203-276): every update form passes the official checker for panel widths
    1, 3, 5, 32 in fp32; the three forms agree within 2e-5; tf32-input
    without repair fails the factor gate, R maintenance alone still fails it,
    R maintenance plus panel refresh passes with the diagnostics bounds;
  * mathematics: the compact-WY T reproduces the product of the reflectors;
    with both repairs every panel and R row is an fp32 quantity, so the
    result matches the fp32 factorisation to fp32 rounding;
  * planted mistakes (mutation flags) are caught.
The input generator is the restated official one (fastqr.cases); its draw
stream is not pinned against the reference's, so the reference's seeds name
inputs of the same family, not the same matrices.
"""
import numpy as np
import pytest
import torch

from fastqr.cases import Case, generate
from oracle import checker
from oracle import mixed as M


def case(batch, n, cond, seed, kind="dense"):
    return generate(Case(batch=batch, n=n, cond=cond, seed=seed, case=kind))


def f32(*xs):
    return np.array(xs, dtype=np.float32)


def device_rne(x, drop_bits):
    """The kernel's rounding: integer round to nearest even, `drop_bits` low bits cleared."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    half = (1 << (drop_bits - 1)) - 1
    u = (u + half + ((u >> drop_bits) & 1)) & ~np.uint64((1 << drop_bits) - 1)
    return (u & 0xFFFFFFFF).astype(np.uint32).view(np.float32)


def test_tf32_rounding_closed_forms():
    ulp = 2.0 ** -10  # 11 significant bits at [1, 2)
    x = f32(1 + ulp / 2, 1 + 3 * ulp / 2, 1 + ulp / 4, 1 + 3 * ulp / 4, 2 - ulp / 2, -(1 + 3 * ulp / 2), 0.0, 3.0,
            2.0 ** -20 * (1 + ulp / 2))
    want = f32(1.0, 1 + 2 * ulp, 1.0, 1 + ulp, 2.0, -(1 + 2 * ulp), 0.0, 3.0, 2.0 ** -20)
    np.testing.assert_array_equal(M.quantize_tf32(x), want)


def test_bf16_rounding_closed_forms():
    ulp = 2.0 ** -7  # 8 significant bits at [1, 2)
    x = f32(1 + ulp / 2, 1 + 3 * ulp / 2, 1 + ulp / 4, 2 - ulp / 2, -(1 + 3 * ulp / 2), 1 + ulp)
    want = f32(1.0, 1 + 2 * ulp, 1.0, 2.0, -(1 + 2 * ulp), 1 + ulp)
    np.testing.assert_array_equal(M.quantize_bf16(x), want)


def test_fp16_rounding_closed_forms():
    x = f32(2049.0, 2051.0, 65504.0, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11)
    want = f32(2048.0, 2052.0, 65504.0, 1.0, 1.0 + 2.0 ** -9)
    np.testing.assert_array_equal(M.round_operand(x, "fp16-input"), want)


@pytest.mark.parametrize("mode,drop,bound", [("tf32-input", 13, 2.0 ** -11), ("bf16-input", 16, 2.0 ** -8)])
def test_rounding_matches_the_kernel_formula_bit_for_bit(mode, drop, bound):
    rng = np.random.default_rng(5)
    x = rng.standard_normal(1_000_000).astype(np.float32) * np.float32(3.0)
    # exact ties and near-ties: random high bits, low `drop` bits set to the halfway pattern (+-1)
    hi = rng.integers(0x30000000, 0x50000000, 200_000, dtype=np.uint64) & ~np.uint64((1 << drop) - 1)
    for delta in (-1, 0, 1):
        ties = (hi | np.uint64(1 << (drop - 1))) + np.uint64(delta + 1) - np.uint64(1)
        x = np.concatenate([x, ties.astype(np.uint32).view(np.float32)])
    got = M.round_operand(x, mode)
    np.testing.assert_array_equal(got.view(np.uint32), device_rne(x, drop).view(np.uint32))
    np.testing.assert_array_equal(M.round_operand(got, mode), got)  # idempotent
    rel = np.abs(got.astype(np.float64) - x) / np.abs(x.astype(np.float64))
    assert rel.max() <= bound


def test_compact_wy_t_reproduces_the_reflector_product():
    a = case(3, 12, 2, 11)
    h, t = torch.geqrf(a[:, :, :5])
    h, t = h.numpy(), t.numpy()
    v = M.panel_v(h)
    T = M.compact_wy_t(v, t)
    block = np.eye(12) - v.astype(np.float64) @ T @ np.swapaxes(v, 1, 2)
    prod = np.broadcast_to(np.eye(12), (3, 12, 12)).copy()
    for j in range(5):  # H_0 H_1 ... H_4
        vj = v[:, :, j].astype(np.float64)
        prod = prod - t[:, j, None, None] * (prod @ vj[:, :, None]) @ vj[:, None, :]
    np.testing.assert_allclose(block, prod, atol=2e-6)
    assert np.all(np.tril(T, -1) == 0)


@pytest.mark.parametrize("update_mode", M.UPDATE_MODES)
@pytest.mark.parametrize("panel_width", [1, 3, 5, 32])
def test_fp32_passes_the_official_checker(panel_width, update_mode):
    # the reference's test_blocked_qr_reference_passes_official_checker... (tests/test_qr_smoke.py:203-215)
    a = case(3, 8, 1, 321)
    h, tau = M.blocked_geqrf_mixed(a, panel_width=panel_width, update_mode=update_mode)
    ok, msg = checker.official_check(a, h, tau)
    assert ok, msg
    assert h.shape == (3, 8, 8) and tau.shape == (3, 8) and h.dtype == np.float32


def test_update_forms_agree():
    # tests/test_qr_smoke.py:261-276: sequential, explicit-transform and compact-WY updates of one panel
    a = case(2, 10, 2, 333, "mixed").numpy()
    ph, pt = (x.numpy() for x in torch.geqrf(torch.from_numpy(a[:, :, :4].copy())))
    outs = []
    for fn in (M.apply_reflectors, M.apply_block_full, M.apply_compact_wy):
        x = a[:, :, 4:].copy()
        fn(x, ph, pt)
        outs.append(x)
    np.testing.assert_allclose(outs[1], outs[0], rtol=2e-5, atol=2e-5)
    np.testing.assert_allclose(outs[2], outs[0], rtol=2e-5, atol=2e-5)
    h, tau = M.blocked_geqrf_mixed(a, panel_width=4, update_mode="compact-wy")
    ok, msg = checker.official_check(a, h, tau)
    assert ok, msg


def test_tf32_update_fails_then_repairs_pass():
    # tests/test_qr_smoke.py:218-258
    a = case(2, 8, 1, 444)
    kw = dict(panel_width=3, update_mode="compact-wy", precision_mode="tf32-input")
    h, tau = M.blocked_geqrf_mixed(a, **kw)
    ok, msg = checker.official_check(a, h, tau)
    assert not ok and "R - Q.T @ A is too large" in msg
    h, tau = M.blocked_geqrf_mixed(a, r_maintenance_mode="panel-prefix", **kw)
    ok, msg = checker.official_check(a, h, tau)
    assert not ok and "R - Q.T @ A is too large" in msg
    h, tau = M.blocked_geqrf_mixed(a, r_maintenance_mode="panel-prefix", panel_refresh_mode="prefix", **kw)
    ok, msg = checker.official_check(a, h, tau)
    assert ok, msg
    d = checker.diagnose(a, h, tau)
    assert d["factor_scaled_max"] < 20.0 and d["orth_scaled_max"] < 100.0


@pytest.mark.parametrize("mode", ["tf32-input", "fp16-input", "bf16-input"])
def test_reduced_precision_fails_the_gate_at_64_and_full_repair_restores_fp32(mode):
    a = case(3, 64, 1, 7)
    h, tau = M.blocked_geqrf_mixed(a, 16, "compact-wy", mode)
    ok, msg = checker.official_check(a, h, tau)
    assert not ok and "R - Q.T @ A is too large" in msg
    hf, tf = M.blocked_geqrf_mixed(a, 16, "compact-wy", "fp32")
    hr, tr = M.blocked_geqrf_mixed(a, 16, "compact-wy", mode, "panel-prefix", "prefix")
    ok, msg = checker.official_check(a, hr, tr)
    assert ok, msg
    # every panel and R row recomputed in fp32: the fp32 factorisation to rounding
    assert np.abs(hr - hf).max() <= 1e-4 * np.abs(hf).max()
    assert np.abs(tr - tf).max() <= 1e-4


def test_panel_refresh_alone_fixes_the_reflectors_not_r():
    # refreshed panels are fp32 quantities: tau, V and diag(R) match fp32;
    # the R rows right of each panel still carry the reduced-precision update
    a = case(3, 64, 1, 8)
    hf, tf = M.blocked_geqrf_mixed(a, 16, "compact-wy", "fp32")
    h, tau = M.blocked_geqrf_mixed(a, 16, "compact-wy", "bf16-input", panel_refresh_mode="prefix")
    assert np.abs(tau - tf).max() <= 1e-4
    np.testing.assert_allclose(np.tril(h), np.tril(hf), atol=1e-4 * np.abs(hf).max())
    ok, msg = checker.official_check(a, h, tau)
    assert not ok and "R - Q.T @ A is too large" in msg


@pytest.mark.parametrize("mutation", [1, 2, 3])
def test_planted_mistakes_are_caught(mutation):
    a = case(3, 64, 1, 7)
    if mutation == 1:  # T for T^T: fp32 result no longer a QR of A
        h, tau = M.blocked_geqrf_mixed(a, 16, "compact-wy", "fp32", mutation=1)
        assert not checker.official_check(a, h, tau)[0]
    elif mutation == 2:  # refresh short of one reflector
        h, tau = M.blocked_geqrf_mixed(a, 16, "compact-wy", "tf32-input", "panel-prefix", "prefix", mutation=2)
        assert not checker.official_check(a, h, tau)[0]
    else:  # rounding dropped: the reduced mode then passes where it must fail
        h, tau = M.blocked_geqrf_mixed(a, 16, "compact-wy", "tf32-input", mutation=3)
        assert checker.official_check(a, h, tau)[0]


def test_argument_errors_mirror_the_reference():
    a = case(1, 4, 1, 1)
    for kw, text in [(dict(panel_width=0), "panel_width must be positive"),
                     (dict(update_mode="x"), "update_mode must be one of"),
                     (dict(precision_mode="fp8"), "precision_mode must be one of"),
                     (dict(r_maintenance_mode="x"), "r_maintenance_mode must be one of"),
                     (dict(panel_refresh_mode="x"), "panel_refresh_mode must be one of")]:
        with pytest.raises(ValueError, match=text):
            M.blocked_geqrf_mixed(a, **kw)
