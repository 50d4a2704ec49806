"""Host-side checks that need no GPU: the C ABI library, argument validation,
the Python mirror of the reference interface, workload generators, bench CLI.

Nothing here launches a kernel: every fastqr_geqrf_f32 call below is rejected
by validation (or is an empty batch) before any HIP call is made.
"""
import ctypes
import inspect
import os
import re
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

import fastqr
from fastqr import _lib, inputs, workspace

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "fastqr.h"


def header_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fastqr_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    declared = header_functions()
    assert declared, "no functions parsed from include/fastqr.h"
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in fastqr.h but not exported"
    assert sorted(_lib.EXPORTED_SYMBOLS) == declared


def test_version_and_path_names():
    lib = fastqr.cdll()
    assert lib.fastqr_version() == 1
    assert lib.fastqr_path_name(1) == b"wave64"
    assert lib.fastqr_path_name(64) == b"wave64"
    assert lib.fastqr_path_name(65) == b"lds"
    assert lib.fastqr_path_name(176) == b"lds"
    assert lib.fastqr_path_name(177) == b"blocked"
    assert fastqr.ext().version() == 1
    assert fastqr.path_for(4096) == "blocked"


def test_workspace_bytes():
    lib = fastqr.cdll()
    assert lib.fastqr_workspace_bytes(20, 32) == 0  # wave path needs none
    assert lib.fastqr_workspace_bytes(40, 176) == 0  # nor does the LDS-resident path
    assert lib.fastqr_workspace_bytes(0, 512) == 0
    small = lib.fastqr_workspace_bytes(1, 512)
    assert small > 0 and small % 256 == 0
    # the T slots (12 of 32 x 32 floats per matrix) scale with the batch
    assert lib.fastqr_workspace_bytes(640, 512) >= 640 * 12 * 32 * 32 * 4


def _call(lib, A=8, b=2, n=100, a_s=(None,), H=16, h_s=None, tau=32, t_s=None, ws=64, ws_bytes=1 << 20):
    a_s0, a_s1, a_s2 = (n * n, n, 1) if a_s == (None,) else a_s
    h_s0, h_s1, h_s2 = (n * n, 1, n) if h_s is None else h_s
    t_s0, t_s1 = (n, 1) if t_s is None else t_s
    # fake, never-dereferenced "device" addresses far apart (validation only)
    base = 1 << 40
    return lib.fastqr_geqrf_f32(base * A if A else None, b, n, a_s0, a_s1, a_s2, base * H if H else None, h_s0,
                                h_s1, h_s2, base * tau if tau else None, t_s0, t_s1, base * ws if ws else None,
                                ws_bytes, None)


def test_argument_validation_returns_codes_without_launching():
    lib = fastqr.cdll()
    assert _call(lib, b=0) == _lib.FASTQR_OK  # empty batch: nothing to do
    assert _call(lib, n=0) == _lib.FASTQR_OK
    assert _call(lib, n=-3) == _lib.FASTQR_EINVAL
    assert _call(lib, A=0) == _lib.FASTQR_EINVAL
    assert b"non-null" in lib.fastqr_last_error()
    assert _call(lib, n=9000) == _lib.FASTQR_EINVAL
    # blocked path needs contiguous columns of H and a workspace
    assert _call(lib, n=200, h_s=(40000, 200, 1)) == _lib.FASTQR_ELAYOUT
    assert b"contiguous columns" in lib.fastqr_last_error()
    assert _call(lib, n=200, ws_bytes=16) == _lib.FASTQR_EWORKSPACE
    assert _call(lib, n=200, ws=0) == _lib.FASTQR_EWORKSPACE
    # the LDS-resident path (n <= 176) takes any H strides and no workspace
    # (the fake addresses are never dereferenced: only validation runs here)
    # A and H overlapping with different layouts
    assert _call(lib, n=100, A=16, a_s=(10000, 100, 1)) == _lib.FASTQR_EOVERLAP
    assert _call(lib, n=32, A=16, a_s=(1024, 32, 1)) == _lib.FASTQR_EOVERLAP
    assert _call(lib, t_s=(100, 0)) == _lib.FASTQR_EINVAL
    assert _call(lib, a_s=(-1, 100, 1)) == _lib.FASTQR_EINVAL


def test_noalloc_rejects_sizes_beyond_its_scratch_without_launching():
    # fake, never-dereferenced addresses: the size check comes before any HIP call
    lib = fastqr.cdll()
    base = 1 << 40

    def call(b, n):
        return lib.fastqr_geqrf_f32_noalloc(8 * base, b, n, n * n, n, 1, 16 * base, n * n, 1, n, 32 * base, n, 1,
                                            None)

    assert lib.fastqr_workspace_bytes(683, 512) > _lib.NOALLOC_SCRATCH_BYTES >= lib.fastqr_workspace_bytes(682, 512)
    assert call(683, 512) == _lib.FASTQR_EWORKSPACE
    assert b"fastqr_geqrf_f32_noalloc holds at most" in lib.fastqr_last_error()
    assert call(2, 4096) == _lib.FASTQR_EWORKSPACE
    assert call(2, 2100) == _lib.FASTQR_EWORKSPACE
    assert call(0, 512) == _lib.FASTQR_OK  # empty batch: nothing to do
    assert call(1, 9000) == _lib.FASTQR_EINVAL


def test_forced_error_hook_round_trip():
    lib = fastqr.cdll()
    lib.fastqr_debug_force_error(-99)
    assert _call(lib) == -99
    assert b"forced error" in lib.fastqr_last_error()
    # the hook fires once; the next (invalid) call reports its own error
    assert _call(lib, A=0) == _lib.FASTQR_EINVAL


def test_profile_hooks_without_work():
    _lib.profile_enable(True)
    stats = _lib.profile_collect()
    _lib.profile_enable(False)
    assert set(stats) == set(_lib.PROFILE_KINDS)
    assert all(v["launches"] == 0 for v in stats.values())
    assert fastqr.cdll().fastqr_profile_collect(7, None, None, None, None) == _lib.FASTQR_EINVAL


def test_custom_kernel_interface_matches_reference():
    # official/submission.py:5-6 / tests/test_case_files.py:64-69: exactly custom_kernel(data)
    params = list(inspect.signature(fastqr.custom_kernel).parameters)
    assert params == ["data"]
    sys.path.insert(0, str(ROOT / "fast-qr_amd"))
    import submission  # noqa: F401  (the drop-in module)

    assert submission.custom_kernel is fastqr.custom_kernel


def test_custom_kernel_rejects_bad_inputs_loudly():
    with pytest.raises(TypeError):
        fastqr.custom_kernel(torch.zeros((2, 4, 4), dtype=torch.float64))
    with pytest.raises(ValueError):
        fastqr.custom_kernel(torch.zeros((2, 4, 5)))
    with pytest.raises(ValueError):
        fastqr.custom_kernel(torch.zeros((2, 4, 4)))  # CPU tensor: no silent fallback
    with pytest.raises(TypeError):
        fastqr.custom_kernel(np.zeros((2, 4, 4), np.float32))


def test_column_major_allocator_layout():
    # tests/test_qr_smoke.py:8088-8095 of the reference
    data = torch.empty((3, 16, 16))
    h = fastqr.allocate_column_major_H(3, 16, data)
    assert h.shape == (3, 16, 16) and h.dtype == torch.float32 and h.stride() == (256, 1, 16)
    tau = fastqr.allocate_tau(3, 16, data)
    assert tau.shape == (3, 16) and tau.stride() == (16, 1)


def test_output_workspace_cache_is_per_input(monkeypatch):
    # tests/test_qr_smoke.py:8097-8143 of the reference
    workspace.clear()
    monkeypatch.setenv("FASTQR_OUTPUT_WORKSPACE_CACHE", "1")
    data_a = torch.empty((3, 16, 16))
    data_b = torch.empty((3, 16, 16))
    h_a = fastqr.allocate_column_major_H(3, 16, data_a)
    h_a.fill_(1.0)
    h_a_again = fastqr.allocate_column_major_H(3, 16, data_a)
    h_b = fastqr.allocate_column_major_H(3, 16, data_b)
    assert h_a_again.data_ptr() == h_a.data_ptr()
    assert h_b.data_ptr() != h_a.data_ptr()
    tau_a = fastqr.allocate_tau(3, 16, data_a)
    tau_a.fill_(7.0)
    tau_zero = fastqr.allocate_tau(3, 16, data_a, zero=True)
    assert tau_zero.data_ptr() == tau_a.data_ptr() and not tau_zero.any()
    h2, t2 = fastqr.allocate_h_tau(3, 16, data_b)
    assert h2.data_ptr() == h_b.data_ptr() and t2.data_ptr() != tau_a.data_ptr()
    # a freed input drops its cache entries
    key_count = len(workspace._OUTPUT_CACHE)
    del data_b, h_b, h2, t2
    import gc

    gc.collect()
    assert len(workspace._OUTPUT_CACHE) < key_count
    monkeypatch.setenv("FASTQR_OUTPUT_WORKSPACE_CACHE", "0")
    assert fastqr.allocate_column_major_H(3, 16, data_a).data_ptr() != h_a.data_ptr()


def test_workload_generators_are_seeded_and_structured():
    s = inputs.Shape(8, 64, "c3mixed", 11)
    a1, a2 = inputs.generate(s), inputs.generate(s)
    assert torch.equal(a1, a2) and a1.dtype == torch.float32 and a1.is_contiguous()
    labels = inputs.structure_labels(s)
    assert labels.count("rankdef") == 2 and labels.count("clustered") == 2 and labels.count("dense") == 4
    for i, lab in enumerate(labels):
        sv = torch.linalg.svdvals(a1[i].double())
        if lab == "rankdef":
            assert sv[31] > 0.99 and sv[32] < 1e-5
        elif lab == "clustered":
            assert sv[31] > 0.99 and 5e-7 < sv[32] < 2e-6
    s4 = inputs.Shape(8, 300, "c4mixed", 12)
    a4 = inputs.generate(s4)
    for i, lab in enumerate(inputs.structure_labels(s4)):
        if lab == "nearrank":
            sv = torch.linalg.svdvals(a4[i].double())
            assert sv[300 - 257] > 0.99 and sv[300 - 256] < 2e-7
    assert inputs.flops(2, 3) == pytest.approx(2 * 4 * 27 / 3)
    assert inputs.bytes_moved(1, 4) == 8 * 16 + 16


def test_bench_input_count_matches_official_formula():
    # official/eval.py:167-175; tests/test_case_files.py:731-736 of the reference
    sys.path.insert(0, str(ROOT))
    import bench

    assert bench.count_for(20, 32) == 50
    assert bench.count_for(640, 512) == 1
    assert bench.count_for(60, 1024) == 1
    assert bench.count_for(2, 4096) == 2


def test_bench_refuses_multi_gpu():
    env = dict(os.environ)
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       env=env, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def _orgqr_call(lib, H=8, b=2, n=100, h_s=None, tau=32, t_s=None, Q=16, q_s=None, ws=64, ws_bytes=1 << 30):
    h_s0, h_s1, h_s2 = (n * n, 1, n) if h_s is None else h_s
    q_s0, q_s1, q_s2 = (n * n, 1, n) if q_s is None else q_s
    t_s0, t_s1 = (n, 1) if t_s is None else t_s
    base = 1 << 40  # fake, never-dereferenced addresses (validation only)
    return lib.fastqr_orgqr_f32(base * H if H else None, b, n, h_s0, h_s1, h_s2, base * tau if tau else None,
                                t_s0, t_s1, base * Q if Q else None, q_s0, q_s1, q_s2, base * ws if ws else None,
                                ws_bytes, None)


def test_orgqr_argument_validation_returns_codes_without_launching():
    lib = fastqr.cdll()
    assert lib.fastqr_orgqr_workspace_bytes(0, 64) == 0
    assert lib.fastqr_orgqr_workspace_bytes(100000, 32) == 0  # one kernel, no scratch
    assert _orgqr_call(lib, n=32, ws=0, ws_bytes=0, H=0) == _lib.FASTQR_EINVAL  # reaches the pointer check
    one = lib.fastqr_orgqr_workspace_bytes(1, 512)
    assert one > 0 and one % 256 == 0
    assert lib.fastqr_orgqr_workspace_bytes(640, 512) >= 640 * one - 255
    assert _orgqr_call(lib, b=0) == _lib.FASTQR_OK
    assert _orgqr_call(lib, n=0) == _lib.FASTQR_OK
    assert _orgqr_call(lib, n=-1) == _lib.FASTQR_EINVAL
    assert _orgqr_call(lib, n=5000) == _lib.FASTQR_EINVAL
    assert _orgqr_call(lib, Q=0) == _lib.FASTQR_EINVAL
    assert b"non-null" in lib.fastqr_last_error()
    assert _orgqr_call(lib, q_s=(10000, 100, 1)) == _lib.FASTQR_ELAYOUT
    assert b"contiguous columns" in lib.fastqr_last_error()
    assert _orgqr_call(lib, ws_bytes=16) == _lib.FASTQR_EWORKSPACE
    assert _orgqr_call(lib, ws=0) == _lib.FASTQR_EWORKSPACE
    # H and Q overlapping with different layouts; tau inside Q
    assert _orgqr_call(lib, H=16, h_s=(10000, 100, 1)) == _lib.FASTQR_EOVERLAP
    assert _orgqr_call(lib, tau=16) == _lib.FASTQR_EOVERLAP
    lib.fastqr_debug_force_error(-99)
    assert _orgqr_call(lib) == -99


def _ormqr_call(lib, H=8, b=2, m=100, r=100, h_s=None, tau=32, t_s=None, C=16, k=40, c_s=None, tr=1, ws=64,
                ws_bytes=1 << 30):
    h_s0, h_s1, h_s2 = (m * r, 1, m) if h_s is None else h_s
    c_s0, c_s1, c_s2 = (m * k, 1, m) if c_s is None else c_s
    t_s0, t_s1 = (r, 1) if t_s is None else t_s
    base = 1 << 40  # fake, never-dereferenced addresses (validation only)
    return lib.fastqr_ormqr_f32(base * H if H else None, b, m, r, h_s0, h_s1, h_s2, base * tau if tau else None,
                                t_s0, t_s1, base * C if C else None, k, c_s0, c_s1, c_s2, tr,
                                base * ws if ws else None, ws_bytes, None)


def test_ormqr_argument_validation_returns_codes_without_launching():
    lib = fastqr.cdll()
    assert lib.fastqr_ormqr_workspace_bytes(0, 64, 64, 8) == 0
    assert lib.fastqr_ormqr_workspace_bytes(2, 64, 0, 8) == 0
    assert lib.fastqr_ormqr_workspace_bytes(2, 64, 64, 0) == 0
    assert lib.fastqr_ormqr_workspace_bytes(2, 64, 65, 8) == 0  # r > m: rejected by the call itself
    one = lib.fastqr_ormqr_workspace_bytes(1, 512, 512, 100)
    assert one >= 16 * 32 * 32 * 4 and one % 256 == 0  # a T factor per 32-column panel
    assert lib.fastqr_ormqr_workspace_bytes(640, 512, 512, 100) >= 640 * one - 255
    # above 2048 rows also a group T and the row-split partial products, bounded in k
    tall = lib.fastqr_ormqr_workspace_bytes(2, 4096, 4096, 4096)
    assert tall > lib.fastqr_ormqr_workspace_bytes(2, 2048, 2048, 4096) > 0
    assert lib.fastqr_ormqr_workspace_bytes(2, 4096, 4096, 100000) == tall
    # nothing to do: empty batch, no rows, no columns of C, no reflectors (Q = I)
    for kw in ({"b": 0}, {"m": 0, "r": 0}, {"k": 0}, {"r": 0}):
        assert _ormqr_call(lib, **kw) == _lib.FASTQR_OK
    assert _ormqr_call(lib, r=101) == _lib.FASTQR_EINVAL  # more reflectors than rows
    assert b"exceed" in lib.fastqr_last_error()
    assert _ormqr_call(lib, m=5000, r=10) == _lib.FASTQR_EINVAL
    assert _ormqr_call(lib, k=-1) == _lib.FASTQR_EINVAL
    assert _ormqr_call(lib, C=0) == _lib.FASTQR_EINVAL
    assert b"non-null" in lib.fastqr_last_error()
    assert _ormqr_call(lib, c_s=(4000, 40, 1)) == _lib.FASTQR_ELAYOUT  # row-major C
    assert b"C must have contiguous columns" in lib.fastqr_last_error()
    assert _ormqr_call(lib, h_s=(10000, 100, 1)) == _lib.FASTQR_ELAYOUT  # row-major H
    assert _ormqr_call(lib, c_s=(10, 1, 100)) == _lib.FASTQR_ELAYOUT  # batch stride inside a matrix
    assert _ormqr_call(lib, ws_bytes=16) == _lib.FASTQR_EWORKSPACE
    assert _ormqr_call(lib, ws=0) == _lib.FASTQR_EWORKSPACE
    assert _ormqr_call(lib, C=8) == _lib.FASTQR_EOVERLAP  # C on top of H
    assert _ormqr_call(lib, tau=16) == _lib.FASTQR_EOVERLAP  # tau inside C
    lib.fastqr_debug_force_error(-99)
    assert _ormqr_call(lib) == -99


def test_householder_product_rejects_bad_inputs_loudly():
    h = torch.zeros((2, 8, 8))
    with pytest.raises(ValueError):
        fastqr.householder_product(h, torch.zeros((2, 8)))  # CPU tensors
    with pytest.raises(TypeError):
        fastqr.householder_product(h.double(), torch.zeros((2, 8)))
    with pytest.raises(ValueError):
        fastqr.householder_product(torch.zeros((2, 8, 7)), torch.zeros((2, 8)))
    with pytest.raises(ValueError):
        fastqr.householder_product(h, torch.zeros((2, 7)))


def test_apply_q_rejects_bad_inputs_loudly():
    h = torch.zeros((2, 8, 8))
    with pytest.raises(ValueError):
        fastqr.apply_q(h, torch.zeros((2, 8)), torch.zeros((2, 8, 3)))  # CPU tensors
    with pytest.raises(ValueError):
        fastqr.apply_q(torch.zeros((2, 8, 9)), torch.zeros((2, 9)), torch.zeros((2, 8, 3)))  # r > m
    with pytest.raises(ValueError):
        fastqr.apply_q(h, torch.zeros((2, 8)), torch.zeros((2, 7, 3)))  # C rows
    with pytest.raises(TypeError):
        fastqr.apply_q(h, torch.zeros((2, 8)), torch.zeros((2, 8, 3), dtype=torch.float64))


def test_missing_native_library_fails_loudly(monkeypatch, tmp_path):
    # no fallback: without the library every entry point raises
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libfastqr.so")
    monkeypatch.setattr(_lib, "EXT_PATH", tmp_path / "_fastqr_py.so")
    monkeypatch.setattr(_lib, "_cdll", None)
    monkeypatch.setattr(_lib, "_ext", None)
    with pytest.raises(fastqr.FastQRUnavailable):
        _lib.cdll()
    with pytest.raises(fastqr.FastQRUnavailable):
        _lib.ext()


def _mixed(lib, A=8, b=2, n=100, H=16, h_s=None, tau=32, pw=32, prec=0, flags=0, ws=64, ws_bytes=1 << 30):
    h_s0, h_s1, h_s2 = (n * n, 1, n) if h_s is None else h_s
    base = 1 << 40  # fake, never-dereferenced addresses (validation only)
    return lib.fastqr_geqrf_mixed_f32(base * A if A else None, b, n, n * n, n, 1, base * H if H else None, h_s0,
                                      h_s1, h_s2, base * tau if tau else None, n, 1, pw, prec, flags,
                                      base * ws if ws else None, ws_bytes, None)


def test_mixed_entry_validates_without_launching():
    lib = fastqr.cdll()
    assert _mixed(lib, b=0) == _lib.FASTQR_OK and _mixed(lib, n=0) == _lib.FASTQR_OK
    assert _mixed(lib, pw=8) == _lib.FASTQR_EINVAL
    assert b"panel_width must be 16 or 32" in lib.fastqr_last_error()
    assert _mixed(lib, prec=7) == _lib.FASTQR_EINVAL
    assert _mixed(lib, flags=4) == _lib.FASTQR_EINVAL
    assert b"unknown flags" in lib.fastqr_last_error()
    assert _mixed(lib, n=3000) == _lib.FASTQR_EINVAL
    assert _mixed(lib, A=0) == _lib.FASTQR_EINVAL
    assert _mixed(lib, h_s=(20000, 100, 1)) == _lib.FASTQR_ELAYOUT
    assert _mixed(lib, A=16) == _lib.FASTQR_EOVERLAP  # the repairs read A again: no overlap at all
    assert b"A and H overlap" in lib.fastqr_last_error()
    assert _mixed(lib, ws_bytes=64) == _lib.FASTQR_EWORKSPACE
    assert _mixed(lib, ws=0) == _lib.FASTQR_EWORKSPACE
    lib.fastqr_debug_force_error(-99)
    assert _mixed(lib) == -99


def test_mixed_workspace_bytes():
    lib = fastqr.cdll()
    plain = lib.fastqr_geqrf_mixed_workspace_bytes(2, 100, 32, 0)
    refresh = lib.fastqr_geqrf_mixed_workspace_bytes(2, 100, 32, _lib.FASTQR_MIXED_PANEL_REFRESH)
    both = lib.fastqr_geqrf_mixed_workspace_bytes(2, 100, 32, 3)
    assert plain >= 2 * 12 * 32 * 32 * 4 and plain % 256 == 0
    assert plain < refresh < both
    assert both >= plain + 2 * 100 * 100 * 4  # R maintenance holds a copy of the batch
    for bad in ((0, 100, 32, 0), (2, 0, 32, 0), (2, 100, 8, 0), (2, 100, 32, 4), (2, 4096, 32, 0)):
        assert lib.fastqr_geqrf_mixed_workspace_bytes(*bad) == 0


def test_mixed_wrapper_rejects_bad_arguments_before_any_device_work():
    a = torch.zeros((1, 8, 8))
    for kw, text in [(dict(panel_width=0), "panel_width must be positive"),
                     (dict(panel_width=24), "panel_width must be one of"),
                     (dict(update_mode="reflectors"), "update_mode must be one of"),
                     (dict(precision_mode="fp8"), "precision_mode must be one of"),
                     (dict(r_maintenance_mode="x"), "r_maintenance_mode must be one of"),
                     (dict(panel_refresh_mode="x"), "panel_refresh_mode must be one of")]:
        with pytest.raises(ValueError, match=text):
            fastqr.blocked_geqrf_mixed(a, **kw)
    with pytest.raises(ValueError, match="CUDA"):
        fastqr.blocked_geqrf_mixed(a)  # a CPU tensor: no fallback
