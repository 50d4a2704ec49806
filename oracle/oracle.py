"""CPU oracle for batched Householder QR — TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's CPU-baseline leg may
import this module, and only as the checker.  The product path
(fast-qr_amd/fastqr) never imports it and has no CPU fallback.

Two oracles live here:

* ``geqrf_lapack`` — the reference's own path: ``torch.geqrf`` on CPU tensors
  (official/reference.py:145-147 ``ref_kernel``; submissions/baseline_geqrf.py:5-6).
  It returns H in the column-major layout (stride (n*n, 1, n)) the reference
  kernels write.
* ``geqrf_restated`` / ``geqrf_restated_blocked`` — the C restatement in
  oracle/hhqr.c of the reference's own kernel algorithm (reflector convention
  submissions/candidate.py:654-668, column loop 146-226, slarft T 2544-2584,
  compact-WY update tools/blocked_qr_reference.py:112-122).  It is pinned
  against ``geqrf_lapack``, scipy's LAPACK ``sgeqrf`` and closed forms in
  tests/test_oracle.py.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_lib = None


def build(force: bool = False) -> Path:
    """Compile oracle/hhqr.c with gcc (oracle/Makefile)."""
    if force or not LIB_PATH.exists() or LIB_PATH.stat().st_mtime < (HERE / "hhqr.c").stat().st_mtime:
        subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(LIB_PATH))
        i64 = ctypes.c_int64
        fp = ctypes.POINTER(ctypes.c_float)
        dp = ctypes.POINTER(ctypes.c_double)
        _lib.orc_geqrf_unblocked_f32.argtypes = [i64, i64, fp, i64, i64, i64, fp, fp, ctypes.c_int]
        _lib.orc_geqrf_unblocked_f32.restype = ctypes.c_int
        _lib.orc_geqrf_unblocked_f64.argtypes = [i64, i64, fp, i64, i64, i64, dp, dp]
        _lib.orc_geqrf_unblocked_f64.restype = ctypes.c_int
        _lib.orc_geqrf_blocked_f32.argtypes = [i64, i64, i64, fp, i64, i64, i64, fp, fp, ctypes.c_int]
        _lib.orc_geqrf_blocked_f32.restype = ctypes.c_int
        _lib.orc_larft_f32.argtypes = [i64, i64, fp, i64, fp, fp]
        _lib.orc_larft_f32.restype = ctypes.c_int
        _lib.orc_reflector_f32.argtypes = [
            ctypes.c_float, ctypes.c_float, ctypes.c_int,
            ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_float),
            ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_int),
        ]
        _lib.orc_reflector_f32.restype = None
    return _lib


def _fptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _dptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_double))


def _as_f32_batch(a) -> np.ndarray:
    try:
        import torch

        if isinstance(a, torch.Tensor):
            a = a.detach().cpu().numpy()
    except ImportError:  # pragma: no cover
        pass
    a = np.asarray(a, dtype=np.float32)
    if a.ndim != 3 or a.shape[1] != a.shape[2]:
        raise ValueError("expected a (batch, n, n) array")
    return a


def _colmajor_out(b: int, n: int, dtype) -> np.ndarray:
    # (b, n, n) array whose memory is column-major per matrix: element (i, j)
    # at offset j*n + i, i.e. strides (n*n, 1, n) in elements.
    buf = np.empty((b, n, n), dtype=dtype)  # buf[b, j, i] == H[b, i, j]
    return buf


def reflector(alpha: float, sigma: float, mutation: int = 0):
    """(beta, tau, denom, active) of the reference's reflector."""
    beta, tau, denom, active = ctypes.c_float(), ctypes.c_float(), ctypes.c_float(), ctypes.c_int()
    lib().orc_reflector_f32(alpha, sigma, mutation, ctypes.byref(beta), ctypes.byref(tau),
                            ctypes.byref(denom), ctypes.byref(active))
    return beta.value, tau.value, denom.value, bool(active.value)


def geqrf_restated(a, mutation: int = 0) -> tuple[np.ndarray, np.ndarray]:
    """Unblocked fp32 restatement. Returns (H, tau); H is (b, n, n) with H[b, i, j]."""
    a = _as_f32_batch(a)
    b, n, _ = a.shape
    s0, s1, s2 = (s // 4 for s in a.strides)
    buf = _colmajor_out(b, n, np.float32)
    tau = np.empty((b, n), dtype=np.float32)
    rc = lib().orc_geqrf_unblocked_f32(b, n, _fptr(a), s0, s1, s2, _fptr(buf), _fptr(tau), mutation)
    if rc != 0:
        raise RuntimeError(f"oracle error {rc}")
    return np.swapaxes(buf, 1, 2), tau


def geqrf_restated_f64(a) -> tuple[np.ndarray, np.ndarray]:
    a = _as_f32_batch(a)
    b, n, _ = a.shape
    s0, s1, s2 = (s // 4 for s in a.strides)
    buf = _colmajor_out(b, n, np.float64)
    tau = np.empty((b, n), dtype=np.float64)
    rc = lib().orc_geqrf_unblocked_f64(b, n, _fptr(a), s0, s1, s2, _dptr(buf), _dptr(tau))
    if rc != 0:
        raise RuntimeError(f"oracle error {rc}")
    return np.swapaxes(buf, 1, 2), tau


def geqrf_restated_blocked(a, nb: int, mutation: int = 0) -> tuple[np.ndarray, np.ndarray]:
    a = _as_f32_batch(a)
    b, n, _ = a.shape
    s0, s1, s2 = (s // 4 for s in a.strides)
    buf = _colmajor_out(b, n, np.float32)
    tau = np.empty((b, n), dtype=np.float32)
    rc = lib().orc_geqrf_blocked_f32(b, n, nb, _fptr(a), s0, s1, s2, _fptr(buf), _fptr(tau), mutation)
    if rc != 0:
        raise RuntimeError(f"oracle error {rc}")
    return np.swapaxes(buf, 1, 2), tau


def larft(v: np.ndarray, tau: np.ndarray) -> np.ndarray:
    """T (nb x nb, upper) for an m x nb unit-lower-trapezoidal V (below-diagonal part used)."""
    v = np.asfortranarray(np.asarray(v, dtype=np.float32))
    tau = np.ascontiguousarray(np.asarray(tau, dtype=np.float32))
    m, nb = v.shape
    t = np.zeros((nb, nb), dtype=np.float32, order="F")
    rc = lib().orc_larft_f32(m, nb, _fptr(v), m, _fptr(tau), _fptr(t))
    if rc != 0:
        raise RuntimeError(f"oracle error {rc}")
    return np.ascontiguousarray(t)


def orgqr_restated(h, tau, mutation: int = 0) -> np.ndarray:
    """Q = H_0 H_1 ... H_{n-1} from compact factors, in fp64 (numpy).

    The product torch.linalg.householder_product forms for the reference's
    checker (official/reference.py:199): reflectors applied to I from the
    last to the first (LAPACK sorg2r's order), v_k = (0, .., 0, 1, h[k+1:, k]).
    ``mutation`` plants a mistake for the tests: 1 applies them first to last
    (giving Q^T).
    """
    h = np.asarray(h, dtype=np.float64)
    tau = np.asarray(tau, dtype=np.float64)
    single = h.ndim == 2
    if single:
        h, tau = h[None], tau[None]
    b, n, _ = h.shape
    q = np.broadcast_to(np.eye(n), (b, n, n)).copy()
    order = range(n) if mutation == 1 else range(n - 1, -1, -1)
    for k in order:
        v = np.concatenate([np.ones((b, 1)), h[:, k + 1:, k]], axis=1)  # (b, n - k)
        w = np.einsum("bi,bij->bj", v, q[:, k:, :])
        q[:, k:, :] -= tau[:, k, None, None] * v[:, :, None] * w[:, None, :]
    return q[0] if single else q


def geqrf_lapack(a):
    """The reference's own path: batched torch.geqrf on CPU (fp32, MKL LAPACK)."""
    import torch

    if not isinstance(a, torch.Tensor):
        a = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))
    return torch.geqrf(a.detach().cpu().to(torch.float32))


def default_threads() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1
