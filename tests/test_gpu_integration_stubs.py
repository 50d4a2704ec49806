"""The ctypes stubs a maintainer would add to bind the C ABI directly
(the reference loads its kernels through torch extensions,
submissions/candidate.py:1333-1353, 4445-4457), run as written with device
pointers on torch's current stream and checked against the oracle: CPU
torch.geqrf (the reference's own path), torch.linalg.householder_product
(official/reference.py:199) and torch.ormqr (submissions/candidate.py:7231-7237)
in fp64.  Tolerances: the stated fp32 gates (|R_ii| and tau within 1e-4
relative through the oracle's agreement check; ||Q - Q_ref||_F <= 1e-5 n;
||X - X_ref||_F <= 1e-5 m ||C||_F)."""
import ctypes
import sys
from pathlib import Path

import pytest
import torch

from oracle import checker

pytestmark = pytest.mark.gpu

LIB = Path(__file__).resolve().parent.parent / "fast-qr_amd" / "fastqr" / "libfastqr.so"


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def lib():
    lib = ctypes.CDLL(str(LIB))
    i64, vp = ctypes.c_int64, ctypes.c_void_p
    lib.fastqr_geqrf_f32.argtypes = [vp, i64, i64, i64, i64, i64, vp, i64, i64, i64,
                                     vp, i64, i64, vp, ctypes.c_size_t, vp]
    lib.fastqr_geqrf_f32.restype = ctypes.c_int
    lib.fastqr_workspace_bytes.argtypes = [i64, i64]
    lib.fastqr_workspace_bytes.restype = ctypes.c_size_t
    lib.fastqr_last_error.restype = ctypes.c_char_p
    lib.fastqr_orgqr_f32.argtypes = [vp, i64, i64, i64, i64, i64, vp, i64, i64,
                                     vp, i64, i64, i64, vp, ctypes.c_size_t, vp]
    lib.fastqr_orgqr_f32.restype = ctypes.c_int
    lib.fastqr_orgqr_workspace_bytes.argtypes = [i64, i64]
    lib.fastqr_orgqr_workspace_bytes.restype = ctypes.c_size_t
    lib.fastqr_ormqr_f32.argtypes = [vp, i64, i64, i64, i64, i64, i64, vp, i64, i64,
                                     vp, i64, i64, i64, i64, ctypes.c_int, vp, ctypes.c_size_t, vp]
    lib.fastqr_ormqr_f32.restype = ctypes.c_int
    lib.fastqr_ormqr_workspace_bytes.argtypes = [i64, i64, i64, i64]
    lib.fastqr_ormqr_workspace_bytes.restype = ctypes.c_size_t
    lib.fastqr_geqrf_mixed_f32.argtypes = [vp, i64, i64, i64, i64, i64, vp, i64, i64, i64, vp, i64, i64,
                                           i64, ctypes.c_int, ctypes.c_int, vp, ctypes.c_size_t, vp]
    lib.fastqr_geqrf_mixed_f32.restype = ctypes.c_int
    lib.fastqr_geqrf_mixed_workspace_bytes.argtypes = [i64, i64, i64, ctypes.c_int]
    lib.fastqr_geqrf_mixed_workspace_bytes.restype = ctypes.c_size_t
    return lib


def geqrf_mixed(lib, data, h, tau, panel_width, precision, flags):
    b, n, _ = data.shape
    ws_bytes = lib.fastqr_geqrf_mixed_workspace_bytes(b, n, panel_width, flags)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=data.device)
    rc = lib.fastqr_geqrf_mixed_f32(data.data_ptr(), b, n, *data.stride(), h.data_ptr(), *h.stride(),
                                    tau.data_ptr(), *tau.stride(), panel_width, precision, flags,
                                    ws.data_ptr(), ws_bytes,
                                    torch.cuda.current_stream(data.device).cuda_stream)
    if rc != 0:
        raise RuntimeError(lib.fastqr_last_error().decode())


@pytest.mark.parametrize("precision,flags,gates", [(0, 0, True), (3, 0, False), (3, 3, True)])
def test_mixed_stub_on_device_pointers(cuda, lib, precision, flags, gates):
    """bf16-input bare fails the gates, with both repairs (flags 3) passes, as
    the reference's prototype does in tf32 (tests/test_qr_smoke.py:218-258)."""
    _say(f"[stub mixed] precision={precision} flags={flags}")
    g = torch.Generator().manual_seed(71)
    a = torch.randn((3, 96, 96), generator=g, dtype=torch.float32)
    d = a.to(cuda)
    h = torch.empty_strided((3, 96, 96), (96 * 96, 1, 96), dtype=torch.float32, device=cuda)
    tau = torch.empty((3, 96), dtype=torch.float32, device=cuda)
    geqrf_mixed(lib, d, h, tau, 32, precision, flags)
    torch.cuda.synchronize()
    ok, msg = checker.official_check(a, h.cpu(), tau.cpu())
    assert ok == gates, msg


def geqrf(lib, data, h, tau):
    b, n, _ = data.shape
    ws_bytes = lib.fastqr_workspace_bytes(b, n)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=data.device)
    rc = lib.fastqr_geqrf_f32(data.data_ptr(), b, n, *data.stride(),
                              h.data_ptr(), *h.stride(), tau.data_ptr(), *tau.stride(),
                              ws.data_ptr(), ws_bytes,
                              torch.cuda.current_stream(data.device).cuda_stream)
    if rc != 0:
        raise RuntimeError(lib.fastqr_last_error().decode())


def householder_product(lib, h, tau):
    b, n, _ = h.shape
    q = torch.empty_strided((b, n, n), (n * n, 1, n), dtype=torch.float32, device=h.device)
    ws_bytes = lib.fastqr_orgqr_workspace_bytes(b, n)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=h.device)
    rc = lib.fastqr_orgqr_f32(h.data_ptr(), b, n, *h.stride(), tau.data_ptr(), *tau.stride(),
                              q.data_ptr(), *q.stride(), ws.data_ptr(), ws_bytes,
                              torch.cuda.current_stream(h.device).cuda_stream)
    if rc != 0:
        raise RuntimeError(lib.fastqr_last_error().decode())
    return q


def ormqr_(lib, h, tau, c, transpose):
    b, m, r = h.shape
    ws_bytes = lib.fastqr_ormqr_workspace_bytes(b, m, r, c.shape[2])
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=h.device)
    rc = lib.fastqr_ormqr_f32(h.data_ptr(), b, m, r, *h.stride(), tau.data_ptr(), *tau.stride(),
                              c.data_ptr(), c.shape[2], *c.stride(), int(transpose),
                              ws.data_ptr(), ws_bytes,
                              torch.cuda.current_stream(h.device).cuda_stream)
    if rc != 0:
        raise RuntimeError(lib.fastqr_last_error().decode())


@pytest.mark.parametrize("batch,n", [(5, 40), (4, 150), (3, 400), (2, 1100)])
def test_stubs_with_device_pointers(cuda, lib, batch, n):
    _say(f"[ctypes stubs] batch={batch} n={n}")
    a = torch.randn((batch, n, n), generator=torch.Generator().manual_seed(4000 + n))
    data = a.to(cuda)
    h = torch.empty_strided((batch, n, n), (n * n, 1, n), dtype=torch.float32, device=cuda)
    tau = torch.empty((batch, n), dtype=torch.float32, device=cuda)
    geqrf(lib, data, h, tau)
    q = householder_product(lib, h, tau)
    c = torch.randn((batch, n, 24), generator=torch.Generator().manual_seed(4001 + n))
    x = c.transpose(-1, -2).contiguous().transpose(-1, -2).to(cuda)  # contiguous columns
    ormqr_(lib, h, tau, x, True)
    torch.cuda.synchronize()
    h_c, tau_c = h.cpu(), tau.cpu()
    ok, msg = checker.official_check(a, h_c, tau_c)
    assert ok, msg
    h_ref, tau_ref = torch.geqrf(a)
    ag = checker.rdiag_tau_agreement(a, h_c, tau_c, h_ref, tau_ref)
    assert ag.ok, ag.message()
    q_ref = torch.linalg.householder_product(h_c.double(), tau_c.double())
    assert torch.linalg.matrix_norm(q.cpu().double() - q_ref).max().item() <= 1e-5 * n
    x_ref = torch.ormqr(h_c.double(), tau_c.double(), c.double(), left=True, transpose=True)
    err = (torch.linalg.matrix_norm(x.cpu().double() - x_ref) / torch.linalg.matrix_norm(c.double())).max().item()
    assert err <= 1e-5 * n, err
