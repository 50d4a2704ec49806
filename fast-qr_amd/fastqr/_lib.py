"""Loader for the gfx950 C-ABI library (libfastqr.so) and its CPython binding.

The product path has no CPU or torch fallback: if the native library is
missing or fails to load, every entry point raises ``FastQRUnavailable``.
"""
from __future__ import annotations

import ctypes
import importlib.util
import os
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libfastqr.so"
EXT_PATH = PKG_DIR / "_fastqr_py.so"

# status codes, include/fastqr.h
FASTQR_OK = 0
FASTQR_EINVAL = -1
FASTQR_EWORKSPACE = -2
FASTQR_ELAYOUT = -3
FASTQR_EOVERLAP = -4
FASTQR_ETESTHOOK = -99
# operand precision and repair flags of fastqr_geqrf_mixed_f32 (FASTQR_PREC_*, FASTQR_MIXED_*)
FASTQR_PREC_FP32 = 0
FASTQR_PREC_TF32_INPUT = 1
FASTQR_PREC_FP16_INPUT = 2
FASTQR_PREC_BF16_INPUT = 3
FASTQR_MIXED_R_MAINTENANCE = 1
FASTQR_MIXED_PANEL_REFRESH = 2
# size of the static device scratch of fastqr_geqrf_f32_noalloc (FASTQR_NOALLOC_SCRATCH_BYTES)
NOALLOC_SCRATCH_BYTES = 32 << 20

# every symbol include/fastqr.h declares
EXPORTED_SYMBOLS = (
    "fastqr_geqrf_f32",
    "fastqr_geqrf_f32_noalloc",
    "fastqr_workspace_bytes",
    "fastqr_orgqr_f32",
    "fastqr_orgqr_workspace_bytes",
    "fastqr_ormqr_f32",
    "fastqr_ormqr_workspace_bytes",
    "fastqr_geqrf_mixed_f32",
    "fastqr_geqrf_mixed_workspace_bytes",
    "fastqr_path_name",
    "fastqr_last_error",
    "fastqr_version",
    "fastqr_debug_force_error",
    "fastqr_profile_enable",
    "fastqr_profile_collect",
    "fastqr_profile_kind_name",
)
PROFILE_KINDS = ("copy", "panel", "update", "wave64", "lds", "update_rowsplit")


class FastQRUnavailable(RuntimeError):
    """The native library is not built or cannot be loaded."""


class FastQRError(RuntimeError):
    """A non-zero status from fastqr_geqrf_f32."""

    def __init__(self, code: int, message: str):
        super().__init__(f"fastqr error {code}: {message}")
        self.code = code
        self.message = message


_cdll = None
_ext = None


def cdll() -> ctypes.CDLL:
    """ctypes view of libfastqr.so with argtypes for every exported symbol."""
    global _cdll
    if _cdll is None:
        if not LIB_PATH.exists():
            raise FastQRUnavailable(
                f"{LIB_PATH} is not built; run `make -C {PKG_DIR.parent}` or __graft_entry__.build()"
            )
        try:
            lib = ctypes.CDLL(str(LIB_PATH))
        except OSError as exc:  # pragma: no cover - depends on the host
            raise FastQRUnavailable(f"cannot load {LIB_PATH}: {exc}") from exc
        i64, vp, sz = ctypes.c_int64, ctypes.c_void_p, ctypes.c_size_t
        lib.fastqr_geqrf_f32.argtypes = [vp, i64, i64, i64, i64, i64, vp, i64, i64, i64, vp, i64, i64, vp, sz, vp]
        lib.fastqr_geqrf_f32.restype = ctypes.c_int
        lib.fastqr_geqrf_f32_noalloc.argtypes = [vp, i64, i64, i64, i64, i64, vp, i64, i64, i64, vp, i64, i64, vp]
        lib.fastqr_geqrf_f32_noalloc.restype = ctypes.c_int
        lib.fastqr_workspace_bytes.argtypes = [i64, i64]
        lib.fastqr_orgqr_f32.argtypes = [vp, i64, i64, i64, i64, i64, vp, i64, i64, vp, i64, i64, i64, vp, sz, vp]
        lib.fastqr_orgqr_f32.restype = ctypes.c_int
        lib.fastqr_orgqr_workspace_bytes.argtypes = [i64, i64]
        lib.fastqr_orgqr_workspace_bytes.restype = sz
        lib.fastqr_ormqr_f32.argtypes = [vp, i64, i64, i64, i64, i64, i64, vp, i64, i64, vp, i64, i64, i64, i64,
                                         ctypes.c_int, vp, sz, vp]
        lib.fastqr_ormqr_f32.restype = ctypes.c_int
        lib.fastqr_ormqr_workspace_bytes.argtypes = [i64, i64, i64, i64]
        lib.fastqr_ormqr_workspace_bytes.restype = sz
        lib.fastqr_workspace_bytes.restype = sz
        lib.fastqr_geqrf_mixed_f32.argtypes = [vp, i64, i64, i64, i64, i64, vp, i64, i64, i64, vp, i64, i64, i64,
                                               ctypes.c_int, ctypes.c_int, vp, sz, vp]
        lib.fastqr_geqrf_mixed_f32.restype = ctypes.c_int
        lib.fastqr_geqrf_mixed_workspace_bytes.argtypes = [i64, i64, i64, ctypes.c_int]
        lib.fastqr_geqrf_mixed_workspace_bytes.restype = sz
        lib.fastqr_path_name.argtypes = [i64]
        lib.fastqr_path_name.restype = ctypes.c_char_p
        lib.fastqr_last_error.argtypes = []
        lib.fastqr_last_error.restype = ctypes.c_char_p
        lib.fastqr_version.argtypes = []
        lib.fastqr_version.restype = ctypes.c_int
        lib.fastqr_debug_force_error.argtypes = [ctypes.c_int]
        lib.fastqr_debug_force_error.restype = None
        lib.fastqr_profile_enable.argtypes = [ctypes.c_int]
        lib.fastqr_profile_enable.restype = ctypes.c_int
        dp = ctypes.POINTER(ctypes.c_double)
        lib.fastqr_profile_collect.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_int64), dp, dp, dp]
        lib.fastqr_profile_collect.restype = ctypes.c_int
        lib.fastqr_profile_kind_name.argtypes = [ctypes.c_int]
        lib.fastqr_profile_kind_name.restype = ctypes.c_char_p
        _cdll = lib
    return _cdll


def ext():
    """The CPython binding module (_fastqr_py), loaded from this directory."""
    global _ext
    if _ext is None:
        if not EXT_PATH.exists():
            raise FastQRUnavailable(f"{EXT_PATH} is not built; run `make -C {PKG_DIR.parent}`")
        cdll()  # load libfastqr.so first so the binding resolves against this copy
        spec = importlib.util.spec_from_file_location("fastqr._fastqr_py", EXT_PATH)
        if spec is None or spec.loader is None:  # pragma: no cover
            raise FastQRUnavailable(f"cannot import {EXT_PATH}")
        mod = importlib.util.module_from_spec(spec)
        try:
            spec.loader.exec_module(mod)
        except ImportError as exc:  # pragma: no cover
            raise FastQRUnavailable(f"cannot import {EXT_PATH}: {exc}") from exc
        sys.modules.setdefault("fastqr._fastqr_py", mod)
        _ext = mod
    return _ext


def profile_enable(on: bool) -> None:
    cdll().fastqr_profile_enable(1 if on else 0)


def profile_collect() -> dict[str, dict[str, float]]:
    """Per kernel kind: launches, ms (summed kernel time), flops, bytes."""
    lib = cdll()
    out = {}
    for kind, name in enumerate(PROFILE_KINDS):
        launches = ctypes.c_int64()
        ms, fl, by = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
        rc = lib.fastqr_profile_collect(kind, ctypes.byref(launches), ctypes.byref(ms), ctypes.byref(fl),
                                        ctypes.byref(by))
        if rc != 0:
            raise FastQRError(rc, lib.fastqr_last_error().decode())
        out[name] = {"launches": launches.value, "ms": ms.value, "flops": fl.value, "bytes": by.value}
    return out


def loaded_paths() -> list[str]:
    """Shared objects of this package currently mapped into the process."""
    out = []
    try:
        with open("/proc/self/maps") as fh:
            for line in fh:
                if str(PKG_DIR) in line and line.rstrip().endswith(".so"):
                    p = line.split()[-1]
                    if p not in out:
                        out.append(p)
    except OSError:  # pragma: no cover
        pass
    return out


def is_built() -> bool:
    return LIB_PATH.exists() and EXT_PATH.exists()


def env_flag(name: str, default: bool) -> bool:
    raw = os.environ.get(name)
    if raw is None or raw.strip() == "":
        return default
    return raw.strip().lower() not in {"0", "false", "no", "off"}
