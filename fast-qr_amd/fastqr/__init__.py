"""fastqr — batched fp32 Householder QR for AMD Instinct MI355X (gfx950).

Drop-in for the reference submission entry point ``custom_kernel(data) -> (H, tau)``.
"""
from ._lib import FastQRError, FastQRUnavailable, cdll, ext, is_built, loaded_paths
from .mixed import blocked_geqrf_mixed
from .orgqr import apply_q, householder_product
from .qr import custom_kernel, geqrf_into, path_for
from .workspace import allocate_column_major_H, allocate_h_tau, allocate_tau

__all__ = [
    "FastQRError",
    "FastQRUnavailable",
    "allocate_column_major_H",
    "allocate_h_tau",
    "allocate_tau",
    "apply_q",
    "blocked_geqrf_mixed",
    "cdll",
    "custom_kernel",
    "ext",
    "geqrf_into",
    "householder_product",
    "is_built",
    "loaded_paths",
    "path_for",
]
