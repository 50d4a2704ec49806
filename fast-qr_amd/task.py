"""Interface types of the submission entry point (official/task.py:4-13).

``NotRequired`` is in ``typing`` from Python 3.11; on older interpreters it
and a ``TypedDict`` that understands it come from ``typing_extensions``.
"""
from typing import TypeVar

try:
    from typing import NotRequired, TypedDict
except ImportError:  # Python < 3.11
    from typing_extensions import NotRequired, TypedDict

import torch

input_t = TypeVar("input_t", bound=torch.Tensor)
output_t = TypeVar("output_t", bound=tuple[torch.Tensor, torch.Tensor])


class TestSpec(TypedDict):
    batch: int
    n: int
    cond: int
    seed: int
    case: NotRequired[str]
