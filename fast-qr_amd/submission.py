"""Drop-in submission module: the reference evaluator does
``from submission import custom_kernel`` (official/eval.py:126, 184) with this
directory on sys.path."""
from fastqr import custom_kernel  # noqa: F401
