"""``asc.adv`` names that kernel signatures on the hot path refer to.

Only ``TCubeTiling`` is provided, so that ``tiling: asc.adv.TCubeTiling``
annotations (python/tutorials/05_matmul_leakyrelu/matmul_leakyrelu.py:27-28)
evaluate.  On the reference it is the CANN tiling library's per-core GEMM split
(python/asc/language/adv/tiling.py); the MI355X kernels choose their own tiles,
so an instance here only carries whatever fields the caller sets.  The rest of
asc1's adv API (Matmul, TQue pipes, ...) addresses Ascend hardware units and is
not provided.
"""
from __future__ import annotations


class TCubeTiling:
    """Attribute container standing for the reference's TCubeTiling struct."""

    def __init__(self, **fields):
        self.__dict__.update(fields)

    def __repr__(self) -> str:
        return f"TCubeTiling({', '.join(f'{k}={v!r}' for k, v in self.__dict__.items())})"
