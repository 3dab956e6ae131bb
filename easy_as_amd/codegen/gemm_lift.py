"""Recognise tile-GEMM kernels in the IR and replace them with a tuned MFMA GEMM.

Placeholder: no kernel is lifted yet, every thread-mode kernel takes the
literal lowering.
"""

from __future__ import annotations

from typing import Any

from ..ir import IRModule


def try_lift(ir: IRModule, block: int) -> Any:
    return None
