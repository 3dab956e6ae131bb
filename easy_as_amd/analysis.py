"""IR analyses shared by the codegen and the runtime."""

from __future__ import annotations

from .ir import IRModule


def infer_writes(ir: IRModule) -> frozenset[str]:
    """Names of buffer arguments that are targets of ``store`` / ``mma_store``.

    Decides which kernel pointers are emitted non-const and which host arrays
    are copied back after a launch (reference: ``eas/analysis.py:8-27``).
    """
    names = {inst.out.id: str(inst.args[0]) for inst in ir.insts if inst.op == "arg" and inst.out is not None}
    return frozenset(
        names[inst.args[0].id]
        for inst in ir.insts
        if inst.op in ("store", "mma_store") and inst.args[0].id in names
    )
