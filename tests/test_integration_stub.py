"""The ctypes binding of the repository's integration guide (its one fenced block that starts
with ``# integration-stub``), executed as written.

CPU: the stub binds every symbol it names and compiles an eas kernel's HIP
source.  GPU: it runs the reference's add kernel end to end through the bare C
ABI, bit-exact against the oracle.
"""

from __future__ import annotations

import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]


def _stub() -> dict:
    text = (ROOT / "INTEGRATION.md").read_text()
    blocks = re.findall(r"```python\n(# integration-stub.*?)```", text, flags=re.S)
    assert len(blocks) == 1, "the integration guide must hold exactly one integration-stub block"
    ns: dict = {"__name__": "integration_stub"}
    exec(compile(blocks[0], "INTEGRATION.md:integration-stub", "exec", dont_inherit=True), ns)
    return ns


def test_stub_binds_and_compiles():
    import importlib

    importlib.import_module("easy_as_amd.runtime.hip_ext")._share_process_hip_runtime()
    ns = _stub()
    abi = ns["HipABI"](str(ROOT / "easy_as_amd" / "libeas_hip.so"))
    assert abi.lib.eas_hip_abi_version() >= 2
    code = abi.compile_code('extern "C" __global__ void k(float* x) { x[threadIdx.x] = 2.0f; }', "k")
    assert code[:4] == b"\x7fELF"
    assert ns["pack_kernargs"]([("u32", 7), ("ptr", type("P", (), {"value": 1})())]) == \
        b"\x07\0\0\0" + b"\0" * 4 + b"\x01" + b"\0" * 7


@pytest.mark.gpu
def test_stub_runs_add_bit_exact():
    import importlib

    from oracle import ops

    importlib.import_module("easy_as_amd.runtime.hip_ext")._share_process_hip_runtime()
    ns = _stub()
    abi = ns["HipABI"](str(ROOT / "easy_as_amd" / "libeas_hip.so"))
    assert abi.lib.eas_hip_is_available() == 1
    n = 4099
    a = np.random.default_rng(0).standard_normal(n, dtype=np.float32)
    b = np.random.default_rng(1).standard_normal(n, dtype=np.float32)
    c = ns["run_add"](abi, a, b)
    assert np.array_equal(c.view(np.uint32), ops.add_f32(a, b).view(np.uint32))


@pytest.mark.gpu
def test_stub_runs_lifted_matmul():
    # the reference's simdgroup-MMA matmul, lifted to the MFMA GEMM, through the bare C ABI's
    # reference-convention launch; every output against float64 (f16 products are exact in f32)
    import importlib
    import math

    import kernels as K

    importlib.import_module("easy_as_amd.runtime.hip_ext")._share_process_hip_runtime()
    ns = _stub()
    abi = ns["HipABI"](str(ROOT / "easy_as_amd" / "libeas_hip.so"))
    for m, n, k in ((300, 520, 200), (512, 1024, 4100)):
        a = np.random.default_rng(0).uniform(-1, 1, m * k).astype(np.float16)
        b = np.random.default_rng(1).uniform(-1, 1, k * n).astype(np.float16)
        ck = K.matmul_mma_kernel.compile(a, b, np.zeros(1, np.float32), m, n, BM=32, BN=32, BK=8, K=k, NT=512)
        assert ck.geometry.kind == "gemm"
        c = ns["run_matmul"](abi, ck, a, b, m, n).reshape(m, n)
        ref = a.astype(np.float64).reshape(m, k) @ b.astype(np.float64).reshape(k, n)
        assert float(np.abs(c - ref).max() / np.abs(ref).max()) <= 1e-5 * math.sqrt(k)
