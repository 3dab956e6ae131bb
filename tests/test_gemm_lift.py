"""The GEMM lift replaces a kernel only when it has proved it is a dense GEMM."""

from __future__ import annotations

import numpy as np
import pytest

import kernels as K
from easy_as_amd.codegen import gemm_lift
from easy_as_amd.codegen.gemm_lift import Unsupported, analyze
from easy_as_amd.compiler import optimize_ir, trace_to_ir
from easy_as_amd.ir import DType

f16 = lambda n: np.zeros(n, np.float16)  # noqa: E731
f32 = lambda n: np.zeros(n, np.float32)  # noqa: E731


def _ir(kern, *args, **kw):
    kern._extract_runtime_options(kw)
    meta, rargs = kern._bind_and_split(*args, **kw)
    return optimize_ir(trace_to_ir(kern.fn, rargs, meta))


def _variant(v, bm=32, bn=32, bk=8, k=64, a=f16, c=f32):
    nt = (bm // 8) * (bn // 8) * 32
    return _ir(K.matmul_mma_variant_kernel, a(8), a(8), c(8), 64, 64, BM=bm, BN=bn, BK=bk, K=k, NT=nt, VARIANT=v), nt


@pytest.mark.parametrize("bm,bn,bk,k", [(32, 32, 8, 64), (32, 32, 16, 100), (16, 32, 8, 4100), (32, 16, 8, 24), (8, 8, 8, 8)])
def test_reference_mma_kernel_is_lifted(bm, bn, bk, k):
    nt = (bm // 8) * (bn // 8) * 32
    spec = analyze(_ir(K.matmul_mma_kernel, f16(8), f16(8), f32(8), 64, 64, BM=bm, BN=bn, BK=bk, K=k, NT=nt), nt)
    assert (spec.a, spec.b, spec.c, spec.m_sym, spec.n_sym) == ("a", "b", "c", "M", "N")
    assert (spec.K, spec.TM, spec.TN, spec.row_axis) == (k, bm, bn, 1)
    assert spec.c_dtype == DType.F32 and not spec.c_f16


def test_f16_output_and_f32_inputs_are_lifted():
    spec = analyze(_ir(K.matmul_mma_f16out_kernel, f16(8), f16(8), f16(8), 64, 64, BM=32, BN=32, BK=8, K=64, NT=512), 512)
    assert spec.c_dtype == DType.F16 and spec.c_f16
    spec = analyze(_ir(K.matmul_mma_kernel, f32(8), f32(8), f32(8), 64, 64, BM=32, BN=32, BK=8, K=64, NT=512), 512)
    assert spec.a_dtype == DType.F32 and spec.b_dtype == DType.F32


@pytest.mark.parametrize("variant", [1, 2, 3, 4, 5, 6, 7, 8, 11, 12])
def test_non_gemm_variants_are_not_lifted(variant):
    ir, nt = _variant(variant)
    with pytest.raises(Unsupported):
        analyze(ir, nt)


@pytest.mark.parametrize("variant,row_axis", [(0, 1), (9, 1), (10, 0)])
def test_equivalent_gemm_variants_are_lifted(variant, row_axis):
    ir, nt = _variant(variant)
    spec = analyze(ir, nt)
    assert spec.row_axis == row_axis and spec.K == 64


def test_compile_routes_lifted_and_literal_kernels():
    z = f16(8)
    ck = K.matmul_mma_variant_kernel.compile(z, z, f32(8), 64, 64, BM=32, BN=32, BK=8, K=64, NT=512, VARIANT=0)
    assert ck.geometry.kind == "gemm" and "__builtin_amdgcn_mfma_f32_32x32x16_f16" in ck.src
    ck = K.matmul_mma_variant_kernel.compile(z, z, f32(8), 64, 64, BM=32, BN=32, BK=8, K=64, NT=512, VARIANT=1)
    assert ck.geometry.kind == "thread" and "mfma" not in ck.src


def test_lift_can_be_disabled(monkeypatch):
    import eas

    monkeypatch.setenv("EAS_HIP_DISABLE_GEMM_LIFT", "1")
    z = f16(8)
    ck = eas.kernel(K.matmul_mma_kernel.fn).compile(z, z, f32(8), 64, 64, BM=32, BN=32, BK=8, K=64, NT=512)
    assert ck.geometry.kind == "thread"


def test_non_gemm_kernels_are_untouched():
    # a dot over global memory (gemv) and elementwise kernels keep their literal lowering
    ck = K.gemv_dot_kernel.compile(f32(8), f32(8), f32(8), 64, 32, 64, BLOCK=64)
    assert ck.geometry.kind != "gemm"
    ck = K.add_kernel.compile(f32(8), f32(8), f32(8), 8, BLOCK=256)
    assert ck.geometry.kind == "spmd"


# ---- fp32 threadgroup-tile (mk.dot) pattern ------------------------------------


def _tiled(kern, *args, **meta):
    z = np.zeros(8, np.float32)
    return kern.compile(z, z, z, *args, **meta)


@pytest.mark.parametrize("bm,bn,bk,k,nt", [(32, 32, 32, 1024, 256), (16, 64, 16, 640, 256), (32, 32, 32, 1000, 256),
                                           (16, 16, 16, 40, 64)])
def test_reference_tiled_kernel_is_lifted(bm, bn, bk, k, nt):
    ck = _tiled(K.matmul_tiled_kernel, 64, 64, 0, 0, BM=bm, BN=bn, BK=bk, K=k, NT=nt)
    assert ck.geometry.kind == "gemm"
    p = ck.geometry.params
    assert (p["TM"], p["TN"], p["K"]) == (bm, bn, k)
    assert (p["m_sym"], p["n_sym"], p["row_base"], p["col_base"], p["col_masked"]) == ("M", "N", "PID_M_BASE",
                                                                                        "PID_N_BASE", True)


def test_full_tile_kernel_is_lifted_without_bounds():
    ck = _tiled(K.matmul_tiled_full_kernel, 64, 64, BM=16, BN=64, BK=16, K=640, NT=256)
    p = ck.geometry.params
    assert ck.geometry.kind == "gemm" and p["m_sym"] is None and p["col_masked"] is False
    assert p["row_base"] is None and p["col_base"] is None


@pytest.mark.parametrize("variant", [1, 2, 3, 4, 5, 6, 7])
def test_non_gemm_tiled_variants_are_not_lifted(variant):
    ck = _tiled(K.matmul_tiled_variant_kernel, 64, 64, BM=16, BN=16, BK=16, K=48, NT=64, VARIANT=variant)
    assert ck.geometry.kind == "thread"
    with pytest.raises(Unsupported):
        gemm_lift.analyze_dot(ck.ir, 64)


@pytest.mark.parametrize("variant", [0, 8, 9])
def test_equivalent_tiled_variants_are_lifted(variant):
    ck = _tiled(K.matmul_tiled_variant_kernel, 64, 64, BM=16, BN=16, BK=16, K=48, NT=64, VARIANT=variant)
    assert ck.geometry.kind == "gemm" and ck.geometry.params["K"] == 48


def test_tiled_launch_rectangles():
    from easy_as_amd.runtime.hip import plan_launch

    ck = _tiled(K.matmul_tiled_kernel, 100, 200, 0, 0, BM=32, BN=32, BK=32, K=64, NT=256)
    z = np.zeros(100 * 64, np.float32)
    args = {"a": z, "b": np.zeros(64 * 200, np.float32), "c": np.zeros(100 * 200, np.float32), "M": 100, "N": 200,
            "PID_M_BASE": 0, "PID_N_BASE": 0}
    plan = plan_launch(ck, args, grid=(7, 4, 1))
    assert plan.hidden == (0, 100, 0, 200) and plan.grid == (2 * 4, 1, 1)
    # the edge strips of the reference's split launch: origin = tile * base, clamped to M / N
    plan = plan_launch(ck, {**args, "PID_N_BASE": 6}, grid=(1, 4, 1))
    assert plan.hidden == (0, 100, 192, 200) and plan.grid == (2, 1, 1)
    plan = plan_launch(ck, {**args, "PID_M_BASE": 3}, grid=(6, 1, 1))
    assert plan.hidden == (96, 100, 0, 192) and plan.grid == (3, 1, 1)
    # a launch that would touch memory past a buffer raises instead of running
    with pytest.raises(ValueError):
        plan_launch(ck, {**args, "a": np.zeros(10, np.float32)}, grid=(7, 4, 1))
    full = _tiled(K.matmul_tiled_full_kernel, 96, 192, BM=32, BN=32, BK=32, K=64, NT=256)
    plan = plan_launch(full, {"a": np.zeros(96 * 64, np.float32), "b": np.zeros(64 * 200, np.float32),
                              "c": np.zeros(96 * 200, np.float32), "M": 96, "N": 200}, grid=(6, 3, 1))
    assert plan.hidden == (0, 96, 0, 192)
