"""bench.py's command line, its GEMM phase-stamp instrumentation and its load-cost microbenchmark.

The CPU tests check argument handling and that the stamped copies of the 8-wave and fp32 GEMM
sources are built (the edits find their anchors in the generated source, and hiprtc compiles the
result), and that the microbenchmark source compiles with every case; the GPU tests run the
stamped kernels and the microbenchmark once and check what they report."""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import pytest

import eas

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402
import kernels as K  # noqa: E402


def _main(monkeypatch, *argv: str) -> int:
    monkeypatch.setattr(sys, "argv", ["bench.py", *argv])
    return bench.main()


@pytest.mark.parametrize("argv", [
    ("--gpus", "2"),
    ("--workload", "add", "--shape", "64,64,64"),
    ("--workload", "mma", "--shape", "64,64"),
    ("--workload", "mma", "--shape", "64,0,64"),
    ("--workload", "add", "--phases"),
    ("--workload", "add", "--data", "ones"),
])
def test_refused_arguments_exit_2(monkeypatch, argv):
    assert _main(monkeypatch, *argv) == 2


def test_shape_override_changes_only_the_shape(monkeypatch):
    monkeypatch.setitem(bench.SHAPE_OVERRIDE, "mma", (4096, 4096, 512))
    kname, m, n, k, da, db, desc = bench._config("mma")
    assert (kname, m, n, k, da, db) == ("matmul_mma_kernel", 4096, 4096, 512, "u", "u")
    assert "shape override" in desc and "K=512" in desc
    assert bench._config("prefill")[1:4] == (8192, 8192, 8192)


def _pp_source(name: str):
    import torch

    from easy_as_amd.runtime.hip import plan_launch

    kname, m, n, k, *_ = bench._config(name)
    dt = torch.bfloat16 if name.endswith("bf16") else torch.float16
    a, b = torch.empty(m * k, dtype=dt), torch.empty(k * n, dtype=dt)
    c = torch.empty(m * n, dtype=torch.float16 if name == "prefill" else torch.float32)
    ck = getattr(K, kname).compile(a, b, c, m, n, BM=32, BN=32, BK=8, K=k, NT=512)
    plan = plan_launch(ck, {"a": a, "b": b, "c": c, "M": m, "N": n},
                       grid=(K.cdiv(n, 32), K.cdiv(m, 32), 1), compute_units=256)
    return ck, plan


@pytest.mark.parametrize("name", ["mma", "prefill", "mma_bf16"])
def test_stamped_source_finds_every_anchor(name):
    ck, plan = _pp_source(name)
    assert plan.entry.endswith("__pp")
    src = bench._stamped_pp_source(ck.src, plan.entry)
    for slot in range(5):
        assert f"EAS_STAMP({slot});" in src
    assert "EAS_STAMP_XCD();" in src and "__eas_stamps) {" in src
    assert not src.startswith("// eas-launch")  # the stamped copy has one more argument


def test_stamped_source_compiles():
    from easy_as_amd.runtime.hip import compile_code
    from easy_as_amd.runtime.hip_ext import load_hip_ext

    mod = load_hip_ext(require=False)
    if mod is None:
        pytest.skip("the _hip extension is not built")
    ck, plan = _pp_source("mma")
    code = compile_code(mod, bench._stamped_pp_source(ck.src, plan.entry), ck.ir.name)
    assert code[:4] == b"\x7fELF"


def test_stamped_source_rejects_an_unexpected_shape():
    ck, plan = _pp_source("mma")
    with pytest.raises(RuntimeError, match="unexpected GEMM source shape"):
        bench._stamped_pp_source(ck.src.replace("    if (g == 1) __syncthreads();\n    for (int kt", "    for (int kt"),
                                 plan.entry)


def _f32_source(name: str):
    from easy_as_amd.runtime.hip import plan_launch

    kname, m, n, k, *_ = bench._config(name)
    z = np.zeros(1, np.float32)
    ck = K.matmul_tiled_kernel.compile(z, z, z, m, n, 0, 0, BM=32, BN=32, BK=32, K=k, NT=256)
    plan = plan_launch(ck, {"M": m, "N": n, "PID_M_BASE": 0, "PID_N_BASE": 0},
                       grid=(K.cdiv(n, 32), K.cdiv(m, 32), 1), compute_units=256)
    return ck, plan.entry or ck.geometry.entry


@pytest.mark.parametrize("name, entry", [("tiled1024", "matmul_tiled_kernel"),
                                         ("tiled2048", "matmul_tiled_kernel__t128")])
def test_stamped_f32_source_stamps_only_its_entry(name, entry):
    from easy_as_amd.runtime.hip import compile_code
    from easy_as_amd.runtime.hip_ext import load_hip_ext

    ck, got = _f32_source(name)
    assert got == entry
    src = bench._stamped_f32_source(ck.src, entry)
    for slot in range(5):
        assert src.count(f"EAS_F32_STAMP({slot});") == 1
    assert src.count("EAS_F32_CLOCK(6);") == src.count("EAS_F32_CLOCK(7);") == src.count("EAS_F32_XCD();") == 1
    assert src.count("unsigned long long* __restrict__ __eas_stamps") == 1
    mod = load_hip_ext(require=False)
    if mod is not None:
        assert compile_code(mod, src, ck.ir.name)[:4] == b"\x7fELF"
    with pytest.raises(RuntimeError, match="unexpected fp32 GEMM source shape"):
        bench._stamped_f32_source(ck.src.replace("  __syncthreads();  // stage 0 landed\n", "  __syncthreads();\n"),
                                  entry)


def _ws_source(m, n, k):
    from easy_as_amd.runtime.hip import plan_launch

    z = np.zeros(1, np.float16)
    ck = K.matmul_mma_kernel.compile(z, z, np.zeros(1, np.float32), m, n, BM=32, BN=32, BK=8, K=k, NT=512)
    plan = plan_launch(ck, {"M": m, "N": n}, grid=(K.cdiv(n, 32), K.cdiv(m, 32), 1), compute_units=256)
    return ck, plan.entry


@pytest.mark.parametrize("mnk, entry", [((2048, 2048, 2048), "matmul_mma_kernel__t128"),
                                        ((512, 14336, 1024), "matmul_mma_kernel__t128x256"),
                                        ((1024, 1024, 1024), "matmul_mma_kernel__t64x64")])
def test_stamped_ws_source_stamps_only_its_entry(mnk, entry):
    from easy_as_amd.runtime.hip import compile_code
    from easy_as_amd.runtime.hip_ext import load_hip_ext

    ck, got = _ws_source(*mnk)
    assert got == entry
    src = bench._stamped_ws_source(ck.src, entry)
    for slot in range(5):
        assert src.count(f"EAS_WS_STAMP({slot});") == 1
    assert src.count("EAS_WS_CLOCK(6);") == src.count("EAS_WS_CLOCK(7);") == src.count("EAS_WS_XCD();") == 1
    assert src.count("unsigned long long* __restrict__ __eas_stamps") == 2  # the body and the entry
    assert src.count(", nullptr);") == 3  # the other tile entries pass no stamp buffer
    mod = load_hip_ext(require=False)
    if mod is not None:
        assert compile_code(mod, src, ck.ir.name)[:4] == b"\x7fELF"
    with pytest.raises(RuntimeError, match="unexpected f16 GEMM source shape"):
        bench._stamped_ws_source(ck.src.replace("  __syncthreads();  // stage 0 landed\n  afrag_t", "  afrag_t"),
                                 entry)


@pytest.mark.parametrize("mnk, entry", [((2048, 2048, 2048), "matmul_mma_kernel__t128"),
                                        ((512, 14336, 1024), "matmul_mma_kernel__t128x256"),
                                        ((2048, 1024, 2048), "matmul_mma_kernel__t128x64")])
def test_stamped_ws_source_under_the_32x32_mfma(monkeypatch, mnk, entry):
    # EAS_HIP_GEMM_MFMA=32 changes the 128 x 128 and 128 x 256 entries' body; the stamps follow it
    monkeypatch.setenv("EAS_HIP_GEMM_MFMA", "32")
    z = np.zeros(1, np.float16)
    m, n, k = mnk
    ck = eas.kernel(K.matmul_mma_kernel.fn).compile(z, z, np.zeros(1, np.float32), m, n, BM=32, BN=32, BK=8, K=k,
                                                    NT=512)
    assert "eas_gemm_t128<CT, K, 128, 32>" in ck.src
    src = bench._stamped_ws_source(ck.src, entry)
    assert src.count("EAS_WS_STAMP(0);") == 1 and src.count(", nullptr);") == 3
    assert src.count(f"eas_gemm_t128<CT, K, {128 if entry.endswith('t128') else 256}, 32>") >= 1


@pytest.mark.gpu
@pytest.mark.parametrize("shape, workgroups, mfma_clocks", [((2048, 2048, 2048), 256, 256),
                                                            ((512, 14336, 1024), 224, 512),
                                                            ((1024, 1024, 1024), 256, 64)])
def test_phases_of_the_128_row_entries(monkeypatch, shape, workgroups, mfma_clocks):
    import torch

    from easy_as_amd.runtime import get_runtime

    monkeypatch.setitem(bench.SHAPE_OVERRIDE, "mma", shape)
    print(f"phases: mma {shape}", flush=True)
    ph = bench._gemm_phases("mma", get_runtime("hip"), torch, trials=2, lead=3)
    assert ph["workgroups"] == workgroups and ph["mfma_clocks_per_stage"] == mfma_clocks
    assert 0 < ph["prologue"] < ph["loop_median"] < ph["end_median"] <= ph["end_last"] < 1000
    assert mfma_clocks <= ph["loop_clocks_per_stage"] < max(8 * mfma_clocks, 1024)
    assert 0.5 < ph["loop_shader_GHz"] < 3.0


@pytest.mark.gpu
@pytest.mark.parametrize("name, stages, mfma_clocks", [("tiled1024", 32, 1024), ("tiled2048", 64, 4096)])
def test_phases_of_the_fp32_entries(name, stages, mfma_clocks):
    import torch

    from easy_as_amd.runtime import get_runtime

    print(f"phases: {name}", flush=True)
    ph = bench._gemm_phases(name, get_runtime("hip"), torch, trials=2, lead=3)
    assert ph["workgroups"] == 256 and ph["mfma_clocks_per_stage"] == mfma_clocks
    assert ph["workgroup_to_xcd_is_modulo_8"] is True and len(ph["loop_median_per_xcd"]) == 8
    assert 0 < ph["prologue"] < ph["loop_median"] < ph["end_median"] <= ph["end_last"] < 1000
    # a stage costs at least its MFMAs; the shader clock is a plausible one
    assert mfma_clocks <= ph["loop_clocks_per_stage"] < 2 * mfma_clocks
    assert 0.5 < ph["loop_shader_GHz"] < 3.0


@pytest.mark.gpu
def test_phases_of_a_short_k_launch(monkeypatch):
    import torch

    from easy_as_amd.runtime import get_runtime

    monkeypatch.setitem(bench.SHAPE_OVERRIDE, "mma", (4096, 4096, 512))
    print("phases: mma 4096 x 4096 x 512", flush=True)
    ph = bench._gemm_phases("mma", get_runtime("hip"), torch, trials=2, lead=3)
    assert ph["entry"] == "matmul_mma_kernel__pp" and ph["workgroups"] == 256
    assert ph["workgroup_to_xcd_is_modulo_8"] is True
    assert len(ph["loop_median_per_xcd"]) == 8
    assert 0 < ph["prologue"] < ph["loop_median"] < ph["end_median"] <= ph["end_last"]
    assert ph["loop_min"] <= ph["loop_median"] <= ph["loop_max"]
    assert ph["store_issue"] > 0 and ph["store_complete"] >= 0
    # 16 stages of BK = 32: a few microseconds of loop, well under a millisecond
    assert np.isfinite(ph["end_last"]) and ph["end_last"] < 1000


def test_loadcost_source_has_every_case():
    from easy_as_amd.runtime.hip import compile_code
    from easy_as_amd.runtime.hip_ext import load_hip_ext

    entries = [e for e, _, _ in bench._LOADCOST_CASES]
    assert len(set(entries)) == len(entries)
    for e, nw, _ in bench._LOADCOST_CASES:
        assert f"LC_ENTRY({e}," in bench._LOADCOST_SRC and nw in (4, 8)
    mod = load_hip_ext(require=False)
    if mod is None:
        pytest.skip("the _hip extension is not built")
    code = compile_code(mod, bench._LOADCOST_SRC, "loadcost")
    assert code[:4] == b"\x7fELF"


@pytest.mark.gpu
def test_loadcost_runs(capsys):
    import torch

    from easy_as_amd.runtime import get_runtime

    print("loadcost microbenchmark", flush=True)
    assert bench._loadcost_main(get_runtime("hip"), torch, iters=200) == 0
    line = json.loads(capsys.readouterr().out.strip().splitlines()[-1])
    rows = {r["entry"]: r for r in line["cases"]}
    # MFMAs alone run at one per 64 clocks; loads a sibling issues with SGPR addressing are free
    assert 1000 < rows["lc_w4_mfma"]["simd_clocks_per_16_mfma_median"] < 1100
    assert rows["lc_w8_salu_producers2"]["loads_per_16_sibling_mfma"] == 2.0


@pytest.mark.gpu
def test_dispatch_probe_measures_a_rate():
    # the empty kernel the add line is compared with: 2^21 workgroups of 32 threads (the add's
    # launch at N = 2^28) dispatch at a few workgroups per ns on one MI355X
    from easy_as_amd.runtime import get_runtime

    print("dispatch probe", flush=True)
    rate = bench._dispatch_probe(get_runtime("hip"), 1 << 21, 32, trials=3)
    assert 1.0 < rate < 50.0, rate
