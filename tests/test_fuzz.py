"""Differential tests on seeded random eas programs (``tests/fuzz_kernels.py``).

CPU: every generated program traces, passes the IR verifier after the pass pipeline, lowers to
gfx950 HIP and compiles with hiprtc, and runs in the oracle interpreter.  GPU: every output
element of the HIP launch equals the oracle's bit for bit (NaN matches NaN), for SPMD kernels and
for thread-mode kernels with and without a threadgroup-memory exchange.  Together they cover the
DSL's arithmetic (f32 and f16, fused and unfused products), u32 index math with wrap-around,
masks, where, conversions and two stores to the same element."""

from __future__ import annotations

import numpy as np
import pytest

import fuzz_kernels as F
from oracle import interp

CPU_SEEDS = range(24)
GPU_SEEDS = range(200)


def _args(seed: int):
    mode, n, block = F.case(seed)
    src = F.spmd_source(seed) if mode == "spmd" else F.thread_source(seed)
    return mode, n, block, src


def test_generator_is_deterministic_and_varied():
    assert F.spmd_source(3) == F.spmd_source(3) and F.thread_source(4) == F.thread_source(4)
    srcs = {F.spmd_source(s) for s in range(20)}
    assert len(srcs) == 20
    joined = "".join(srcs) + "".join(F.thread_source(s) for s in range(20))
    for op in ("mk.fma(", "mk.where(", "mk.to_f16(", "mk.to_f32(", " // ", " % ", " < ", " & ", " | ", "~",
               "mk.barrier()", "mk.alloc_tg(", "mk.lane_id()", "mk.sg_id()"):
        assert op in joined, op


@pytest.mark.parametrize("seed", CPU_SEEDS)
def test_random_program_compiles_and_runs_in_the_oracle(seed):
    from easy_as_amd.runtime.hip import compile_code
    from easy_as_amd.runtime.hip_ext import load_hip_ext

    mode, n, block, src = _args(seed)
    k = F.build(src)
    x, y, z, h, out, out16 = F.inputs(seed, n)
    ck = k.compile(x, y, z, h, out, out16, n, BLOCK=block)
    assert ck.launch_mode == mode
    ref = interp.run_kernel(k, x, y, z, h, out, out16, n, BLOCK=block)
    assert ref["out"].shape == (n,) and ref["out16"].shape == (n,)
    mod = load_hip_ext(require=False)
    if mod is None:
        pytest.skip("the _hip extension is not built")
    assert compile_code(mod, ck.src, ck.ir.name)[:4] == b"\x7fELF"


def test_same_values_treats_nans_alike_and_nothing_else():
    a = np.array([1.0, np.nan, -0.0], np.float32)
    assert F.same_values(a, np.array([1.0, -np.nan, -0.0], np.float32))
    assert not F.same_values(a, np.array([1.0, np.nan, 0.0], np.float32))  # -0 vs +0
    assert not F.same_values(a, np.array([1.0, 2.0, -0.0], np.float32))


@pytest.mark.gpu
@pytest.mark.parametrize("seed", GPU_SEEDS)
def test_random_program_matches_the_oracle_on_the_gpu(seed, gpu_runtime):
    mode, n, block, src = _args(seed)
    print(f"fuzz seed {seed}: {mode} N={n} BLOCK={block}", flush=True)
    k = F.build(src)
    x, y, z, h, out, out16 = F.inputs(seed, n)
    ref = interp.run_kernel(k, x, y, z, h, out, out16, n, BLOCK=block)
    k(x, y, z, h, out, out16, n, BLOCK=block)
    for name, got in (("out", out), ("out16", out16)):
        if not F.same_values(got, ref[name]):
            bad = np.flatnonzero(got.view(np.uint32 if got.dtype == np.float32 else np.uint16)
                                 != ref[name].view(np.uint32 if got.dtype == np.float32 else np.uint16))
            i = int(bad[0])
            pytest.fail(f"seed {seed} ({mode}, N={n}, BLOCK={block}): {name}[{i}] = {got[i]!r}, oracle "
                        f"{ref[name][i]!r}; {bad.size} elements differ\n{src}")
