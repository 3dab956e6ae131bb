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

CPU_SEEDS = list(range(24)) + list(range(200, 212))
GPU_SEEDS = range(260)




def test_generator_is_deterministic_and_varied():
    assert F.case(3) == F.case(3) and F.case(4) == F.case(4)
    cases = [F.case(s) for s in range(40)]
    assert len({c["src"] for c in cases}) == 40
    joined = "".join(c["src"] for c in cases)
    for op in ("mk.fma(", "mk.where(", "mk.to_f16(", "mk.to_f32(", " // ", " % ", " < ", " & ", " | ", "~",
               "mk.barrier()", "mk.alloc_tg(", "mk.lane_id()", "mk.sg_id()", "mk.dot(", "mk.program_id(1)",
               "alpha", " S", "tgs = mk.alloc_tg(BLOCK)", "mk.to_u32("):
        assert op in joined, op
    assert any(c["options"].get("_grid") for c in cases)


def _run_oracle(c: dict, args: tuple) -> dict:
    return interp.run_kernel(F.build(c["src"]), *args, BLOCK=c["BLOCK"], **c["options"])


@pytest.mark.parametrize("seed", CPU_SEEDS)
def test_random_program_compiles_and_runs_in_the_oracle(seed):
    from easy_as_amd.runtime.hip import compile_code
    from easy_as_amd.runtime.hip_ext import load_hip_ext

    c = F.case(seed)
    k = F.build(c["src"])
    args = F.inputs(seed, c["N"])
    ck = k.compile(*args, BLOCK=c["BLOCK"])
    assert ck.launch_mode == c["mode"]
    ref = _run_oracle(c, args)
    assert ref["out"].shape == (c["N"],) and ref["out16"].shape == (c["N"],)
    mod = load_hip_ext(require=False)
    if mod is None:
        pytest.skip("the _hip extension is not built")
    assert compile_code(mod, ck.src, ck.ir.name)[:4] == b"\x7fELF"


def test_exchange_cases_run_whole_threadgroups():
    # a threadgroup-memory exchange reads slots other threads wrote: a partial last threadgroup
    # would read slots no thread wrote, so those cases need N to be a multiple of BLOCK (the
    # BLOCKs from seed 200 on do not all divide 2048)
    for seed in range(0, 460):
        c = F.case(seed)
        if "mk.barrier()" in c["src"] and c["mode"] == "thread":
            assert c["N"] % c["BLOCK"] == 0 and c["N"] >= 2048, (seed, c["N"], c["BLOCK"])


def test_same_values_treats_nans_alike_and_nothing_else():
    a = np.array([1.0, np.nan, -0.0], np.float32)
    assert F.same_values(a, np.array([1.0, -np.nan, -0.0], np.float32))
    assert not F.same_values(a, np.array([1.0, np.nan, 0.0], np.float32))  # -0 vs +0
    assert not F.same_values(a, np.array([1.0, 2.0, -0.0], np.float32))


@pytest.mark.gpu
@pytest.mark.parametrize("seed", GPU_SEEDS)
def test_random_program_matches_the_oracle_on_the_gpu(seed, gpu_runtime):
    c = F.case(seed)
    print(f"fuzz seed {seed}: {c['mode']} N={c['N']} BLOCK={c['BLOCK']} {c['options']}", flush=True)
    k = F.build(c["src"])
    args = F.inputs(seed, c["N"])
    ref = _run_oracle(c, args)
    k(*args, BLOCK=c["BLOCK"], **c["options"])
    for name, got in (("out", args[4]), ("out16", args[5])):
        if not F.same_values(got, ref[name]):
            bits = np.uint32 if got.dtype == np.float32 else np.uint16
            bad = np.flatnonzero(got.view(bits) != ref[name].view(bits))
            i = int(bad[0])
            pytest.fail(f"seed {seed} ({c['mode']}, N={c['N']}, BLOCK={c['BLOCK']}, {c['options']}): {name}[{i}] = "
                        f"{got[i]!r}, oracle {ref[name][i]!r}; {bad.size} elements differ\n{c['src']}")


_MAPPINGS = [{"EAS_HIP_SPMD_WG": "64"}, {"EAS_HIP_SPMD_WG": "256"}, {"EAS_HIP_SPMD_LPT": "16"},
             {"EAS_HIP_SPMD_UNROLL": "2", "EAS_HIP_SPMD_WG": "32"}]


@pytest.mark.gpu
@pytest.mark.parametrize("env", _MAPPINGS, ids=lambda e: ",".join(f"{k[13:]}={v}" for k, v in e.items()))
@pytest.mark.parametrize("seed", range(0, 80, 2))  # the SPMD cases
def test_random_spmd_program_under_every_mapping(seed, env, gpu_runtime, monkeypatch):
    """The SPMD emitter's other workgroup mappings (threads per workgroup, lanes per thread,
    programs per workgroup, split programs) give the same bits as the oracle."""
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    c = F.case(seed)
    assert c["mode"] == "spmd"
    print(f"fuzz seed {seed} {env}: N={c['N']} BLOCK={c['BLOCK']} {c['options']}", flush=True)
    k = F.build(c["src"])
    args = F.inputs(seed, c["N"])
    ref = _run_oracle(c, args)
    k(*args, BLOCK=c["BLOCK"], **c["options"])
    for name, got in (("out", args[4]), ("out16", args[5])):
        assert F.same_values(got, ref[name]), f"seed {seed} {env}: {name} differs\n{c['src']}"


def _lanes_seeds() -> list[int]:
    """The thread-mode cases the emitter takes as lanes of one program per threadgroup (element
    streams without barriers, threadgroup memory, thread positions or dot)."""
    seeds = []
    for seed in range(1, 260, 2):
        c = F.case(seed)
        if c["mode"] != "thread":
            continue
        opts = {k: v for k, v in c["options"].items() if not k.startswith("_")}
        if F.build(c["src"]).compile(*F.inputs(seed, c["N"]), BLOCK=c["BLOCK"], **opts).geometry.params.get("lanes"):
            seeds.append(seed)
    return seeds


def test_some_thread_cases_are_emitted_as_lanes():
    seeds = _lanes_seeds()
    assert len(seeds) >= 15, seeds


_LANES_ENVS = [{"EAS_HIP_THREAD_LANES": "0"}, {"EAS_HIP_SPMD_WG": "256"}, {"EAS_HIP_SPMD_LPT": "16"},
               {"EAS_HIP_SPMD_UNROLL": "2", "EAS_HIP_SPMD_WG": "32"}]


@pytest.mark.gpu
@pytest.mark.parametrize("env", _LANES_ENVS, ids=lambda e: ",".join(f"{k[8:]}={v}" for k, v in e.items()))
def test_random_thread_program_as_lanes_and_one_thread_per_thread(env, gpu_runtime, monkeypatch):
    """The thread-mode cases emitted as lanes, again with the conversion off (one HIP thread per
    Metal thread) and under other workgroup mappings of the lanes: the same bits as the oracle."""
    seeds = _lanes_seeds()
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    for seed in seeds:
        c = F.case(seed)
        print(f"fuzz seed {seed} {env}: N={c['N']} BLOCK={c['BLOCK']} {c['options']}", flush=True)
        k = F.build(c["src"])
        args = F.inputs(seed, c["N"])
        ref = _run_oracle(c, args)
        k(*args, BLOCK=c["BLOCK"], **c["options"])
        for name, got in (("out", args[4]), ("out16", args[5])):
            assert F.same_values(got, ref[name]), f"seed {seed} {env}: {name} differs\n{c['src']}"

