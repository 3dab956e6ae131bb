"""GPU: kernels launched through ``eas._hip`` exactly as the reference runtime launches them.

The reference's ``MetalRuntime.run`` compiles with ``compile(src, name)``, builds argv
from buffer capsules and packed scalars (eas/runtime/metal.py:142-242) and calls
``launch(pipeline, argv, writable, threads_per_grid, threads_per_threadgroup)``
(metal.py:341-346) or ``launch_async`` + ``synchronize``; ``launch_tg`` takes
threadgroup counts (_metal.mm:1232-1379).  Each test here does the same against
``eas._hip`` and checks the outputs against the oracle bit for bit, including the
threads past a non-uniform last threadgroup.  Calls shaped for a different
convention are refused before anything launches.
"""

from __future__ import annotations

import numpy as np
import pytest

import kernels as K
from conftest import seeded_normal
from easy_as_amd.runtime.hip import pack_scalar
from easy_as_amd.runtime.hip_ext import load_hip_ext
from metal_dispatch import reference_dispatch
from oracle import ops

pytestmark = pytest.mark.gpu


def _bits_equal(x, y) -> bool:
    x, y = np.asarray(x), np.asarray(y)
    return x.shape == y.shape and x.dtype == y.dtype and np.array_equal(x.view(np.uint8), y.view(np.uint8))


def _argv(mod, ck, host_args):
    """argv, writable and copy-backs as the reference's _build_argv makes them: a device buffer
    per array (copied in), packed little-endian scalars."""
    argv, writable, back = [], [], []
    for a in ck.ir.args:
        v = host_args[a.name]
        if a.kind == "buffer":
            buf = mod.alloc_buffer(v.nbytes, "private")
            mod.copy_from_host(buf, v)
            w = a.name in ck.writes
            argv.append(buf)
            writable.append(w)
            if w:
                back.append((buf, v))
        else:
            argv.append(pack_scalar(a.dtype, v))
            writable.append(False)
    return argv, writable, back


def _run(mod, ck, host_args, *, grid=None, form="launch"):
    pipeline = mod.compile(ck.src, ck.geometry.entry)
    argv, writable, back = _argv(mod, ck, host_args)
    tpg, tptg = reference_dispatch(ck, host_args, grid=grid)
    if form == "launch":
        mod.launch(pipeline, argv, writable, tpg, tptg)
    elif form == "async":
        mod.synchronize(mod.launch_async(pipeline, argv, writable, tpg, tptg))
    else:
        groups = grid if grid is not None else tpg
        mod.launch_tg(pipeline, argv, writable, groups, tptg)
    for buf, arr in back:
        mod.copy_to_host(buf, arr)


@pytest.fixture(scope="module")
def hip():
    return load_hip_ext(require=True)


@pytest.mark.parametrize("form", ["launch", "async"])
@pytest.mark.parametrize("n,block", [(1031, 256), (1 << 20, 256), (4099, 1024), (1, 1024)])
def test_spmd_add_through_reference_launch(hip, form, n, block):
    a, b = seeded_normal(0, n), seeded_normal(1, n)
    c = np.full(n + 5, np.nan, np.float32)
    ck = K.add_kernel.compile(a, b, c, n, BLOCK=block)
    _run(hip, ck, {"a": a, "b": b, "c": c, "N": n}, form=form)
    assert _bits_equal(c[:n], ops.add_f32(a, b)) and np.all(np.isnan(c[n:]))


def test_spmd_fma_through_reference_launch_tg(hip):
    # SPMD threadgroups are single programs, so launch_tg takes the program count too
    n = 4099
    a, b, c = seeded_normal(0, n), seeded_normal(1, n), seeded_normal(2, n)
    d = np.zeros(n, np.float32)
    ck = K.fma_kernel.compile(a, b, c, d, n, BLOCK=256)
    _run(hip, ck, {"a": a, "b": b, "c": c, "d": d, "N": n}, form="launch_tg")
    assert _bits_equal(d, ops.fmaf(a, b, c))


@pytest.mark.parametrize("form", ["launch", "async"])
def test_thread_mode_non_uniform_last_threadgroup(hip, form):
    # 1000 threads in threadgroups of 256: the last 24 threads of the fourth group do nothing
    n = 1000
    a, b, c = seeded_normal(0, 1024), seeded_normal(1, 1024), seeded_normal(2, 1024)
    d = np.full(1024, 7.0, np.float32)
    ck = K.simple_fma_kernel.compile(a, b, c, d, n, BLOCK=256)
    _run(hip, ck, {"a": a, "b": b, "c": c, "d": d, "N": n}, form=form)
    assert _bits_equal(d[:n], ops.fmaf(a[:n], b[:n], c[:n])) and np.all(d[n:] == 7.0)


@pytest.mark.parametrize("form", ["launch", "launch_tg"])
def test_thread_mode_2d_grid(hip, form):
    # out[r, c] = r over a (W/BLOCK) x H grid (tests/test_callable_grid.py:40-52)
    h, w, block = 5, 10, 4
    out = np.full(h * w + 3, -1.0, np.float32)
    ck = K.grid_callable_kernel.compile(out, h, w, BLOCK=block)
    grid = (-(-w // block), h, 1)
    _run(hip, ck, {"out": out, "H": h, "W": w}, grid=grid, form=form)
    assert np.array_equal(out[:h * w].reshape(h, w), np.repeat(np.arange(h, dtype=np.float32), w).reshape(h, w))
    assert np.all(out[h * w:] == -1.0)


def test_calls_shaped_for_another_convention_are_refused(hip):
    n = 1031
    a, b = seeded_normal(0, n), seeded_normal(1, n)
    c = np.zeros(n, np.float32)
    ck = K.add_kernel.compile(a, b, c, n, BLOCK=256)
    pipeline = hip.compile(ck.src, ck.geometry.entry)
    argv, writable, _ = _argv(hip, ck, {"a": a, "b": b, "c": c, "N": n})
    # the hidden extent is the launch's job: an argv that already carries it does not match
    with pytest.raises(ValueError, match="does not match"):
        hip.launch(pipeline, argv + [pack_scalar(ck.ir.args[-1].dtype, 5)], writable + [False], 5, (1, 1, 1))
    # a thread-count call shaped for a BLOCK-thread kernel
    with pytest.raises(ValueError, match=r"\(1, 1, 1\)"):
        hip.launch(pipeline, argv, writable, 1031, 256)
    # the workgroup form needs the hidden extent after the arguments
    with pytest.raises(ValueError, match="does not match"):
        hip.launch_groups(pipeline, argv, writable, (10, 1, 1), (32, 1, 1))
    assert hip.kernel_shape(pipeline)["kind"] == "spmd"
    # a lifted GEMM: a partial threadgroup, a buffer too short for the launch
    ha, hb = np.zeros(64 * 64, np.float16), np.zeros(64 * 64, np.float16)
    hc = np.zeros(64 * 64, np.float32)
    gk = K.matmul_mma_kernel.compile(ha, hb, hc, 64, 64, BM=32, BN=32, BK=8, K=64, NT=512)
    gp = hip.compile(gk.src, gk.geometry.entry)
    gargv, gw, _ = _argv(hip, gk, {"a": ha, "b": hb, "c": hc, "M": 64, "N": 64})
    with pytest.raises(ValueError, match="whole threadgroups"):
        hip.launch(gp, gargv, gw, (2 * 512 - 64, 2, 1), (512, 1, 1))
    short, _, _ = _argv(hip, gk, {"a": ha[:-1], "b": hb, "c": hc, "M": 64, "N": 64})
    with pytest.raises(ValueError, match="holds"):
        hip.launch(gp, short, gw, (2 * 512, 2, 1), (512, 1, 1))


# The reference's matmul kernels through the reference's launch, as metal.py:142-346 drives it:
# compile(src, name) once, argv of buffer capsules and packed scalars, launch with threads per
# grid (gx * BLOCK, gy, 1) and (BLOCK, 1, 1), or launch_tg with the threadgroup counts.  The
# library plans the lifted GEMM (entry, workgroups, covered rectangle) from M, N and the buffers.
# Every output against a float64 matmul of the same inputs: <= 1e-5 sqrt(K) relative to max|R|
# (f16 products are exact in f32; the fp32 tiled bar of the configs).
_REF_MATMULS = [
    # (kernel, M, N, K, form)
    ("mma", 4096, 4096, 4100, "launch"),
    ("mma", 4096, 4096, 4096, "launch_tg"),
    ("mma", 300, 520, 200, "launch"),
    ("mma", 257, 264, 72, "async"),
    ("mma", 16, 14336, 4096, "launch_tg"),
    ("mma", 1024, 1024, 1024, "launch"),
    ("tiled", 1024, 1024, 1024, "launch"),
    ("tiled", 1024, 1024, 1024, "launch_tg"),
    ("tiled", 300, 200, 64, "async"),
]


@pytest.mark.parametrize("case", _REF_MATMULS, ids=lambda c: f"{c[0]}-{c[1]}x{c[2]}x{c[3]}-{c[4]}")
def test_lifted_matmuls_through_reference_launch(hip, case):
    import math

    import torch

    kind, m, n, k, form = case
    rng_a, rng_b = np.random.default_rng(0), np.random.default_rng(1)
    if kind == "mma":
        a = rng_a.uniform(-1, 1, m * k).astype(np.float16)
        b = rng_b.uniform(-1, 1, k * n).astype(np.float16)
        c = np.full(m * n, np.nan, np.float32)
        ck = K.matmul_mma_kernel.compile(a, b, c, m, n, BM=32, BN=32, BK=8, K=k, NT=512)
        args = {"a": a, "b": b, "c": c, "M": m, "N": n}
        grid = K.mma_grid({"BM": 32, "BN": 32}, args)
    else:
        a = (rng_a.standard_normal(m * k, dtype=np.float32) / np.float32(math.sqrt(k))).astype(np.float32)
        b = (rng_b.standard_normal(k * n, dtype=np.float32) / np.float32(math.sqrt(k))).astype(np.float32)
        c = np.full(m * n, np.nan, np.float32)
        ck = K.matmul_tiled_kernel.compile(a, b, c, m, n, 0, 0, BM=32, BN=32, BK=32, K=k, NT=256)
        args = {"a": a, "b": b, "c": c, "M": m, "N": n, "PID_M_BASE": 0, "PID_N_BASE": 0}
        grid = (K.cdiv(n, 32), K.cdiv(m, 32), 1)
    assert ck.geometry.kind == "gemm"
    print(f"reference launch of the lifted {kind} matmul {m}x{n}x{k} by {form}", flush=True)
    _run(hip, ck, args, grid=grid, form=form)
    ref = torch.from_numpy(a).cuda().double().reshape(m, k) @ torch.from_numpy(b).cuda().double().reshape(k, n)
    got = torch.from_numpy(c).cuda().double().reshape(m, n)
    assert bool(torch.isfinite(got).all())
    err = float((got - ref).abs().max() / ref.abs().max())
    assert err <= 1e-5 * math.sqrt(k), err


def test_lifted_matmul_launch_covering_no_output_runs_nothing(hip):
    # the tiled kernel offsets its threadgroup ids by PID_M_BASE: a base past M covers no row of C
    m, n, k = 96, 64, 32
    a, b = np.ones(m * k, np.float32), np.ones(k * n, np.float32)
    c = np.full(m * n, 7.0, np.float32)
    ck = K.matmul_tiled_kernel.compile(a, b, c, m, n, 0, 0, BM=32, BN=32, BK=32, K=k, NT=256)
    args = {"a": a, "b": b, "c": c, "M": m, "N": n, "PID_M_BASE": 3, "PID_N_BASE": 0}
    _run(hip, ck, args, grid=(2, 3, 1), form="launch")
    assert np.all(c == 7.0)
    # the rows from base 1 on: rows 32-95 hold K, rows 0-31 are untouched
    args["PID_M_BASE"] = 1
    _run(hip, ck, args, grid=(2, 3, 1), form="launch_tg")
    out = c.reshape(m, n)
    assert np.all(out[:32] == 7.0) and np.all(out[32:] == float(k))
