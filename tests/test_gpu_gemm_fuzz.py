"""Seeded random shapes through the lifted GEMMs, against float64.

32 cases.  Each draws a kernel from the reference's workloads (f16-input simdgroup MMA with f32
or f16 output, the bf16 variant, the fp32 threadgroup-tile kernel) and M, N, K from 1 to ~800 on a
log scale, so the cases cover:
* skinny and full-tile launches;
* odd K (A rows not 4-byte aligned) and K below one stage;
* N not a multiple of 4, and every entry the launch plan picks by itself;
* each shape again on the 128 x 128, 128 x 256 and 128 x 64-tile entries
  (``EAS_HIP_GEMM_ENTRY=tile128``, ``tile128x256``, ``tile128x64``), which the plan picks by
  itself only for launches of more than 128 rows.

Each case also runs once through the reference's native launch convention
(``_hip.launch(pipeline, argv, writable, threads_per_grid, threads_per_threadgroup)``,
argv of device buffers and packed scalars as eas/runtime/metal.py:142-346 builds it),
which the C library plans (``eas_hip_plan_gemm``).

Every output is checked with the tolerances the parity bars state.  The output buffer is
longer than M x N, and its tail must keep its sentinel (no write past C)."""

from __future__ import annotations

import math
import random

import numpy as np
import pytest

import kernels as K
from oracle import ops

pytestmark = pytest.mark.gpu

CASES = range(32)
KINDS = ("f16_f32", "f16_f16", "bf16_f32", "tiled_f32")
PAD = 1031


def _shape(seed: int) -> tuple[str, int, int, int]:
    r = random.Random(50_000 + seed)
    kind = KINDS[seed % len(KINDS)]

    def dim(hi: int) -> int:
        return max(1, int(round(math.exp(r.uniform(0.0, math.log(hi))))))

    return kind, dim(800), dim(900), dim(700)


def _native_launch(rt, kern, host: dict, meta: dict, grid) -> None:
    """Run `kern` on `host` (NumPy arrays and scalars, the kernel's argument names) through
    ``_hip.launch`` with the reference runtime's argv and sizes; copy the written buffers back."""
    from easy_as_amd.runtime.hip import pack_scalar

    mod = rt._mod()
    ck = kern.compile(*[host[n] for n in kern.sig.parameters if n not in meta], **meta)
    pipeline = rt.kernel_handle(ck)
    argv, writable, back = [], [], []
    for a in ck.ir.args:
        v = host[a.name]
        if a.kind == "buffer":
            if not isinstance(v, np.ndarray):  # a torch CPU tensor: a NumPy view of the same memory
                import torch

                v = v.view(torch.int16).numpy() if v.dtype == torch.bfloat16 else v.numpy()
            buf = mod.alloc_buffer(v.nbytes, "private")
            mod.copy_from_host(buf, v)
            argv.append(buf)
            writable.append(a.name in ck.writes)
            if a.name in ck.writes:
                back.append((buf, v))
        else:
            argv.append(pack_scalar(a.dtype, v))
            writable.append(False)
    block = ck.block_size
    mod.launch(pipeline, argv, writable, (grid[0] * block, grid[1], grid[2]), (block, 1, 1))
    for buf, v in back:
        mod.copy_to_host(buf, v)


def test_shapes_cover_the_edges():
    shapes = [_shape(s) for s in CASES]
    assert any(k % 2 for _, _, _, k in shapes) and any(n % 4 for _, _, n, _ in shapes)
    assert any(m <= 16 for _, m, _, _ in shapes) and any(m > 256 for _, m, _, _ in shapes)
    assert any(k < 32 for _, _, _, k in shapes) and {s[0] for s in shapes} == set(KINDS)


@pytest.mark.parametrize("seed", CASES)
def test_random_shape_matches_float64(gpu_runtime, monkeypatch, seed):
    torch = pytest.importorskip("torch")
    kind, m, n, k = _shape(seed)
    print(f"gemm fuzz {seed}: {kind} M={m} N={n} K={k}", flush=True)
    rng = np.random.default_rng(seed)
    if kind == "tiled_f32":
        a = (rng.standard_normal(m * k, dtype=np.float32) / np.float32(math.sqrt(k))).astype(np.float32)
        b = (rng.standard_normal(k * n, dtype=np.float32) / np.float32(math.sqrt(k))).astype(np.float32)
        bm, bn, bk, nt = (32, 32, 32, 256) if seed % 8 < 4 else (16, 64, 16, 256)
        ref = ops.matmul_ref(a.reshape(m, k), b.reshape(k, n))
        bar = 1e-5 * math.sqrt(k)

        def run():
            c = np.full(m * n + PAD, np.nan, np.float32)
            K.matmul_tiled_kernel(a, b, c, m, n, 0, 0, BM=bm, BN=bn, BK=bk, K=k, NT=nt,
                                  _grid=(K.cdiv(n, bn), K.cdiv(m, bm), 1), _tptg=(nt, 1, 1))
            return c

        def run_native():
            c = np.full(m * n + PAD, np.nan, np.float32)
            _native_launch(gpu_runtime, K.matmul_tiled_kernel,
                           {"a": a, "b": b, "c": c, "M": m, "N": n, "PID_M_BASE": 0, "PID_N_BASE": 0},
                           {"BM": bm, "BN": bn, "BK": bk, "K": k, "NT": nt}, (K.cdiv(n, bn), K.cdiv(m, bm), 1))
            return c
    elif kind == "bf16_f32":
        a_bits = ops.f32_to_bf16(rng.uniform(-1, 1, m * k).astype(np.float32))
        b_bits = ops.f32_to_bf16(rng.uniform(-1, 1, k * n).astype(np.float32))
        ta = torch.from_numpy(a_bits.view(np.int16)).view(torch.bfloat16)
        tb = torch.from_numpy(b_bits.view(np.int16)).view(torch.bfloat16)
        ref = ops.matmul_ref(ops.bf16_to_f32(a_bits).reshape(m, k), ops.bf16_to_f32(b_bits).reshape(k, n))
        bar = 1e-5 * math.sqrt(k)

        def run():
            tc = torch.full((m * n + PAD,), float("nan"), dtype=torch.float32)
            K.matmul_mma_bf16_kernel(ta, tb, tc, m, n, BM=32, BN=32, BK=8, K=k, NT=512, OUT16=False,
                                     _grid=K.mma_grid, _tptg=(512, 1, 1))
            return tc.numpy()

        def run_native():
            tc = torch.full((m * n + PAD,), float("nan"), dtype=torch.float32)
            meta = {"BM": 32, "BN": 32, "BK": 8, "K": k, "NT": 512, "OUT16": False}
            _native_launch(gpu_runtime, K.matmul_mma_bf16_kernel, {"a": ta, "b": tb, "c": tc, "M": m, "N": n},
                           meta, K.mma_grid(meta, {"M": m, "N": n}))
            return tc.numpy()
    else:
        a = rng.uniform(-1, 1, m * k).astype(np.float16)
        b = rng.uniform(-1, 1, k * n).astype(np.float16)
        out16 = kind == "f16_f16"
        kern = K.matmul_mma_f16out_kernel if out16 else K.matmul_mma_kernel
        ref = ops.matmul_ref(a.reshape(m, k).astype(np.float32), b.reshape(k, n).astype(np.float32))
        bar = 2e-3 if out16 else 1e-5 * math.sqrt(k)

        def run():
            c = np.full(m * n + PAD, np.nan, np.float16 if out16 else np.float32)
            kern(a, b, c, m, n, BM=32, BN=32, BK=8, K=k, NT=512, _grid=K.mma_grid, _tptg=(512, 1, 1))
            return c

        def run_native():
            c = np.full(m * n + PAD, np.nan, np.float16 if out16 else np.float32)
            meta = {"BM": 32, "BN": 32, "BK": 8, "K": k, "NT": 512}
            _native_launch(gpu_runtime, kern, {"a": a, "b": b, "c": c, "M": m, "N": n}, meta,
                           K.mma_grid(meta, {"M": m, "N": n}))
            return c
    # the entry the launch plan picks, and the smaller-tile entries on every shape (their edge tiles,
    # K tails and zero-filled stages)
    for choice in ("auto", "tile128", "tile128x256", "tile128x64", "tile64", "native"):
        monkeypatch.setenv("EAS_HIP_GEMM_ENTRY", "auto" if choice == "native" else choice)
        c = run_native() if choice == "native" else run()
        got, tail = c[:m * n], c[m * n:]
        assert np.isnan(tail).all(), f"{kind} {choice} M={m} N={n} K={k}: wrote past C"
        assert np.isfinite(got).all(), f"{kind} {choice} M={m} N={n} K={k}: an output was not written"
        err = ops.rel_err(np.asarray(got, np.float64).reshape(m, n), ref)
        assert err <= min(2e-2, bar), f"{kind} {choice} M={m} N={n} K={k}: rel err {err:.3e} > {bar:.3e}"
