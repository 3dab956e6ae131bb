"""GPU parity of the bfloat16 additions: SPMD add, conversions and the bf16 MFMA GEMM.

bfloat16 is not among the reference's dtypes; its semantics here are fixed by
the oracle (``oracle.ops.f32_to_bf16`` / ``add_bf16``, pinned in
tests/test_oracle.py against exact rational rounding and torch's conversion):

* elementwise results are bit-exact (a NaN only has to stay a NaN);
* the GEMM (bf16 A and B, f32 accumulate) is held to the f16-input bar,
  ``max|C - R| / max|R| <= 2e-2`` with R the float64 matmul of the bf16 inputs,
  and, since products of bf16 values are exact in f32, to ``1e-5 * sqrt(K)``
  for an f32 output (a bf16 output adds one rounding of at most 2^-9 relative).
"""

from __future__ import annotations

import math

import numpy as np
import pytest

import kernels as K
from conftest import seeded_normal
from oracle import ops

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _bf16(bits: np.ndarray, device: str = "cuda") -> "torch.Tensor":
    """A torch bfloat16 tensor holding the given 16-bit patterns."""
    t = torch.from_numpy(np.ascontiguousarray(bits, np.uint16).view(np.int16).copy()).view(torch.bfloat16)
    return t.to(device)


def _bits(t: "torch.Tensor") -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _same_bf16(got: np.ndarray, want: np.ndarray) -> bool:
    """Bit equality with every NaN pattern treated as one."""
    gn, wn = np.isnan(ops.bf16_to_f32(got)), np.isnan(ops.bf16_to_f32(want))
    return bool(np.array_equal(gn, wn) and np.array_equal(got[~gn], want[~wn]))


_SPECIAL_F32 = np.array([0.0, -0.0, 1.0, -1.0, 1 + 2.0 ** -8, 1 + 3 * 2.0 ** -8, 3.0e38, -3.0e38,
                         np.finfo(np.float32).max, 2.0 ** -133, -2.0 ** -134, 1e-39, np.inf, -np.inf, np.nan],
                        np.float32)


def _ties(n: int, seed: int) -> np.ndarray:
    """binary32 values whose low 16 bits sit at, just below and just above a bf16 tie."""
    rng = np.random.default_rng(seed)
    hi = rng.integers(0, 2 ** 16, n, dtype=np.uint64).astype(np.uint32) << 16
    low = rng.choice(np.array([0x8000, 0x7FFF, 0x8001, 0, 0xFFFF], np.uint32), n)
    return (hi | low).view(np.float32)


@pytest.mark.parametrize("n", [1031, 1 << 20])
def test_add_bf16_bit_exact(gpu_runtime, n):
    a = ops.f32_to_bf16(seeded_normal(0, n) * np.float32(4.0))
    b = ops.f32_to_bf16(seeded_normal(1, n))
    # the ends of the bf16 range: overflow to inf, cancellation to +0, subnormals, NaN propagation
    k = min(n, _SPECIAL_F32.size)
    a[:k] = ops.f32_to_bf16(_SPECIAL_F32[:k])
    b[:k] = ops.f32_to_bf16(_SPECIAL_F32[::-1][:k])
    ta, tb = _bf16(a), _bf16(b)
    tc = torch.full((n,), float("nan"), dtype=torch.bfloat16, device="cuda")
    K.add_bf16_kernel(ta, tb, tc, n, BLOCK=256)
    torch.cuda.synchronize()
    assert _same_bf16(_bits(tc), ops.add_bf16(a, b))


def test_add_bf16_host_tensors_copy_back(gpu_runtime):
    n = 4099
    a = ops.f32_to_bf16(seeded_normal(2, n))
    b = ops.f32_to_bf16(seeded_normal(3, n))
    ta, tb = _bf16(a, "cpu"), _bf16(b, "cpu")
    tc = torch.zeros(n, dtype=torch.bfloat16)
    K.add_bf16_kernel(ta, tb, tc, n, BLOCK=1024)
    assert _same_bf16(_bits(tc), ops.add_bf16(a, b))


def test_bf16_conversion_bit_exact(gpu_runtime):
    x = np.concatenate([_SPECIAL_F32, _ties(5000, 7), seeded_normal(4, 5000) * np.float32(1e4)]).astype(np.float32)
    n = x.size
    y = torch.zeros(n, dtype=torch.bfloat16, device="cuda")
    z = torch.zeros(n, dtype=torch.float32, device="cuda")
    K.bf16_convert_kernel(torch.from_numpy(x).cuda(), y, z, n, BLOCK=256)
    torch.cuda.synchronize()
    want_y = ops.f32_to_bf16(x)
    assert _same_bf16(_bits(y), want_y)
    with np.errstate(all="ignore"):
        want_z = ops.bf16_to_f32(want_y) * x  # one binary32 RNE product
    got_z = z.cpu().numpy()
    assert np.array_equal(np.isnan(got_z), np.isnan(want_z))
    ok = ~np.isnan(want_z)
    assert np.array_equal(got_z[ok].view(np.uint32), want_z[ok].view(np.uint32))


def _gemm(m, n, k, *, out16=False, f32_in=False, seed=0, device="cuda"):
    rng = np.random.default_rng(seed)
    a32 = rng.uniform(-1, 1, m * k).astype(np.float32)
    b32 = rng.uniform(-1, 1, k * n).astype(np.float32)
    a_bits, b_bits = ops.f32_to_bf16(a32), ops.f32_to_bf16(b32)
    if f32_in:  # the kernel rounds the f32 inputs to bf16 tiles itself
        ta, tb = torch.from_numpy(a32).to(device), torch.from_numpy(b32).to(device)
    else:
        ta, tb = _bf16(a_bits, device), _bf16(b_bits, device)
    tc = torch.full((m * n,), float("nan"), dtype=torch.bfloat16 if out16 else torch.float32, device=device)
    nt = 512
    K.matmul_mma_bf16_kernel(ta, tb, tc, m, n, BM=32, BN=32, BK=8, K=k, NT=nt, OUT16=out16, _grid=K.mma_grid,
                             _tptg=(nt, 1, 1))
    if device == "cuda":
        torch.cuda.synchronize()
    c = ops.bf16_to_f32(_bits(tc)) if out16 else tc.cpu().numpy()
    ref = ops.matmul_ref(ops.bf16_to_f32(a_bits).reshape(m, k), ops.bf16_to_f32(b_bits).reshape(k, n))
    return np.asarray(c, np.float64).reshape(m, n), ref


def _check(c, ref, k, out16):
    err = ops.rel_err(c, ref)
    assert err <= 2e-2, err
    assert err <= (2.0 ** -8 if out16 else 1e-5 * math.sqrt(k)), err


@pytest.mark.parametrize("mnk", [(256, 256, 256), (300, 520, 200), (257, 264, 72), (520, 256, 1000),
                                 (130, 136, 8), (300, 256, 50),
                                 # skinny path (1, 2, 4 and 8 row tiles) and its unaligned fallback
                                 (16, 640, 1000), (33, 200, 40), (64, 136, 4096), (100, 101, 64)])
@pytest.mark.parametrize("out16", [False, True])
def test_bf16_mma_matches_f64(gpu_runtime, mnk, out16):
    m, n, k = mnk
    c, ref = _gemm(m, n, k, out16=out16)
    _check(c, ref, k, out16)


@pytest.mark.parametrize("mnk", [(300, 260, 64), (16, 96, 72)])
def test_bf16_mma_rounds_f32_inputs(gpu_runtime, mnk):
    m, n, k = mnk
    c, ref = _gemm(m, n, k, f32_in=True, seed=1)
    _check(c, ref, k, False)


def test_bf16_mma_host_tensors(gpu_runtime):
    c, ref = _gemm(130, 264, 72, out16=True, seed=2, device="cpu")
    _check(c, ref, 72, True)


@pytest.mark.parametrize("mnk", [(300, 520, 200), (520, 256, 1000), (129, 300, 8)])
def test_bf16_gemm_entries_agree(gpu_runtime, monkeypatch, mnk):
    """The 8-wave, 128 x 128, 128 x 256, 128 x 64 and 4-wave entries run the same bf16 MFMA sequence
    per output."""
    from easy_as_amd.runtime.hip import plan_launch

    m, n, k = mnk
    z = torch.zeros(1, dtype=torch.bfloat16, device="cuda")
    ck = K.matmul_mma_bf16_kernel.compile(z, z, torch.zeros(1, device="cuda"), m, n, BM=32, BN=32, BK=8, K=k,
                                          NT=512)
    outs = {}
    for choice, entry in (("8wave", "matmul_mma_bf16_kernel__pp"), ("tile128", "matmul_mma_bf16_kernel__t128"),
                          ("tile128x256", "matmul_mma_bf16_kernel__t128x256"),
                          ("tile128x64", "matmul_mma_bf16_kernel__t128x64"),
                          ("tile64", "matmul_mma_bf16_kernel__t64x64"), ("4wave", None)):
        monkeypatch.setenv("EAS_HIP_GEMM_ENTRY", choice)
        args = {"a": torch.zeros(m * k, dtype=torch.bfloat16, device="cuda"),
                "b": torch.zeros(k * n, dtype=torch.bfloat16, device="cuda"),
                "c": torch.zeros(m * n, device="cuda"), "M": m, "N": n}
        assert plan_launch(ck, args, grid=K.mma_grid({"BM": 32, "BN": 32}, args)).entry == entry
        c, ref = _gemm(m, n, k, seed=3)
        _check(c, ref, k, False)
        outs[choice] = c
    for choice in ("8wave", "tile128", "tile128x256", "tile128x64", "tile64"):
        assert ops.rel_err(outs[choice], outs["4wave"]) <= 1e-6, choice
