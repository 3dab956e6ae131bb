"""GPU parity of simdgroup-MMA matmul kernels (lifted to the MFMA GEMM, or literal).

Tolerance: ``max|C - R| / max|R| <= 2e-2`` for f16 inputs with f32 accumulate,
R = float64 matmul of the f16-rounded inputs (examples/matmul_simdgroup.py:218-222
checks against an f16 matmul).  Products of f16 values are exact in f32, so the
tests also hold the tighter ``1e-5 * sqrt(K)``.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

import kernels as K
from oracle import interp, ops

pytestmark = pytest.mark.gpu


def _inputs(m, n, k, dtype=np.float16, seed=0):
    rng = np.random.default_rng(seed)
    a = rng.uniform(-1, 1, m * k).astype(dtype)
    b = rng.uniform(-1, 1, k * n).astype(dtype)
    return a, b


def _mma(kern, a, b, c, m, n, k, bm=32, bn=32, bk=8, **extra):
    nt = (bm // 8) * (bn // 8) * 32
    kern(a, b, c, m, n, BM=bm, BN=bn, BK=bk, K=k, NT=nt, _grid=K.mma_grid, _tptg=(nt, 1, 1), **extra)


def _check(c, a, b, m, n, k):
    ref = ops.matmul_ref(a.reshape(m, k).astype(np.float32), b.reshape(k, n).astype(np.float32))
    err = ops.rel_err(np.asarray(c, np.float64).reshape(m, n), ref)
    assert err <= 2e-2
    assert err <= 1e-5 * math.sqrt(k), err


@pytest.mark.parametrize("mnk,tile", [((64, 64, 64), (32, 32, 8)), ((300, 520, 200), (32, 32, 8)),
                                      ((33, 17, 100), (32, 32, 16)), ((257, 300, 72), (16, 32, 8)),
                                      ((512, 512, 512), (32, 64, 16)),
                                      # HBM->LDS path: M/N edge tiles, K tail of 8, K below one stage
                                      ((257, 264, 72), (32, 32, 8)), ((130, 136, 8), (32, 32, 8)),
                                      ((64, 520, 24), (32, 32, 8)), ((520, 256, 1000), (32, 32, 8)),
                                      # register body: A rows 4-byte aligned (K % 8 = 2) and 2-byte (odd K)
                                      ((300, 256, 50), (32, 32, 8)), ((260, 264, 33), (32, 32, 8))])
def test_lifted_mma_matmul_matches_f64(gpu_runtime, mnk, tile):
    m, n, k = mnk
    bm, bn, bk = tile
    ck = K.matmul_mma_kernel.compile(np.zeros(1, np.float16), np.zeros(1, np.float16), np.zeros(1, np.float32),
                                     m, n, BM=bm, BN=bn, BK=bk, K=k, NT=(bm // 8) * (bn // 8) * 32)
    assert ck.geometry.kind == "gemm"
    a, b = _inputs(m, n, k)
    c = np.full(m * n, np.nan, np.float32)
    _mma(K.matmul_mma_kernel, a, b, c, m, n, k, bm, bn, bk)
    _check(c, a, b, m, n, k)


@pytest.mark.parametrize("mnk", [(1, 104, 72), (5, 640, 40), (16, 200, 1000), (12, 64, 8), (16, 136, 4096),
                                 # 2, 4 and 8 row tiles of 16 (17-128 rows)
                                 (17, 300, 72), (32, 640, 1000), (33, 200, 40), (48, 128, 8), (64, 136, 4096),
                                 (65, 300, 72), (100, 200, 1000), (128, 136, 4096)])
def test_skinny_path_matches_f64(gpu_runtime, mnk):
    m, n, k = mnk
    a, b = _inputs(m, n, k)
    c = np.full(m * n, np.nan, np.float32)
    _mma(K.matmul_mma_kernel, a, b, c, m, n, k)
    _check(c, a, b, m, n, k)


@pytest.mark.parametrize("mnk,dtype", [((1, 16448, 64), np.float16), ((16, 16390, 200), np.float16),
                                       ((7, 16448, 36), np.float16), ((16, 16390, 40), np.float32),
                                       ((12, 28672, 1000), np.float16),
                                       # 2 and 4 row tiles of 16 (17-64 rows)
                                       ((17, 16448, 72), np.float16), ((32, 16390, 200), np.float16),
                                       ((48, 16448, 1000), np.float16), ((64, 20480, 64), np.float16),
                                       ((40, 16390, 36), np.float16), ((64, 16448, 40), np.float32),
                                       # 8 row tiles (65-128 rows): 2-stage rings, two reduction passes
                                       ((65, 16448, 72), np.float16), ((128, 16390, 200), np.float16),
                                       ((100, 20480, 1000), np.float16), ((128, 16448, 36), np.float16)])
def test_skinny_path_on_128_column_groups(gpu_runtime, mnk, dtype):
    """Up to 128 rows with more 64-column groups than CUs: one workgroup per 128 columns (a last
    group of 64 or 6 columns; K % 8 != 0 and f32 inputs take the path without the DMA, 64 columns
    at a time)."""
    from easy_as_amd.runtime.hip import plan_launch

    m, n, k = mnk
    a, b = _inputs(m, n, k, dtype)
    ck = K.matmul_mma_kernel.compile(a, b, np.zeros(1, np.float32), m, n, BM=32, BN=32, BK=8, K=k, NT=512)
    args = {"a": a, "b": b, "M": m, "N": n}
    assert plan_launch(ck, args, grid=K.mma_grid({"BM": 32, "BN": 32}, args)).grid == (-(-n // 128), 1, 1)
    c = np.full(m * n, np.nan, np.float32)
    _mma(K.matmul_mma_kernel, a, b, c, m, n, k)
    _check(c, a.astype(np.float16), b.astype(np.float16), m, n, k)


@pytest.mark.parametrize("mnk,dtype", [((7, 101, 64), np.float16), ((16, 96, 72), np.float32),
                                       ((40, 101, 64), np.float16), ((64, 96, 72), np.float32),
                                       ((100, 101, 64), np.float16)])
def test_skinny_fallback_unaligned_or_f32(gpu_runtime, mnk, dtype):
    m, n, k = mnk  # N = 101: rows of B are not 16-byte aligned; f32 inputs are rounded to f16
    a, b = _inputs(m, n, k, dtype)
    c = np.full(m * n, np.nan, np.float32)
    _mma(K.matmul_mma_kernel, a, b, c, m, n, k)
    _check(c, a.astype(np.float16), b.astype(np.float16), m, n, k)


@pytest.mark.parametrize("m,n", [(16, 14336), (64, 14336), (128, 14336), (16, 28672)])
def test_decode_shape_f16_out(gpu_runtime, m, n):
    import torch

    k = 4096
    rng = np.random.default_rng(3)
    a = rng.standard_normal(m * k, dtype=np.float32).astype(np.float16)
    b = (0.02 * rng.standard_normal(k * n, dtype=np.float32)).astype(np.float16)
    tc = torch.full((m * n,), float("nan"), device="cuda", dtype=torch.float16)
    _mma(K.matmul_mma_f16out_kernel, torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda(), tc, m, n, k)
    torch.cuda.synchronize()
    c = tc.float().cpu().numpy().reshape(m, n)
    ref = ops.matmul_ref(a.reshape(m, k), b.reshape(k, n))
    assert np.isfinite(c).all() and ops.rel_err(c, ref) <= 2e-3


@pytest.mark.parametrize("k", [36, 4100])
def test_row_tail_chunk_does_not_leak_the_next_row(gpu_runtime, k):
    # K % 8 == 4: rows of A are 8-byte aligned and the last 16-byte chunk of row r holds the first
    # halves of row r + 1.  An inf there must only affect row r + 1 of C.
    m, n = 64, 128
    a, b = _inputs(m, n, k, seed=9)
    a = a.reshape(m, k)
    a[5, 0] = np.inf
    c = np.full(m * n, np.nan, np.float32)
    _mma(K.matmul_mma_kernel, a.reshape(-1), b, c, m, n, k)
    c = c.reshape(m, n)
    ok = np.ones(m, bool)
    ok[5] = False
    assert np.isfinite(c[ok]).all() and not np.isfinite(c[5]).all()
    ref = ops.matmul_ref(a[ok].astype(np.float32), b.reshape(k, n))
    assert ops.rel_err(c[ok], ref) <= 1e-5 * math.sqrt(k)


def test_rows_past_k_are_never_read(gpu_runtime):
    # B is followed by NaN padding and A rows end where the next begins: a K-tail
    # stage that read past K would put NaN (B) or wrong values (A) into C.
    m, n, k = 96, 128, 40
    a, b = _inputs(m, n, k)
    b_pad = np.concatenate([b, np.full(64 * n, np.nan, np.float16)])
    c = np.zeros(m * n, np.float32)
    _mma(K.matmul_mma_kernel, a, b_pad, c, m, n, k)
    assert np.isfinite(c).all()
    _check(c, a, b, m, n, k)


def test_lifted_partial_grid_writes_only_its_rectangle(gpu_runtime):
    m, n, k = 200, 300, 64
    a, b = _inputs(m, n, k)
    c = np.full(m * n, 7.0, np.float32)
    K.matmul_mma_kernel(a, b, c, m, n, BM=32, BN=32, BK=8, K=k, NT=512, _grid=(3, 2, 1), _tptg=(512, 1, 1))
    ref = ops.matmul_ref(a.reshape(m, k), b.reshape(k, n))
    got = c.reshape(m, n)
    assert ops.rel_err(got[:64, :96], ref[:64, :96]) <= 1e-5 * math.sqrt(k)
    assert np.all(got[64:, :] == 7.0) and np.all(got[:, 96:] == 7.0)


def test_lifted_f16_output_rounds_accumulator(gpu_runtime):
    m, n, k = 96, 160, 128
    a, b = _inputs(m, n, k)
    c = np.zeros(m * n, np.float16)
    _mma(K.matmul_mma_f16out_kernel, a, b, c, m, n, k)
    ref = ops.matmul_ref(a.reshape(m, k), b.reshape(k, n))
    # within one f16 rounding of the f32 accumulation
    assert ops.rel_err(c.astype(np.float64).reshape(m, n), ref) <= 2e-3


def test_lifted_f32_inputs_are_rounded_to_f16(gpu_runtime):
    m, n, k = 64, 96, 64
    a, b = _inputs(m, n, k, np.float32)
    c = np.zeros(m * n, np.float32)
    _mma(K.matmul_mma_kernel, a, b, c, m, n, k)
    a16, b16 = a.astype(np.float16), b.astype(np.float16)
    _check(c, a16, b16, m, n, k)


def test_swapped_grid_axes_variant(gpu_runtime):
    m, n, k = 100, 70, 64
    a, b = _inputs(m, n, k)
    c = np.zeros(m * n, np.float32)
    K.matmul_mma_variant_kernel(a, b, c, m, n, BM=32, BN=32, BK=8, K=k, NT=512, VARIANT=10,
                                _grid=(K.cdiv(m, 32), K.cdiv(n, 32), 1), _tptg=(512, 1, 1))
    _check(c, a, b, m, n, k)


def test_unlifted_variant_runs_literally_and_matches_oracle(gpu_runtime):
    # VARIANT=1 skips the last k block: not a GEMM, so the literal MMA lowering runs.
    m, n, k = 40, 48, 32
    a, b = _inputs(m, n, k)
    c = np.zeros(m * n, np.float32)
    K.matmul_mma_variant_kernel(a, b, c, m, n, BM=32, BN=32, BK=8, K=k, NT=512, VARIANT=1,
                                _grid=K.mma_grid, _tptg=(512, 1, 1))
    ref = interp.run_kernel(K.matmul_mma_variant_kernel, a, b, np.zeros(m * n, np.float32), m, n,
                            BM=32, BN=32, BK=8, K=k, NT=512, VARIANT=1, _grid=K.mma_grid)["c"]
    assert ops.rel_err(c.reshape(m, n), ref.reshape(m, n)) <= 1e-6
    full = ops.matmul_ref(a.reshape(m, k), b.reshape(k, n))
    assert ops.rel_err(c.reshape(m, n), full) > 1e-2  # really is missing a k block


@pytest.mark.parametrize("k", [4096, 4100])
def test_full_size_4096_sampled_rows(gpu_runtime, k):
    """BASELINE sizes (4096 x 4096 x K): every output row computed on the GPU;
    a seeded sample of 48 rows checked against float64 on the host."""
    import torch

    m = n = 4096
    a, b = _inputs(m, n, k, seed=1)
    ta = torch.from_numpy(a).cuda()
    tb = torch.from_numpy(b).cuda()
    tc = torch.full((m * n,), float("nan"), device="cuda", dtype=torch.float32)
    _mma(K.matmul_mma_kernel, ta, tb, tc, m, n, k)
    torch.cuda.synchronize()
    c = tc.cpu().numpy().reshape(m, n)
    assert np.isfinite(c).all()
    rows = np.sort(np.random.default_rng(7).choice(m, 48, replace=False))
    ref = a.reshape(m, k)[rows].astype(np.float64) @ b.reshape(k, n).astype(np.float64)
    assert ops.rel_err(c[rows], ref) <= 1e-5 * math.sqrt(k)


@pytest.mark.parametrize("mnk", [(300, 520, 200), (257, 264, 72), (520, 256, 1000), (136, 128, 36), (129, 300, 8),
                                 (130, 260, 4100), (100, 20000, 72)])
def test_gemm_entries_agree(gpu_runtime, monkeypatch, mnk):
    """The 8-wave (ping-pong), 128 x 128, 128 x 256, 128 x 64 and 4-wave entries on the same launch:
    each within tolerance of float64 (edge tiles, K tails of 8 and of 4, one stage, 129 rows: just above
    the skinny path)."""
    from easy_as_amd.runtime.hip import plan_launch

    m, n, k = mnk
    a, b = _inputs(m, n, k, seed=4)
    ck = K.matmul_mma_kernel.compile(a, b, np.zeros(1, np.float32), m, n, BM=32, BN=32, BK=8, K=k, NT=512)
    args = {"a": a, "b": b, "c": np.zeros(m * n, np.float32), "M": m, "N": n}
    outs = {}
    for choice, entry in (("8wave", "matmul_mma_kernel__pp"), ("tile128", "matmul_mma_kernel__t128"),
                          ("tile128x256", "matmul_mma_kernel__t128x256"), ("tile128x64", "matmul_mma_kernel__t128x64"),
                          ("tile64", "matmul_mma_kernel__t64x64"), ("4wave", None)):
        monkeypatch.setenv("EAS_HIP_GEMM_ENTRY", choice)
        assert plan_launch(ck, args, grid=K.mma_grid({"BM": 32, "BN": 32}, args)).entry == entry
        c = np.full(m * n, np.nan, np.float32)
        _mma(K.matmul_mma_kernel, a, b, c, m, n, k)
        _check(c, a, b, m, n, k)
        outs[choice] = c.reshape(m, n).astype(np.float64)
    # the same MFMA sequence per output element: equal up to f32 rounding (at most 128 rows the
    # 4-wave entry runs the skinny path, whose waves split K: another summation order)
    tol = 1e-6 if m > 128 else 1e-5 * math.sqrt(k)
    for choice in ("8wave", "tile128", "tile128x256", "tile128x64", "tile64"):
        assert ops.rel_err(outs[choice], outs["4wave"]) <= tol, choice
    if m <= 128 and -(-n // 64) > 256:  # more 64-column groups than CUs: 128-column skinny groups
        monkeypatch.setenv("EAS_HIP_GEMM_ENTRY", "auto")
        plan = plan_launch(ck, args, grid=K.mma_grid({"BM": 32, "BN": 32}, args))
        assert plan.entry is None and plan.grid == (-(-n // 128), 1, 1)


@pytest.mark.parametrize("mnk", [(300, 520, 200), (257, 264, 72), (520, 256, 1000), (130, 260, 4100),
                                 (1024, 1024, 1024)])
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("choice", ["8wave", "tile128", "tile128x256"])  # 128 x 64 is 16 x 16 x 32 only
def test_entries_with_32x32x16_mfma(gpu_runtime, monkeypatch, mnk, dtype, choice):
    """EAS_HIP_GEMM_MFMA=32: the 8-wave entry's 4 x 2 tiles of v_mfma_f32_32x32x16 per wave, and the
    128 x 128 and 128 x 256 entries' 2 x 2 (2 x 4), against float64 and against the default 16 x 16 x 32 bodies on
    the same launch (same products, other summation order inside an MFMA: equal to f32 rounding)."""
    import torch

    import eas

    m, n, k = mnk
    a, b = _inputs(m, n, k, seed=6)
    if dtype == "bf16":
        a32, b32 = (torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16) for x in (a, b))
        a, b = (t.float().numpy() for t in (a32, b32))
        da, db = a32.cuda(), b32.cuda()
        src_kernel = K.matmul_mma_bf16_kernel
    else:
        da, db = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
        src_kernel = K.matmul_mma_kernel
    monkeypatch.setenv("EAS_HIP_GEMM_ENTRY", choice)
    outs = {}
    for mi in ("32", "16"):
        monkeypatch.setenv("EAS_HIP_GEMM_MFMA", mi)
        kern = eas.kernel(src_kernel.fn)
        ck = kern.compile(da, db, torch.zeros(1, device="cuda"), m, n, BM=32, BN=32, BK=8, K=k, NT=512)
        assert f"eas_gemm_pp<CT, K, {mi}>" in ck.src and f"eas_gemm_t128<CT, K, 128, {mi}>" in ck.src
        assert f"eas_gemm_t128<CT, K, 256, {mi}>" in ck.src
        tc = torch.full((m * n,), float("nan"), device="cuda", dtype=torch.float32)
        _mma(kern, da, db, tc, m, n, k)
        torch.cuda.synchronize()
        outs[mi] = tc.cpu().numpy()
        _check(outs[mi], a, b, m, n, k)
    assert ops.rel_err(outs["32"].reshape(m, n).astype(np.float64), outs["16"].reshape(m, n).astype(np.float64)) <= 1e-6


@pytest.mark.parametrize("choice,entry", [("8wave", "matmul_mma_kernel__pp"), ("tile128", "matmul_mma_kernel__t128"),
                                          ("tile128x256", "matmul_mma_kernel__t128x256"),
                                          ("tile128x64", "matmul_mma_kernel__t128x64"),
                                          ("tile64", "matmul_mma_kernel__t64x64")])
def test_dma_entry_guard_for_an_operand_it_cannot_see(gpu_runtime, monkeypatch, choice, entry):
    """An eas.Tensor viewing torch memory at a 2-byte offset: the plan cannot see the address,
    picks a DMA entry, and the entry's own check sends the launch to its element-wise guard.
    The same view as a torch tensor is planned onto the 4-wave entry."""
    import torch

    import eas
    from easy_as_amd.runtime.hip import plan_launch

    monkeypatch.setenv("EAS_HIP_GEMM_ENTRY", choice)
    m, n, k = 160, 160, 64
    a, b = _inputs(m, n, k, seed=5)
    store = torch.zeros(m * k + 1, dtype=torch.float16, device="cuda")
    store[1:] = torch.from_numpy(a).cuda()
    ta = store[1:]
    assert ta.data_ptr() % 4 == 2
    tb = torch.from_numpy(b).cuda()
    ck = K.matmul_mma_kernel.compile(a, b, np.zeros(1, np.float32), m, n, BM=32, BN=32, BK=8, K=k, NT=512)
    grid = (K.cdiv(m, 32), K.cdiv(n, 32), 1)
    assert plan_launch(ck, {"a": ta, "b": tb, "M": m, "N": n}, grid=grid).entry is None
    ea = eas.tensor(ta, device="hip")
    assert plan_launch(ck, {"a": ea, "b": tb, "M": m, "N": n}, grid=grid).entry == entry
    for a_arg in (ta, ea):
        tc = torch.full((m * n,), float("nan"), device="cuda", dtype=torch.float32)
        _mma(K.matmul_mma_kernel, a_arg, tb, tc, m, n, k)
        torch.cuda.synchronize()
        _check(tc.cpu().numpy(), a, b, m, n, k)


# The configurations' own shapes and distributions, every output element checked.  The reference is
# a float64 matmul of the same (f16/bf16-rounded) operands, computed by torch on the GPU so that
# the 8192^3 case stays fast; tolerances as above: max|C - R| / max|R| <= 1e-5 sqrt(K) with an f32
# output, <= 2e-3 with an f16 output (one rounding of the f32 accumulator to 11 significant bits).
_BASELINE_SHAPES = [
    # (kernel, M, N, K, operand dtype, A distribution, B distribution, f16 output)
    ("matmul_mma_kernel", 4096, 4096, 4096, "f16", "u", "u", False),
    ("matmul_mma_kernel", 4096, 4096, 4100, "f16", "u", "u", False),
    ("matmul_mma_bf16_kernel", 4096, 4096, 4096, "bf16", "u", "u", False),
    ("matmul_mma_f16out_kernel", 16, 14336, 4096, "f16", "n1", "n02", True),
    ("matmul_mma_f16out_kernel", 8192, 8192, 8192, "f16", "n1", "n02", True),
    ("matmul_tiled_kernel", 1024, 1024, 1024, "f32", "ns", "ns", False),
    ("matmul_tiled_kernel", 2048, 2048, 2048, "f32", "ns", "ns", False),
]


# LLM-linear shapes on each entry the launch plan picks by itself (which one is asserted), every
# output checked the same way: 128 x 256, 128 x 128 and 64 x 64 tiles, 128-column skinny groups
# (2 and 8 row tiles), and the 128-tile entry for a launch of more than 16 rows too wide for one
# round of 128-column groups.
_PLAN_SHAPES = [
    ("matmul_mma_kernel", 512, 14336, 1024, "f16", "n1", "n02", False, "__t128x256"),
    ("matmul_mma_kernel", 2048, 2048, 2048, "f16", "u", "u", False, "__t128"),
    ("matmul_mma_kernel", 1024, 1024, 1024, "f16", "u", "u", False, "__t64x64"),
    ("matmul_mma_f16out_kernel", 48, 28672, 2048, "f16", "n1", "n02", True, ""),
    ("matmul_mma_f16out_kernel", 128, 28672, 1024, "f16", "n1", "n02", True, ""),
    ("matmul_mma_f16out_kernel", 100, 40960, 512, "f16", "n1", "n02", True, "__t128"),
]


@pytest.mark.parametrize("case", _PLAN_SHAPES, ids=lambda c: f"{c[0]}-{c[1]}x{c[2]}x{c[3]}")
def test_plan_entries_on_llm_shapes_every_output_vs_float64(gpu_runtime, case):
    import torch

    from easy_as_amd.runtime.hip import plan_launch

    kname, m, n, k, op, da, db, out16, suffix = case
    z = torch.zeros(1, dtype=torch.float16, device="cuda")
    ck = getattr(K, kname).compile(z, z, z if out16 else torch.zeros(1, device="cuda"), m, n, BM=32, BN=32, BK=8,
                                   K=k, NT=512)
    args = {"M": m, "N": n}
    entry = plan_launch(ck, args, grid=K.mma_grid({"BM": 32, "BN": 32}, args)).entry
    assert entry == (kname + suffix if suffix else None), entry
    test_baseline_shapes_every_output_vs_float64(gpu_runtime, case[:8])


@pytest.mark.parametrize("case", _BASELINE_SHAPES, ids=lambda c: f"{c[0]}-{c[1]}x{c[2]}x{c[3]}")
def test_baseline_shapes_every_output_vs_float64(gpu_runtime, case):
    import torch

    kname, m, n, k, op, da, db, out16 = case
    gen = torch.Generator(device="cuda").manual_seed(m + 3 * n + 7 * k)
    dt = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[op]

    def draw(dist, numel):
        if dist == "u":  # U(-1, 1)
            x = torch.rand(numel, generator=gen, device="cuda", dtype=torch.float32) * 2 - 1
        else:  # N(0, 1), N(0, 0.02), or N(0, 1) / sqrt(K) for the fp32 tiled matmul
            x = torch.randn(numel, generator=gen, device="cuda", dtype=torch.float32)
            x = x * {"n1": 1.0, "n02": 0.02, "ns": 1.0 / math.sqrt(k)}[dist]
        return x.to(dt)

    a, b = draw(da, m * k), draw(db, k * n)
    c = torch.full((m * n,), float("nan"), device="cuda", dtype=torch.float16 if out16 else torch.float32)
    kern = getattr(K, kname)
    if kname == "matmul_tiled_kernel":
        kern(a, b, c, m, n, 0, 0, BM=32, BN=32, BK=32, K=k, NT=256, _grid=(K.cdiv(n, 32), K.cdiv(m, 32), 1),
             _tptg=(256, 1, 1))
    else:
        _mma(kern, a, b, c, m, n, k)
    torch.cuda.synchronize()
    ref = a.double().reshape(m, k) @ b.double().reshape(k, n)
    got = c.double().reshape(m, n)
    assert bool(torch.isfinite(got).all())
    err = float((got - ref).abs().max() / ref.abs().max())
    assert err <= (2e-3 if out16 else 1e-5 * math.sqrt(k)), err


_MMA_TILES = [(8, 8, 8), (16, 16, 8), (64, 32, 8), (8, 64, 8), (64, 16, 8), (32, 32, 32)]
_TILED_TILES = [(16, 16, 8), (32, 64, 16), (64, 64, 8), (8, 32, 32), (64, 16, 4), (32, 32, 8)]


@pytest.mark.parametrize("mnk", [(300, 520, 200), (77, 130, 33)])
@pytest.mark.parametrize("kind,tile", [("mma", t) for t in _MMA_TILES] + [("tiled", t) for t in _TILED_TILES])
def test_lift_over_tile_parameters(gpu_runtime, kind, tile, mnk):
    """The reference kernels at tile shapes other than the examples' (8 x 8 to 64 x 64, BK 4-32):
    the lift accepts each, the launch plan maps the reference grid onto its own tile per
    threadgroup, and every output matches float64, with nothing written past C."""
    m, n, k = mnk
    bm, bn, bk = tile
    pad = 37
    if kind == "mma":
        nt = (bm // 8) * (bn // 8) * 32
        a, b = _inputs(m, n, k)
        c = np.full(m * n + pad, np.nan, np.float32)
        ck = K.matmul_mma_kernel.compile(a, b, c, m, n, BM=bm, BN=bn, BK=bk, K=k, NT=nt)
        _mma(K.matmul_mma_kernel, a, b, c, m, n, k, bm, bn, bk)
        ref = ops.matmul_ref(a.reshape(m, k).astype(np.float32), b.reshape(k, n).astype(np.float32))
    else:
        nt = bm * (bn // 4)
        a, b = _inputs(m, n, k, np.float32)
        c = np.full(m * n + pad, np.nan, np.float32)
        ck = K.matmul_tiled_kernel.compile(a, b, c, m, n, 0, 0, BM=bm, BN=bn, BK=bk, K=k, NT=nt)
        K.matmul_tiled_kernel(a, b, c, m, n, 0, 0, BM=bm, BN=bn, BK=bk, K=k, NT=nt,
                              _grid=(K.cdiv(n, bn), K.cdiv(m, bm), 1), _tptg=(nt, 1, 1))
        ref = ops.matmul_ref(a.reshape(m, k), b.reshape(k, n))
    assert ck.geometry.kind == "gemm", (kind, tile)
    assert np.all(np.isnan(c[m * n:])), "wrote past C"
    assert np.isfinite(c[:m * n]).all(), "an output was not written"
    err = ops.rel_err(np.asarray(c[:m * n], np.float64).reshape(m, n), ref)
    assert err <= 1e-5 * math.sqrt(k), (kind, tile, mnk, err)

