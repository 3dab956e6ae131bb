"""GPU parity: the HIP path against the oracle on seeded inputs.

Bit-exact for f32 add / fma and integer index work; matmul within
``max|C-R|/max|R| <= 1e-5*sqrt(K)`` (f32) and ``<= 2e-2`` (f16 inputs, f32
accumulate).  Counterparts of the reference's device tests (test_add.py,
test_fma.py, test_matmul*.py, test_threadgroup_memory.py, test_local_and_lane_id.py,
test_callable_grid.py, test_tptg_override.py, test_grid_infer.py,
test_dot_dynamic_k.py, test_kernel_cache.py, test_tensor.py, test_torch_interop.py).
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest

import eas
import kernels as K
from eas import mk
from conftest import seeded_normal
from oracle import interp, ops

pytestmark = pytest.mark.gpu


def _bits_equal(x: np.ndarray, y: np.ndarray) -> bool:
    x, y = np.asarray(x), np.asarray(y)
    return x.shape == y.shape and x.dtype == y.dtype and np.array_equal(x.view(np.uint8), y.view(np.uint8))


# -- elementwise ------------------------------------------------------------------


@pytest.mark.parametrize("n", [1, 255, 1031, 4099, 1 << 20])
@pytest.mark.parametrize("block", [256, 1024])
def test_add_numpy_bit_exact(gpu_runtime, n, block):
    a, b = seeded_normal(0, n), seeded_normal(1, n)
    c = np.full(n, np.nan, np.float32)
    K.add_kernel(a, b, c, n, BLOCK=block)
    assert _bits_equal(c, ops.add_f32(a, b))


def test_add_golden_fixture(gpu_runtime):
    from pathlib import Path

    g = np.load(Path(__file__).parent / "golden" / "add_f32_n1031.npz")
    c = np.zeros_like(g["a"])
    K.add_kernel(g["a"], g["b"], c, int(g["a"].size), BLOCK=256)
    assert _bits_equal(c, g["c"])


def test_add_masked_tail_leaves_rest_untouched(gpu_runtime):
    n, cap = 1031, 2048
    a, b = seeded_normal(0, cap), seeded_normal(1, cap)
    c = np.full(cap, 7.0, np.float32)
    K.add_kernel(a, b, c, n, BLOCK=256)
    assert _bits_equal(c[:n], ops.add_f32(a[:n], b[:n]))
    assert np.all(c[n:] == 7.0)


def test_add_f16_bit_exact(gpu_runtime):
    n = 4099
    a, b = seeded_normal(0, n, np.float16), seeded_normal(1, n, np.float16)
    c = np.zeros(n, np.float16)
    K.add_kernel(a, b, c, n, BLOCK=256)
    assert _bits_equal(c, (a.astype(np.float32) + b.astype(np.float32)).astype(np.float16))


def test_add_device_tensors_and_unaligned_view(gpu_runtime):
    n = 4099
    a_np, b_np = seeded_normal(0, n), seeded_normal(1, n)
    a, b = eas.tensor(a_np, device="hip"), eas.tensor(b_np, device="hip")
    c = eas.empty_like(a)
    K.add_kernel(a, b, c, n, BLOCK=256)
    assert _bits_equal(c.numpy(), ops.add_f32(a_np, b_np))


@pytest.mark.parametrize("n", [1031, 1 << 20])
def test_fma_spmd_bit_exact_vs_fmaf(gpu_runtime, n):
    a, b, c = seeded_normal(0, n), seeded_normal(1, n), seeded_normal(2, n)
    d = np.zeros(n, np.float32)
    K.fma_kernel(a, b, c, d, n, BLOCK=256)
    assert _bits_equal(d, ops.fmaf(a, b, c))


def test_fma_thread_mode_and_explicit(gpu_runtime):
    n = 1031
    a, b, c = seeded_normal(0, n), seeded_normal(1, n), seeded_normal(2, n)
    d = np.zeros(n, np.float32)
    K.simple_fma_kernel(a, b, c, d, n, BLOCK=256)
    assert _bits_equal(d, ops.fmaf(a, b, c))
    d2 = np.zeros(n, np.float32)
    K.explicit_fma_kernel(a, b, c, d2, n, BLOCK=256)
    assert _bits_equal(d2, ops.fmaf(a, b, c))


@eas.kernel
def _thread_add_f16(a, b, c, N, BLOCK: eas.constexpr):
    offs = mk.program_id(0) * BLOCK + mk.tid(0, BLOCK)
    m = offs < N
    mk.store(c, offs, mk.load(a, offs, m) + mk.load(b, offs, m), m)


@pytest.mark.parametrize("block", [3, 100, 200, 1000])
def test_blocks_that_are_not_powers_of_two(gpu_runtime, block):
    """SPMD add and fma and the thread-mode fma at BLOCKs whose thread count per program the
    default 32-thread workgroup does not divide (200, 1000) or does not fill (3, 100): every lane."""
    n = 7 * block + 5
    a, b, c = seeded_normal(0, n), seeded_normal(1, n), seeded_normal(2, n)
    out = np.full(n + 3, np.nan, np.float32)
    eas.kernel(K.add_kernel.fn)(a, b, out, n, BLOCK=block)
    assert _bits_equal(out[:n], ops.add_f32(a, b)) and np.all(np.isnan(out[n:])), block
    for kern in (K.fma_kernel, K.simple_fma_kernel):
        out = np.full(n + 3, np.nan, np.float32)
        eas.kernel(kern.fn)(a, b, c, out, n, BLOCK=block)
        assert _bits_equal(out[:n], ops.fmaf(a, b, c)) and np.all(np.isnan(out[n:])), (kern.name, block)


@pytest.mark.parametrize("lanes", ["1", "0"])
@pytest.mark.parametrize("block", [32, 64, 256, 1024])
def test_thread_mode_element_streams(gpu_runtime, monkeypatch, block, lanes):
    """Thread-mode element kernels emitted as lanes of one program per threadgroup (the default)
    and one thread per Metal thread give the same bits: odd sizes, a thread count below the
    kernel's own bound (only that many threads exist), explicit threadgroup grids, f16."""
    monkeypatch.setenv("EAS_HIP_THREAD_LANES", lanes)
    fma, add16 = eas.kernel(K.simple_fma_kernel.fn), eas.kernel(_thread_add_f16.fn)
    n_max = 5 * block + 7
    a, b, c = seeded_normal(0, n_max), seeded_normal(1, n_max), seeded_normal(2, n_max)
    want = ops.fmaf(a, b, c)
    for n in (1, block - 1, block, 3 * block + 1, n_max):
        d = np.full(n_max + 5, np.nan, np.float32)
        fma(a, b, c, d, n, BLOCK=block)
        assert _bits_equal(d[:n], want[:n]) and np.all(np.isnan(d[n:])), (block, n)
    assert fma.compile(a, b, c, d, 8, BLOCK=block).geometry.params.get("lanes", False) == (lanes == "1")
    # 900 threads of a kernel bounded by N = n_max: the threads past 900 do not exist
    nt = min(900, n_max - 1)
    d = np.full(n_max, np.nan, np.float32)
    fma(a, b, c, d, n_max, BLOCK=block, _nthreads=nt)
    assert _bits_equal(d[:nt], want[:nt]) and np.all(np.isnan(d[nt:])), (block, nt)
    # an explicit grid of threadgroups: every thread of them exists; the kernel's mask stops at N
    d = np.full(n_max, np.nan, np.float32)
    fma(a, b, c, d, 2 * block + 3, BLOCK=block, _grid=(2, 1, 1))
    assert _bits_equal(d[:2 * block], want[:2 * block]) and np.all(np.isnan(d[2 * block:]))
    d = np.full(n_max, np.nan, np.float32)
    fma(a, b, c, d, 2 * block + 3, BLOCK=block, _grid=(4, 1, 1))
    assert _bits_equal(d[:2 * block + 3], want[:2 * block + 3]) and np.all(np.isnan(d[2 * block + 3:]))
    h1, h2 = a.astype(np.float16), b.astype(np.float16)
    o = np.full(n_max, np.float16(7), np.float16)
    add16(h1, h2, o, n_max - 2, BLOCK=block)
    assert _bits_equal(o[:n_max - 2], ops.add_f16(h1[:n_max - 2], h2[:n_max - 2])) and np.all(o[n_max - 2:] == 7)


def test_fma_known_answer_differs_from_two_roundings(gpu_runtime):
    # (1+2^-23)(1-2^-23) - 1 = -2^-46 exactly; mul-then-add gives 0.
    e = np.float32(2.0 ** -23)
    a = np.array([1 + e] * 4, np.float32)
    b = np.array([1 - e] * 4, np.float32)
    c = np.array([-1.0] * 4, np.float32)
    d = np.zeros(4, np.float32)
    K.fma_kernel(a, b, c, d, 4, BLOCK=256)
    assert np.all(d == np.float32(-(2.0 ** -46)))


def test_unfused_mul_add_rounds_twice(gpu_runtime):
    n = 1031
    a, b, c = seeded_normal(0, n), seeded_normal(1, n), seeded_normal(2, n)
    d, e = np.zeros(n, np.float32), np.zeros(n, np.float32)
    K.multi_use_mul_kernel(a, b, c, d, e, n, BLOCK=128)
    prod = (a * b).astype(np.float32)
    assert _bits_equal(d, (prod + c).astype(np.float32))
    assert _bits_equal(e, prod)


def test_subnormal_results_are_not_flushed(gpu_runtime):
    """f32 subnormals are kept (the HIP build uses no fast-math and no flush to zero): products
    below 2^-126 and sums with subnormal addends equal NumPy's IEEE binary32 results bit for bit,
    and the fma corner fixture (subnormal inputs and outputs, signed zeros, NaN) matches on the
    GPU, NaN for NaN."""
    rng = np.random.default_rng(21)
    n = 4099

    def scaled(lo: int, hi: int) -> np.ndarray:
        return (rng.uniform(1, 2, n) * np.exp2(rng.integers(lo, hi, n)) * rng.choice([-1.0, 1.0], n)).astype(np.float32)

    a, b, c = scaled(-75, -55), scaled(-75, -55), scaled(-149, -126)
    prod = a * b
    assert np.count_nonzero((prod != 0) & (np.abs(prod) < np.finfo(np.float32).tiny)) > n // 4
    d, e = np.zeros(n, np.float32), np.zeros(n, np.float32)
    K.multi_use_mul_kernel(a, b, c, d, e, n, BLOCK=128)
    assert _bits_equal(e, prod)
    assert _bits_equal(d, prod + c)
    g = np.load(Path(__file__).parent / "golden" / "fma_f32_corners.npz")
    out = np.zeros_like(g["d"])
    K.fma_kernel(g["a"], g["b"], g["c"], out, len(out), BLOCK=256)
    nan = np.isnan(g["d"])
    assert np.array_equal(np.isnan(out), nan) and _bits_equal(out[~nan], g["d"][~nan])


def test_axpy_scalar_runtime_arg_and_cache(gpu_runtime):
    n = 1031
    a, b = seeded_normal(0, n), seeded_normal(1, n)
    for alpha in (2.0, 3.5):
        c = np.zeros(n, np.float32)
        K.axpy_kernel(a, b, c, n, alpha, BLOCK=256)
        assert _bits_equal(c, ops.fmaf(a, np.float32(alpha), b))


def test_spmd_lanes_exchange_through_threadgroup_memory(gpu_runtime):
    n = 1000
    a = seeded_normal(0, n)
    out = np.zeros(n, np.float32)
    K.spmd_tg_rotate_kernel(a, out, n, BLOCK=256)
    ref = interp.run_kernel(K.spmd_tg_rotate_kernel, a, np.zeros(n, np.float32), n, BLOCK=256)["out"]
    assert _bits_equal(out, ref)


_SPMD_ENVS = [{}, {"EAS_HIP_SPMD_WG": "32"}, {"EAS_HIP_SPMD_WG": "64"}, {"EAS_HIP_SPMD_WG": "256"},
              {"EAS_HIP_SPMD_WG": "1024"}, {"EAS_HIP_SPMD_NT": "0"}, {"EAS_HIP_SPMD_UNROLL": "4"},
              {"EAS_HIP_SPMD_LPT": "16"}, {"EAS_HIP_SPMD_LPT": "16", "EAS_HIP_SPMD_WG": "32"}]


@pytest.mark.parametrize("env", _SPMD_ENVS, ids=lambda e: ",".join(f"{k.replace('EAS_HIP_SPMD_', '')}={v}" for k, v in e.items()) or "default")
@pytest.mark.parametrize("block", [256, 1024])
def test_spmd_emitter_variants_bit_exact(gpu_runtime, monkeypatch, env, block):
    # every SPMD mapping the emitter can take (workgroup size, split programs, unroll, lanes per
    # thread, plain or nontemporal accesses) on odd sizes, against the oracle
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    n = (1 << 16) + 5 * block + 3
    a, b, c = seeded_normal(0, n), seeded_normal(1, n), seeded_normal(2, n)
    add, fma, copy, fill = (eas.kernel(k.fn) for k in (K.add_kernel, K.fma_kernel, K.copy_kernel, K.fill_kernel))
    first_k, rot = eas.kernel(K.add_first_lane_kernel.fn), eas.kernel(K.spmd_tg_rotate_kernel.fn)
    out = np.full(n, np.nan, np.float32)
    add(a, b, out, n, BLOCK=block)
    assert _bits_equal(out, ops.add_f32(a, b)), env
    out = np.full(n, np.nan, np.float32)
    fma(a, b, c, out, n, BLOCK=block)
    assert _bits_equal(out, ops.fmaf(a, b, c)), env
    out = np.full(n + 7, 5.0, np.float32)
    copy(a, out, n, BLOCK=block)
    assert _bits_equal(out[:n], a) and np.all(out[n:] == 5.0), env
    out = np.full(n + 7, 5.0, np.float32)
    fill(out, n, BLOCK=block)
    assert np.all(out[:n] == 1.0) and np.all(out[n:] == 5.0), env
    progs = -(-n // block)
    out, first = np.full(n, np.nan, np.float32), np.full(progs + 3, 9.0, np.float32)
    first_k(a, b, out, first, n, BLOCK=block)
    assert _bits_equal(out, ops.add_f32(a, b)), env
    assert _bits_equal(first[:progs], ops.add_f32(a[::block], b[::block])) and np.all(first[progs:] == 9.0), env
    out = np.full(n, np.nan, np.float32)
    rot(a, out, n, BLOCK=block)
    padded = np.zeros(progs * block, np.float32)
    padded[:n] = a
    assert _bits_equal(out, np.roll(padded.reshape(progs, block), -1, axis=1).reshape(-1)[:n]), env


@pytest.fixture(scope="module")
def inputs_n2e28():
    """a, b, c ~ N(0,1) float32 from seeds 0, 1, 2, N = 2^28 (1 GiB each)."""
    n = 1 << 28
    return n, seeded_normal(0, n), seeded_normal(1, n), seeded_normal(2, n)


@pytest.mark.parametrize("block", [256, 1024])
def test_add_and_fma_n2e28_every_output_bit_exact(gpu_runtime, inputs_n2e28, block):
    """configs[1] at its own size on device-resident torch tensors: every one of the 2^28
    outputs of c = a + b and d = a*b + c (one fused rounding) against the oracle."""
    import torch

    n, a, b, c = inputs_n2e28
    dev = torch.device("cuda:0")
    ta, tb, tc = (torch.from_numpy(x).to(dev) for x in (a, b, c))
    out = torch.full((n,), float("nan"), dtype=torch.float32, device=dev)
    K.add_kernel(ta, tb, out, n, BLOCK=block)
    torch.cuda.synchronize()
    assert _bits_equal(out.cpu().numpy(), ops.add_f32(a, b))
    out.fill_(float("nan"))
    K.fma_kernel(ta, tb, tc, out, n, BLOCK=block)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    step = 1 << 26
    for s in range(0, n, step):
        assert _bits_equal(got[s:s + step], ops.fmaf(a[s:s + step], b[s:s + step], c[s:s + step])), s
    # the reference's own fma kernel, thread mode (tests/test_fma.py:13-23), emitted as lanes
    out.fill_(float("nan"))
    K.simple_fma_kernel(ta, tb, tc, out, n, BLOCK=block)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for s in range(0, n, step):
        assert _bits_equal(got[s:s + step], ops.fmaf(a[s:s + step], b[s:s + step], c[s:s + step])), ("thread", s)
    del ta, tb, tc, out
    torch.cuda.empty_cache()


def _f16_triples(n: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Seeded f16 operands with frequent cancellation, plus the triple on which the
    reference's half(fma(float...)) and a single rounding of the exact value differ."""
    a, b = seeded_normal(0, n, np.float16), seeded_normal(1, n, np.float16)
    c = seeded_normal(2, n, np.float16)
    c[::3] = (-(a[::3].astype(np.float32) * b[::3].astype(np.float32)) * np.float32(1.0009765625)).astype(np.float16)
    a[0], b[0], c[0] = np.float16(1044 * 2.0 ** -10), np.float16(2009 * 2.0 ** -22), np.float16(1.0)
    return a, b, c


@pytest.mark.parametrize("kern", ["fma_kernel", "simple_fma_kernel"])
def test_f16_mul_then_add_rounds_twice_in_f16(gpu_runtime, kern):
    # on f16 values the fusion pass does not apply (eas/compiler.py:1019-1096 fuses f32 only):
    # the product is rounded to f16, then the sum
    n = 4099
    a, b, c = _f16_triples(n)
    d = np.zeros(n, np.float16)
    getattr(K, kern)(a, b, c, d, n, BLOCK=256)
    assert _bits_equal(d, ops.add_f16(ops.mul_f16(a, b), c))
    assert d[0] == np.float16(1.0)


def test_f16_explicit_fma_is_half_of_fmaf(gpu_runtime):
    # mk.fma on f16 values: half(fma((float)x, (float)y, (float)z)) (eas/codegen/msl.py:291-294)
    n = 4099
    a, b, c = _f16_triples(n)
    d = np.zeros(n, np.float16)
    K.explicit_fma_kernel(a, b, c, d, n, BLOCK=256)
    assert _bits_equal(d, ops.fma_f16(a, b, c))
    assert d[0] == np.float16(1.0)  # the double-rounding witness


# -- thread mode / index known answers -----------------------------------------------


def test_local_and_lane_and_sg_ids(gpu_runtime):
    n = 128 * 3
    out = np.zeros(n, np.float32)
    K.local_id_kernel(out, n, BLOCK=128)
    assert np.array_equal(out, (np.arange(n) % 128).astype(np.float32))
    out = np.zeros(256, np.float32)
    K.lane_id_kernel(out, 256, BLOCK=256)
    assert np.array_equal(out, (np.arange(256) % 32).astype(np.float32))
    out = np.zeros(256, np.float32)
    K.sg_id_kernel(out, 256, BLOCK=256)
    assert np.array_equal(out, (np.arange(256) // 32).astype(np.float32))


def test_callable_grid(gpu_runtime):
    h, w, block = 5, 10, 4
    out = np.zeros(h * w, np.float32)
    K.grid_callable_kernel(out, h, w, BLOCK=block, _grid=lambda meta, args: (K.cdiv(args["W"], meta["BLOCK"]), args["H"], 1))
    assert np.array_equal(out.reshape(h, w), np.repeat(np.arange(h, dtype=np.float32), w).reshape(h, w))


def test_tptg_must_match_and_arange(gpu_runtime):
    n = 1024 + 7
    out = np.zeros(n, np.float32)
    with pytest.raises(ValueError):
        K.tptg_independent_kernel(out, n, BLOCK=256, _tptg=64)
    with pytest.raises(ValueError):
        K.tptg_independent_kernel(out, n, BLOCK=256, _tptg=(128, 1, 1))
    K.tptg_independent_kernel(out, n, BLOCK=256, _tptg=(256, 1, 1))
    assert np.array_equal(out, np.arange(n, dtype=np.float32))


def test_threadgroup_copy_exact(gpu_runtime):
    n = 4096 + 7
    a = seeded_normal(0, n)
    out = np.zeros(n, np.float32)
    K.tg_copy_kernel(a, out, n, BLOCK=256)
    assert _bits_equal(out, a)


def test_grid_inferred_from_hw(gpu_runtime):
    h, w = 11, 77
    a, b = seeded_normal(0, h * w), seeded_normal(1, h * w)
    c = eas.empty(h * w, device="hip")
    K.add2d_hw_kernel(eas.tensor(a, device="hip"), eas.tensor(b, device="hip"), c, h, w, BLOCK=32)
    assert _bits_equal(c.numpy(), ops.add_f32(a, b))


@pytest.mark.parametrize("k", [7, 31, 64])
def test_dot_dynamic_k_partial_workgroup(gpu_runtime, k):
    m = 33
    a2, x = seeded_normal(0, m * k).reshape(m, k), seeded_normal(1, k)
    y = np.zeros(m, np.float32)
    K.gemv_dot_kernel(a2.reshape(-1), x, y, m, k, m, BLOCK=64)
    ref = np.array([ops.dot_f32(a2[r], x) for r in range(m)], np.float32)
    assert _bits_equal(y, ref)


def test_dot_f16_tn4(gpu_runtime):
    kk, groups = 8, 16
    a = seeded_normal(0, kk, np.float16)
    b = seeded_normal(1, groups * 4 + kk, np.float16)
    out = np.zeros(groups * 4, np.float32)
    K.dot_f16_tn4_kernel(a, b, out, kk, BLOCK=128, _grid=(groups, 1, 1))
    ref = interp.run_kernel(K.dot_f16_tn4_kernel, a, b, np.zeros(groups * 4, np.float32), kk, BLOCK=128, _grid=(groups, 1, 1))["out"]
    assert _bits_equal(out, ref)


# -- matmul ------------------------------------------------------------------------------


def test_naive_matmul_bit_exact_vs_oracle(gpu_runtime):
    m, n, k, block = 32, 100, 16, 64
    a2, b2 = seeded_normal(0, m * k).reshape(m, k), seeded_normal(1, k * n).reshape(k, n)
    c = np.zeros(m * n, np.float32)
    K.matmul_kernel(a2.reshape(-1), b2.reshape(-1), c, m, n, BLOCK=block, K=k, _grid=(m, K.cdiv(n, block)))
    ref = interp.run_kernel(K.matmul_kernel, a2.reshape(-1), b2.reshape(-1), np.zeros(m * n, np.float32), m, n,
                            BLOCK=block, K=k, _grid=(m, K.cdiv(n, block)))["c"]
    assert _bits_equal(c, ref)
    assert ops.rel_err(c.reshape(m, n), ops.matmul_ref(a2, b2)) <= 1e-5 * math.sqrt(k)


def test_naive_matmul_on_gpu_eas_tensors(gpu_runtime):
    # reference: tests/test_matmul.py:63-93 (the same kernel on device eas.Tensors, M=8, N=48,
    # K=16, BLOCK=32 over an (M, N tiles) grid)
    m, n, k, block = 8, 48, 16, 32
    a2, b2 = seeded_normal(0, m * k).reshape(m, k), seeded_normal(1, k * n).reshape(k, n)
    a, b = eas.tensor(a2.reshape(-1), device="hip"), eas.tensor(b2.reshape(-1), device="hip")
    c = eas.empty(m * n, device="hip")
    K.matmul_kernel(a, b, c, m, n, BLOCK=block, K=k, _grid=(m, K.cdiv(n, block)))
    ref = interp.run_kernel(K.matmul_kernel, a2.reshape(-1), b2.reshape(-1), np.zeros(m * n, np.float32), m, n,
                            BLOCK=block, K=k, _grid=(m, K.cdiv(n, block)))["c"]
    got = c.numpy()
    assert _bits_equal(got, ref)
    assert ops.rel_err(got.reshape(m, n), ops.matmul_ref(a2, b2)) <= 1e-5 * math.sqrt(k)


@pytest.mark.parametrize("mnk", [(33, 65, 48), (64, 64, 32), (17, 130, 31)])
def test_tiled_matmul_literal_bit_exact(gpu_runtime, monkeypatch, mnk):
    # the literal lowering (lift disabled) keeps the reference's fma order: bit-exact vs the oracle
    monkeypatch.setenv("EAS_HIP_DISABLE_GEMM_LIFT", "1")
    kern = eas.kernel(K.matmul_tiled_kernel.fn)
    m, n, k = mnk
    bm, bn, bk, nt = 16, 64, 16, 256
    a2 = seeded_normal(0, m * k).reshape(m, k) / np.float32(math.sqrt(k))
    b2 = seeded_normal(1, k * n).reshape(k, n)
    c = np.zeros(m * n, np.float32)
    kern(a2.reshape(-1), b2.reshape(-1), c, m, n, 0, 0, BM=bm, BN=bn, BK=bk, K=k, NT=nt,
         _grid=(K.cdiv(n, bn), K.cdiv(m, bm), 1), _tptg=(nt, 1, 1))
    assert kern.compile(a2.reshape(-1), b2.reshape(-1), c, m, n, 0, 0, BM=bm, BN=bn, BK=bk, K=k,
                        NT=nt).geometry.kind == "thread"
    ref = interp.run_kernel(K.matmul_tiled_kernel, a2.reshape(-1), b2.reshape(-1), np.zeros(m * n, np.float32), m, n,
                            0, 0, BM=bm, BN=bn, BK=bk, K=k, NT=nt, _grid=(K.cdiv(n, bn), K.cdiv(m, bm), 1))["c"]
    assert _bits_equal(c, ref)
    assert ops.rel_err(c.reshape(m, n), ops.matmul_ref(a2, b2)) <= 1e-5 * math.sqrt(k)


def _tiled_inputs(m, n, k, seed=0):
    a2 = seeded_normal(seed, m * k).reshape(m, k) / np.float32(math.sqrt(k))
    b2 = seeded_normal(seed + 1, k * n).reshape(k, n) / np.float32(math.sqrt(k))
    return a2, b2


@pytest.mark.parametrize("mnk,tile", [((33, 65, 48), (16, 64, 16, 256)), ((64, 64, 32), (16, 64, 16, 256)),
                                      ((17, 130, 31), (16, 64, 16, 256)), ((300, 260, 1000), (32, 32, 32, 256)),
                                      ((1024, 1024, 1024), (32, 32, 32, 256)), ((130, 70, 30), (16, 16, 16, 64))])
def test_tiled_matmul_lifted_fp32_tolerance(gpu_runtime, mnk, tile):
    # lifted to the fp32 MFMA GEMM (K = 31 and 30: rows not 16-byte aligned, the kernel's fma path)
    m, n, k = mnk
    bm, bn, bk, nt = tile
    a2, b2 = _tiled_inputs(m, n, k)
    c = np.full(m * n, np.nan, np.float32)
    assert K.matmul_tiled_kernel.compile(a2.reshape(-1), b2.reshape(-1), c, m, n, 0, 0, BM=bm, BN=bn, BK=bk, K=k,
                                         NT=nt).geometry.kind == "gemm"
    K.matmul_tiled_kernel(a2.reshape(-1), b2.reshape(-1), c, m, n, 0, 0, BM=bm, BN=bn, BK=bk, K=k, NT=nt,
                          _grid=(K.cdiv(n, bn), K.cdiv(m, bm), 1), _tptg=(nt, 1, 1))
    assert ops.rel_err(c.reshape(m, n), ops.matmul_ref(a2, b2)) <= 1e-5 * math.sqrt(k)


@pytest.mark.parametrize("choice", ["auto", "tile128"])
def test_tiled_matmul_split_launch_like_the_reference(gpu_runtime, monkeypatch, choice):
    # examples/matmul_tiled.py's split mode: the full-tile kernel on the interior, the masked
    # kernel with tile bases on the right strip, the bottom strip and the corner
    monkeypatch.setenv("EAS_HIP_GEMM_ENTRY", choice)
    m, n, k = 100, 200, 64
    bm, bn, bk, nt = 32, 32, 32, 256
    a2, b2 = _tiled_inputs(m, n, k, seed=4)
    c = np.full(m * n, np.nan, np.float32)
    gx, gy = n // bn, m // bm
    meta = dict(BM=bm, BN=bn, BK=bk, K=k, NT=nt, _tptg=(nt, 1, 1))
    A, B = a2.reshape(-1), b2.reshape(-1)
    K.matmul_tiled_full_kernel(A, B, c, m, n, _grid=(gx, gy, 1), **meta)
    K.matmul_tiled_kernel(A, B, c, m, n, 0, gx, _grid=(K.cdiv(n, bn) - gx, gy, 1), **meta)
    K.matmul_tiled_kernel(A, B, c, m, n, gy, 0, _grid=(gx, K.cdiv(m, bm) - gy, 1), **meta)
    K.matmul_tiled_kernel(A, B, c, m, n, gy, gx, _grid=(K.cdiv(n, bn) - gx, K.cdiv(m, bm) - gy, 1), **meta)
    assert np.isfinite(c).all()
    assert ops.rel_err(c.reshape(m, n), ops.matmul_ref(a2, b2)) <= 1e-5 * math.sqrt(k)


@pytest.mark.parametrize("mnk", [(300, 260, 1000), (130, 300, 40), (257, 132, 36), (2048, 2048, 256),
                                 (2048, 2048, 100), (4096, 3000, 96)])
def test_tiled_fp32_entries_agree(gpu_runtime, monkeypatch, mnk):
    """The fp32 GEMM's 128 x 128-tile entry and its 64 x 64 default on the same launch (edge
    tiles, K tails of 8 and 4 elements; 2048² picks the 128 tiles by itself, also with a K tail;
    4096 x 3000 runs four 128 x 128 tiles per CU with a partial last column of tiles)."""
    from easy_as_amd.runtime.hip import plan_launch

    m, n, k = mnk
    a2, b2 = _tiled_inputs(m, n, k, seed=11)
    A, B = a2.reshape(-1), b2.reshape(-1)
    meta = dict(BM=32, BN=32, BK=32, K=k, NT=256)
    grid = (K.cdiv(n, 32), K.cdiv(m, 32), 1)
    ck = K.matmul_tiled_kernel.compile(A, B, np.zeros(1, np.float32), m, n, 0, 0, **meta)
    args = {"a": A, "b": B, "c": np.zeros(m * n, np.float32), "M": m, "N": n, "PID_M_BASE": 0, "PID_N_BASE": 0}
    auto = plan_launch(ck, args, grid=grid).entry
    assert auto == ("matmul_tiled_kernel__t128" if m >= 2048 else None)
    ref = ops.matmul_ref(a2, b2)
    outs = {}
    for choice, entry in (("tile128", "matmul_tiled_kernel__t128"), ("auto", auto), ("4wave", None)):
        monkeypatch.setenv("EAS_HIP_GEMM_ENTRY", choice)
        assert plan_launch(ck, args, grid=grid).entry == entry
        c = np.full(m * n, np.nan, np.float32)
        K.matmul_tiled_kernel(A, B, c, m, n, 0, 0, _grid=grid, _tptg=(256, 1, 1), **meta)
        assert np.isfinite(c).all()
        assert ops.rel_err(c.reshape(m, n), ref) <= 1e-5 * math.sqrt(k)
        outs[choice] = c


def test_tiled_rows_past_k_are_never_read(gpu_runtime):
    m, n, k = 64, 128, 40
    a2, b2 = _tiled_inputs(m, n, k, seed=8)
    b_pad = np.concatenate([b2.reshape(-1), np.full(64 * n, np.nan, np.float32)])
    c = np.zeros(m * n, np.float32)
    K.matmul_tiled_kernel(a2.reshape(-1), b_pad, c, m, n, 0, 0, BM=32, BN=32, BK=32, K=k, NT=256,
                          _grid=(K.cdiv(n, 32), K.cdiv(m, 32), 1), _tptg=(256, 1, 1))
    assert np.isfinite(c).all()
    assert ops.rel_err(c.reshape(m, n), ops.matmul_ref(a2, b2)) <= 1e-5 * math.sqrt(k)


def test_tiled_partial_grid_touches_only_its_rectangle(gpu_runtime):
    m, n, k = 96, 160, 64
    a2, b2 = _tiled_inputs(m, n, k, seed=6)
    c = np.full(m * n, 7.0, np.float32)
    K.matmul_tiled_kernel(a2.reshape(-1), b2.reshape(-1), c, m, n, 1, 2, BM=32, BN=32, BK=32, K=k, NT=256,
                          _grid=(2, 1, 1), _tptg=(256, 1, 1))
    got = c.reshape(m, n)
    ref = ops.matmul_ref(a2, b2)
    assert ops.rel_err(got[32:64, 64:128], ref[32:64, 64:128]) <= 1e-5 * math.sqrt(k)
    got[32:64, 64:128] = 7.0
    assert np.all(got == 7.0)


@pytest.mark.parametrize("mnk", [(64, 64, 64), (40, 72, 24), (33, 17, 16)])
def test_mma_matmul_small(gpu_runtime, mnk):
    m, n, k = mnk
    bm, bn, bk = 32, 32, 8
    nt = (bm // 8) * (bn // 8) * 32
    rng = np.random.default_rng(0)
    a = rng.uniform(-1, 1, m * k).astype(np.float16)
    b = rng.uniform(-1, 1, k * n).astype(np.float16)
    c = np.zeros(m * n, np.float32)
    K.matmul_mma_kernel(a, b, c, m, n, BM=bm, BN=bn, BK=bk, K=k, NT=nt, _grid=K.mma_grid, _tptg=(nt, 1, 1))
    ref = ops.matmul_ref(a.reshape(m, k), b.reshape(k, n))
    assert ops.rel_err(c.reshape(m, n), ref) <= 2e-2
    assert ops.rel_err(c.reshape(m, n), ref) <= 1e-5 * math.sqrt(k)  # f32 accumulation of exact products


# -- interop ------------------------------------------------------------------------------


def test_torch_rocm_tensors_zero_copy(gpu_runtime):
    import torch

    n = 4096 + 3
    a = torch.randn(n, device="cuda", dtype=torch.float32)
    b = torch.randn(n, device="cuda", dtype=torch.float32)
    c = torch.empty_like(a)
    K.add_kernel(a, b, c, n, BLOCK=256)
    torch.cuda.synchronize()
    assert _bits_equal(c.cpu().numpy(), ops.add_f32(a.cpu().numpy(), b.cpu().numpy()))


def test_dlpack_roundtrip_with_torch(gpu_runtime):
    import torch

    x = torch.arange(1024, device="cuda", dtype=torch.float32)
    t = eas.tensor(x, device="hip")
    assert t.device == "hip" and t.shape == (1024,)
    y = t.to_torch("hip")
    assert y.device.type == "cuda" and torch.equal(y, x)
    y.add_(1.0)  # shares memory with x
    torch.cuda.synchronize()
    assert float(x[5].item()) == 6.0
    host = eas.tensor(np.ones(8, np.float16), device="hip").to("cpu")
    assert host.dtype == np.float16 and np.all(host.numpy() == 1)


def test_async_launches_and_synchronize(gpu_runtime):
    n = 1 << 16
    a, b = seeded_normal(0, n), seeded_normal(1, n)
    ta, tb = eas.tensor(a, device="hip"), eas.tensor(b, device="hip")
    outs = [eas.empty(n, device="hip") for _ in range(4)]
    for o in outs:
        K.add_kernel(ta, tb, o, n, BLOCK=256, _sync=False)
    gpu_runtime.synchronize()
    for o in outs:
        assert _bits_equal(o.numpy(), ops.add_f32(a, b))


@pytest.mark.parametrize("limit", [2, 0])
def test_in_flight_limit_bounds_pending_launches(monkeypatch, limit):
    """EAS_MAX_IN_FLIGHT (eas/runtime/metal.py:52-67, 340-352): at most that many async launches
    stay pending; the oldest is waited on first.  0 means no bound."""
    from easy_as_amd.runtime.hip import HipRuntime

    monkeypatch.setenv("EAS_MAX_IN_FLIGHT", str(limit))
    rt = HipRuntime()
    n = 1 << 20
    a, b = seeded_normal(0, n), seeded_normal(1, n)
    ta, tb = eas.tensor(a, device="hip"), eas.tensor(b, device="hip")
    outs = [eas.empty(n, device="hip") for _ in range(16)]
    ck = K.add_kernel.compile(ta, tb, outs[0], n, BLOCK=256)
    seen = []
    for o in outs:
        rt.run(ck, {"a": ta, "b": tb, "c": o, "N": n}, {"BLOCK": 256}, sync=False)
        seen.append(len(rt._pending))
    if limit:
        assert max(seen) == limit and seen[:limit] == list(range(1, limit + 1))
    else:
        assert seen == list(range(1, 17))
    # launches share completion events in batches of at most min(16, limit) launches, so waiting
    # on the oldest pending launch waits for at most `limit` launches and leaves the rest in flight
    mod = rt._mod()
    for p in rt._pending:
        info = mod.pending_info(p)
        if not info["released"]:
            assert info["limit"] == (min(16, limit) if limit else 16) and info["launches"] <= info["limit"], info
    rt.synchronize()
    assert len(rt._pending) == 0
    want = ops.add_f32(a, b)
    for o in outs:
        assert _bits_equal(o.numpy(), want)


def test_async_batches_close_when_the_stream_changes(gpu_runtime):
    """A completion batch belongs to one stream and is closed (its event recorded) as soon as an
    async launch arrives on another stream, so it is never recorded on a stream long after its
    last launch; launches on both streams complete, bit-exact."""
    import torch

    hip = gpu_runtime._mod()
    n = 1 << 16
    a, b = seeded_normal(0, n), seeded_normal(1, n)
    ta, tb = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    outs = [torch.zeros(n, device="cuda") for _ in range(6)]
    ck = K.add_kernel.compile(ta, tb, outs[0], n, BLOCK=256)
    side = torch.cuda.Stream()
    gpu_runtime.synchronize()  # no batch left open by earlier launches
    torch.cuda.synchronize()
    pend = []
    for i, o in enumerate(outs):
        with torch.cuda.stream(side if i % 3 == 2 else torch.cuda.current_stream()):
            gpu_runtime.run(ck, {"a": ta, "b": tb, "c": o, "N": n}, {"BLOCK": 256}, sync=False)
        pend.append(gpu_runtime._pending[-1])
    infos = [hip.pending_info(p) for p in pend]
    # launches 0-1 on the main stream, 2 on the side stream, 3-4 main, 5 side: each stream switch
    # closed the batch before it
    assert [i["launches"] for i in infos] == [2, 2, 1, 2, 2, 1]
    assert all(i["closed"] for i in infos[:5]) and not infos[5]["closed"]
    assert len({i["stream"] for i in infos}) == 2
    with pytest.raises(ValueError, match="batch"):
        hip.launch_groups_async(gpu_runtime.kernel_handle(ck), [], [], (1, 1, 1), (64, 1, 1), batch=0)
    gpu_runtime.synchronize()
    torch.cuda.synchronize()
    want = ops.add_f32(a, b)
    for o in outs:
        assert _bits_equal(o.cpu().numpy(), want)


def test_launches_follow_torch_current_stream(gpu_runtime):
    """An eas launch with torch GPU tensors goes on torch's current stream: inputs that torch
    writes on a side stream (after a long matmul, so they land late) are seen by the kernel,
    and torch work queued after it on that stream sees the kernel's output."""
    import torch

    n = 1 << 22
    a_np, b_np = seeded_normal(0, n), seeded_normal(1, n)
    ha, hb = torch.from_numpy(a_np).cuda(), torch.from_numpy(b_np).cuda()
    a = torch.zeros(n, device="cuda")
    b = torch.zeros(n, device="cuda")
    c = torch.zeros(n, device="cuda")
    big = torch.ones(4096, 4096, device="cuda")
    torch.cuda.synchronize()
    side = torch.cuda.Stream()  # default priority
    with torch.cuda.stream(side):
        for _ in range(4):
            big = big @ big * (1.0 / 4096)  # a few ms of work ahead of the input copies
        a.copy_(ha)  # device-to-device, queued behind the matmuls; the host does not wait
        b.copy_(hb)
        K.add_kernel(a, b, c, n, BLOCK=256, _sync=False)
        d = c * 1.0  # torch work after the kernel on the same stream
    gpu_runtime.synchronize()
    side.synchronize()
    want = ops.add_f32(a_np, b_np)
    assert _bits_equal(c.cpu().numpy(), want)
    assert _bits_equal(d.cpu().numpy(), want)


_TUNE_BLOCKS = (64, 256, 1024)


@eas.autotune(configs=[eas.Config(meta={"BLOCK": b}) for b in _TUNE_BLOCKS], key=["N"], warmup=1, repeat=3)
@eas.kernel
def _tuned_add_hip(a, b, c, N, BLOCK: eas.constexpr = 64):
    pid = mk.program_id(0)
    offs = pid * BLOCK + mk.arange(0, BLOCK)
    mask = offs < N
    mk.store(c, offs, mk.load(a, offs, mask) + mk.load(b, offs, mask), mask)


class _CountingRuntime:
    """The HIP runtime, with every benchmark() call recorded and its timing checked."""

    def __init__(self, rt):
        self.rt, self.benchmarked = rt, []

    def benchmark(self, ck, runtime_args, meta, **kw):
        self.benchmarked.append(int(meta["BLOCK"]))
        t = self.rt.benchmark(ck, runtime_args, meta, **kw)
        assert 0.0 < t < 1.0
        return t

    def __getattr__(self, name):
        return getattr(self.rt, name)


def test_autotune_on_hip_times_each_config_once_per_key(gpu_runtime, monkeypatch):
    """@eas.autotune with real HIP-event timings (eas/autotune.py:9-57, eas/kernel.py:73-127):
    each config is benchmarked once per key value, the chosen config runs and is cached, and the
    result is the bit-exact sum whichever BLOCK won."""
    import importlib

    eas_kernel = importlib.import_module("easy_as_amd.kernel")
    rt = _CountingRuntime(gpu_runtime)
    monkeypatch.setattr(eas_kernel, "get_runtime", lambda *a, **k: rt)
    _tuned_add_hip._tuned_cache.clear()  # the choice is per process; start from none
    for n in (1 << 20, 4099):
        a_np, b_np = seeded_normal(0, n), seeded_normal(1, n)
        a, b = eas.tensor(a_np, device="hip"), eas.tensor(b_np, device="hip")
        for _ in range(2):
            c = eas.tensor(np.full(n, np.nan, np.float32), device="hip")
            _tuned_add_hip(a, b, c, n)
            gpu_runtime.synchronize()
            assert _bits_equal(c.numpy(), ops.add_f32(a_np, b_np))
    assert sorted(rt.benchmarked) == sorted(2 * _TUNE_BLOCKS)
    assert len(_tuned_add_hip._tuned_cache) == 2
    assert {int(cfg.meta["BLOCK"]) for cfg in _tuned_add_hip._tuned_cache.values()} <= set(_TUNE_BLOCKS)


def test_benchmark_returns_positive_seconds(gpu_runtime):
    n = 1 << 20
    a = eas.tensor(seeded_normal(0, n), device="hip")
    c = eas.empty(n, device="hip")
    ck = K.add_kernel.compile(a, a, c, n, BLOCK=256)
    t = gpu_runtime.benchmark(ck, {"a": a, "b": a, "c": c, "N": n}, {"BLOCK": 256}, repeat=5, warmup=2)
    assert 0.0 < t < 1.0
