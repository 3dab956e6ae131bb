"""The oracle itself, checked before it is trusted (CPU only).

The reference holds no golden vectors for this path (all of its test inputs are
unseeded), so the oracle is pinned by:

* closed forms: binary32 RNE addition is numpy's float32 ``+``; a correctly
  rounded fma is checked against an independent restatement (``fmaf_rto``,
  exact binary64 product + TwoSum + round-to-odd) on random and special values,
  and against textbook known answers where fused and unfused results differ;
* a planted mistake: an unfused "fma" placed in the oracle must fail the corner
  cases, so the checks can tell the two apart;
* the committed golden fixtures (fixed bits over time);
* the reference's own known-answer tests for index/mask work, run through the
  interpreter (tests/test_local_and_lane_id.py:53,73, tests/test_callable_grid.py:51,
  tests/test_tptg_override.py:47, tests/test_threadgroup_memory.py:89,
  tests/test_grid_infer.py:45-61);
* brute force on tiny inputs for dot / matmul / the MMA interpreter.
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest

import kernels as K
from oracle import interp, ops

GOLDEN = Path(__file__).resolve().parent / "golden"

F32 = np.finfo(np.float32)
SPECIALS = np.array([0.0, -0.0, 1.0, -1.0, 0.5, 2.0 ** -23, 1 + 2.0 ** -23, 1 - 2.0 ** -24, 3.0, -7.25,
                     F32.tiny, -F32.tiny, F32.smallest_subnormal, 3e-39, F32.max, -F32.max, 1e30, -1e-30,
                     np.inf, -np.inf, np.nan], np.float32)


def _bits(x: np.ndarray) -> np.ndarray:
    """uint32 view with every NaN mapped to one pattern (payloads are not part of the contract)."""
    x = np.asarray(x, np.float32).copy()
    x[np.isnan(x)] = np.float32(np.nan)
    return x.view(np.uint32)


def _unfused_fma(a, b, c):
    # planted mistake: two roundings (product to binary32, then the sum)
    a, b, c = (np.asarray(v, np.float32) for v in (a, b, c))
    with np.errstate(all="ignore"):
        return (a * b) + c


# ---- add ---------------------------------------------------------------------

def test_add_is_binary32_rne():
    rng = np.random.default_rng(5)
    a = rng.standard_normal(100_000, dtype=np.float32) * np.float32(1e3)
    b = rng.standard_normal(100_000, dtype=np.float32)
    assert np.array_equal(_bits(ops.add_f32(a, b)), _bits(a + b))
    x, y = np.meshgrid(SPECIALS, SPECIALS)
    with np.errstate(all="ignore"):
        assert np.array_equal(_bits(ops.add_f32(x, y)), _bits(x + y))


def test_add_known_answers():
    # 1 + 2^-24 rounds to 1 (tie to even); 1 + 3*2^-24 rounds up to 1 + 2^-22
    got = ops.add_f32(np.array([1.0, 1.0, F32.max], np.float32),
                      np.array([2.0 ** -24, 3 * 2.0 ** -24, F32.max], np.float32))
    assert got[0] == np.float32(1.0)
    assert got[1] == np.float32(1 + 2.0 ** -22)
    assert np.isinf(got[2])


# ---- fma ---------------------------------------------------------------------

def test_fmaf_matches_independent_round_to_odd_random():
    rng = np.random.default_rng(6)
    n = 200_000
    a = rng.standard_normal(n, dtype=np.float32)
    b = rng.standard_normal(n, dtype=np.float32)
    # c close to -a*b makes heavy cancellation frequent
    c = (-(a.astype(np.float64) * b) * (1 + rng.standard_normal(n) * 1e-6)).astype(np.float32)
    c[::2] = rng.standard_normal(n // 2, dtype=np.float32) * np.float32(4.0)
    assert np.array_equal(_bits(ops.fmaf(a, b, c)), _bits(ops.fmaf_rto(a, b, c)))


def test_fmaf_matches_independent_round_to_odd_specials():
    a, b, c = np.meshgrid(SPECIALS, SPECIALS, SPECIALS, indexing="ij")
    a, b, c = a.ravel(), b.ravel(), c.ravel()
    got = ops.fmaf(a, b, c)
    want = ops.fmaf_rto(a, b, c)
    assert np.array_equal(_bits(got), _bits(want))


def test_fmaf_matches_exact_rational_on_wide_exponents():
    # exact value via Python integers/fractions, rounded once to binary32
    from fractions import Fraction

    rng = np.random.default_rng(7)
    a = (rng.standard_normal(400) * 2.0 ** rng.integers(-60, 60, 400)).astype(np.float32)
    b = (rng.standard_normal(400) * 2.0 ** rng.integers(-60, 60, 400)).astype(np.float32)
    c = (rng.standard_normal(400) * 2.0 ** rng.integers(-120, 120, 400)).astype(np.float32)
    got = ops.fmaf(a, b, c)
    for i in range(400):
        exact = Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i]))
        want = _round_f32(exact)
        assert got[i].view(np.uint32) == want.view(np.uint32), (a[i], b[i], c[i])


def _round_f32(q) -> np.float32:
    """Round a Fraction to binary32, round-to-nearest-even (normal and subnormal range)."""
    from fractions import Fraction

    if q == 0:
        return np.float32(0.0)
    sign = -1 if q < 0 else 1
    q = abs(q)
    e = q.numerator.bit_length() - q.denominator.bit_length()
    if Fraction(2) ** e > q:
        e -= 1
    e = max(e, -126)  # subnormals share the minimum exponent
    scale = Fraction(2) ** (23 - e)
    m = q * scale
    fl = m.numerator // m.denominator
    rem = m - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    val = Fraction(fl) / scale
    return np.float32(sign * float(val)) if val < Fraction(2) ** 128 else np.float32(sign * np.inf)


def test_fmaf_known_answers_differ_from_unfused():
    e = np.float32(2.0 ** -23)
    a = np.array([1 + e, 1 + e, 0.1], np.float32)
    b = np.array([1 - e, 1 + e, 10.0], np.float32)
    c = np.array([-1.0, -1.0, -1.0], np.float32)
    got = ops.fmaf(a, b, c)
    # (1+e)(1-e) - 1 = -e^2 exactly; unfused rounds the product to 1 and gives 0
    assert got[0] == np.float32(-(2.0 ** -46))
    # (1+e)^2 - 1 = 2e + e^2 exactly representable
    assert got[1] == np.float32(2.0 ** -22 + 2.0 ** -46)
    # 0.1f * 10 - 1 is the binary32 rounding error of 0.1f, times 10
    assert got[2] == np.float32(float(np.float32(0.1)) * 10 - 1)
    unfused = _unfused_fma(a, b, c)
    assert unfused[0] == 0.0 and got[0] != unfused[0]


def test_planted_unfused_mistake_is_caught():
    d = np.load(GOLDEN / "fma_f32_corners.npz")
    wrong = _unfused_fma(d["a"], d["b"], d["c"])
    assert not np.array_equal(_bits(wrong), _bits(d["d"]))
    assert not np.array_equal(_bits(wrong), _bits(ops.fmaf_rto(d["a"], d["b"], d["c"])))


def test_planted_wrong_rounding_in_rto_is_caught():
    # a round-to-odd restatement that forgets the odd fix-up is a double-rounding fma
    a, b, c = np.meshgrid(SPECIALS, SPECIALS, SPECIALS, indexing="ij")
    a, b, c = a.ravel(), b.ravel(), c.ravel()
    rng = np.random.default_rng(8)
    ra, rb = rng.standard_normal((2, 50_000), dtype=np.float32)
    rc = (-(ra.astype(np.float64) * rb)).astype(np.float32) + rng.standard_normal(50_000, dtype=np.float32) * 1e-7
    a, b, c = np.concatenate([a, ra]), np.concatenate([b, rb]), np.concatenate([c, rc.astype(np.float32)])
    with np.errstate(all="ignore"):
        double_rounded = (a.astype(np.float64) * b + c).astype(np.float32)
    assert not np.array_equal(_bits(double_rounded), _bits(ops.fmaf(a, b, c)))


# ---- golden fixtures ---------------------------------------------------------

@pytest.mark.parametrize("n", [1031, 4099])
def test_golden_add_and_fma(n):
    d = np.load(GOLDEN / f"add_f32_n{n}.npz")
    assert np.array_equal(_bits(ops.add_f32(d["a"], d["b"])), _bits(d["c"]))
    assert np.array_equal(_bits(d["a"] + d["b"]), _bits(d["c"]))
    f = np.load(GOLDEN / f"fma_f32_n{n}.npz")
    assert np.array_equal(_bits(ops.fmaf(f["a"], f["b"], f["c"])), _bits(f["d"]))
    assert np.array_equal(_bits(ops.fmaf_rto(f["a"], f["b"], f["c"])), _bits(f["d"]))


def test_golden_fixture_inputs_are_the_seeded_ones():
    d = np.load(GOLDEN / "add_f32_n1031.npz")
    assert np.array_equal(d["a"], np.random.default_rng(0).standard_normal(1031, dtype=np.float32))
    assert np.array_equal(d["b"], np.random.default_rng(1).standard_normal(1031, dtype=np.float32))


def test_golden_fma_corners():
    d = np.load(GOLDEN / "fma_f32_corners.npz")
    assert np.array_equal(_bits(ops.fmaf(d["a"], d["b"], d["c"])), _bits(d["d"]))
    assert np.array_equal(_bits(ops.fmaf_rto(d["a"], d["b"], d["c"])), _bits(d["d"]))


# ---- dot / matmul ------------------------------------------------------------

def test_dot_is_ascending_fma_chain():
    rng = np.random.default_rng(9)
    a = rng.standard_normal(257, dtype=np.float32)
    b = rng.standard_normal(257, dtype=np.float32)
    acc = np.float32(0.0)
    for k in range(257):
        acc = ops.fmaf_rto(a[k:k + 1], b[k:k + 1], np.array([acc], np.float32))[0]
    assert ops.dot_f32(a, b).view(np.uint32) == acc.view(np.uint32)
    # and it is not the pairwise or unfused sum in general
    assert abs(float(ops.dot_f32(a, b)) - float(np.dot(a.astype(np.float64), b))) < 1e-4


def test_matmul_ref_against_brute_force_and_identity():
    rng = np.random.default_rng(10)
    a = rng.standard_normal((5, 7))
    b = rng.standard_normal((7, 3))
    brute = np.array([[sum(a[i, k] * b[k, j] for k in range(7)) for j in range(3)] for i in range(5)])
    assert np.allclose(ops.matmul_ref(a, b), brute, rtol=1e-13, atol=1e-13)
    assert np.array_equal(ops.matmul_ref(a, np.eye(7)), a)
    assert ops.rel_err(brute * (1 + 1e-3), brute) == pytest.approx(1e-3, rel=1e-6)


# ---- interpreter: reference known-answer tests -------------------------------

def test_interp_add_is_bit_exact():
    d = np.load(GOLDEN / "add_f32_n1031.npz")
    out = interp.run_kernel(K.add_kernel, d["a"], d["b"], np.zeros(1031, np.float32), 1031, BLOCK=256)["c"]
    assert np.array_equal(_bits(out), _bits(d["c"]))


def test_interp_fused_and_unfused_fma_rules():
    d = np.load(GOLDEN / "fma_f32_n1031.npz")
    z = np.zeros(1031, np.float32)
    out = interp.run_kernel(K.simple_fma_kernel, d["a"], d["b"], d["c"], z, 1031, BLOCK=256)["d"]
    assert np.array_equal(_bits(out), _bits(d["d"]))
    # a mul with two users is not fused (compiler.py:1019-1096): two roundings
    res = interp.run_kernel(K.multi_use_mul_kernel, d["a"], d["b"], d["c"], z, z.copy(), 1031, BLOCK=256)
    with np.errstate(all="ignore"):
        prod = d["a"] * d["b"]
    assert np.array_equal(_bits(res["d"]), _bits(prod + d["c"]))


def test_interp_local_and_lane_ids():
    n = 128 * 3
    out = interp.run_kernel(K.local_id_kernel, np.zeros(n, np.float32), n, BLOCK=128)["out"]
    assert np.array_equal(out, (np.arange(n) % 128).astype(np.float32))
    out = interp.run_kernel(K.lane_id_kernel, np.zeros(256, np.float32), 256, BLOCK=256)["out"]
    assert np.array_equal(out, (np.arange(256) % 32).astype(np.float32))


def test_interp_callable_grid_rows():
    h, w = 5, 10
    out = interp.run_kernel(K.grid_callable_kernel, np.zeros(h * w, np.float32), h, w, BLOCK=4,
                            _grid=lambda meta, args: (K.cdiv(int(args["W"]), int(meta["BLOCK"])), int(args["H"]), 1))
    assert np.array_equal(out["out"].reshape(h, w), np.repeat(np.arange(h, dtype=np.float32), w).reshape(h, w))


def test_interp_tptg_independent_arange_and_tg_copy():
    n = 1000
    out = interp.run_kernel(K.tptg_independent_kernel, np.zeros(n, np.float32), n, BLOCK=256)["out"]
    assert np.array_equal(out, np.arange(n, dtype=np.float32))
    a = np.random.default_rng(11).standard_normal(300, dtype=np.float32)
    out = interp.run_kernel(K.tg_copy_kernel, a, np.zeros(300, np.float32), 300, BLOCK=128)["out"]
    assert np.array_equal(_bits(out), _bits(a))


@pytest.mark.parametrize("n,block", [(1000, 256), (256, 256), (3000, 1024), (1, 128)])
def test_interp_spmd_threadgroup_rotate_closed_form(n, block):
    # the kernel's own statement: out[p*BLOCK + l] = a'[p*BLOCK + (l+1) % BLOCK], a' = a with 0 past N;
    # written with numpy index arithmetic, independently of the interpreter
    a = np.random.default_rng(14).standard_normal(n, dtype=np.float32)
    out = interp.run_kernel(K.spmd_tg_rotate_kernel, a, np.full(n, np.nan, np.float32), n, BLOCK=block)["out"]
    progs = -(-n // block)
    padded = np.zeros(progs * block, np.float32)
    padded[:n] = a
    want = np.roll(padded.reshape(progs, block), -1, axis=1).reshape(-1)[:n]
    assert np.array_equal(_bits(out), _bits(want))
    if n > 2:
        # a planted off-by-one (rotation the other way) is told apart
        wrong = np.roll(padded.reshape(progs, block), 1, axis=1).reshape(-1)[:n]
        assert not np.array_equal(_bits(wrong), _bits(want))


def test_interp_masked_tail_leaves_outside_untouched():
    a = np.ones(1031, np.float32)
    res = interp.run_kernel(K.add_kernel, a, a, np.full(1100, 7.0, np.float32), 1031, BLOCK=256)["c"]
    assert np.all(res[:1031] == 2.0) and np.all(res[1031:] == 7.0)


def test_interp_mma_matches_brute_force():
    m, n, k = 40, 48, 16
    rng = np.random.default_rng(12)
    a = rng.uniform(-1, 1, m * k).astype(np.float16)
    b = rng.uniform(-1, 1, k * n).astype(np.float16)
    out = interp.run_kernel(K.matmul_mma_kernel, a, b, np.zeros(m * n, np.float32), m, n,
                            BM=32, BN=32, BK=8, K=k, NT=512, _grid=K.mma_grid)["c"]
    a64, b64 = a.astype(np.float64).reshape(m, k), b.astype(np.float64).reshape(k, n)
    brute = np.array([[math.fsum(a64[i, kk] * b64[kk, j] for kk in range(k)) for j in range(n)] for i in range(m)])
    assert ops.rel_err(out.reshape(m, n), brute) <= 1e-6


def test_interp_tiled_matmul_matches_brute_force():
    m, n, k = 20, 24, 40
    rng = np.random.default_rng(13)
    a = (rng.standard_normal(m * k) / math.sqrt(k)).astype(np.float32)
    b = (rng.standard_normal(k * n) / math.sqrt(k)).astype(np.float32)
    out = interp.run_kernel(K.matmul_tiled_kernel, a, b, np.zeros(m * n, np.float32), m, n, 0, 0,
                            BM=16, BN=16, BK=16, K=k, NT=64, _grid=(K.cdiv(n, 16), K.cdiv(m, 16), 1))["c"]
    ref = ops.matmul_ref(a.reshape(m, k), b.reshape(k, n))
    assert ops.rel_err(out.reshape(m, n), ref) <= 1e-5 * math.sqrt(k)


# ---- bfloat16 (an addition to the reference's dtypes) -------------------------

def _bf16_of_rational(q, negative_zero: bool = False) -> int:
    """bfloat16 bit pattern of the exact rational ``q`` rounded to nearest even,
    from the definition: 8 significant bits, exponents down to -126 (subnormal
    spacing 2^-133), overflow to infinity past the largest finite value.  A zero
    result keeps the sign of ``q`` (``negative_zero`` for an exact -0)."""
    from fractions import Fraction

    q = Fraction(q)
    sign = 0x8000 if q < 0 or (q == 0 and negative_zero) else 0
    a = abs(q)
    if a == 0:
        return sign
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, -126)
    ulp = Fraction(2) ** (e - 7)
    n = round(a / ulp)  # Fraction rounds half to even
    r = n * ulp
    if r >= Fraction(2) ** 128 - Fraction(2) ** (127 - 8):  # at or past the halfway point above max
        return sign | 0x7F80
    return sign | int(np.array([float(r)], np.float32).view(np.uint32)[0] >> 16)


def _bf16_probe_values() -> np.ndarray:
    rng = np.random.default_rng(11)
    vals = [rng.standard_normal(2000, dtype=np.float32) * np.float32(100.0),
            rng.integers(0, 2 ** 32, 3000, dtype=np.uint64).astype(np.uint32).view(np.float32)]
    # exact ties and near-ties: low 16 bits 0x8000 (tie), 0x7FFF, 0x8001, for even and odd kept bits
    hi = rng.integers(0, 2 ** 16, 400, dtype=np.uint64).astype(np.uint32) << 16
    for low in (0x8000, 0x7FFF, 0x8001, 0x0000, 0xFFFF):
        vals.append((hi | np.uint32(low)).view(np.float32))
    vals.append(SPECIALS)
    v = np.concatenate(vals).astype(np.float32)
    return v[~np.isnan(v)]


def test_bf16_rounding_matches_exact_rational_rounding():
    from fractions import Fraction

    x = _bf16_probe_values()
    got = ops.f32_to_bf16(x)
    fin = np.isfinite(x)
    want = np.array([_bf16_of_rational(Fraction(float(v)), bool(np.signbit(v))) for v in x[fin]], np.uint16)
    assert np.array_equal(got[fin], want)
    assert np.array_equal(got[~fin], np.where(x[~fin] > 0, 0x7F80, 0xFF80).astype(np.uint16))
    # the widening is exact, and a bf16 value converts to itself
    assert np.array_equal(ops.f32_to_bf16(ops.bf16_to_f32(got)), got)


def test_bf16_rounding_matches_torch_and_keeps_nans():
    torch = pytest.importorskip("torch")
    x = _bf16_probe_values()
    t = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ops.f32_to_bf16(x), t)
    nan = ops.f32_to_bf16(np.array([np.nan, -np.nan], np.float32))
    assert np.all(np.isnan(ops.bf16_to_f32(nan)))


def test_bf16_known_answers():
    one = 0x3F80
    u = np.array([0x7F7F7FFF, 0x7F7F8000], np.uint32).view(np.float32)  # below / at the tie above max finite
    x = np.array([1 + 2.0 ** -8,               # tie between 1 and 1 + 2^-7: even is 1
                  1 + 3 * 2.0 ** -8,           # tie between 1 + 2^-7 and 1 + 2^-6: even is 1 + 2^-6
                  1 + 2.0 ** -8 + 2.0 ** -20,  # just above the tie: up
                  F32.max,                     # past the tie above bf16's largest finite value: inf
                  u[0], u[1],
                  -2.0 ** -134,                # half of the smallest subnormal 2^-133: tie to -0
                  -3 * 2.0 ** -135], np.float32)  # 0.75 of it: -2^-133
    got = ops.f32_to_bf16(x)
    assert got.tolist() == [one, one + 2, one + 1, 0x7F80, 0x7F7F, 0x7F80, 0x8000, 0x8001]


def test_bf16_planted_truncation_fails_the_rational_check():
    from fractions import Fraction

    x = _bf16_probe_values()
    x = x[np.isfinite(x)]
    truncated = (x.view(np.uint32) >> 16).astype(np.uint16)  # round toward zero: a plausible mistake
    want = np.array([_bf16_of_rational(Fraction(float(v)), bool(np.signbit(v))) for v in x], np.uint16)
    assert not np.array_equal(truncated, want)


def test_add_bf16_is_the_correctly_rounded_exact_sum():
    from fractions import Fraction

    rng = np.random.default_rng(12)
    a = ops.f32_to_bf16(rng.standard_normal(3000, dtype=np.float32) * np.float32(2.0) ** rng.integers(-30, 30, 3000))
    b = ops.f32_to_bf16(rng.standard_normal(3000, dtype=np.float32) * np.float32(2.0) ** rng.integers(-30, 30, 3000))
    # add the cases with exponent gaps where binary32 must round before bfloat16 does
    a = np.concatenate([a, ops.f32_to_bf16(np.array([1.0, 1.0, 1.0, 2.0 ** 100, 1.5], np.float32))])
    b = np.concatenate([b, ops.f32_to_bf16(np.array([2.0 ** -8 + 2.0 ** -15, 2.0 ** -30, -2.0 ** -9, 1.0, 2.0 ** -8],
                                                    np.float32))])
    got = ops.add_bf16(a, b)
    fa, fb = ops.bf16_to_f32(a), ops.bf16_to_f32(b)
    want = np.array([_bf16_of_rational(Fraction(float(x)) + Fraction(float(y))) for x, y in zip(fa, fb)], np.uint16)
    assert np.array_equal(got, want)


# ---- binary16 arithmetic (mul, add, the reference's f16 fma) ------------------------

def _f16_of_rational(q) -> np.float16:
    """Round the exact rational ``q`` to binary16, nearest even, from the definition: 11
    significant bits, exponents down to -14 (subnormal spacing 2^-24), infinity from the
    halfway point above the largest finite value (65504 + 16) on."""
    from fractions import Fraction

    q = Fraction(q)
    if q == 0:
        return np.float16(0.0)
    sign = -1 if q < 0 else 1
    a = abs(q)
    if a >= 65520:
        return np.float16(sign * np.inf)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, -14)
    ulp = Fraction(2) ** (e - 10)
    r = round(a / ulp) * ulp  # Fraction rounds half to even
    return np.float16(sign * float(r))


def _f16_probe_pairs(n: int, seed: int) -> tuple[np.ndarray, np.ndarray]:
    """Random finite binary16 bit patterns (every exponent, subnormals included)."""
    rng = np.random.default_rng(seed)
    x = rng.integers(0, 1 << 16, (2, n * 2), dtype=np.uint32).astype(np.uint16).view(np.float16)
    fin = np.isfinite(x[0]) & np.isfinite(x[1])
    return x[0][fin][:n], x[1][fin][:n]


def _f16_bits(x) -> np.ndarray:
    x = np.asarray(x, np.float16).copy()
    x[np.isnan(x)] = np.float16(np.nan)
    return x.view(np.uint16)


def test_f16_mul_and_add_round_once():
    from fractions import Fraction

    a, b = _f16_probe_pairs(3000, 15)
    prod, summ = ops.mul_f16(a, b), ops.add_f16(a, b)
    want_p = [_f16_of_rational(Fraction(float(x)) * Fraction(float(y))) for x, y in zip(a, b)]
    want_s = [_f16_of_rational(Fraction(float(x)) + Fraction(float(y))) for x, y in zip(a, b)]
    # the sign of an exact zero result is not part of this check (compare values for zeros)
    for got, want in ((prod, want_p), (summ, want_s)):
        want = np.array(want, np.float16)
        nz = want != 0
        assert np.array_equal(_f16_bits(got[nz]), _f16_bits(want[nz]))
        assert np.all(got[~nz] == 0)


def test_f16_fma_is_fmaf_then_binary16():
    from fractions import Fraction

    a, b = _f16_probe_pairs(1500, 16)
    c, _ = _f16_probe_pairs(1500, 17)
    # magnitudes near a*b make cancellation (and so rounding at low exponents) frequent
    with np.errstate(over="ignore"):
        c[::2] = (-(a[::2].astype(np.float32) * b[::2].astype(np.float32)) * np.float32(1.001)).astype(np.float16)
    ok = np.isfinite(c)
    a, b, c = a[ok], b[ok], c[ok]
    got = ops.fma_f16(a, b, c)
    for i in range(a.size):
        exact = Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i]))
        r32 = _round_f32(exact)
        want = np.float16(np.inf if np.isinf(r32) else 0.0) if not np.isfinite(r32) else \
            _f16_of_rational(Fraction(float(r32)))
        if want == 0:
            assert got[i] == 0, (a[i], b[i], c[i])
        else:
            assert _f16_bits(got[i]) == _f16_bits(want), (a[i], b[i], c[i])


def test_f16_fma_double_rounding_witness():
    # a*b + c = 1 + 2^-11 + 244 * 2^-32: just above the binary16 midpoint between 1 and
    # 1 + 2^-10.  Rounded to binary32 first it becomes the midpoint itself, which binary16
    # rounds to even (1.0); rounded once it goes up.  The reference's half(fma(float...))
    # gives 1.0, so an oracle that rounded the exact value once would fail here.
    from fractions import Fraction

    a = np.array([1044 * 2.0 ** -10], np.float16)
    b = np.array([2009 * 2.0 ** -22], np.float16)
    c = np.array([1.0], np.float16)
    exact = Fraction(1044, 2 ** 10) * Fraction(2009, 2 ** 22) + 1
    assert exact - 1 - Fraction(1, 2 ** 11) == Fraction(244, 2 ** 32)
    assert ops.fma_f16(a, b, c)[0] == np.float16(1.0)
    assert _f16_of_rational(exact) == np.float16(1 + 2.0 ** -10)
    # unfused f16 (mul rounded to binary16, then add): a third answer
    assert ops.add_f16(ops.mul_f16(a, b), c)[0] == np.float16(1.0)
