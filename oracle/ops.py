"""Oracle arithmetic: closed forms the eas hot path must reproduce.

TEST INFRASTRUCTURE ONLY.  Imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` as the checker; the product
(``easy_as_amd``) never imports anything under ``oracle/``.

* ``add_f32``      — binary32 RNE addition (examples/add.py:23-31).
* ``fmaf``         — correctly rounded f32 fused multiply-add, via the C
                     restatement ``oracle/fmaf.c`` (glibc ``fmaf``);
                     the fused op comes from eas/compiler.py:1019-1096.
* ``fmaf_rto``     — an independent numpy implementation of the same function
                     (exact product in binary64, TwoSum, round-to-odd, then one
                     RNE rounding to binary32: Boldo & Melquiond, "Emulation of
                     FMA and correctly rounded sums: proved algorithms using
                     rounding to odd", IEEE TC 2008).  Used only to pin
                     ``fmaf``; the two must agree bit for bit.
* ``mul_f16``, ``add_f16`` — binary16 arithmetic rounded once to binary16
                     (MSL ``half`` operators, eas/codegen/msl.py:224-237).
* ``fma_f16``      — the reference's f16 fma: fmaf in binary32, then binary16
                     (eas/codegen/msl.py:291-294).
* ``matmul_ref``   — float64 matmul reference (tests/test_matmul.py:55).
* ``f32_to_bf16``  — binary32 -> bfloat16, round to nearest even, as 16-bit
                     patterns; ``bf16_to_f32`` widens them back (exact).
* ``add_bf16``     — bf16 + bf16: the binary32 sum rounded once to bfloat16.
                     bfloat16 is not among the reference's dtypes (it is this
                     backend's addition), so there is no reference call site:
                     both are pinned against exact rational rounding and
                     against torch's bfloat16 conversion in tests/test_oracle.py.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle.so"

_lib: ctypes.CDLL | None = None


def build() -> Path:
    """Compile oracle/fmaf.c (gcc) into oracle/_build/liboracle.so."""
    subprocess.run(["make", "-C", str(HERE)], check=True, stdout=subprocess.DEVNULL)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        fp = ctypes.POINTER(ctypes.c_float)
        L.eas_oracle_add_f32.argtypes = [fp, fp, fp, ctypes.c_size_t]
        L.eas_oracle_fmaf.argtypes = [fp, fp, fp, fp, ctypes.c_size_t]
        L.eas_oracle_dot_f32.argtypes = [fp, ctypes.c_size_t, fp, ctypes.c_size_t, ctypes.c_size_t]
        L.eas_oracle_dot_f32.restype = ctypes.c_float
        _lib = L
    return _lib


def _f32(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32)


def _ptr(x: np.ndarray) -> ctypes._Pointer:
    return x.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def add_f32(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a, b = np.broadcast_arrays(_f32(a), _f32(b))
    a, b = _f32(a), _f32(b)
    out = np.empty_like(a)
    lib().eas_oracle_add_f32(_ptr(a), _ptr(b), _ptr(out), a.size)
    return out


def fmaf(a: np.ndarray, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    """Correctly rounded ``a*b+c`` in binary32 (C fmaf), broadcasting numpy-style."""
    a, b, c = np.broadcast_arrays(_f32(a), _f32(b), _f32(c))
    a, b, c = _f32(a), _f32(b), _f32(c)
    out = np.empty_like(a)
    lib().eas_oracle_fmaf(_ptr(a), _ptr(b), _ptr(c), _ptr(out), a.size)
    return out


def fmaf_rto(a: np.ndarray, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    """Correctly rounded binary32 fma without an fma instruction (see module doc)."""
    a64 = np.asarray(a, np.float32).astype(np.float64)
    b64 = np.asarray(b, np.float32).astype(np.float64)
    c64 = np.asarray(c, np.float32).astype(np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        p = a64 * b64  # exact: 24+24 significant bits fit in 53
        s = p + c64
        # TwoSum: e = (p + c) - s exactly
        bb = s - p
        e = (p - (s - bb)) + (c64 - bb)
        finite = np.isfinite(s) & np.isfinite(e)
        bits = s.view(np.int64)
        inexact = finite & (e != 0)
        even = (bits & 1) == 0
        # round to odd: an inexact result with an even last bit moves one ulp toward the exact value
        fix = inexact & even
        toward = np.where(e > 0, np.inf, -np.inf)
        s = np.where(fix, np.nextafter(s, toward), s)
        return s.astype(np.float32)  # results past the binary32 range become inf


def _f16(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float16)


def mul_f16(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """binary16 ``a * b`` rounded once to binary16 (MSL ``half * half``, eas/codegen/msl.py:224-237).
    The binary32 product of two binary16 values is exact (11 + 11 significant bits fit in
    24), so converting it to binary16 (RNE) is the single rounding."""
    with np.errstate(over="ignore", invalid="ignore"):
        return (_f16(a).astype(np.float32) * _f16(b).astype(np.float32)).astype(np.float16)


def add_f16(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """binary16 ``a + b`` rounded to binary16 (MSL ``half + half``, eas/codegen/msl.py:224-237):
    the binary32 sum, then binary16.  Rounding twice is innocuous for addition here
    because binary32's 24 bits are at least 2 * 11 + 2 (Figueroa, SIGNUM 1995)."""
    with np.errstate(over="ignore", invalid="ignore"):
        return (_f16(a).astype(np.float32) + _f16(b).astype(np.float32)).astype(np.float16)


def fma_f16(a: np.ndarray, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    """The reference's f16 fma, ``half(fma((float)x, (float)y, (float)z))``
    (eas/codegen/msl.py:291-294): the exact ``a*b+c`` rounded once to binary32, then
    to binary16.  This double rounding is the reference's definition and can differ
    from rounding the exact value to binary16 once (the oracle tests hold a case)."""
    with np.errstate(over="ignore", invalid="ignore"):
        return fmaf(_f16(a).astype(np.float32), _f16(b).astype(np.float32),
                    _f16(c).astype(np.float32)).astype(np.float16)


def dot_f32(a: np.ndarray, b: np.ndarray) -> np.float32:
    """One dot product with the reference's accumulation order (fma per k, k ascending)."""
    a, b = _f32(a), _f32(b)
    return np.float32(lib().eas_oracle_dot_f32(_ptr(a), 1, _ptr(b), 1, a.size))


def matmul_ref(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """float64 matmul of the given (already rounded) operands."""
    return np.asarray(a, np.float64) @ np.asarray(b, np.float64)


def rel_err(c: np.ndarray, ref: np.ndarray) -> float:
    """``max|C - R| / max|R|`` — the matmul parity metric."""
    ref = np.asarray(ref, np.float64)
    denom = float(np.max(np.abs(ref))) or 1.0
    return float(np.max(np.abs(np.asarray(c, np.float64) - ref))) / denom


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """bfloat16 bit patterns (uint16) of binary32 ``x``, rounded to nearest even.

    bfloat16 keeps binary32's sign and 8-bit exponent and the top 7 stored
    significand bits, so rounding is on the low 16 bits: add half an ulp minus
    one plus the kept last bit, then drop them (a carry may ripple into the
    exponent, which is right: it rounds up to the next binade or to infinity).
    A NaN stays a NaN: its top half with the quiet bit set."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    keep = (u >> 16) & 1
    r = ((u + 0x7FFF + keep) >> 16) & 0xFFFF
    nan = np.isnan(np.asarray(x, np.float32))
    r = np.where(nan, ((u >> 16) | 0x40) & 0xFFFF, r)
    return r.astype(np.uint16)


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    """binary32 values of bfloat16 bit patterns (exact)."""
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def add_bf16(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """bf16 + bf16 on bit patterns: the binary32 sum (RNE) rounded to bfloat16 (RNE).
    binary32's 24 bits are at least twice bfloat16's 8 plus 2, so this double
    rounding equals rounding the exact sum once (Figueroa, "When is double
    rounding innocuous?", SIGNUM 1995)."""
    return f32_to_bf16(add_f32(bf16_to_f32(a), bf16_to_f32(b)))
