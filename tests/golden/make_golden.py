"""Writes the small golden fixtures under tests/golden/ (run from the repo root).

Inputs are seeded (numpy PCG64, seeds a=0, b=1, c=2; standard normal float32);
expected outputs come from the oracle's closed forms: binary32 RNE addition
and the correctly rounded fmaf of oracle/fmaf.c.  The reference holds no golden
vectors of its own (all of its test inputs are unseeded), so these fixtures
pin this build's oracle and HIP path to fixed bits.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import ops  # noqa: E402

OUT = Path(__file__).resolve().parent


def normal(seed: int, n: int) -> np.ndarray:
    return np.random.default_rng(seed).standard_normal(n, dtype=np.float32)


def main() -> None:
    for n in (1031, 4099):
        a, b, c = normal(0, n), normal(1, n), normal(2, n)
        np.savez(OUT / f"add_f32_n{n}.npz", a=a, b=b, c=ops.add_f32(a, b))
        np.savez(OUT / f"fma_f32_n{n}.npz", a=a, b=b, c=c, d=ops.fmaf(a, b, c))
    # fma corner cases: cancellation, signed zeros, subnormals, overflow, inf/nan
    e = np.float32(2.0 ** -23)
    tiny = np.float32(np.finfo(np.float32).smallest_subnormal)
    big = np.float32(np.finfo(np.float32).max)
    a = np.array([1 + e, 1 + e, -0.0, 0.0, tiny, 3e-39, big, big, np.inf, np.nan, 1.5, -2.0], np.float32)
    b = np.array([1 - e, 1 + e, 0.0, -0.0, 0.5, 1e-6, 2.0, -1.0, 0.0, 1.0, 2 ** -126, 0.375], np.float32)
    c = np.array([-1.0, -1.0, 0.0, -0.0, 0.0, tiny, -big, big, 1.0, 0.0, -(2 ** -125), 0.75], np.float32)
    np.savez(OUT / "fma_f32_corners.npz", a=a, b=b, c=c, d=ops.fmaf(a, b, c))


if __name__ == "__main__":
    main()
