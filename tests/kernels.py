"""User kernels exercised by the tests, bench and smoke run.

These are eas user programs (the workloads the reference's examples and tests
define), written against the public DSL.  Sources in the reference:
add ``examples/add.py:23-31``; fma ``tests/test_fma.py:13-39, 135-148,
187-196``; naive matmul ``tests/test_matmul.py:15-28``; tiled fp32 matmul
``examples/matmul_tiled.py:27-230`` and ``tests/test_matmul_tiled.py:19-99``;
simdgroup-MMA matmul ``examples/matmul_simdgroup.py:29-127``; the small
index/known-answer kernels from the reference test files named below.
"""

from __future__ import annotations

import eas
from eas import mk


def cdiv(a: int, b: int) -> int:
    return (a + b - 1) // b


# -- elementwise (SPMD) --------------------------------------------------------


@eas.kernel
def add_kernel(a, b, c, N, BLOCK: eas.constexpr):
    pid = mk.program_id(0)
    offs = pid * BLOCK + mk.arange(0, BLOCK)
    mask = offs < N
    mk.store(c, offs, mk.load(a, offs, mask) + mk.load(b, offs, mask), mask)


@eas.kernel
def copy_kernel(a, c, N, BLOCK: eas.constexpr):
    """c = a: a plain copy of known size, used to calibrate HBM byte counters."""
    pid = mk.program_id(0)
    offs = pid * BLOCK + mk.arange(0, BLOCK)
    mask = offs < N
    mk.store(c, offs, mk.load(a, offs, mask), mask)


@eas.kernel
def read_kernel(a, c, N, BLOCK: eas.constexpr):
    """Reads a; writes c only where a < -3e38 (never for N(0,1) data): HBM read traffic alone."""
    pid = mk.program_id(0)
    offs = pid * BLOCK + mk.arange(0, BLOCK)
    mask = offs < N
    x = mk.load(a, offs, mask)
    mk.store(c, offs, x, mask & (x < -3.0e38))


@eas.kernel
def fill_kernel(c, N, BLOCK: eas.constexpr):
    """c = 1.0: HBM write traffic alone."""
    pid = mk.program_id(0)
    offs = pid * BLOCK + mk.arange(0, BLOCK)
    mk.store(c, offs, 1.0, offs < N)


@eas.kernel
def fma_kernel(a, b, c, d, N, BLOCK: eas.constexpr):
    """d = a * b + c; the IR pass fuses it into one fma (single rounding)."""
    pid = mk.program_id(0)
    offs = pid * BLOCK + mk.arange(0, BLOCK)
    mask = offs < N
    mk.store(d, offs, mk.load(a, offs, mask) * mk.load(b, offs, mask) + mk.load(c, offs, mask), mask)


@eas.kernel
def axpy_kernel(a, b, c, N, alpha, BLOCK: eas.constexpr):
    """tests/test_kernel_cache.py:14-24."""
    pid = mk.program_id(0)
    offs = pid * BLOCK + mk.arange(0, BLOCK)
    mask = offs < N
    mk.store(c, offs, mk.load(a, offs, mask) * alpha + mk.load(b, offs, mask), mask)


@eas.kernel
def spmd_tg_rotate_kernel(a, out, N, BLOCK: eas.constexpr):
    """SPMD program that rotates its lanes by one through threadgroup memory:
    out[p*BLOCK + l] = a'[p*BLOCK + (l+1) % BLOCK] with a' = a masked to 0 past N.
    Lanes of one program exchange data, so once a program is spread over
    several threads the store and the load need a barrier between them."""
    pid = mk.program_id(0)
    lanes = mk.arange(0, BLOCK)
    offs = pid * BLOCK + lanes
    mask = offs < N
    tg = mk.alloc_tg(BLOCK)
    mk.store(tg, lanes, mk.load(a, offs, mask))
    mk.store(out, offs, mk.load(tg, (lanes + 1) % BLOCK), mask)


@eas.kernel
def add_first_lane_kernel(a, b, c, first, N, BLOCK: eas.constexpr):
    """c = a + b, and first[p] = a[p*BLOCK] + b[p*BLOCK] for each program p: a
    program-uniform load and store next to the lane streams (one store per program)."""
    pid = mk.program_id(0)
    offs = pid * BLOCK + mk.arange(0, BLOCK)
    mask = offs < N
    mk.store(c, offs, mk.load(a, offs, mask) + mk.load(b, offs, mask), mask)
    mk.store(first, pid, mk.load(a, pid * BLOCK) + mk.load(b, pid * BLOCK))


# -- thread mode -----------------------------------------------------------------


@eas.kernel
def simple_fma_kernel(a, b, c, d, N, BLOCK: eas.constexpr):
    pid = mk.program_id(0)
    offs = pid * BLOCK + mk.tid(0, BLOCK)
    mask = offs < N
    d_val = mk.load(a, offs, mask) * mk.load(b, offs, mask) + mk.load(c, offs, mask)
    mk.store(d, offs, d_val, mask)


@eas.kernel
def explicit_fma_kernel(a, b, c, d, N, BLOCK: eas.constexpr):
    pid = mk.program_id(0)
    offs = pid * BLOCK + mk.tid(0, BLOCK)
    mask = offs < N
    mk.store(d, offs, mk.fma(mk.load(a, offs, mask), mk.load(b, offs, mask), mk.load(c, offs, mask)), mask)


@eas.kernel
def multi_use_mul_kernel(a, b, c, d, e, N, BLOCK: eas.constexpr):
    pid = mk.program_id(0)
    offs = pid * BLOCK + mk.tid(0, BLOCK)
    mask = offs < N
    a_val = mk.load(a, offs, mask)
    b_val = mk.load(b, offs, mask)
    c_val = mk.load(c, offs, mask)
    mul_result = a_val * b_val
    mk.store(d, offs, mul_result + c_val, mask)
    mk.store(e, offs, mk.where(mask, mul_result, c_val), mask)


@eas.kernel
def matmul_kernel(a, b, c, M, N, BLOCK: eas.constexpr, K: eas.constexpr):
    row = mk.program_id(0)
    tile = mk.program_id(1)
    col = tile * BLOCK + mk.tid(0, BLOCK)
    out = row * N + col
    mask = mk.where(row < M, col < N, False)
    acc = 0.0
    for k in range(K):
        acc = acc + mk.load(a, row * K + k, mask) * mk.load(b, k * N + col, mask)
    mk.store(c, out, acc, mask)


@eas.kernel
def gemv_dot_kernel(a, x, y, M, K, N, BLOCK: eas.constexpr):
    pid = mk.program_id(0)
    row = pid * BLOCK + mk.tid(0, BLOCK)
    mask = row < M
    mk.store(y, row, mk.dot(a, row * K, 1, x, 0, 1, K), mask)


@eas.kernel
def tg_copy_kernel(a, out, N, BLOCK: eas.constexpr):
    pid = mk.program_id(0)
    tid = mk.tid(0, BLOCK)
    offs = pid * BLOCK + tid
    mask = offs < N
    scratch = mk.alloc_tg(BLOCK)
    mk.store(scratch, tid, mk.load(a, offs, mask))
    mk.barrier()
    mk.store(out, offs, mk.load(scratch, tid), mask)


@eas.kernel
def local_id_kernel(out, N, BLOCK: eas.constexpr):
    pid = mk.program_id(0)
    _ = mk.tid(0, BLOCK)
    lid = mk.local_id(0)
    offs = pid * BLOCK + lid
    mk.store(out, offs, mk.to_f32(lid), offs < N)


@eas.kernel
def lane_id_kernel(out, N, BLOCK: eas.constexpr):
    pid = mk.program_id(0)
    tid = pid * BLOCK + mk.tid(0, BLOCK)
    mk.store(out, tid, mk.to_f32(mk.lane_id()), tid < N)


@eas.kernel
def sg_id_kernel(out, N, BLOCK: eas.constexpr):
    pid = mk.program_id(0)
    tid = pid * BLOCK + mk.tid(0, BLOCK)
    mk.store(out, tid, mk.to_f32(mk.sg_id()), tid < N)


@eas.kernel
def grid_callable_kernel(out, H, W, BLOCK: eas.constexpr):
    tile = mk.program_id(0)
    row = mk.program_id(1)
    col = tile * BLOCK + mk.tid(0, BLOCK)
    mk.store(out, row * W + col, mk.to_f32(row), mk.where(row < H, col < W, False))


@eas.kernel
def tptg_independent_kernel(out, N, BLOCK: eas.constexpr):
    pid = mk.program_id(0)
    offs = pid * BLOCK + mk.tid(0, BLOCK)
    mk.store(out, offs, mk.to_f32(offs), offs < N)


@eas.kernel
def add2d_shape_kernel(a, b, c, M, N, BLOCK: eas.constexpr):
    """2-D add whose grid comes from ``_shape`` (tests/test_grid_infer.py:25-32)."""
    tile = mk.program_id(0)
    row = mk.program_id(1)
    col = tile * BLOCK + mk.tid(0, BLOCK)
    offs = row * N + col
    mask = mk.where(row < M, col < N, False)
    mk.store(c, offs, mk.load(a, offs, mask) + mk.load(b, offs, mask), mask)


@eas.kernel
def add2d_hw_kernel(a, b, c, H, W, BLOCK: eas.constexpr):
    tile = mk.program_id(0)
    row = mk.program_id(1)
    col = tile * BLOCK + mk.tid(0, BLOCK)
    offs = row * W + col
    mask = mk.where(row < H, col < W, False)
    mk.store(c, offs, mk.load(a, offs, mask) + mk.load(b, offs, mask), mask)


@eas.kernel
def dot_f16_tn4_kernel(a, b, out, K, BLOCK: eas.constexpr):
    pid = mk.program_id(0)
    _ = mk.tid(0, BLOCK)
    base = pid * 4
    d0 = mk.dot(a, 0, 1, b, base, 1, K)
    d1 = mk.dot(a, 0, 1, b, base + 1, 1, K)
    d2 = mk.dot(a, 0, 1, b, base + 2, 1, K)
    d3 = mk.dot(a, 0, 1, b, base + 3, 1, K)
    mk.store(out, base + 0, d0, True)
    mk.store(out, base + 1, d1, True)
    mk.store(out, base + 2, d2, True)
    mk.store(out, base + 3, d3, True)


@eas.kernel
def matmul_tiled_kernel(a, b, c, M, N, PID_M_BASE, PID_N_BASE, BM: eas.constexpr, BN: eas.constexpr,
                        BK: eas.constexpr, K: eas.constexpr, NT: eas.constexpr):
    """fp32 tiled matmul with padded threadgroup tiles (examples/matmul_tiled.py:27-131)."""
    pid_n = mk.program_id(0) + PID_N_BASE
    pid_m = mk.program_id(1) + PID_M_BASE
    tid = mk.tid(0, NT)
    tn = 4
    if BN % tn != 0:
        raise ValueError("BN must be divisible by 4 for TN=4 mapping")
    ng = BN // tn
    if NT != BM * ng:
        raise ValueError("NT must equal BM*(BN/4) for this tiled mapping")
    lda = BK + 1
    ldb = BN + 1
    rm = tid // ng
    cg = tid % ng
    tile_m = pid_m * BM
    tile_n = pid_n * BN
    row = tile_m + rm
    col0 = tile_n + cg * tn
    As = mk.alloc_tg(BM * lda)
    Bs = mk.alloc_tg(BK * ldb)
    acc0 = acc1 = acc2 = acc3 = 0.0
    row_ok = row < M
    c_row_base = row * N
    for k0 in range(0, K, BK):
        for i in range(0, BM * BK, NT):
            a_idx = tid + i
            in_tile = a_idx < (BM * BK)
            a_r = a_idx // BK
            a_c = a_idx % BK
            a_row = tile_m + a_r
            a_mask = in_tile & (a_row < M) & ((k0 + a_c) < K)
            mk.store(As, a_r * lda + a_c, mk.load(a, a_row * K + k0 + a_c, a_mask), in_tile)
        for i in range(0, BK * BN, NT):
            b_idx = tid + i
            in_tile = b_idx < (BK * BN)
            b_r = b_idx // BN
            b_c = b_idx % BN
            b_mask = in_tile & ((k0 + b_r) < K) & ((tile_n + b_c) < N)
            mk.store(Bs, b_r * ldb + b_c, mk.load(b, (k0 + b_r) * N + tile_n + b_c, b_mask), in_tile)
        mk.barrier()
        a_base = rm * lda
        b_base = cg * tn
        acc0 = acc0 + mk.dot(As, a_base, 1, Bs, b_base + 0, ldb, BK)
        acc1 = acc1 + mk.dot(As, a_base, 1, Bs, b_base + 1, ldb, BK)
        acc2 = acc2 + mk.dot(As, a_base, 1, Bs, b_base + 2, ldb, BK)
        acc3 = acc3 + mk.dot(As, a_base, 1, Bs, b_base + 3, ldb, BK)
        mk.barrier()
    base = c_row_base + col0
    mk.store(c, base + 0, acc0, row_ok & (col0 + 0 < N))
    mk.store(c, base + 1, acc1, row_ok & (col0 + 1 < N))
    mk.store(c, base + 2, acc2, row_ok & (col0 + 2 < N))
    mk.store(c, base + 3, acc3, row_ok & (col0 + 3 < N))


@eas.kernel
def matmul_tiled_full_kernel(a, b, c, M, N, BM: eas.constexpr, BN: eas.constexpr, BK: eas.constexpr,
                             K: eas.constexpr, NT: eas.constexpr):
    """Interior-tile fp32 tiled matmul without bounds checks (examples/matmul_tiled.py:132-230):
    valid only for grids of whole tiles and K divisible by BK."""
    pid_n = mk.program_id(0)
    pid_m = mk.program_id(1)
    tid = mk.tid(0, NT)
    tn = 4
    ng = BN // tn
    if NT != BM * ng or (BM * BK) % NT or (BK * BN) % NT:
        raise ValueError("full kernel needs NT = BM*BN/4 dividing both tile loads")
    lda = BK + 1
    ldb = BN + 1
    rm = tid // ng
    cg = tid % ng
    tile_m = pid_m * BM
    tile_n = pid_n * BN
    row = tile_m + rm
    col0 = tile_n + cg * tn
    As = mk.alloc_tg(BM * lda)
    Bs = mk.alloc_tg(BK * ldb)
    acc0 = acc1 = acc2 = acc3 = 0.0
    for k0 in range(0, K, BK):
        for i in range(0, BM * BK, NT):
            a_idx = tid + i
            a_r = a_idx // BK
            a_c = a_idx % BK
            mk.store(As, a_r * lda + a_c, mk.load(a, (tile_m + a_r) * K + k0 + a_c, True), True)
        for i in range(0, BK * BN, NT):
            b_idx = tid + i
            b_r = b_idx // BN
            b_c = b_idx % BN
            mk.store(Bs, b_r * ldb + b_c, mk.load(b, (k0 + b_r) * N + tile_n + b_c, True), True)
        mk.barrier()
        a_base = rm * lda
        b_base = cg * tn
        acc0 = acc0 + mk.dot(As, a_base, 1, Bs, b_base + 0, ldb, BK)
        acc1 = acc1 + mk.dot(As, a_base, 1, Bs, b_base + 1, ldb, BK)
        acc2 = acc2 + mk.dot(As, a_base, 1, Bs, b_base + 2, ldb, BK)
        acc3 = acc3 + mk.dot(As, a_base, 1, Bs, b_base + 3, ldb, BK)
        mk.barrier()
    base = row * N + col0
    mk.store(c, base + 0, acc0, True)
    mk.store(c, base + 1, acc1, True)
    mk.store(c, base + 2, acc2, True)
    mk.store(c, base + 3, acc3, True)


@eas.kernel
def matmul_tiled_variant_kernel(a, b, c, M, N, BM: eas.constexpr, BN: eas.constexpr, BK: eas.constexpr,
                                K: eas.constexpr, NT: eas.constexpr, VARIANT: eas.constexpr):
    """matmul_tiled_kernel (without tile bases) with one deliberate change selected by VARIANT
    (0 = none).  Variants 1-7 are not GEMMs and must not be lifted; 8-9 are equivalent rewrites."""
    pid_n = mk.program_id(0)
    pid_m = mk.program_id(1)
    tid = mk.tid(0, NT)
    tn = 4
    ng = BN // tn
    lda = BK + 1
    ldb = BN + 1
    rm = tid // ng
    cg = tid % ng
    tile_m = pid_m * BM
    tile_n = pid_n * BN
    row = tile_m + rm
    col0 = tile_n + cg * tn
    As = mk.alloc_tg(BM * lda)
    Bs = mk.alloc_tg(BK * ldb)
    acc = [0.0, 0.0, 0.0, 0.0]
    row_ok = row < M
    k_start = BK if VARIANT == 1 else 0          # 1: skips the first k block
    for k0 in range(k_start, K, BK):
        for i in range(0, BM * BK, NT):
            a_idx = tid + i
            in_tile = a_idx < (BM * BK)
            a_r = a_idx // BK
            a_c = a_idx % BK
            a_row = tile_m + a_r
            a_mask = in_tile & (a_row < M) & ((k0 + a_c) < K)
            if VARIANT == 6:                       # 6: A masked by the column bound
                a_mask = in_tile & (a_row < N) & ((k0 + a_c) < K)
            src = b if VARIANT == 4 else a         # 4: A read from B
            mk.store(As, a_r * lda + a_c, mk.load(src, a_row * K + k0 + a_c, a_mask), in_tile)
        for i in range(0, BK * BN, NT):
            b_idx = tid + i
            in_tile = b_idx < (BK * BN)
            b_r = b_idx // BN
            b_c = b_idx % BN
            b_mask = in_tile & ((k0 + b_r) < K) & ((tile_n + b_c) < N)
            mk.store(Bs, b_r * ldb + b_c, mk.load(b, (k0 + b_r) * N + tile_n + b_c, b_mask), in_tile)
        mk.barrier()
        a_base = rm * lda
        b_base = cg * tn
        kd = BK - 1 if VARIANT == 5 else BK        # 5: each dot drops its last k
        bst = ldb + 1 if VARIANT == 2 else ldb     # 2: B walked with the wrong stride
        for j in range(4):
            d = mk.dot(As, a_base, 1, Bs, b_base + j, bst, kd)
            acc[j] = d + acc[j] if VARIANT == 8 else acc[j] + d   # 8: operands of the add swapped
        mk.barrier()
    for j in range(4):
        jj = 3 - j if VARIANT == 3 else j          # 3: outputs stored to mirrored columns
        mask = row_ok & (col0 + j < N)
        if VARIANT == 7:                           # 7: a store mask on the wrong index
            mask = (col0 + j < M) & (col0 + j < N)
        if VARIANT == 9:                           # 9: equivalent mask written the other way round
            mask = (col0 + j < N) & row_ok
        mk.store(c, row * N + col0 + jj, acc[j], mask)


@eas.kernel
def matmul_mma_kernel(a, b, c, M, N, BM: eas.constexpr, BN: eas.constexpr, BK: eas.constexpr,
                      K: eas.constexpr, NT: eas.constexpr):
    """Simdgroup 8x8x8 MMA matmul, f16 operands in threadgroup memory, f32
    accumulate; the C tile goes through threadgroup memory and is copied out
    with bounds checks (examples/matmul_simdgroup.py:29-127)."""
    if BM % 8 != 0 or BN % 8 != 0 or BK % 8 != 0:
        raise ValueError("BM/BN/BK must be divisible by 8 for 8x8 MMA")
    if NT != (BM // 8) * (BN // 8) * 32:
        raise ValueError("NT must be (BM/8)*(BN/8)*32 for 8x8 MMA")
    pid_n = mk.program_id(0)
    pid_m = mk.program_id(1)
    tid = mk.tid(0, NT)
    sg = mk.sg_id()
    base_m = pid_m * BM
    base_n = pid_n * BN
    sgn = BN // 8
    sg_m = sg // sgn
    sg_n = sg % sgn
    lda = BK + 1
    ldb = BN + 1
    ldc = BN + 1
    As = mk.alloc_tg_f16(BM * lda)
    Bs = mk.alloc_tg_f16(BK * ldb)
    Cs = mk.alloc_tg(BM * ldc)
    acc = mk.mma_zero()
    for k0 in range(0, K, BK):
        for i in range(0, BM * BK, NT):
            a_idx = tid + i
            a_r = a_idx // BK
            a_c = a_idx % BK
            a_row = base_m + a_r
            a_col = k0 + a_c
            in_tile = a_idx < BM * BK
            a_mask = mk.where(in_tile, mk.where(a_row < M, a_col < K, False), False)
            mk.store(As, a_r * lda + a_c, mk.to_f16(mk.load(a, a_row * K + a_col, a_mask)), in_tile)
        for i in range(0, BK * BN, NT):
            b_idx = tid + i
            b_r = b_idx // BN
            b_c = b_idx % BN
            b_row = k0 + b_r
            b_col = base_n + b_c
            in_tile = b_idx < BK * BN
            b_mask = mk.where(in_tile, mk.where(b_row < K, b_col < N, False), False)
            mk.store(Bs, b_r * ldb + b_c, mk.to_f16(mk.load(b, b_row * N + b_col, b_mask)), in_tile)
        mk.barrier()
        for kk in range(0, BK, 8):
            acc = mk.mma(As, (sg_m * 8) * lda + kk, lda, Bs, kk * ldb + (sg_n * 8), ldb, acc)
        mk.barrier()
    mk.mma_store(Cs, (sg_m * 8) * ldc + (sg_n * 8), ldc, acc)
    mk.barrier()
    for i in range(0, BM * BN, NT):
        c_idx = tid + i
        r = c_idx // BN
        cc = c_idx % BN
        row = base_m + r
        col = base_n + cc
        mk.store(c, row * N + col, mk.load(Cs, r * ldc + cc, True), mk.where(row < M, col < N, False))


@eas.kernel
def matmul_mma_f16out_kernel(a, b, c, M, N, BM: eas.constexpr, BN: eas.constexpr, BK: eas.constexpr,
                             K: eas.constexpr, NT: eas.constexpr):
    """matmul_mma_kernel with an f16 output buffer: the copy-out rounds the f32
    accumulator with mk.to_f16 (the LLM-linear variant)."""
    if BM % 8 != 0 or BN % 8 != 0 or BK % 8 != 0:
        raise ValueError("BM/BN/BK must be divisible by 8 for 8x8 MMA")
    if NT != (BM // 8) * (BN // 8) * 32:
        raise ValueError("NT must be (BM/8)*(BN/8)*32 for 8x8 MMA")
    pid_n = mk.program_id(0)
    pid_m = mk.program_id(1)
    tid = mk.tid(0, NT)
    sg = mk.sg_id()
    base_m = pid_m * BM
    base_n = pid_n * BN
    sgn = BN // 8
    sg_m = sg // sgn
    sg_n = sg % sgn
    lda = BK + 1
    ldb = BN + 1
    ldc = BN + 1
    As = mk.alloc_tg_f16(BM * lda)
    Bs = mk.alloc_tg_f16(BK * ldb)
    Cs = mk.alloc_tg(BM * ldc)
    acc = mk.mma_zero()
    for k0 in range(0, K, BK):
        for i in range(0, BM * BK, NT):
            a_idx = tid + i
            a_r = a_idx // BK
            a_c = a_idx % BK
            a_row = base_m + a_r
            a_col = k0 + a_c
            in_tile = a_idx < BM * BK
            a_mask = mk.where(in_tile, mk.where(a_row < M, a_col < K, False), False)
            mk.store(As, a_r * lda + a_c, mk.to_f16(mk.load(a, a_row * K + a_col, a_mask)), in_tile)
        for i in range(0, BK * BN, NT):
            b_idx = tid + i
            b_r = b_idx // BN
            b_c = b_idx % BN
            b_row = k0 + b_r
            b_col = base_n + b_c
            in_tile = b_idx < BK * BN
            b_mask = mk.where(in_tile, mk.where(b_row < K, b_col < N, False), False)
            mk.store(Bs, b_r * ldb + b_c, mk.to_f16(mk.load(b, b_row * N + b_col, b_mask)), in_tile)
        mk.barrier()
        for kk in range(0, BK, 8):
            acc = mk.mma(As, (sg_m * 8) * lda + kk, lda, Bs, kk * ldb + (sg_n * 8), ldb, acc)
        mk.barrier()
    mk.mma_store(Cs, (sg_m * 8) * ldc + (sg_n * 8), ldc, acc)
    mk.barrier()
    for i in range(0, BM * BN, NT):
        c_idx = tid + i
        r = c_idx // BN
        cc = c_idx % BN
        row = base_m + r
        col = base_n + cc
        mk.store(c, row * N + col, mk.to_f16(mk.load(Cs, r * ldc + cc, True)), mk.where(row < M, col < N, False))


def mma_grid(meta, rargs):
    return (cdiv(int(rargs["N"]), int(meta["BN"])), cdiv(int(rargs["M"]), int(meta["BM"])), 1)


@eas.kernel
def matmul_mma_variant_kernel(a, b, c, M, N, BM: eas.constexpr, BN: eas.constexpr, BK: eas.constexpr,
                              K: eas.constexpr, NT: eas.constexpr, VARIANT: eas.constexpr):
    """matmul_mma_kernel with one deliberate change selected by VARIANT (0 = none).

    Used to check that the GEMM lift proves what it replaces: variants 1-8 are
    not dense GEMMs (or not with these masks) and must keep the literal
    lowering; variants 9-10 are GEMMs written differently and may be lifted.
      1 last k block skipped        2 A rows shifted by one       3 column mask uses M
      4 output stored transposed    5 B row stride is M           6 half the tile stored
      7 A fragment stride off       8 one output element stored twice
      9 k blocks in reverse order  10 rows on program_id(0), cols on program_id(1)
     11 output stored without its row mask (rows past M written, as zeros)
     12 output stored without its column mask
    """
    V = VARIANT
    pid_n = mk.program_id(1 if V == 10 else 0)
    pid_m = mk.program_id(0 if V == 10 else 1)
    tid = mk.tid(0, NT)
    sg = mk.sg_id()
    base_m = pid_m * BM
    base_n = pid_n * BN
    sgn = BN // 8
    sg_m = sg // sgn
    sg_n = sg % sgn
    lda = BK + 1
    ldb = BN + 1
    ldc = BN + 1
    As = mk.alloc_tg_f16(BM * lda)
    Bs = mk.alloc_tg_f16(BK * ldb)
    Cs = mk.alloc_tg(BM * ldc)
    acc = mk.mma_zero()
    kblocks = list(range(0, K, BK))
    if V == 1:
        kblocks = kblocks[:-1]
    if V == 9:
        kblocks = kblocks[::-1]
    for k0 in kblocks:
        for i in range(0, BM * BK, NT):
            a_idx = tid + i
            a_r = a_idx // BK
            a_c = a_idx % BK
            a_row = base_m + a_r + (1 if V == 2 else 0)
            a_col = k0 + a_c
            in_tile = a_idx < BM * BK
            a_mask = mk.where(in_tile, mk.where(a_row < M, a_col < K, False), False)
            mk.store(As, a_r * lda + a_c, mk.to_f16(mk.load(a, a_row * K + a_col, a_mask)), in_tile)
        for i in range(0, BK * BN, NT):
            b_idx = tid + i
            b_r = b_idx // BN
            b_c = b_idx % BN
            b_row = k0 + b_r
            b_col = base_n + b_c
            in_tile = b_idx < BK * BN
            b_mask = mk.where(in_tile, mk.where(b_row < K, b_col < N, False), False)
            stride = M if V == 5 else N
            mk.store(Bs, b_r * ldb + b_c, mk.to_f16(mk.load(b, b_row * stride + b_col, b_mask)), in_tile)
        mk.barrier()
        for kk in range(0, BK, 8):
            a_stride = lda + 1 if V == 7 else lda
            acc = mk.mma(As, (sg_m * 8) * lda + kk, a_stride, Bs, kk * ldb + (sg_n * 8), ldb, acc)
        mk.barrier()
    mk.mma_store(Cs, (sg_m * 8) * ldc + (sg_n * 8), ldc, acc)
    mk.barrier()
    total = BM * BN // 2 if V == 6 else BM * BN
    for i in range(0, total, NT):
        c_idx = tid + i
        r = c_idx // BN
        cc = c_idx % BN
        row = base_m + r
        col = base_n + cc
        col_bound = M if V == 3 else N
        mask = mk.where(row < M, col < col_bound, False)
        if V == 11:
            mask = col < col_bound
        if V == 12:
            mask = row < M
        off = col * N + row if V == 4 else row * N + col
        mk.store(c, off, mk.load(Cs, r * ldc + cc, True), mask)
    if V == 8:
        mk.store(c, base_m * N + base_n, mk.load(Cs, 0, True), mk.where(base_m < M, base_n < N, False))


@eas.kernel
def matmul_mma_bf16_kernel(a, b, c, M, N, BM: eas.constexpr, BN: eas.constexpr, BK: eas.constexpr,
                           K: eas.constexpr, NT: eas.constexpr, OUT16: eas.constexpr = False):
    """matmul_mma_kernel with bf16 threadgroup tiles (``mk.alloc_tg_bf16``; inputs
    rounded with ``mk.to_bf16``, a no-op for bf16 inputs); with OUT16 the copy-out
    rounds the f32 accumulator into a bf16 ``c``.  bf16 is an addition to the
    reference's dtypes."""
    if BM % 8 != 0 or BN % 8 != 0 or BK % 8 != 0:
        raise ValueError("BM/BN/BK must be divisible by 8 for 8x8 MMA")
    if NT != (BM // 8) * (BN // 8) * 32:
        raise ValueError("NT must be (BM/8)*(BN/8)*32 for 8x8 MMA")
    pid_n = mk.program_id(0)
    pid_m = mk.program_id(1)
    tid = mk.tid(0, NT)
    sg = mk.sg_id()
    base_m = pid_m * BM
    base_n = pid_n * BN
    sgn = BN // 8
    sg_m = sg // sgn
    sg_n = sg % sgn
    lda = BK + 1
    ldb = BN + 1
    ldc = BN + 1
    As = mk.alloc_tg_bf16(BM * lda)
    Bs = mk.alloc_tg_bf16(BK * ldb)
    Cs = mk.alloc_tg(BM * ldc)
    acc = mk.mma_zero()
    for k0 in range(0, K, BK):
        for i in range(0, BM * BK, NT):
            a_idx = tid + i
            a_r = a_idx // BK
            a_c = a_idx % BK
            a_row = base_m + a_r
            a_col = k0 + a_c
            in_tile = a_idx < BM * BK
            a_mask = mk.where(in_tile, mk.where(a_row < M, a_col < K, False), False)
            mk.store(As, a_r * lda + a_c, mk.to_bf16(mk.load(a, a_row * K + a_col, a_mask)), in_tile)
        for i in range(0, BK * BN, NT):
            b_idx = tid + i
            b_r = b_idx // BN
            b_c = b_idx % BN
            b_row = k0 + b_r
            b_col = base_n + b_c
            in_tile = b_idx < BK * BN
            b_mask = mk.where(in_tile, mk.where(b_row < K, b_col < N, False), False)
            mk.store(Bs, b_r * ldb + b_c, mk.to_bf16(mk.load(b, b_row * N + b_col, b_mask)), in_tile)
        mk.barrier()
        for kk in range(0, BK, 8):
            acc = mk.mma(As, (sg_m * 8) * lda + kk, lda, Bs, kk * ldb + (sg_n * 8), ldb, acc)
        mk.barrier()
    mk.mma_store(Cs, (sg_m * 8) * ldc + (sg_n * 8), ldc, acc)
    mk.barrier()
    for i in range(0, BM * BN, NT):
        c_idx = tid + i
        r = c_idx // BN
        cc = c_idx % BN
        row = base_m + r
        col = base_n + cc
        v = mk.load(Cs, r * ldc + cc, True)
        mk.store(c, row * N + col, mk.to_bf16(v) if OUT16 else v, mk.where(row < M, col < N, False))


@eas.kernel
def add_bf16_kernel(a, b, c, N, BLOCK: eas.constexpr):
    """SPMD add on bf16 buffers (each sum computed in f32 and rounded once to bf16)."""
    offs = mk.program_id(0) * BLOCK + mk.arange(0, BLOCK)
    mask = offs < N
    mk.store(c, offs, mk.load(a, offs, mask) + mk.load(b, offs, mask), mask)


@eas.kernel
def bf16_convert_kernel(x, y, z, N, BLOCK: eas.constexpr):
    """y = bf16(x) (round to nearest even), z = f32(bf16(x)) * x (a product of a bf16
    value and an f32 value, rounded to f32)."""
    offs = mk.program_id(0) * BLOCK + mk.tid(0, BLOCK)
    mask = offs < N
    v = mk.load(x, offs, mask)
    h = mk.to_bf16(v)
    mk.store(y, offs, h, mask)
    mk.store(z, offs, mk.to_f32(h) * v, mask)
