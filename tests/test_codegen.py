"""Structure of the emitted gfx950 HIP source (CPU only, no GPU).

Each test mirrors one of the reference's codegen tests, stated for the HIP text
this backend emits instead of the Metal text:

* ``tests/test_f16_codegen.py:24-32``        f16 buffers -> ``const _Float16*`` (read) / ``_Float16*`` (written)
* ``tests/test_spmd_codegen.py:20-37``       SPMD mode, block size, program ids only (no thread ids)
* ``tests/test_fma.py:44-121``               ``fma`` emitted, early return for a single-store mask, no per-load branches
* ``tests/test_dot_f16_codegen.py:38-59``    f16 dot loads widened to float; TN4 vector load under an alignment test
* ``tests/test_dot_codegen_unique_vars.py``  repeated dot groups do not redeclare their index variables
* ``tests/test_matmul_tiled.py:126``         the literal tiled lowering reads four B columns with one vector load
* ``tests/test_mma_codegen.py:34-39``        the MMA kernel lowers to MFMA
* ``tests/test_threadgroup_memory.py:60-75`` the barrier of a masked threadgroup copy is never inside a mask guard
* ``tests/test_dot_dynamic_k.py:52-59``      a ``dot`` over a runtime K is a loop over K, not unrolled
* ``tests/test_local_and_lane_id.py:32-39``  local, lane and simdgroup ids come from the thread index

The last test compiles every emitted source with hiprtc for gfx950 (no GPU is
needed for that), which is what proves a redeclaration or any other C++ error
absent.
"""

from __future__ import annotations

import re

import numpy as np
import pytest

import eas
from eas import mk

import kernels as K


@eas.kernel
def add_f16_kernel(a, b, c, N, BLOCK: eas.constexpr):
    pid = mk.program_id(0)
    offs = pid * BLOCK + mk.arange(0, BLOCK)
    mask = offs < N
    av = mk.load(a, offs, mask)
    bv = mk.load(b, offs, mask)
    mk.store(c, offs, av + bv, mask)


@eas.kernel
def simple_fma_kernel(a, b, c, d, N, BLOCK: eas.constexpr):
    pid = mk.program_id(0)
    offs = pid * BLOCK + mk.tid(0, BLOCK)
    mask = offs < N
    d_val = mk.load(a, offs, mask) * mk.load(b, offs, mask) + mk.load(c, offs, mask)
    mk.store(d, offs, d_val, mask)


@eas.kernel
def matmul_with_fma(a, b, c, M, N, BLOCK: eas.constexpr, K: eas.constexpr):
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
def dot_f16_scalar_kernel(a, b, out, K, BLOCK: eas.constexpr):
    pid = mk.program_id(0)
    offs = pid * BLOCK + mk.tid(0, BLOCK)
    v = mk.dot(a, offs * K, 1, b, 0, 1, K)
    mk.store(out, offs, v, offs < (BLOCK * 2))


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
def many_dot_kernel(out, K: eas.constexpr, BLOCK: eas.constexpr):
    _ = mk.tid(0, BLOCK)
    As = mk.alloc_tg(1 * K)
    Bs = mk.alloc_tg(K * 1)
    mk.barrier()
    acc = 0.0
    for _i in range(20):
        acc = acc + mk.dot(As, 0, 1, Bs, 0, 1, K)
    mk.store(out, 0, acc, True)


def _h(n: int) -> np.ndarray:
    return np.zeros(n, np.float16)


def _f(n: int) -> np.ndarray:
    return np.zeros(n, np.float32)


def _params(src: str, name: str) -> list[str]:
    """The parameter declarations of kernel ``name`` in ``src``, one per entry."""
    m = re.search(rf"\b{re.escape(name)}\(\s*(.*?)\)\s*\{{", src, re.S)
    assert m, f"kernel {name} not found"
    return [p.strip() for p in m.group(1).split(",")]


def test_f16_buffers_emit_half_pointers():
    ck = add_f16_kernel.compile(_h(256), _h(256), _h(256), 256, BLOCK=256)
    params = _params(ck.src, "add_f16_kernel")
    assert "const _Float16* __restrict__ a" in params
    assert "const _Float16* __restrict__ b" in params
    assert "_Float16* __restrict__ c" in params  # written: not const


def test_spmd_mode_block_size_and_program_ids_only():
    block = 128
    ck = K.add_kernel.compile(_f(1027), _f(1027), _f(1027), 1027, BLOCK=block)
    assert ck.launch_mode == "spmd" and int(ck.block_size) == block
    params = _params(ck.src, "add_kernel")
    # an SPMD launch counts programs, not threads
    assert "const uint32_t __eas_nprog" in params and not any("__eas_nthreads" in p for p in params)
    # each program's BLOCK lanes are spread over threads: no per-program serial lane loop
    assert not re.search(rf"for \(uint32_t \w+ = 0; \w+ < {block}u;", ck.src)
    assert "__pid < __eas_nprog" in ck.src


def test_fma_emitted_with_early_return_for_single_store_mask(monkeypatch):
    # the one-thread-per-thread emitter (the lanes form is checked below)
    monkeypatch.setenv("EAS_HIP_THREAD_LANES", "0")
    z = _f(256)
    ck = eas.kernel(simple_fma_kernel.fn).compile(z, z, z, z.copy(), 256, BLOCK=256)
    assert "__builtin_fmaf(" in ck.src
    assert re.search(r"\bif \(!v\d+\) return;", ck.src)
    assert not re.search(r"\bif \(v\d+\) \{", ck.src)


def test_matmul_fma_chain_has_no_per_load_branches():
    m, n, k = 32, 64, 8
    ck = matmul_with_fma.compile(_f(m * k), _f(k * n), _f(m * n), m, n, BLOCK=32, K=k)
    src = ck.src
    assert src.split('extern "C"', 1)[1].count("__builtin_fmaf(") == k
    assert re.search(r"\bif \(!v\d+\) return;", src)
    assert not re.search(r"\bif \(v\d+\) \{", src)
    lines = src.split("\n")
    per_load_branches = sum(
        1 for i, line in enumerate(lines[:-1])
        if "= 0.0f;" in line and "if (" in lines[i + 1] and "{" in lines[i + 1] and "[" in lines[i + 1])
    assert per_load_branches == 0
    # every load is a plain indexed read after the guard
    assert len(re.findall(r"= (a|b)\[v\d+\];", src)) == 2 * k


def test_dot_f16_scalar_loads_cast_to_float():
    ck = dot_f16_scalar_kernel.compile(_h(256), _h(256), _f(256), 8, BLOCK=128)
    params = _params(ck.src, "dot_f16_scalar_kernel")
    assert "const _Float16* __restrict__ a" in params
    assert "const _Float16* __restrict__ b" in params
    assert "float* __restrict__ out" in params
    assert "(float)a[" in ck.src and "(float)b[" in ck.src


def test_dot_f16_tn4_uses_vector_load_when_aligned():
    ck = dot_f16_tn4_kernel.compile(_h(256), _h(256), _f(256), 8, BLOCK=128)
    src = ck.src
    # four adjacent B columns: one 8-byte half4 load when the address allows it,
    # element loads otherwise (the reference tests the index with ``& 3u``)
    assert "*(const eas_f16x4*)" in src
    assert re.search(r"\(\(\(uint64_t\)__bp\) & 7ull\) == 0ull", src)
    assert src.count("__builtin_fmaf(") == 8  # 4 on the vector path, 4 on the element path


def test_dot_groups_do_not_redeclare_index_variables():
    ck = many_dot_kernel.compile(_f(1), K=16, BLOCK=32)
    src = ck.src
    assert "uint a_idx =" not in src
    # the index pair of every dot lives in its own scope
    assert src.count("{ uint32_t __ai =") == 20
    assert len(re.findall(r"^\s*uint32_t __ai\b", src, re.M)) == 0


def test_literal_tiled_lowering_reads_b_columns_as_float4(monkeypatch):
    monkeypatch.setenv("EAS_HIP_DISABLE_GEMM_LIFT", "1")
    z = _f(64 * 64)
    ck = eas.kernel(K.matmul_tiled_kernel.fn).compile(z, z, z.copy(), 64, 64, 0, 0, BM=32, BN=32, BK=16, K=64,
                                                      NT=256)
    assert ck.launch_mode == "thread"
    assert "*(const eas_f32x4*)" in ck.src
    assert "__shared__" in ck.src and "__syncthreads();" in ck.src


def test_mma_kernel_lowers_to_mfma():
    ck = K.matmul_mma_kernel.compile(_h(64 * 64), _h(64 * 64), _f(64 * 64), 64, 64, BM=32, BN=32, BK=8, K=64,
                                     NT=512)
    assert "__builtin_amdgcn_mfma_f32_32x32x16_f16" in ck.src
    # the 8-wave and smaller-tile entries' bodies run 16 x 16 x 32 MFMAs unless EAS_HIP_GEMM_MFMA=32 asks
    # otherwise
    assert "__builtin_amdgcn_mfma_f32_16x16x32_f16" in ck.src
    assert "eas_gemm_pp<CT, K, 16>" in ck.src and "eas_gemm_t128<CT, K, 128, 16>" in ck.src
    assert "eas_gemm_t128<CT, K, 256, 16>" in ck.src


def test_pp_mfma_switch_is_validated(monkeypatch):
    # read when a GEMM source is emitted: a fresh kernel object picks it up
    h, f = np.zeros(8, np.float16), np.zeros(8, np.float32)
    monkeypatch.setenv("EAS_HIP_GEMM_MFMA", "32")
    ck = eas.kernel(K.matmul_mma_kernel.fn).compile(h, h, f, 4096, 4096, BM=32, BN=32, BK=8, K=4096, NT=512)
    assert "eas_gemm_pp<CT, K, 32>" in ck.src and "eas_gemm_t128<CT, K, 128, 32>" in ck.src
    monkeypatch.setenv("EAS_HIP_GEMM_MFMA", "8")
    with pytest.raises(ValueError, match="EAS_HIP_GEMM_MFMA must be 16 or 32"):
        eas.kernel(K.matmul_mma_kernel.fn).compile(h, h, f, 4096, 4096, BM=32, BN=32, BK=8, K=4096, NT=512)


def _one_thread_per_thread(kern, *args, **meta):
    """``kern`` compiled on the one-thread-per-thread emitter (``EAS_HIP_THREAD_LANES=0``)."""
    import os

    old = os.environ.get("EAS_HIP_THREAD_LANES")
    os.environ["EAS_HIP_THREAD_LANES"] = "0"
    try:
        return eas.kernel(kern.fn).compile(*args, **meta)
    finally:
        if old is None:
            del os.environ["EAS_HIP_THREAD_LANES"]
        else:
            os.environ["EAS_HIP_THREAD_LANES"] = old


def _sources() -> list[tuple[str, str]]:
    h, f = _h(256), _f(256)
    cks = [
        ("add_f16_kernel", add_f16_kernel.compile(h, h, h.copy(), 256, BLOCK=256)),
        ("simple_fma_kernel", simple_fma_kernel.compile(f, f, f, f.copy(), 256, BLOCK=256)),
        ("simple_fma_kernel_one_thread", _one_thread_per_thread(simple_fma_kernel, f, f, f, f.copy(), 256, BLOCK=256)),
        ("add2d_hw_kernel", K.add2d_hw_kernel.compile(f, f, f.copy(), 4, 64, BLOCK=32)),
        ("grid_callable_kernel", K.grid_callable_kernel.compile(f, 4, 64, BLOCK=64)),
        ("matmul_with_fma", matmul_with_fma.compile(f, f, f.copy(), 32, 64, BLOCK=32, K=8)),
        ("dot_f16_scalar_kernel", dot_f16_scalar_kernel.compile(h, h, f, 8, BLOCK=128)),
        ("dot_f16_tn4_kernel", dot_f16_tn4_kernel.compile(h, h, f, 8, BLOCK=128)),
        ("many_dot_kernel", many_dot_kernel.compile(_f(1), K=16, BLOCK=32)),
    ]
    return [(name, ck.src) for name, ck in cks]


@pytest.mark.parametrize("name,src", _sources(), ids=lambda v: v if isinstance(v, str) and len(v) < 40 else "src")
def test_emitted_source_compiles_for_gfx950(name, src):
    from easy_as_amd.runtime.hip import COMPILE_OPTIONS
    from easy_as_amd.runtime.hip_ext import load_hip_ext

    mod = load_hip_ext(require=True)
    code = mod.compile_to_code(src, f"{name}.hip", list(COMPILE_OPTIONS))
    assert code[:4] == b"\x7fELF"



_OBJDUMP = "/opt/rocm/lib/llvm/bin/llvm-objdump"


@pytest.mark.parametrize("spmd", [False, True])
def test_f16_fma_keeps_two_roundings_in_the_code_object(tmp_path, spmd):
    # half(fma((float)x, (float)y, (float)z)) rounds twice; LLVM would otherwise merge the
    # f32 fma and the narrowing into v_fma_mixlo_f16, which rounds the exact value once
    import os
    import subprocess

    from easy_as_amd.runtime.hip import COMPILE_OPTIONS
    from easy_as_amd.runtime.hip_ext import load_hip_ext

    if not os.path.exists(_OBJDUMP):
        pytest.skip("llvm-objdump not installed")

    @eas.kernel
    def spmd_fma_f16(a, b, c, d, N, BLOCK: eas.constexpr):
        offs = mk.program_id(0) * BLOCK + mk.arange(0, BLOCK)
        m = offs < N
        mk.store(d, offs, mk.fma(mk.load(a, offs, m), mk.load(b, offs, m), mk.load(c, offs, m)), m)

    h = _h(256)
    kern = spmd_fma_f16 if spmd else K.explicit_fma_kernel
    ck = kern.compile(h, h, h, h.copy(), 256, BLOCK=256)
    assert "eas_fma_f16(" in ck.src
    code = load_hip_ext(require=True).compile_to_code(ck.src, "fma_f16.hip", list(COMPILE_OPTIONS))
    path = tmp_path / "k.co"
    path.write_bytes(code)
    asm = subprocess.run([_OBJDUMP, "-d", "--mcpu=gfx950", str(path)], capture_output=True, text=True,
                         check=True).stdout
    assert "v_fma_mixlo_f16" not in asm and "v_fma_mixhi_f16" not in asm
    assert "v_cvt_f16_f32" in asm


@pytest.mark.parametrize("spmd", [False, True])
def test_f16_conversion_of_an_f32_product_rounds_twice_in_the_code_object(tmp_path, spmd):
    # to_f16(a * b) with f32 a, b: the product rounds to binary32, then to binary16.  Without the
    # conversion helper LLVM folds the multiply into v_fma_mixlo_f16 / v_mad_mixlo_f16 (one
    # rounding of the exact product), which a random-program test found differing on the GPU.
    import os
    import subprocess

    from easy_as_amd.runtime.hip import COMPILE_OPTIONS
    from easy_as_amd.runtime.hip_ext import load_hip_ext

    if not os.path.exists(_OBJDUMP):
        pytest.skip("llvm-objdump not installed")

    @eas.kernel
    def spmd_narrow(a, b, d, N, BLOCK: eas.constexpr):
        offs = mk.program_id(0) * BLOCK + mk.arange(0, BLOCK)
        m = offs < N
        mk.store(d, offs, mk.to_f16(mk.load(a, offs, m) * mk.load(b, offs, m)), m)

    @eas.kernel
    def thread_narrow(a, b, d, N, BLOCK: eas.constexpr):
        i = mk.tid(0, BLOCK)
        m = i < N
        mk.store(d, i, mk.to_f16(mk.load(a, i, m) * mk.load(b, i, m)), m)

    f = np.zeros(256, np.float32)
    ck = (spmd_narrow if spmd else thread_narrow).compile(f, f, _h(256), 256, BLOCK=256)
    assert "eas_f32_to_f16(" in ck.src
    code = load_hip_ext(require=True).compile_to_code(ck.src, "narrow.hip", list(COMPILE_OPTIONS))
    path = tmp_path / "k.co"
    path.write_bytes(code)
    asm = subprocess.run([_OBJDUMP, "-d", "--mcpu=gfx950", str(path)], capture_output=True, text=True,
                         check=True).stdout
    assert not re.search(r"v_(fma|mad)_mix(lo|hi)_f16", asm)
    assert "v_cvt_f16_f32" in asm and "v_mul_f32" in asm

# ---- bfloat16 (an addition to the reference's dtypes) ---------------------------

def test_bf16_buffers_lower_to_bf16_pointers_and_f32_arithmetic():
    torch = pytest.importorskip("torch")
    z = torch.zeros(256, dtype=torch.bfloat16)
    ck = K.add_bf16_kernel.compile(z, z, z.clone(), 256, BLOCK=256)
    params = _params(ck.src, "add_bf16_kernel")
    assert "const __bf16* __restrict__ a" in params and "__bf16* __restrict__ c" in params
    # each sum is formed in f32 and rounded once; loads and stores stay 16-byte vectors
    assert re.search(r"\(\(__bf16\)\(\(float\)v\d+\[0\] \+ \(float\)v\d+\[0\]\)\)", ck.src)
    assert "eas_bf16x8" in ck.src
    ck = K.bf16_convert_kernel.compile(np.zeros(64, np.float32), torch.zeros(64, dtype=torch.bfloat16),
                                       np.zeros(64, np.float32), 64, BLOCK=64)
    assert "eas_f32_to_bf16(v" in ck.src and "((float)(v" in ck.src


def test_bf16_mma_lifts_to_bf16_mfma():
    torch = pytest.importorskip("torch")
    z = torch.zeros(64 * 64, dtype=torch.bfloat16)
    ck = K.matmul_mma_bf16_kernel.compile(z, z, np.zeros(64 * 64, np.float32), 64, 64, BM=32, BN=32, BK=8, K=64,
                                          NT=512)
    assert ck.geometry.kind == "gemm" and ck.geometry.params["op_dtype"] == "bf16"
    assert ck.geometry.params["pp_entry"] == "matmul_mma_bf16_kernel__pp"
    assert "__builtin_amdgcn_mfma_f32_32x32x16_bf16" in ck.src and "mfma_f32_32x32x16_f16" not in ck.src
    # f32 inputs rounded to bf16 tiles: the lift keeps bf16 operands, the DMA entries drop out
    f = np.zeros(64 * 64, np.float32)
    ck = K.matmul_mma_bf16_kernel.compile(f, f, f, 64, 64, BM=32, BN=32, BK=8, K=64, NT=512)
    assert ck.geometry.params["op_dtype"] == "bf16" and ck.geometry.params["pp_entry"] is None


def _bf16_sources() -> list[tuple[str, str]]:
    torch = pytest.importorskip("torch")
    z, f = torch.zeros(64 * 64, dtype=torch.bfloat16), np.zeros(64 * 64, np.float32)
    return [
        ("add_bf16_kernel", K.add_bf16_kernel.compile(z, z, z.clone(), 256, BLOCK=256).src),
        ("bf16_convert_kernel", K.bf16_convert_kernel.compile(f, z, f.copy(), 64, BLOCK=64).src),
        ("matmul_mma_bf16_kernel", K.matmul_mma_bf16_kernel.compile(z, z, z.clone(), 64, 64, BM=32, BN=32, BK=8,
                                                                    K=64, NT=512, OUT16=True).src),
    ]


def test_bf16_sources_compile_for_gfx950():
    from easy_as_amd.runtime.hip import COMPILE_OPTIONS
    from easy_as_amd.runtime.hip_ext import load_hip_ext

    mod = load_hip_ext(require=True)
    for name, src in _bf16_sources():
        assert mod.compile_to_code(src, f"{name}.hip", list(COMPILE_OPTIONS))[:4] == b"\x7fELF", name


def _kernel_body(src: str, name: str) -> list[str]:
    """The lines of kernel ``name``'s body (after its opening brace, up to its closing one)."""
    lines = src.splitlines()
    start = next(i for i, x in enumerate(lines) if re.search(rf"\b{name}\(", x) and "__global__" in x)
    while not lines[start].rstrip().endswith("{"):
        start += 1
    body, depth = [], 1
    for x in lines[start + 1:]:
        depth += x.count("{") - x.count("}")
        if depth <= 0:
            break
        body.append(x)
    return body


@pytest.mark.parametrize("n", [515, 256 * 2 + 3, 7])
def test_barrier_of_a_masked_tg_copy_is_never_inside_a_mask_guard(n):
    # reference: tests/test_threadgroup_memory.py:60-75 (the masked copy at N = 2*256 + 3).  Every
    # thread of a workgroup must reach __syncthreads(): it sits at function scope (brace depth 1),
    # no statement before it returns early, and the masked lanes are predicated instead.
    a = np.zeros(n, np.float32)
    ck = K.tg_copy_kernel.compile(a, np.empty_like(a), n, BLOCK=256)
    assert ck.launch_mode == "thread" and ck.writes == frozenset({"out"})
    body = _kernel_body(ck.src, "tg_copy_kernel")
    depth, barriers = 1, 0
    for x in body:
        if "__syncthreads()" in x:
            barriers += 1
            assert depth == 1 and x.startswith("  __syncthreads();"), x
        if barriers == 0:
            assert not re.search(r"\breturn\b", x), f"early return before the barrier: {x}"
        depth += x.count("{") - x.count("}")
    assert barriers == 1
    # the masked store and load stay guarded per thread
    assert any(re.match(r"\s+if \(.*\) \{ out\[", x) for x in body)
    assert re.search(r"__shared__ .*float v\d+\[256\];", "\n".join(body))


def test_dot_over_a_runtime_k_is_a_loop_not_unrolled():
    # reference: tests/test_dot_dynamic_k.py:52-59 (gemv with K a runtime scalar, M = 8, K = 11)
    a, x, y = np.zeros(88, np.float32), np.zeros(11, np.float32), np.zeros(8, np.float32)
    ck = K.gemv_dot_kernel.compile(a, x, y, 8, 11, 8, BLOCK=64)
    body = "\n".join(_kernel_body(ck.src, "gemv_dot_kernel"))
    loop = re.search(r"for \(uint32_t (k\d+) = 0; \1 < K; \+\+\1\)", body)
    assert loop, body
    # one fma in the loop body, whatever K is: the same source serves every K
    assert body.count("__builtin_fmaf") == 1
    for k in (7, 31, 64, 4096):
        other = K.gemv_dot_kernel.compile(np.zeros(8 * k, np.float32), np.zeros(k, np.float32), y, 8, k, 8, BLOCK=64)
        assert other.src == ck.src


def test_local_lane_and_simdgroup_ids_come_from_the_thread_index():
    # reference: tests/test_local_and_lane_id.py:32-39 (the Metal kernels declare
    # [[thread_position_in_threadgroup]] and [[thread_index_in_simdgroup]]).  HIP has those as
    # builtins: on the one-thread-per-thread emitter the local id is threadIdx.x, and the 32-lane
    # simdgroup of the Metal model maps onto half of a wave64, lane = threadIdx.x & 31 and
    # simdgroup = threadIdx.x >> 5.  The launch's thread count (Metal's non-uniform grid) is a
    # hidden u32 argument after the user's.  (Emitted as lanes, the position is the lane: below.)
    out = np.zeros(256, np.float32)
    want = {"local_id_kernel": r"= threadIdx\.x;", "lane_id_kernel": r"= threadIdx\.x & 31u;",
            "sg_id_kernel": r"= threadIdx\.x >> 5;"}
    for name, pattern in want.items():
        ck = _one_thread_per_thread(getattr(K, name), out, 256, BLOCK=256)
        assert ck.launch_mode == "thread"
        head = ck.src[ck.src.index(f"void __launch_bounds__(256) {name}("):]
        params = head[:head.index("{")]
        assert re.search(r"float\* __restrict__ out,\s*const uint32_t N,\s*const uint32_t __eas_nthreads\)", params)
        body = "\n".join(_kernel_body(ck.src, name))
        assert re.search(pattern, body), (name, body)


def test_thread_element_streams_are_emitted_as_lanes():
    # The reference's thread-mode fma (tests/test_fma.py:13-23): one program of BLOCK lanes per
    # threadgroup, 16-byte nontemporal vectors, and every lane-varying access masked by the live
    # thread count, which stays the kernel's one hidden argument after the user's.
    f = _f(256)
    ck = simple_fma_kernel.compile(f, f, f, f.copy(), 256, BLOCK=256)
    one = _one_thread_per_thread(simple_fma_kernel, f, f, f, f.copy(), 256, BLOCK=256)
    assert ck.launch_mode == one.launch_mode == "thread" and ck.block_size == one.block_size == 256
    geo = ck.geometry
    assert geo.kind == "thread" and geo.params["lanes"] and geo.params["lanes_per_thread"] == 4
    assert (geo.wg_size, geo.split) == (32, 2)  # four HBM streams: 512-byte chunks, as the SPMD fma
    sig = lambda c: c.src[c.src.index("simple_fma_kernel("):c.src.index("{", c.src.index("simple_fma_kernel("))]
    assert sig(ck).replace("__launch_bounds__(32)", "") == sig(one).replace("__launch_bounds__(256)", "")
    assert sig(ck).rstrip().endswith("const uint32_t __eas_nthreads)")
    body = ck.src.split('extern "C"', 1)[1]
    assert body.count("__builtin_nontemporal_load((const eas_f32x4*)") == 3
    assert body.count("__builtin_nontemporal_store((eas_f32x4)") == 1
    assert "__builtin_fmaf(" in body and "__eas_nprog = __eas_nthreads / 256u" in body
    live = re.search(r"bool (v\d+)\[4\];\n  \1\[0\] = v\d+\[0\] < __eas_nthreads;", body)
    assert live, "the live-thread mask"
    # every global access is guarded by a mask that includes it
    masks = set(re.findall(r"(v\d+)\[0\] = v\d+\[0\] && " + live.group(1) + r"\[0\];", body))
    for m in re.findall(r"if \((v\d+)\[0\] && \1\[1\]", body):
        assert m in masks or m == live.group(1), m
    assert len(re.findall(r"if \((v\d+)\[0\] && \1\[1\]", body)) == 4  # three loads, one store


def test_thread_positions_as_lanes():
    # a thread's position in its (BLOCK, 1, 1) threadgroup is its lane of the program:
    # local id = lane, lane id = lane % 32, simdgroup id = lane / 32 (32-lane simdgroups)
    out = _f(256)
    for name, op in (("local_id_kernel", "+ v"), ("lane_id_kernel", "% v"), ("sg_id_kernel", "/ v")):
        ck = eas.kernel(getattr(K, name).fn).compile(out, 256, BLOCK=256)
        assert ck.launch_mode == "thread" and ck.geometry.params.get("lanes"), name
        body = ck.src.split('extern "C"', 1)[1]
        lane = re.search(r"(v\d+)\[0\] = 0u \+ __lbase;", body).group(1)
        assert re.search(rf"= {lane}\[0\] {re.escape(op)}\d+;", body), (name, op)


@pytest.mark.parametrize("case", ["barrier", "dot", "shared_address_load", "lanes_off"])
def test_kernels_that_stay_one_thread_per_thread(case, monkeypatch):
    f, h = _f(256), _h(256)
    if case == "barrier":  # threadgroup memory shared between threads
        ck = K.tg_copy_kernel.compile(f, f.copy(), 256, BLOCK=256)
    elif case == "dot":
        ck = dot_f16_tn4_kernel.compile(h, h, f, 8, BLOCK=128)
    elif case == "shared_address_load":  # a row of A at one address, under each thread's own mask
        ck = K.matmul_kernel.compile(f, f, f.copy(), 8, 48, BLOCK=32, K=4)
    else:
        monkeypatch.setenv("EAS_HIP_THREAD_LANES", "0")
        ck = eas.kernel(simple_fma_kernel.fn).compile(f, f, f, f.copy(), 256, BLOCK=256)
    assert ck.launch_mode == "thread" and not ck.geometry.params.get("lanes")
    assert ck.geometry.wg_size == ck.block_size and "__gid" in ck.src
    monkeypatch.setenv("EAS_HIP_THREAD_LANES", "2")
    with pytest.raises(ValueError, match="EAS_HIP_THREAD_LANES must be 0 or 1"):
        eas.kernel(simple_fma_kernel.fn).compile(f, f, f, f.copy(), 256, BLOCK=256)


_MAPPING_ENVS = [{}, {"EAS_HIP_SPMD_WG": "32"}, {"EAS_HIP_SPMD_WG": "64"}, {"EAS_HIP_SPMD_WG": "1024"},
                 {"EAS_HIP_SPMD_LPT": "16"}, {"EAS_HIP_SPMD_UNROLL": "2"}]
_BLOCKS = sorted(set(range(1, 65)) | {96, 100, 127, 128, 160, 200, 250, 256, 384, 500, 512, 640, 768, 1000, 1024})


@pytest.mark.parametrize("env", _MAPPING_ENVS, ids=lambda e: ",".join(f"{k[13:]}={v}" for k, v in e.items()) or "default")
def test_every_lane_of_a_program_has_a_thread(env, monkeypatch):
    """A program's BLOCK lanes are covered by its T threads (lanes_per_thread each), and those T
    threads by its workgroups: `split` workgroups of `wg` threads, or `ppw` programs of T threads
    in one workgroup.  Before this was checked a BLOCK such as 200 or 1000 (T = 50 or 250 over
    32-thread workgroups) left lanes without a thread."""
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    f = _f(16)
    for kern, args in ((K.add_kernel, (f, f, f, 8)), (K.copy_kernel, (f, f, 8)), (K.fill_kernel, (f, 8)),
                       (K.fma_kernel, (f, f, f, f, 8)), (K.simple_fma_kernel, (f, f, f, f, 8))):
        for block in _BLOCKS:
            if kern is K.simple_fma_kernel and block > 1024:
                continue
            geo = eas.kernel(kern.fn).compile(*args, BLOCK=block).geometry
            if not geo.params.get("lanes_per_thread"):
                assert kern is K.simple_fma_kernel and block == 1  # one thread per Metal thread
                continue
            T, lpt = geo.params["threads_per_program"], geo.params["lanes_per_thread"]
            assert T * lpt == block, (kern.name, block, env)
            if geo.split > 1:
                assert geo.programs_per_wg == 1 and geo.split * geo.wg_size == T, (kern.name, block, env, geo)
            else:
                assert geo.wg_size == T * geo.programs_per_wg <= 1024, (kern.name, block, env, geo)

