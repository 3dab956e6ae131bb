"""IR-level behaviour of the tracer and passes (counterparts of the reference's
test_thread_id_rewrite.py, test_interval_lt_fold.py, test_fma.py fusion rules,
test_bool_simplify.py, test_kernel_cache.py, test_threadgroup_memory.py:58)."""

from __future__ import annotations

import numpy as np
import pytest

import eas
from eas import mk
from eas.compiler import _cse_pure, _dce, _fold_static_lts, _fuse_fma, _rewrite_thread_id, _simplify_bools, trace_to_ir
from eas.ir import Arg, DType, IRModule, Inst, ValueRef, validate_ir

import kernels as K


def _ops(ck) -> list[str]:
    return [i.op for i in ck.ir.insts]


f32 = lambda n: np.zeros(n, np.float32)  # noqa: E731


@eas.kernel
def _simple_add_tid(a, b, c, N, BLOCK: eas.constexpr):
    pid = mk.program_id(0)
    offs = pid * BLOCK + mk.tid(0, BLOCK)
    mask = offs < N
    mk.store(c, offs, mk.load(a, offs, mask) + mk.load(b, offs, mask), mask)


def test_thread_id_rewrite_applies_and_env_disables(monkeypatch):
    ck = _simple_add_tid.compile(f32(4), f32(4), f32(4), 4, BLOCK=256)
    # emitted as lanes of one program per threadgroup, the thread id is the program's base plus a lane
    assert "thread_id" in _ops(ck) and ck.geometry.params.get("lanes") and "__pid" in ck.src
    with monkeypatch.context() as mp:  # one thread per Metal thread: the global thread index
        mp.setenv("EAS_HIP_THREAD_LANES", "0")
        assert "__gid" in eas.kernel(_simple_add_tid.fn).compile(f32(4), f32(4), f32(4), 4, BLOCK=256).src
    monkeypatch.setenv("EAS_DISABLE_THREAD_ID_REWRITE", "1")
    ck2 = eas.kernel(_simple_add_tid.fn).compile(f32(4), f32(4), f32(4), 4, BLOCK=256)
    assert "thread_id" not in _ops(ck2)
    assert "blockIdx.x" in ck2.src and "threadIdx.x" in ck2.src


def test_thread_id_rewrite_requires_single_threadgroup_size():
    pid, block, mul = ValueRef(1, DType.U32), ValueRef(2, DType.U32), ValueRef(3, DType.U32)
    t0, t1, out = ValueRef(4, DType.U32), ValueRef(5, DType.U32), ValueRef(6, DType.U32)
    head = (Inst("program_id", pid, (0,)), Inst("const", block, (256,)), Inst("mul", mul, (pid, block)),
            Inst("tid", t0, (0, 256)))
    multi = IRModule("k", (), head + (Inst("tid", t1, (0, 128)), Inst("add", out, (mul, t0))))
    assert _rewrite_thread_id(multi).insts[-1].op == "add"
    single = IRModule("k", (), head + (Inst("add", out, (mul, t0)),))
    assert _rewrite_thread_id(single).insts[-1].op == "thread_id"
    # operand order of the add and of the mul do not matter
    swapped = IRModule("k", (), (Inst("program_id", pid, (0,)), Inst("const", block, (256,)),
                                 Inst("mul", mul, (block, pid)), Inst("tid", t0, (0, 256)), Inst("add", out, (t0, mul))))
    assert _rewrite_thread_id(swapped).insts[-1].op == "thread_id"


@eas.kernel
def _in_tile_store(src, dst, LIMIT: eas.constexpr, NT: eas.constexpr):
    tid = mk.tid(0, NT)
    for i in range(0, LIMIT, NT):
        idx = tid + i
        mk.store(dst, idx, mk.load(src, idx, True), idx < LIMIT)


def test_interval_fold_removes_provably_true_lt():
    assert "lt" not in _ops(_in_tile_store.compile(f32(64), f32(64), LIMIT=64, NT=16))


def test_interval_fold_keeps_needed_lt():
    assert "lt" in _ops(_in_tile_store.compile(f32(70), f32(70), LIMIT=70, NT=16))


def test_interval_fold_does_not_bound_global_thread_id():
    # offs = pid*BLOCK + tid is the *global* thread index: `offs < 300` must stay a runtime test.
    @eas.kernel
    def k(out, N, BLOCK: eas.constexpr):
        offs = mk.program_id(0) * BLOCK + mk.tid(0, BLOCK)
        mk.store(out, offs, 1.0, offs < 300)

    assert "lt" in _ops(k.compile(f32(4), 4, BLOCK=256))


def test_interval_fold_respects_u32_wraparound():
    @eas.kernel
    def k(out, BLOCK: eas.constexpr):
        t = mk.tid(0, BLOCK)
        big = t + 4294967295  # wraps to t - 1 for t >= 1
        mk.store(out, t, 1.0, big < 8)

    assert "lt" in _ops(k.compile(f32(4), BLOCK=64))


def test_fma_fused_for_single_use_mul():
    ck = K.simple_fma_kernel.compile(f32(4), f32(4), f32(4), f32(4), 4, BLOCK=256)
    assert "fma" in _ops(ck) and "mul" not in _ops(ck)
    assert "__builtin_fmaf(" in ck.src


def test_fma_not_fused_when_mul_has_two_users():
    ck = K.multi_use_mul_kernel.compile(f32(4), f32(4), f32(4), f32(4), f32(4), 4, BLOCK=128)
    assert "fma" not in _ops(ck) and "mul" in _ops(ck) and "add" in _ops(ck)
    assert "__builtin_fmaf" not in ck.src


def test_fma_first_mul_operand_decides():
    # add(mul_multi_use, mul_single_use): the first mul-defined operand is the
    # candidate and it has two users, so nothing fuses (reference rule).
    @eas.kernel
    def k(a, b, out, BLOCK: eas.constexpr):
        t = mk.tid(0, BLOCK)
        x = mk.load(a, t)
        y = mk.load(b, t)
        m1 = x * y
        m2 = y * y
        mk.store(out, t, m1 + m2)
        mk.store(out, t + BLOCK, m1)

    assert "fma" not in _ops(k.compile(f32(4), f32(4), f32(4), BLOCK=64))


def test_fma_not_fused_for_f16():
    @eas.kernel
    def k(a, b, c, out, BLOCK: eas.constexpr):
        t = mk.tid(0, BLOCK)
        mk.store(out, t, mk.load(a, t) * mk.load(b, t) + mk.load(c, t))

    h = np.zeros(4, np.float16)
    assert "fma" not in _ops(k.compile(h, h, h, h, BLOCK=64))


def test_matmul_unrolled_chain_fuses_every_step():
    ck = K.matmul_kernel.compile(f32(4), f32(4), f32(4), 2, 2, BLOCK=32, K=8)
    # acc starts as the literal 0.0, so the first add(0.0, a*b) fuses too: K fmas, no mul left.
    assert _ops(ck).count("fma") == 8
    assert "mul" not in [i.op for i in ck.ir.insts if i.out is not None and i.out.dtype == DType.F32]


def test_bool_where_lowers_to_logical_and():
    @eas.kernel
    def k(out, N, BLOCK: eas.constexpr):
        tid = mk.program_id(0) * BLOCK + mk.tid(0, BLOCK)
        m = mk.where(tid < N, tid < (N + 1), False)
        mk.store(out, tid, mk.to_f32(m), tid < N)

    ck = k.compile(f32(4), 4, BLOCK=256)
    assert "where" not in _ops(ck) and "and" in _ops(ck)
    assert "&&" in ck.src


def test_nested_where_chain_inlines_to_single_if(monkeypatch):
    # the one-thread-per-thread emitter's folding of a single store's boolean mask (a kernel
    # emitted as lanes keeps its masks per lane instead)
    monkeypatch.setenv("EAS_HIP_THREAD_LANES", "0")

    @eas.kernel
    def k(out, N, BLOCK: eas.constexpr):
        tid = mk.tid(0, BLOCK)
        m = mk.where(tid < N, mk.where(tid < (N + 1), mk.where(tid < (N + 2), True, False), False), False)
        mk.store(out, tid, 1.0, m)

    import re

    assert re.search(r"if \(!?\([^\n]*&&[^\n]*&&[^\n]*\)", k.compile(f32(4), 4, BLOCK=256).src)


def test_simplify_bools_constant_folding():
    t, c_t, c_f = ValueRef(0, DType.BOOL), ValueRef(1, DType.BOOL), ValueRef(2, DType.BOOL)
    o1, o2, o3, o4 = (ValueRef(i, DType.BOOL) for i in (3, 4, 5, 6))
    ir = IRModule("k", (Arg("t", DType.BOOL, "scalar"),), (
        Inst("arg", t, ("t", "scalar", DType.BOOL)),
        Inst("const", c_t, (True,)), Inst("const", c_f, (False,)),
        Inst("and", o1, (t, c_f)), Inst("or", o2, (t, c_t)), Inst("not", o3, (c_f,)), Inst("where", o4, (c_t, t, c_f)),
    ))
    out = {i.out.id: i for i in _simplify_bools(ir).insts if i.out is not None}
    assert out[3].op == "const" and out[3].args == (False,)
    assert out[4].op == "const" and out[4].args == (True,)
    assert out[5].op == "const" and out[5].args == (True,)
    assert 6 not in out  # where(True, t, False) is just t


def test_cse_merges_commutative_and_dce_drops_dead():
    a, b = ValueRef(0, DType.U32), ValueRef(1, DType.U32)
    s1, s2, dead = ValueRef(2, DType.U32), ValueRef(3, DType.U32), ValueRef(4, DType.U32)
    buf, m = ValueRef(5, DType.F32), ValueRef(6, DType.BOOL)
    v = ValueRef(7, DType.F32)
    ir = IRModule("k", (Arg("x", DType.F32, "buffer"), Arg("a", DType.U32, "scalar"), Arg("b", DType.U32, "scalar")), (
        Inst("arg", buf, ("x", "buffer", DType.F32)), Inst("arg", a, ("a", "scalar", DType.U32)),
        Inst("arg", b, ("b", "scalar", DType.U32)),
        Inst("add", s1, (a, b)), Inst("add", s2, (b, a)), Inst("mul", dead, (a, a)),
        Inst("const", m, (True,)), Inst("const", v, (1.0,)),
        Inst("store", None, (buf, s1, v, m)), Inst("store", None, (buf, s2, v, m)),
    ))
    out = _dce(_cse_pure(ir))
    validate_ir(out)
    adds = [i for i in out.insts if i.op == "add"]
    assert len(adds) == 1
    assert all(i.op != "mul" for i in out.insts)
    stores = [i for i in out.insts if i.op == "store"]
    assert stores[0].args[1] == stores[1].args[1] == adds[0].out


def test_writes_inference_and_tg_declared():
    ck = K.tg_copy_kernel.compile(f32(4), f32(4), 4, BLOCK=256)
    assert ck.writes == frozenset({"out"})
    assert "__shared__" in ck.src and "__syncthreads();" in ck.src
    assert "const float* __restrict__ a" in ck.src and "float* __restrict__ out" in ck.src


def test_compile_cache_ignores_scalar_values():
    a = f32(8)
    ck1 = K.axpy_kernel.compile(a, a, a, 8, alpha=2.0, BLOCK=256)
    ck2 = K.axpy_kernel.compile(a, a, a, 9, alpha=3.0, BLOCK=256)
    assert ck1 is ck2
    ck3 = K.axpy_kernel.compile(a, a, a, 8, alpha=2.0, BLOCK=128)
    assert ck3 is not ck1


def test_specialisation_key_fast_path_matches_classify_arg():
    import torch

    from eas.compiler import _arg_key, classify_arg

    values = [f32(4), np.zeros(3, np.float16), 7, 2.5, True, np.float32(1.0), np.int64(3), np.float16(2.0),
              torch.zeros(3), torch.zeros(3, dtype=torch.float16), eas.tensor(f32(4))]
    for v in values:
        s = classify_arg(v)
        assert _arg_key(v) == (s.kind, s.dtype, s.device), type(v)
    for bad in (np.zeros(3, np.float64), torch.zeros(3, dtype=torch.int32), "x"):
        with pytest.raises(TypeError):
            _arg_key(bad)


def test_constexpr_removed_runtime_scalar_kept(monkeypatch):
    a = f32(8)
    src = K.add_kernel.to_hip(a, a, a, 8, BLOCK=256)
    assert "const uint32_t N" in src and "BLOCK" not in src
    monkeypatch.setenv("EAS_SPECIALIZE_SCALARS", "N")  # a no-op in the reference too
    assert "const uint32_t N" in K.add_kernel.to_hip(a, a, a, 8, BLOCK=256)


def test_large_unrolled_k_traces_without_recursion():
    ck = K.matmul_kernel.compile(f32(1200), f32(3600), f32(3), 1, 3, BLOCK=2, K=1200, _grid=(1, 2))
    assert _ops(ck).count("load") == 2400


def test_builder_type_errors():
    @eas.kernel
    def bad_mix(a, BLOCK: eas.constexpr):
        mk.store(a, mk.tid(0, BLOCK), mk.load(a, 0) + 1)  # f32 + u32

    with pytest.raises(TypeError):
        bad_mix.compile(f32(4), BLOCK=64)

    @eas.kernel
    def bad_lanes(a, BLOCK: eas.constexpr):
        x = mk.arange(0, BLOCK)
        y = mk.arange(0, BLOCK * 2)
        mk.store(a, x + y, 1.0)

    with pytest.raises(TypeError):
        bad_lanes.compile(f32(4), BLOCK=64)

    @eas.kernel
    def bad_mode(a, BLOCK: eas.constexpr):
        mk.store(a, mk.arange(0, BLOCK) + mk.tid(0, BLOCK), 1.0)

    with pytest.raises(ValueError):
        bad_mode.compile(f32(4), BLOCK=64)

    @eas.kernel
    def neg(a, BLOCK: eas.constexpr):
        mk.store(a, mk.tid(0, BLOCK), 1.0, mk.tid(0, BLOCK) < -1)

    with pytest.raises(ValueError):
        neg.compile(f32(4), BLOCK=64)


def test_meta_must_be_literal():
    with pytest.raises(TypeError):
        K.add_kernel.compile(f32(4), f32(4), f32(4), 4, BLOCK=[256])


def test_validate_ir_rejects_malformed():
    v = ValueRef(0, DType.U32)
    with pytest.raises(ValueError, match="invalid IR"):
        validate_ir(IRModule("k", (), (Inst("const", v, (-1,)),)))
    with pytest.raises(ValueError, match="undefined"):
        validate_ir(IRModule("k", (), (Inst("add", ValueRef(1, DType.U32), (v, v)),)))
    with pytest.raises(ValueError, match="missing arg"):
        validate_ir(IRModule("k", (Arg("x", DType.F32, "buffer"),), ()))


def test_dsl_outside_trace_raises():
    with pytest.raises(RuntimeError):
        mk.program_id(0)


def test_trace_is_thread_local():
    import threading

    errors = []

    def worker():
        try:
            K.add_kernel.compile(f32(4), f32(4), f32(4), 4, BLOCK=64 + 64 * threading.get_ident() % 3)
        except Exception as e:  # pragma: no cover
            errors.append(e)

    ts = [threading.Thread(target=worker) for _ in range(4)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors


def test_bf16_typing_rules():
    torch = pytest.importorskip("torch")
    bf = torch.zeros(64, dtype=torch.bfloat16)

    @eas.kernel
    def bf16_plus_literal(a, BLOCK: eas.constexpr):
        i = mk.tid(0, BLOCK)
        mk.store(a, i, mk.load(a, i) + 1.0)  # bf16 + f32 literal: no implicit conversion

    with pytest.raises(TypeError):
        bf16_plus_literal.compile(bf, BLOCK=64)

    @eas.kernel
    def mixed_mma(c, BLOCK: eas.constexpr):
        _ = mk.tid(0, BLOCK)
        a = mk.alloc_tg_f16(64)
        b = mk.alloc_tg_bf16(64)
        mk.mma_store(c, 0, 8, mk.mma(a, 0, 8, b, 0, 8, mk.mma_zero()))

    with pytest.raises(TypeError, match="bf16"):
        mixed_mma.compile(f32(64), BLOCK=32)

    # the verifier holds the same rule for IR built by hand
    tg_a, tg_b = ValueRef(0, DType.F16), ValueRef(1, DType.BF16)
    z, u = ValueRef(2, DType.SG_F32_8X8), ValueRef(3, DType.U32)
    insts = (Inst("alloc_tg", tg_a, (64,)), Inst("alloc_tg", tg_b, (64,)), Inst("mma_zero", z, ()),
             Inst("const", u, (0,)), Inst("mma", ValueRef(4, DType.SG_F32_8X8), (tg_a, u, u, tg_b, u, u, z)))
    with pytest.raises(ValueError, match="bf16"):
        validate_ir(IRModule("k", (), insts))

    @eas.kernel
    def round_trip(a, b, BLOCK: eas.constexpr):
        i = mk.tid(0, BLOCK)
        mk.store(b, i, mk.to_f32(mk.to_bf16(mk.load(a, i))))

    ck = round_trip.compile(f32(64), f32(64), BLOCK=64)
    assert [i.op for i in ck.ir.insts].count("cast") == 2
    assert any(i.op == "cast" and i.out.dtype == DType.BF16 for i in ck.ir.insts)
