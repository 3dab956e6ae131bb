"""GPU: the call memo's native launch (``HipRuntime.fast_launcher`` over ``_hip.fast_call``).

A repeated call of a kernel with torch GPU tensors or eas.Tensors and Python scalars (the reference's
add and fma kernels, eas/runtime/metal.py:244-352 on each call) is launched by one native
call after its first full-path call.  Each test checks the outputs against the oracle bit
for bit, and that calls the fast launch does not take (another dtype or argument kind, a
non-contiguous tensor, a scalar out of range, a zero extent) behave as on the full path.
"""

from __future__ import annotations

import numpy as np
import pytest

import eas
import kernels as K
from conftest import seeded_normal
from oracle import ops

pytestmark = pytest.mark.gpu


def _bits_equal(x, y) -> bool:
    x, y = np.asarray(x), np.asarray(y)
    return x.shape == y.shape and x.dtype == y.dtype and np.array_equal(x.view(np.uint8), y.view(np.uint8))


def _no_full_path(monkeypatch, rt):
    """Make the full path fail, so a call that succeeds went through the fast launch."""
    def refuse(*a, **k):
        raise AssertionError("the full path ran")

    monkeypatch.setattr(rt, "run", refuse)


@pytest.mark.parametrize("sync", [True, False])
def test_spmd_add_through_the_fast_launch(gpu_runtime, monkeypatch, sync):
    import torch

    k = eas.kernel(K.add_kernel.fn)
    n_max = (1 << 20) + 5
    a_np, b_np = seeded_normal(0, n_max), seeded_normal(1, n_max)
    a, b = torch.from_numpy(a_np).cuda(), torch.from_numpy(b_np).cuda()
    c = torch.full((n_max,), float("nan"), device="cuda")
    k(a, b, c, 1031, BLOCK=256, _sync=sync)  # full path; makes the fast launch
    assert len(k._fast) == 1
    _no_full_path(monkeypatch, gpu_runtime)
    want = ops.add_f32(a_np, b_np)
    for n in (1031, 4099, 1, n_max, 1031):  # a new N plans a new dispatch
        c.fill_(float("nan"))
        k(a, b, c, n, BLOCK=256, _sync=sync)
        gpu_runtime.synchronize()
        torch.cuda.synchronize()
        got = c.cpu().numpy()
        assert _bits_equal(got[:n], want[:n]) and np.all(np.isnan(got[n:])), n


def test_thread_mode_fma_through_the_fast_launch(gpu_runtime, monkeypatch):
    import torch

    k = eas.kernel(K.simple_fma_kernel.fn)
    n = 1000  # four threadgroups of 256, the last 24 threads past N do nothing
    a_np, b_np, c_np = seeded_normal(0, 1024), seeded_normal(1, 1024), seeded_normal(2, 1024)
    a, b, c = (torch.from_numpy(x).cuda() for x in (a_np, b_np, c_np))
    d = torch.full((1024,), 7.0, device="cuda")
    k(a, b, c, d, n, BLOCK=256)
    _no_full_path(monkeypatch, gpu_runtime)
    d.fill_(7.0)
    k(a, b, c, d, n, BLOCK=256)
    got = d.cpu().numpy()
    assert _bits_equal(got[:n], ops.fmaf(a_np[:n], b_np[:n], c_np[:n])) and np.all(got[n:] == 7.0)


def test_f32_scalar_and_calls_the_fast_launch_declines(gpu_runtime):
    import torch

    k = eas.kernel(K.axpy_kernel.fn)
    n = 4099
    a_np, b_np = seeded_normal(0, n), seeded_normal(1, n)
    a, b = torch.from_numpy(a_np).cuda(), torch.from_numpy(b_np).cuda()
    c = torch.zeros(n, device="cuda")
    k(a, b, c, n, 2.0, BLOCK=256)
    assert len(k._fast) == 1
    for alpha in (3.5, 0.25):  # new f32 scalar values through the fast launch
        k(a, b, c, n, alpha, BLOCK=256)
        assert _bits_equal(c.cpu().numpy(), ops.fmaf(a_np, np.float32(alpha), b_np)), alpha
    # NumPy arguments take the full path (staged and copied back)
    c_np = np.zeros(n, np.float32)
    k(a_np, b_np, c_np, n, 2.0, BLOCK=256)
    assert _bits_equal(c_np, ops.fmaf(a_np, np.float32(2.0), b_np))
    # another dtype (f16 tensors, an f16 scalar): a new specialisation on the full path
    h = [torch.from_numpy(x.astype(np.float16)).cuda() for x in (a_np, b_np)]
    hc = torch.zeros(n, dtype=torch.float16, device="cuda")
    k(h[0], h[1], hc, n, np.float16(2.0), BLOCK=256)
    assert len(k._cache) == 3  # f32 GPU tensors, NumPy host arrays, f16 GPU tensors
    want16 = (a_np.astype(np.float16) * np.float16(2.0)).astype(np.float16) + b_np.astype(np.float16)
    assert np.allclose(hc.cpu().numpy().astype(np.float32), want16.astype(np.float32), rtol=2e-3, atol=2e-3)
    # the full path's errors: a non-contiguous tensor, a u32 out of range
    with pytest.raises(ValueError, match="contiguous"):
        k(a, b, torch.zeros(2 * n, device="cuda")[::2], n, 2.0, BLOCK=256)
    with pytest.raises(OverflowError):
        k(a, b, c, 1 << 32, 2.0, BLOCK=256)
    with pytest.raises(OverflowError):  # an f32 scalar beyond the f32 range
        k(a, b, c, n, 1e39, BLOCK=256)
    k(a, b, c, n, float("inf"), BLOCK=256)  # infinities pack as they are
    assert np.all(a_np != 0)  # so every output is an infinity, no NaN
    assert _bits_equal(c.cpu().numpy(), ops.fmaf(a_np, np.float32(np.inf), b_np))
    # a zero extent launches nothing
    c.fill_(5.0)
    k(a, b, c, 0, 2.0, BLOCK=256)
    torch.cuda.synchronize()
    assert bool((c == 5.0).all())


def test_fast_launches_keep_the_in_flight_bound(monkeypatch):
    import torch

    import importlib

    from easy_as_amd.runtime.hip import HipRuntime

    eas_kernel = importlib.import_module("easy_as_amd.kernel")  # the module, not the kernel() it exports

    monkeypatch.setenv("EAS_MAX_IN_FLIGHT", "3")
    rt = HipRuntime()
    monkeypatch.setattr(eas_kernel, "get_runtime", lambda *a, **kw: rt)
    k = eas.kernel(K.add_kernel.fn)
    n = 1 << 20
    a_np, b_np = seeded_normal(0, n), seeded_normal(1, n)
    a, b = torch.from_numpy(a_np).cuda(), torch.from_numpy(b_np).cuda()
    outs = [torch.zeros(n, device="cuda") for _ in range(10)]
    seen = []
    for o in outs:
        k(a, b, o, n, BLOCK=256, _sync=False)
        seen.append(len(rt._pending))
    assert len(k._fast) == 1 and max(seen) == 3
    hip = rt._mod()
    for p in rt._pending:
        info = hip.pending_info(p)
        assert info["released"] or (info["limit"] == 3 and info["launches"] <= 3), info
    rt.synchronize()
    torch.cuda.synchronize()
    want = ops.add_f32(a_np, b_np)
    for o in outs:
        assert _bits_equal(o.cpu().numpy(), want)


@pytest.mark.parametrize("sync", [True, False])
def test_eas_gpu_tensors_through_the_fast_launch(gpu_runtime, monkeypatch, sync):
    """eas.Tensors on the GPU (the reference's own device buffers) take the fast launch on the
    default stream, alone and beside torch GPU tensors (then on torch's current stream)."""
    import torch

    k = eas.kernel(K.add_kernel.fn)
    n_max = (1 << 18) + 3
    a_np, b_np = seeded_normal(0, n_max), seeded_normal(1, n_max)
    a, b = eas.tensor(a_np, device="hip"), eas.tensor(b_np, device="hip")
    c = eas.tensor(np.full(n_max, np.nan, np.float32), device="hip")
    k(a, b, c, 1031, BLOCK=256, _sync=sync)  # full path; makes the fast launch
    assert len(k._fast) == 1
    want = ops.add_f32(a_np, b_np)
    gpu_runtime.synchronize()
    got = c.numpy()
    assert _bits_equal(got[:1031], want[:1031]) and np.all(np.isnan(got[1031:]))
    _no_full_path(monkeypatch, gpu_runtime)
    for n in (4099, 1, n_max):
        k(a, b, c, n, BLOCK=256, _sync=sync)
        gpu_runtime.synchronize()
        got = c.numpy()
        assert _bits_equal(got[:n], want[:n]), n
    # a torch GPU tensor for c: another memo key, run by the full path first and by the memo
    # after, on torch's current stream
    monkeypatch.undo()
    tc = torch.full((n_max,), float("nan"), device="cuda")
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        k(a, b, tc, 777, BLOCK=256, _sync=sync)
        k(a, b, tc, 4099, BLOCK=256, _sync=sync)
    gpu_runtime.synchronize()
    s.synchronize()
    got = tc.cpu().numpy()
    assert _bits_equal(got[:4099], want[:4099]) and np.all(np.isnan(got[4099:]))


def test_eas_tensors_the_fast_launch_declines(gpu_runtime):
    """Host eas.Tensors and GPU ones of another dtype take the full path, with its results and
    errors."""
    k = eas.kernel(K.add_kernel.fn)
    n = 2048
    a_np, b_np = seeded_normal(0, n), seeded_normal(1, n)
    a, b = eas.tensor(a_np, device="hip"), eas.tensor(b_np, device="hip")
    c = eas.empty(n, device="hip")
    k(a, b, c, n, BLOCK=256)
    assert len(k._fast) == 1
    # host eas.Tensors: staged and copied back by the full path
    hc = eas.tensor(np.zeros(n, np.float32))
    k(eas.tensor(a_np), eas.tensor(b_np), hc, n, BLOCK=256)
    assert _bits_equal(hc.numpy(), ops.add_f32(a_np, b_np))
    # f16 GPU tensors: the full path's f16 specialisation
    h = [eas.tensor(x.astype(np.float16), device="hip") for x in (a_np, b_np)]
    hc16 = eas.empty(n, device="hip", dtype=np.float16)
    k(h[0], h[1], hc16, n, BLOCK=256)
    assert _bits_equal(hc16.numpy(), ops.add_f16(a_np.astype(np.float16), b_np.astype(np.float16)))
    # a GPU tensor of another dtype in one slot: the full path's dtype error
    with pytest.raises(TypeError):
        k(a, b, hc16, n, BLOCK=256)
