"""``eas.Tensor`` and DLPack on the host (CPU only), and the device copies (GPU).

Mirrors the reference's ``tests/test_tensor_f16.py:13-23``, ``tests/test_dlpack.py:13-40``,
``tests/test_torch_interop.py:34-45`` (host tensors) and ``tests/test_metal_copy.py:23-41``,
``tests/test_tensor.py:24-58`` (device tensors; the Apple device ``mps`` is ``hip`` here).
Inputs are seeded; every comparison is exact.
"""

from __future__ import annotations

import numpy as np
import pytest

import eas

import kernels as K
from conftest import seeded_normal


# ---- host tensors ---------------------------------------------------------------

def test_cpu_tensor_preserves_float16():
    a = seeded_normal(0, 128, np.float16)
    t = eas.tensor(a, device="cpu")
    assert t.dtype == np.dtype(np.float16) and t.device == "cpu" and t.shape == (128,)
    assert np.array_equal(t.numpy(), a) and t.numpy().dtype == np.float16


def test_empty_float16_and_default_float32():
    t = eas.empty((16, 8), device="cpu", dtype=np.float16)
    assert t.dtype == np.dtype(np.float16) and t.numpy().dtype == np.float16 and t.shape == (16, 8)
    assert eas.empty(5).dtype == np.dtype(np.float32)
    assert eas.empty_like(t).shape == (16, 8) and eas.empty_like(t).dtype == np.float16
    assert t.nbytes == 16 * 8 * 2


def test_other_dtypes_are_converted_or_rejected():
    # Python / float64 data becomes float32 (reference eas/tensor.py:45-49 supports f16 and f32 only)
    assert eas.tensor([1.0, 2.0]).dtype == np.dtype(np.float32)
    with pytest.raises(TypeError):
        eas.tensor(np.zeros(4, np.float64), dtype=np.float64)
    with pytest.raises(TypeError):
        eas.empty(4, dtype=np.int32)
    with pytest.raises(ValueError):
        eas.empty(4, device="mps")
    with pytest.raises(ValueError):
        eas.empty((2, -1))


def test_numpy_dlpack_roundtrip_cpu():
    a = seeded_normal(1, 1024)
    t = eas.tensor(a, device="cpu")
    cap = eas.to_dlpack(t)
    assert type(cap).__name__ == "PyCapsule"
    assert t.__dlpack_device__() == (1, 0)  # kDLCPU

    t2 = eas.from_dlpack(a)
    assert np.array_equal(t2.numpy(), a)
    # NumPy consumes the protocol from objects, not raw capsules
    b = np.from_dlpack(t)
    assert np.array_equal(b, a)
    t3 = eas.from_dlpack(np.from_dlpack(t.numpy()))
    assert np.array_equal(t3.numpy(), a)


def test_numpy_dlpack_roundtrip_cpu_float16():
    a = seeded_normal(2, 1024, np.float16)
    b = np.from_dlpack(eas.tensor(a, device="cpu"))
    assert b.dtype == np.float16 and np.array_equal(b, a)


def test_from_dlpack_rejects_non_float_and_non_producers():
    with pytest.raises(TypeError):
        eas.from_dlpack(np.zeros(4, np.int32))
    with pytest.raises(TypeError):
        eas.from_dlpack(object())
    with pytest.raises(TypeError):
        eas.to_dlpack(np.zeros(4, np.float32))


def test_torch_cpu_tensor_is_wrapped_zero_copy():
    torch = pytest.importorskip("torch")
    n = 1024 + 3
    a_t = torch.zeros(n, device="cpu", dtype=torch.float32)
    a = eas.tensor(a_t, device="cpu")
    a_t.add_(1.0)
    assert np.array_equal(a.numpy(), a_t.numpy())
    a.numpy()[0] = 7.0
    assert float(a_t[0].item()) == 7.0
    # and back: to_torch of a host tensor shares the same memory
    back = eas.to_torch(a)
    back[1] = 5.0
    assert float(a_t[1].item()) == 5.0


def test_hip_tensor_without_a_gpu_fails_loudly():
    from easy_as_amd.runtime.hip_ext import load_hip_ext

    if load_hip_ext(require=True).is_available():
        pytest.skip("a GPU is present; the device tests cover this path")
    with pytest.raises(RuntimeError, match="not available"):
        eas.tensor(np.zeros(4, np.float32), device="hip")
    with pytest.raises(RuntimeError, match="not available"):
        eas.empty(4, device="hip")


# ---- device tensors and copies --------------------------------------------------

@pytest.mark.gpu
def test_private_copy_roundtrip_numpy():
    from easy_as_amd.runtime.hip_ext import load_hip_ext

    mod = load_hip_ext(require=True)
    src = seeded_normal(3, 4096 + 7)
    dst = np.empty_like(src)
    buf = mod.alloc_buffer(int(src.nbytes), "private")
    mod.copy_from_host(buf, src)
    mod.copy_to_host(buf, dst)
    assert np.array_equal(dst.view(np.uint32), src.view(np.uint32))


@pytest.mark.gpu
def test_private_copy_roundtrip_bytearray_and_size_checks():
    from easy_as_amd.runtime.hip_ext import load_hip_ext

    mod = load_hip_ext(require=True)
    nbytes = 8192
    src = bytearray((i * 7 + 3) & 0xFF for i in range(nbytes))
    dst = bytearray(nbytes)
    buf = mod.alloc_buffer(nbytes, "private")
    mod.copy_from_host(buf, src)
    mod.copy_to_host(buf, dst)
    assert dst == src
    # pinned host storage takes the same copies
    pinned = mod.alloc_buffer(nbytes, "shared")
    mod.copy_from_host(pinned, src)
    back = bytearray(nbytes)
    mod.copy_to_host(pinned, back)
    assert back == src
    with pytest.raises(ValueError):
        mod.copy_from_host(buf, bytearray(nbytes + 1))  # larger than the buffer
    with pytest.raises(ValueError):
        mod.copy_to_host(buf, bytearray(nbytes - 1))  # smaller than the buffer
    with pytest.raises(ValueError):
        mod.alloc_buffer(0, "private")


@pytest.mark.gpu
def test_hip_tensor_roundtrip_and_kernel_bit_exact(gpu_runtime):
    n = 4096 + 3
    a_np, b_np = seeded_normal(0, n), seeded_normal(1, n)
    a, b = eas.tensor(a_np, device="hip"), eas.tensor(b_np, device="hip")
    assert a.device == "hip" and a.__dlpack_device__() == (10, 0)  # kDLROCM
    assert np.array_equal(a.numpy(), a_np) and np.array_equal(a.to("cpu").numpy(), a_np)
    c = eas.empty_like(a)
    K.add_kernel(a, b, c, n, BLOCK=256)
    assert np.array_equal(c.numpy().view(np.uint32), (a_np + b_np).view(np.uint32))


@pytest.mark.gpu
def test_cpu_tensors_run_through_the_device_and_copy_back(gpu_runtime):
    n = 4096 + 3
    a_np, b_np = seeded_normal(0, n), seeded_normal(1, n)
    a, b = eas.tensor(a_np, device="cpu"), eas.tensor(b_np, device="cpu")
    c = eas.empty_like(a)
    K.add_kernel(a, b, c, n, BLOCK=256)
    assert c.device == "cpu"
    assert np.array_equal(c.numpy().view(np.uint32), (a_np + b_np).view(np.uint32))
