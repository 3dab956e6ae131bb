"""Host side of the boundary, on the CPU: the C-ABI library, launch planning,
kernel-argument packing, autotune and grid inference.

No GPU compute happens here.  The C-ABI checks call only entry points that need
no device (symbol export, ABI version, hiprtc compilation, error returns); the
runtime checks drive ``HipRuntime`` through a recording stand-in for the
``_hip`` extension.
"""

from __future__ import annotations

import ctypes
import importlib
import re
import struct
from pathlib import Path

import numpy as np
import pytest

import eas
import kernels as K
from eas import mk
from easy_as_amd.runtime.grid import infer_grid, infer_nthreads
from easy_as_amd.runtime.hip import HipRuntime, plan_launch

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "eas_hip.h"
LIB = ROOT / "easy_as_amd" / "libeas_hip.so"
# the module (the package re-exports a function of the same name)
eas_kernel = importlib.import_module("easy_as_amd.kernel")


def _declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(eas_hip_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not LIB.exists():
        pytest.fail(f"{LIB} is not built; run __graft_entry__.build()")
    return ctypes.CDLL(str(LIB))


# ---- C ABI -------------------------------------------------------------------

def test_header_declares_the_boundary():
    names = _declared_functions()
    for required in ("eas_hip_is_available", "eas_hip_compile_source", "eas_hip_kernel_load", "eas_hip_launch",
                     "eas_hip_alloc", "eas_hip_free", "eas_hip_copy_h2d", "eas_hip_copy_d2h", "eas_hip_dlpack_view",
                     "eas_hip_dlpack_make", "eas_hip_stream_synchronize", "eas_hip_event_elapsed_ms"):
        assert required in names


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in _declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_abi_version_matches_header(lib):
    m = re.search(r"#define\s+EAS_HIP_ABI_VERSION\s+(\d+)", HEADER.read_text())
    assert m and lib.eas_hip_abi_version() == int(m.group(1))


def test_compile_source_without_gpu(lib):
    lib.eas_hip_compile_source.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p),
                                           ctypes.c_int, ctypes.POINTER(ctypes.c_void_p),
                                           ctypes.POINTER(ctypes.c_size_t), ctypes.c_char_p, ctypes.c_size_t]
    opts = (ctypes.c_char_p * 2)(b"--offload-arch=gfx950", b"-O3")
    code, size = ctypes.c_void_p(), ctypes.c_size_t()
    log = ctypes.create_string_buffer(4096)
    src = b'extern "C" __global__ void k(float* x) { x[threadIdx.x] += 1.0f; }'
    rc = lib.eas_hip_compile_source(src, b"k.hip", opts, 2, ctypes.byref(code), ctypes.byref(size), log, 4096)
    assert rc == 0, log.value
    head = ctypes.string_at(code, 4)
    lib.eas_hip_free_host.argtypes = [ctypes.c_void_p]
    lib.eas_hip_free_host(code)
    assert head == b"\x7fELF" and size.value > 0
    # a syntax error is EAS_HIP_ERR_COMPILE (-3) with the compiler log filled in
    rc = lib.eas_hip_compile_source(b"this is not C++", b"bad.hip", opts, 2, ctypes.byref(code),
                                    ctypes.byref(size), log, 4096)
    assert rc == -3 and b"error" in log.value


def test_null_arguments_are_invalid(lib):
    lib.eas_hip_last_error.restype = ctypes.c_char_p
    lib.eas_hip_compile_source.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_void_p, ctypes.c_int,
                                           ctypes.c_void_p, ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t]
    assert lib.eas_hip_compile_source(None, None, None, 0, None, None, None, 0) == -1
    assert b"must not be NULL" in lib.eas_hip_last_error()
    lib.eas_hip_compiler_version.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t]
    assert lib.eas_hip_compiler_version(None, None, None, 0) == -1


def test_compiler_version_is_rocm_hiprtc(lib):
    major, minor = ctypes.c_int(), ctypes.c_int()
    path = ctypes.create_string_buffer(512)
    lib.eas_hip_compiler_version.argtypes = [ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int),
                                             ctypes.c_char_p, ctypes.c_size_t]
    assert lib.eas_hip_compiler_version(ctypes.byref(major), ctypes.byref(minor), path, 512) == 0
    assert major.value >= 7 and path.value.endswith(b"libhiprtc.so.7")


def test_compile_after_environment_grows():
    # hiprtc lives in a private link namespace with its own libc; growing the
    # environment (setenv reallocates the array) must not leave it reading freed memory
    import subprocess
    import sys

    script = (
        "import os\n"
        "os.environ['EAS_T_PRE'] = '1'\n"
        "from easy_as_amd.runtime.hip_ext import load_hip_ext\n"
        "m = load_hip_ext(require=True)\n"
        "src = 'extern \"C\" __global__ void k(float* x) { x[threadIdx.x] = %s; }'\n"
        "opts = ['--offload-arch=gfx950', '-O3']\n"
        "m.compile_to_code(src % '1.0f', 'k.hip', opts)\n"
        "for i in range(300): os.environ[f'EAS_T_GROW_{i}'] = 'x' * 64\n"
        "m.compiler_version()\n"
        "assert m.compile_to_code(src % '2.0f', 'k.hip', opts)[:4] == b'\\x7fELF'\n"
        "print('ok')\n"
    )
    r = subprocess.run([sys.executable, "-c", script], cwd=ROOT, capture_output=True, text=True, timeout=300,
                       env={**__import__("os").environ, "PYTHONPATH": str(ROOT)})
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), (r.returncode, r.stderr[-2000:])


def test_no_device_paths_fail_cleanly(lib):
    if lib.eas_hip_is_available() != 0:
        pytest.skip("a GPU is visible; the no-device contract is checked only on CPU hosts")
    buf = ctypes.c_void_p()
    lib.eas_hip_alloc.argtypes = [ctypes.c_size_t, ctypes.c_int, ctypes.POINTER(ctypes.c_void_p)]
    assert lib.eas_hip_alloc(1024, 0, ctypes.byref(buf)) == -2  # EAS_HIP_ERR_NODEV


# ---- grid inference (reference known answers) --------------------------------

def test_infer_grid_from_h_w():
    ck = K.add2d_hw_kernel.compile(np.zeros(1, np.float32), np.zeros(1, np.float32), np.zeros(1, np.float32),
                                   17, 103, BLOCK=32)
    assert infer_grid(ck.ir, {"H": 17, "W": 103}, ck.block_size) == (4, 17, 1)


def test_infer_grid_from_shape_option():
    ck = K.add2d_shape_kernel.compile(np.zeros(1, np.float32), np.zeros(1, np.float32), np.zeros(1, np.float32),
                                      9, 65, BLOCK=16)
    assert infer_grid(ck.ir, {}, ck.block_size, shape=(9, 65)) == (5, 9, 1)


def test_infer_nthreads_rules():
    assert infer_nthreads({"N": 1031}) == 1031
    assert infer_nthreads({"N": 1031}, nthreads=7) == 7
    with pytest.raises(Exception):
        infer_nthreads({})


# ---- launch planning ------------------------------------------------------------

def _add_ck(block=256):
    z = np.zeros(1, np.float32)
    return K.add_kernel.compile(z, z, z, 1031, BLOCK=block)


@pytest.mark.parametrize("block", [256, 1024])
def test_plan_spmd_add_splits_programs(block):
    # c = a + b reads two streams and writes one: 512 bytes of each stream per workgroup
    # (32 threads of 16 bytes), so one BLOCK-lane program spans BLOCK/128 workgroups
    ck = _add_ck(block)
    n = 1 << 28
    plan = plan_launch(ck, {"N": n})
    geo = ck.geometry
    programs = -(-n // block)
    assert geo.wg_size == 32 and geo.programs_per_wg == 1 and geo.split == block // 128
    assert plan.hidden == (programs,)
    assert plan.grid == (programs * geo.split, 1, 1)
    assert plan.block == (32, 1, 1)
    # the split workgroups' lanes cover the program's BLOCK elements exactly
    assert geo.split * geo.wg_size * geo.params["lanes_per_thread"] == block


def test_spmd_workgroup_size_follows_stream_count():
    z = np.zeros(1, np.float32)
    shapes = {name: getattr(K, name).compile(*args, BLOCK=256).geometry for name, args in (
        ("fill_kernel", (z, 1)), ("copy_kernel", (z, z, 1)), ("add_kernel", (z, z, z, 1)),
        ("fma_kernel", (z, z, z, z, 1)), ("read_kernel", (z, z, 1)), ("spmd_tg_rotate_kernel", (z, z, 1)))}
    # bytes per stream per workgroup: 4 KiB (one stream), 1 KiB (two), 512 B (three or more)
    assert (shapes["fill_kernel"].wg_size, shapes["fill_kernel"].programs_per_wg) == (256, 4)
    assert (shapes["copy_kernel"].wg_size, shapes["copy_kernel"].split) == (64, 1)
    assert (shapes["add_kernel"].wg_size, shapes["add_kernel"].split) == (32, 2)
    assert (shapes["fma_kernel"].wg_size, shapes["fma_kernel"].split) == (32, 2)
    # no dense output stream: 64 bytes per thread, 256 threads
    assert shapes["read_kernel"].wg_size == 256
    # threadgroup memory keeps a program in one workgroup
    assert shapes["spmd_tg_rotate_kernel"].split == 1


def test_spmd_workgroup_override_is_validated(monkeypatch):
    z = np.zeros(1, np.float32)
    monkeypatch.setenv("EAS_HIP_SPMD_WG", "1024")
    geo = eas.kernel(K.add_kernel.fn).compile(z, z, z, 1, BLOCK=256).geometry
    assert (geo.wg_size, geo.programs_per_wg, geo.split) == (1024, 16, 1)
    monkeypatch.setenv("EAS_HIP_SPMD_WG", "96")
    with pytest.raises(ValueError, match="EAS_HIP_SPMD_WG"):
        eas.kernel(K.add_kernel.fn).compile(z, z, z, 1, BLOCK=256)


def test_plan_zero_extent_and_tptg_rules(monkeypatch):
    ck = _add_ck()
    assert plan_launch(ck, {"N": 0}) is None
    assert plan_launch(ck, {"N": 10}, grid=(0, 1, 1)) is None
    with pytest.raises(ValueError):
        plan_launch(ck, {"N": 10}, tptg=(256, 1, 1))  # SPMD kernels take (1,1,1)
    tck = K.tptg_independent_kernel.compile(np.zeros(1, np.float32), 10, BLOCK=64)
    assert tck.launch_mode == "thread" and tck.geometry.params.get("lanes")
    # 1000 threads in 16 threadgroups of 64: as lanes, 16 threads of 16-byte vectors per
    # threadgroup, 16 threadgroups per 256-thread workgroup; one thread per Metal thread, one
    # workgroup per threadgroup
    plan = plan_launch(tck, {"N": 1000}, tptg=(64, 1, 1))
    assert plan.grid == (1, 1, 1) and plan.block == (256, 1, 1) and plan.hidden == (1000,)
    monkeypatch.setenv("EAS_HIP_THREAD_LANES", "0")
    one = eas.kernel(K.tptg_independent_kernel.fn).compile(np.zeros(1, np.float32), 10, BLOCK=64)
    plan = plan_launch(one, {"N": 1000}, tptg=(64, 1, 1))
    assert plan.grid == (16, 1, 1) and plan.block == (64, 1, 1) and plan.hidden == (1000,)
    for c in (tck, one):
        with pytest.raises(ValueError):
            plan_launch(c, {"N": 1000}, tptg=(1, 1, 1))


def test_plan_lifted_gemm_covers_the_reference_rectangle():
    f16, f32 = np.zeros(1, np.float16), np.zeros(1, np.float32)
    ck = K.matmul_mma_kernel.compile(f16, f16, f32, 300, 520, BM=32, BN=32, BK=8, K=200, NT=512)
    assert ck.geometry.kind == "gemm"
    plan = plan_launch(ck, {"M": 300, "N": 520}, grid=(17, 10, 1))
    # 6 tiles of 256 x 256, or 15 of 128 x 128, would leave CUs idle: 5 x 9 tiles of 64 x 64
    assert plan.hidden == (0, 300, 0, 520) and plan.grid == (5 * 9, 1, 1)
    assert plan.block == (512, 1, 1) and plan.entry == "matmul_mma_kernel__t64x64"
    plan = plan_launch(ck, {"M": 300, "N": 520}, grid=(3, 2, 1))  # partial grid: 64 x 96 rectangle
    assert plan.hidden == (0, 64, 0, 96) and plan.grid == (2, 1, 1)  # 64 rows: skinny, 64 columns per workgroup
    # M <= 128 (decode-like): one workgroup per 64 columns, on the 4-wave entry
    for m in (16, 17, 64, 128):
        plan = plan_launch(ck, {"M": m, "N": 14336}, grid=(448, K.cdiv(m, 32), 1))
        assert plan.hidden == (0, m, 0, 14336) and plan.grid == (224, 1, 1)
        assert plan.block == (256, 1, 1) and plan.entry is None
    # up to 128 rows: 128 columns per workgroup rather than a second round of CUs
    for m in (16, 17, 64, 65, 128):
        plan = plan_launch(ck, {"M": m, "N": 28672}, grid=(896, K.cdiv(m, 32), 1))
        assert plan.grid == (224, 1, 1) and plan.entry is None
    # 17-128 rows too wide for one round of 128-column groups: 128 x 128 tiles
    plan = plan_launch(ck, {"M": 65, "N": 40960}, grid=(1280, 3, 1))
    assert plan.grid == (320, 1, 1) and plan.entry == "matmul_mma_kernel__t128"
    plan = plan_launch(ck, {"M": 128, "N": 40960}, grid=(1280, 4, 1))
    assert plan.grid == (320, 1, 1) and plan.entry == "matmul_mma_kernel__t128" and plan.block == (512, 1, 1)
    plan = plan_launch(ck, {"M": 16, "N": 16384}, grid=(512, 1, 1))
    assert plan.grid == (256, 1, 1) and plan.entry is None  # 256 groups of 64: still one round
    plan = plan_launch(ck, {"M": 16, "N": 16390}, grid=(513, 1, 1))
    assert plan.grid == (129, 1, 1) and plan.entry is None
    plan = plan_launch(ck, {"M": 129, "N": 14336}, grid=(448, 5, 1))
    assert plan.hidden == (0, 129, 0, 14336) and plan.grid == (2 * 112, 1, 1)
    assert plan.entry == "matmul_mma_kernel__t128"


@pytest.mark.parametrize("mn,entry,grid", [((4096, 4096), "__pp", 256), ((3072, 3072), "__pp", 144),
                                           ((2560, 2560), "__t128x256", 200), ((2048, 2048), "__t128", 256),
                                           ((512, 14336), "__t128x256", 224), ((256, 14336), "__t128", 224),
                                           ((1536, 1536), "__t128", 144), ((1024, 1024), "__t64x64", 256),
                                           ((1280, 1280), "__t64x64", 400), ((2048, 1024), "__t128x64", 256),
                                           ((8192, 8192), "__pp", 1024)])
def test_plan_tile_size_follows_the_cu_count(mn, entry, grid):
    # 256 x 256 tiles unless they would fill at most half of the 256 CUs; then 128 x 128 tiles if
    # they take one round of CUs, else 128 x 256; if 128 x 128 would fill at most half, 64 x 64
    # while they need at most 1.75 rounds, else 128 x 64
    m, n = mn
    f16, f32 = np.zeros(1, np.float16), np.zeros(1, np.float32)
    ck = K.matmul_mma_kernel.compile(f16, f16, f32, m, n, BM=32, BN=32, BK=8, K=64, NT=512)
    plan = plan_launch(ck, {"M": m, "N": n}, grid=(n // 32, m // 32, 1))
    assert plan.entry == "matmul_mma_kernel" + entry and plan.grid == (grid, 1, 1)
    assert plan.block == (512, 1, 1)


def test_plan_fp32_tile_size(monkeypatch):
    # fp32: 128 x 128 tiles while they still give every CU one, else 64 x 64; both entries run
    # 4 consumer and 4 producer waves
    z = np.zeros(1, np.float32)
    for m, entry, grid in ((2048, "matmul_tiled_kernel__t128", 256), (1024, None, 256), (1536, None, 576)):
        ck = K.matmul_tiled_kernel.compile(z, z, z, m, m, 0, 0, BM=32, BN=32, BK=32, K=64, NT=256)
        args = {"M": m, "N": m, "PID_M_BASE": 0, "PID_N_BASE": 0}
        plan = plan_launch(ck, args, grid=(m // 32, m // 32, 1))
        assert plan.entry == entry and plan.grid == (grid, 1, 1) and plan.block == (512, 1, 1)
    ck = K.matmul_tiled_kernel.compile(z, z, z, 2048, 2048, 0, 0, BM=32, BN=32, BK=32, K=62, NT=256)
    assert plan_launch(ck, {"M": 2048, "N": 2048, "PID_M_BASE": 0, "PID_N_BASE": 0},
                       grid=(64, 64, 1)).entry is None  # rows of 62 floats are not 16-byte aligned
    monkeypatch.setenv("EAS_HIP_GEMM_ENTRY", "tile128")
    ck = K.matmul_tiled_kernel.compile(z, z, z, 100, 200, 0, 0, BM=32, BN=32, BK=32, K=64, NT=256)
    plan = plan_launch(ck, {"M": 100, "N": 200, "PID_M_BASE": 0, "PID_N_BASE": 0}, grid=(7, 4, 1))
    assert plan.entry == "matmul_tiled_kernel__t128" and plan.grid == (2, 1, 1)


class _FakeTorchTensor:
    def __init__(self, addr, numel):
        self._addr, self._numel = addr, numel

    def data_ptr(self):
        return self._addr

    def numel(self):
        return self._numel


def test_plan_dma_entries_only_for_operands_the_dma_takes(monkeypatch):
    f16, f32 = np.zeros(1, np.float16), np.zeros(1, np.float32)
    ck = K.matmul_mma_kernel.compile(f16, f16, f32, 512, 512, BM=32, BN=32, BK=8, K=64, NT=512)
    args = {"M": 512, "N": 512}
    monkeypatch.setenv("EAS_HIP_GEMM_ENTRY", "8wave")
    assert plan_launch(ck, args, grid=(16, 16, 1)).entry == "matmul_mma_kernel__pp"
    # odd row stride of B: rows are not 4-byte aligned
    assert plan_launch(ck, {"M": 512, "N": 511}, grid=(16, 16, 1)).entry is None
    # a torch operand at a 2-byte offset
    odd = {**args, "a": _FakeTorchTensor(0x1000002, 512 * 64), "b": _FakeTorchTensor(0x2000000, 64 * 512)}
    assert plan_launch(ck, odd, grid=(16, 16, 1)).entry is None
    even = {**args, "a": _FakeTorchTensor(0x1000004, 512 * 64), "b": _FakeTorchTensor(0x2000000, 64 * 512)}
    assert plan_launch(ck, even, grid=(16, 16, 1)).entry == "matmul_mma_kernel__pp"
    # odd K (rows of A 2-byte aligned) and f32 inputs have no 8-wave entry
    ck_odd = K.matmul_mma_kernel.compile(f16, f16, f32, 512, 512, BM=32, BN=32, BK=8, K=63, NT=512)
    assert ck_odd.geometry.params["pp_entry"] is None and "__pp" not in ck_odd.src and "__t128" not in ck_odd.src
    assert plan_launch(ck_odd, args, grid=(16, 16, 1)).entry is None
    ck32 = K.matmul_mma_kernel.compile(f32, f32, f32, 512, 512, BM=32, BN=32, BK=8, K=64, NT=512)
    assert ck32.geometry.params["pp_entry"] is None and "__pp" not in ck32.src
    assert plan_launch(ck32, args, grid=(16, 16, 1)).block == (256, 1, 1)
    # the entry switch: one entry for every launch the DMA takes, or the automatic choice
    monkeypatch.setenv("EAS_HIP_GEMM_ENTRY", "tile128")
    assert plan_launch(ck, args, grid=(16, 16, 1)).entry == "matmul_mma_kernel__t128"
    monkeypatch.setenv("EAS_HIP_GEMM_ENTRY", "4wave")
    assert plan_launch(ck, args, grid=(16, 16, 1)).entry is None
    monkeypatch.setenv("EAS_HIP_GEMM_ENTRY", "tile128x64")
    assert plan_launch(ck, args, grid=(16, 16, 1)).entry == "matmul_mma_kernel__t128x64"
    monkeypatch.setenv("EAS_HIP_GEMM_ENTRY", "tile64")
    assert plan_launch(ck, args, grid=(16, 16, 1)).entry == "matmul_mma_kernel__t64x64"
    monkeypatch.setenv("EAS_HIP_GEMM_ENTRY", "auto")  # 512 x 512: 16 tiles of 128 x 128, so 64 x 64
    assert plan_launch(ck, args, grid=(16, 16, 1)).entry == "matmul_mma_kernel__t64x64"
    monkeypatch.setenv("EAS_HIP_GEMM_ENTRY", "fastest")
    with pytest.raises(ValueError):
        plan_launch(ck, args, grid=(16, 16, 1))


# ---- kernel-argument packing through a recording extension ------------------------

class _RecordingExt:
    ABI_VERSION = 3

    def __init__(self):
        self.launches, self.h2d, self.d2h, self.allocs = [], [], [], []

    def alloc_buffer(self, nbytes, storage):
        self.allocs.append((nbytes, storage))
        return ("buf", len(self.allocs))

    def copy_from_host(self, buf, arr):
        self.h2d.append((buf, arr.nbytes))

    def copy_to_host(self, buf, arr):
        self.d2h.append((buf, arr.nbytes))

    def compile_to_code(self, src, name, options):
        return b"\x7fELF-recorded"

    def load(self, code, entry, src=None):
        return ("kernel", entry)

    def launch_groups(self, kernel, argv, writable, grid, block, stream=None):
        self.launches.append((kernel, list(argv), list(writable), grid, block))

    def launch_groups_async(self, kernel, argv, writable, grid, block, stream=None, batch=16):
        self.launch_groups(kernel, argv, writable, grid, block, stream)
        self.batches = getattr(self, "batches", []) + [batch]
        return ("pending", len(self.launches))

    def synchronize(self, pending):
        pass

    def queue_synchronize(self, stream=None):
        pass


def test_numpy_add_argv_contract(monkeypatch, tmp_path):
    monkeypatch.setenv("EAS_HIP_CACHE_DIR", str(tmp_path))
    ext = _RecordingExt()
    rt = HipRuntime(ext=ext)
    monkeypatch.setattr(eas_kernel, "get_runtime", lambda *a, **k: rt)
    n = 1031
    a = np.ones(n, np.float32)
    b = np.ones(n, np.float32)
    c = np.zeros(n, np.float32)
    K.add_kernel(a, b, c, n, BLOCK=256)
    assert len(ext.launches) == 1
    kern, argv, writable, grid, block = ext.launches[0]
    assert kern == ("kernel", "add_kernel")
    # IR argument order (a, b, c, N) then the hidden program count
    assert argv[:3] == [("buf", 1), ("buf", 2), ("buf", 3)]
    assert argv[3] == struct.pack("<I", n) and argv[4] == struct.pack("<I", 5)
    assert writable == [False, False, True, False, False]
    # numpy inputs are staged; only the written buffer is copied back (a synchronous launch)
    assert [nb for _, nb in ext.h2d] == [4 * n] * 3
    assert ext.d2h == [(("buf", 3), 4 * n)]


def _recording_runtime(monkeypatch, tmp_path):
    monkeypatch.setenv("EAS_HIP_CACHE_DIR", str(tmp_path))
    ext = _RecordingExt()
    rt = HipRuntime(ext=ext)
    monkeypatch.setattr(eas_kernel, "get_runtime", lambda *a, **k: rt)
    return ext


def test_call_memo_launches_what_the_full_path_launches(monkeypatch, tmp_path):
    """Repeated calls of one argument shape skip binding and specialisation (the call memo); the
    launch they make is the one the full path makes, scalar values included."""
    ext = _recording_runtime(monkeypatch, tmp_path)
    k = eas.kernel(K.axpy_kernel.fn)
    a, b, c = np.ones(1031, np.float32), np.ones(1031, np.float32), np.zeros(1031, np.float32)
    k(a, b, c, 1031, 2.0, BLOCK=256, _sync=True)
    assert len(k._memo) == 1
    k(a, b, c, 1000, 3.5, BLOCK=256, _sync=True)  # memo hit: new scalar values, same kernel
    monkeypatch.setattr(k, "_memo", {})  # the same call through the full path
    k(a, b, c, 1000, 3.5, BLOCK=256, _sync=True)
    assert len(ext.launches) == 3

    def shape(launch):  # NumPy arguments are staged afresh on every call: compare buffer slots
        kern, argv, writable, grid, block = launch
        return kern, [x[0] if isinstance(x, tuple) else x for x in argv], writable, grid, block

    assert shape(ext.launches[1]) == shape(ext.launches[2])
    assert ext.launches[1][1][3] == struct.pack("<I", 1000) and ext.launches[1][1][4] == struct.pack("<f", 3.5)
    assert ext.launches[0][1][3] == struct.pack("<I", 1031)


def test_call_memo_keys_everything_that_selects_a_kernel(monkeypatch, tmp_path):
    ext = _recording_runtime(monkeypatch, tmp_path)
    k = eas.kernel(K.add_kernel.fn)
    f32 = [np.ones(64, np.float32) for _ in range(3)]
    f16 = [np.ones(64, np.float16) for _ in range(3)]
    k(*f32, 64, BLOCK=64)
    k(*f32, 64, BLOCK=128)  # another meta value
    k(*f16, 64, BLOCK=64)  # another dtype
    k(*f32, 64, BLOCK=64, _sync=False)  # another option value
    assert len(k._memo) == 4 and len(k._cache) == 3
    k(*f32, 64, BLOCK=64)
    assert len(k._memo) == 4 and len(ext.launches) == 5
    # launch options other than _sync, keyword runtime arguments and unkeyed types bypass the memo
    k(*f32, 64, BLOCK=64, _grid=(1, 1, 1))
    k(*f32, N=64, BLOCK=64)
    k(*f32, np.uint32(64), BLOCK=64)
    assert len(k._memo) == 4 and len(ext.launches) == 8


def test_call_memo_still_rejects_bad_arguments(monkeypatch, tmp_path):
    _recording_runtime(monkeypatch, tmp_path)
    k = eas.kernel(K.add_kernel.fn)
    a = np.ones(64, np.float32)
    k(a, a, a.copy(), 64, BLOCK=64)
    with pytest.raises(TypeError):
        k(a, a, a.astype(np.float64), 64, BLOCK=64)  # another light key: the full path checks it
    with pytest.raises(ValueError):
        k(a, a, np.ones(128, np.float32)[::2], 64, BLOCK=64)  # same light key, not contiguous


class _FastRuntime:
    """A runtime with a fast launcher: records full-path runs and fast calls, and declines
    (NotImplemented) calls whose first argument is the `decline` object."""

    def __init__(self):
        self.runs, self.fast_calls, self.made = [], [], []
        self.decline = object()

    def run(self, ck, runtime_args, meta, **opts):
        self.runs.append((ck, dict(runtime_args), dict(meta), opts))

    def fast_launcher(self, ck, names, args, sync):
        self.made.append((ck, names, args, sync))

        def launch(call_args):
            self.fast_calls.append((ck, call_args, sync))
            return NotImplemented if call_args[0] is self.decline else None

        return launch


def test_call_memo_takes_the_runtime_fast_launch(monkeypatch):
    rt = _FastRuntime()
    monkeypatch.setattr(eas_kernel, "get_runtime", lambda *a, **k: rt)
    k = eas.kernel(K.add_kernel.fn)
    a = np.ones(64, np.float32)
    k(a, a, a, 64, BLOCK=64, _sync=False)
    # the first call runs the full path and makes the fast launch for its keyword items
    assert len(rt.runs) == 1 and len(rt.made) == 1 and not rt.fast_calls
    ck, names, args, sync = rt.made[0]
    assert names == ("a", "b", "c", "N") and args[3] == 64 and sync is False
    k(a, a, a, 100, BLOCK=64, _sync=False)
    assert len(rt.runs) == 1 and rt.fast_calls[-1][1][3] == 100
    # declined: the memo's full-path launch runs the call
    b = np.ones(64, np.float32)
    rt.decline = b
    k(b, a, a, 64, BLOCK=64, _sync=False)
    assert len(rt.runs) == 2 and rt.runs[-1][1]["a"] is b and rt.runs[-1][3]["sync"] is False
    # other keyword items have their own fast launch; options other than _sync never make one
    k(a, a, a, 64, BLOCK=128, _sync=False)
    assert len(rt.made) == 2 and set(k._fast) == {(("BLOCK", 64), ("_sync", False)), (("BLOCK", 128), ("_sync", False))}
    k(a, a, a, 64, BLOCK=32, _grid=(1, 1, 1))
    assert len(rt.made) == 2


class _FastMakingExt(_RecordingExt):
    """Records the native fast launches HipRuntime.fast_launcher makes and calls."""

    def __init__(self):
        super().__init__()
        self.made, self.calls = [], []

    def fast_make(self, kernel, specs, n_index, sync, batch, tensor_type, streams, eas_type):
        self.made.append((kernel, list(specs), n_index, sync, batch, tensor_type, eas_type))
        return ("fast", len(self.made))

    def fast_call(self, fast, args):
        """Declines as the native call does: an eas.Tensor argument must be on the GPU and of the
        recorded dtype."""
        specs = self.made[fast[1] - 1][1]
        for (kind, expect), v in zip(specs, args):
            if kind == 4 and (getattr(v, "device", None) != "hip" or v.dtype != expect):
                return NotImplemented
        self.calls.append((fast, args))


def test_eas_gpu_tensors_take_the_native_fast_launch(monkeypatch, tmp_path):
    """eas.Tensor arguments key the call memo by dtype and device; GPU ones are passed to the
    native fast launch as their own argument kind, host ones keep the full path (staging)."""
    from easy_as_amd.tensor import Tensor, _HipStorage

    monkeypatch.setenv("EAS_HIP_CACHE_DIR", str(tmp_path))
    ext = _FastMakingExt()
    rt = HipRuntime(ext=ext)
    monkeypatch.setattr(eas_kernel, "get_runtime", lambda *a, **k: rt)
    gpu = [Tensor(shape=(64,), dtype=np.float32, device="hip", hip=_HipStorage(("dev", i), 256)) for i in range(3)]
    k = eas.kernel(K.add_kernel.fn)
    k(*gpu, 64, BLOCK=64)
    assert len(ext.launches) == 1 and ext.launches[0][1][:3] == [("dev", 0), ("dev", 1), ("dev", 2)]
    assert len(ext.made) == 1
    _, specs, n_index, sync, _, _, eas_type = ext.made[0]
    assert specs == [(4, np.dtype(np.float32))] * 3 + [(1, int)] and n_index == 3 and sync and eas_type is Tensor
    k(*gpu, 1000, BLOCK=64)  # the memo hit goes through the fast launch
    assert len(ext.launches) == 1 and ext.calls[-1][1] == (*gpu, 1000)
    # host eas.Tensors: another memo key, staged on the full path, no fast launch
    host = [eas.tensor(np.ones(64, np.float32)) for _ in range(3)]
    k(*host, 64, BLOCK=64)
    k(*host, 64, BLOCK=64)
    assert len(k._memo) == 2 and len(ext.launches) == 3 and len(ext.made) == 1 and len(ext.calls) == 1
    # GPU tensors of another dtype: the fast launch declines them and the full path runs them
    f16 = [Tensor(shape=(64,), dtype=np.float16, device="hip", hip=_HipStorage(("dev", i), 128)) for i in range(3)]
    k(*f16, 64, BLOCK=64)
    assert len(ext.launches) == 4 and len(ext.calls) == 1 and len(k._memo) == 3
    # no fast launch is made for host eas.Tensors, nor for GPU ones of another dtype than the kernel's
    ck32 = k.compile(*gpu, 64, BLOCK=64)
    assert rt.fast_launcher(ck32, ("a", "b", "c", "N"), (*host, 64), True) is None
    assert rt.fast_launcher(ck32, ("a", "b", "c", "N"), (*f16, 64), True) is None
    assert rt.fast_launcher(ck32, ("a", "b", "c", "N"), (*gpu, 64), True) is not None


class _FillingExt(_RecordingExt):
    """Copies back a fixed byte pattern, so a test sees which host memory a result reaches."""

    def copy_to_host(self, buf, arr):
        super().copy_to_host(buf, arr)
        np.asarray(arr).view(np.uint8)[:] = 0x3F


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
def test_torch_host_tensors_are_staged_and_copied_back(monkeypatch, tmp_path, dtype):
    torch = pytest.importorskip("torch")
    monkeypatch.setenv("EAS_HIP_CACHE_DIR", str(tmp_path))
    ext = _FillingExt()
    rt = HipRuntime(ext=ext)
    monkeypatch.setattr(eas_kernel, "get_runtime", lambda *a, **k: rt)
    n = 1031
    dt = getattr(torch, dtype)
    a, b, c = torch.ones(n, dtype=dt), torch.ones(n, dtype=dt), torch.zeros(n, dtype=dt)
    kern = K.add_bf16_kernel if dtype == "bfloat16" else K.add_kernel
    kern(a, b, c, n, BLOCK=256)
    _, argv, writable, _, _ = ext.launches[0]
    # three distinct staged buffers, even though the host views are temporaries
    assert argv[:3] == [("buf", 1), ("buf", 2), ("buf", 3)] and writable[:3] == [False, False, True]
    assert ext.d2h == [(("buf", 3), n * c.element_size())]
    # the result lands in the torch tensor itself; the inputs are untouched
    assert bool((c.view(torch.uint8) == 0x3F).all()) and bool((a == 1).all())


def test_array_passed_twice_is_staged_once_and_copied_back(monkeypatch, tmp_path):
    monkeypatch.setenv("EAS_HIP_CACHE_DIR", str(tmp_path))
    ext = _RecordingExt()
    rt = HipRuntime(ext=ext)
    monkeypatch.setattr(eas_kernel, "get_runtime", lambda *a, **k: rt)
    n = 1031
    a, b = np.ones(n, np.float32), np.ones(n, np.float32)
    K.add_kernel(a, b, a, n, BLOCK=256)  # in place: a = a + b
    _, argv, writable, _, _ = ext.launches[0]
    assert argv[0] == argv[2] == ("buf", 1) and argv[1] == ("buf", 2)
    assert ext.d2h == [(("buf", 1), 4 * n)]


def test_benchmark_rejects_written_numpy_arrays(monkeypatch, tmp_path):
    """As the reference (eas/runtime/metal.py:455-462): timing with a written host array
    would time host copies, so benchmark() refuses it before launching anything."""
    monkeypatch.setenv("EAS_HIP_CACHE_DIR", str(tmp_path))
    ext = _RecordingExt()
    rt = HipRuntime(ext=ext)
    x = np.ones(1031, np.float32)
    ck = K.add_kernel.compile(x, x, x.copy(), 1031, BLOCK=256)
    args = {"a": x, "b": x, "c": np.zeros(1031, np.float32), "N": 1031}
    with pytest.raises(ValueError, match="numpy"):
        rt.benchmark(ck, args, {"BLOCK": 256}, repeat=3)
    assert ext.launches == []
    with pytest.raises(ValueError):
        rt.benchmark(ck, args, {"BLOCK": 256}, repeat=0)


def test_scalar_packing_errors(monkeypatch, tmp_path):
    monkeypatch.setenv("EAS_HIP_CACHE_DIR", str(tmp_path))
    rt = HipRuntime(ext=_RecordingExt())
    monkeypatch.setattr(eas_kernel, "get_runtime", lambda *a, **k: rt)
    x = np.zeros(8, np.float32)
    # the reference's struct.pack raises struct.error (metal.py:28-30); the error here is also an OverflowError
    with pytest.raises(struct.error) as info:
        K.add_kernel(x, x, x, 1 << 32, BLOCK=256)
    assert isinstance(info.value, OverflowError)
    with pytest.raises(ValueError, match="nthreads must be >= 0"):  # the grid rule comes first (grid.py:26-28)
        K.add_kernel(x, x, x, -1, BLOCK=256)
    with pytest.raises(OverflowError):  # an f32 beyond the f32 range, as struct.pack("<f") reports it
        K.axpy_kernel(x, x, x, 8, 1e39, BLOCK=256)
    with pytest.raises(TypeError):
        K.add_kernel(x.astype(np.float64), x, x, 8, BLOCK=256)


# ---- autotune ----------------------------------------------------------------------

class _TimingRuntime:
    """Benchmarks cost 1/BLOCK seconds; records what ran."""

    def __init__(self):
        self.benchmarked, self.ran = [], []

    def benchmark(self, ck, runtime_args, meta, *, repeat, warmup=0, **_):
        self.benchmarked.append(int(meta["BLOCK"]))
        return {64: 3.0, 128: 2.0, 256: 1.0, 1024: 1.5}[int(meta["BLOCK"])]

    def run(self, ck, runtime_args, meta, **_):
        self.ran.append(int(meta["BLOCK"]))


@eas.autotune(configs=[eas.Config(meta={"BLOCK": b}) for b in (64, 128, 256, 1024)], key=["N"], warmup=0, repeat=1)
@eas.kernel
def _tuned_add(a, b, c, N, BLOCK: eas.constexpr = 64):
    pid = mk.program_id(0)
    offs = pid * BLOCK + mk.arange(0, BLOCK)
    mask = offs < N
    mk.store(c, offs, mk.load(a, offs, mask) + mk.load(b, offs, mask), mask)


def test_autotune_benchmarks_once_per_key_and_keeps_fastest(monkeypatch):
    rt = _TimingRuntime()
    monkeypatch.setattr(eas_kernel, "get_runtime", lambda *a, **k: rt)
    x = np.zeros(2000, np.float32)
    _tuned_add(x, x, x, 1027)
    assert sorted(rt.benchmarked) == [64, 128, 256, 1024] and rt.ran == [256]
    _tuned_add(x, x, x, 1027)
    assert len(rt.benchmarked) == 4 and rt.ran == [256, 256]
    _tuned_add(x, x, x, 2000)  # a new key value is tuned again
    assert len(rt.benchmarked) == 8 and rt.ran[-1] == 256


# ---- argument binding ---------------------------------------------------------------

def test_fast_binding_matches_inspect():
    import inspect

    def fn(a, b, c, N, BLOCK: eas.constexpr = 256, scale=1.5):
        pass

    k = eas_kernel.Kernel(fn)
    assert k._plain
    x = np.zeros(4, np.float32)
    calls = [((x, x, x, 4), {}), ((x, x), {"c": x, "N": 7}), ((x, x, x, 4, 128), {"scale": 2.0}),
             ((), {"a": x, "b": x, "c": x, "N": 1, "BLOCK": 64})]
    for args, kw in calls:
        b = inspect.signature(fn).bind(*args, **kw)
        b.apply_defaults()
        want_meta = {n: v for n, v in b.arguments.items() if n == "BLOCK"}
        want_rt = {n: v for n, v in b.arguments.items() if n != "BLOCK"}
        meta, rt = k._bind_and_split(*args, **kw)
        assert meta == want_meta and list(rt) == list(want_rt) and all(rt[n] is want_rt[n] for n in rt)
    # binding errors are inspect's TypeErrors
    for args, kw in [((x, x, x, 4, 1, 2, 3), {}), ((x, x), {}), ((x, x, x, 4), {"a": x}), ((x, x, x, 4), {"M": 1})]:
        with pytest.raises(TypeError):
            k._bind_and_split(*args, **kw)

    def kwonly(a, *, N):
        pass

    assert not eas_kernel.Kernel(kwonly)._plain
    assert eas_kernel.Kernel(kwonly)._bind_and_split(x, N=3) == ({}, {"a": x, "N": 3})


# ---- code-object cache (reference: the pipeline cache, eas/runtime/metal.py:122-132) ----------

class _CountingCompiler:
    """compile_to_code that counts its calls; compiler_version and ABI_VERSION are settable."""

    def __init__(self, tag=("7", "2"), abi=3):
        self.calls, self.tag, self.ABI_VERSION = [], tag, abi

    def compile_to_code(self, src, name, options):
        self.calls.append((name, tuple(options)))
        return b"\x7fELF" + str(len(self.calls)).encode()

    def compiler_version(self):
        return (int(self.tag[0]), int(self.tag[1]), "/opt/rocm/lib/libhiprtc.so.7")


def test_code_object_cache_hits_and_misses(monkeypatch, tmp_path):
    from easy_as_amd.runtime.hip import COMPILE_OPTIONS, compile_code

    monkeypatch.setenv("EAS_HIP_CACHE_DIR", str(tmp_path))
    src = K.add_kernel.compile(np.zeros(1, np.float32), np.zeros(1, np.float32), np.zeros(1, np.float32), 8,
                               BLOCK=256).src
    cc = _CountingCompiler()
    first = compile_code(cc, src, "add_kernel")
    assert len(cc.calls) == 1 and len(list(tmp_path.glob("*.co"))) == 1
    assert compile_code(cc, src, "add_kernel") == first and len(cc.calls) == 1  # hit
    # each part of the key misses: options, entry, source, compiler version, ABI version
    compile_code(cc, src, "add_kernel", COMPILE_OPTIONS[:-1])
    compile_code(cc, src, "other_entry")
    compile_code(cc, src + "\n", "add_kernel")
    assert len(cc.calls) == 4
    for other in (_CountingCompiler(tag=("7", "3")), _CountingCompiler(abi=4)):
        compile_code(other, src, "add_kernel")
        assert len(other.calls) == 1  # a miss: compiled, not read back
    assert len(list(tmp_path.glob("*.co"))) == 6
    # and EAS_HIP_DISABLE_CACHE=1 recompiles
    monkeypatch.setenv("EAS_HIP_DISABLE_CACHE", "1")
    compile_code(cc, src, "add_kernel")
    assert len(cc.calls) == 5


def test_second_process_loads_the_cached_code_object(tmp_path):
    # a first process compiles with the real hiprtc; a second one, whose compiler would fail,
    # gets the identical code object from EAS_HIP_CACHE_DIR
    import os
    import subprocess
    import sys

    script = (
        "import sys, hashlib\n"
        "sys.path[:0] = ['.', 'tests']\n"
        "import numpy as np, kernels as K\n"
        "from easy_as_amd.runtime.hip import compile_code\n"
        "from easy_as_amd.runtime.hip_ext import load_hip_ext\n"
        "mod = load_hip_ext(require=True)\n"
        "z = np.zeros(1, np.float32)\n"
        "src = K.add_kernel.compile(z, z, z, 8, BLOCK=256).src\n"
        "if sys.argv[1] == 'second':\n"
        "    class NoCompiler:\n"
        "        ABI_VERSION = mod.ABI_VERSION\n"
        "        compiler_version = staticmethod(mod.compiler_version)\n"
        "        def compile_to_code(self, *a):\n"
        "            raise AssertionError('compiled again')\n"
        "    mod = NoCompiler()\n"
        "code = compile_code(mod, src, 'add_kernel')\n"
        "assert code[:4] == b'\\x7fELF'\n"
        "print(hashlib.sha256(code).hexdigest())\n"
    )
    env = {**os.environ, "EAS_HIP_CACHE_DIR": str(tmp_path), "PYTHONPATH": str(ROOT)}
    out = []
    for which in ("first", "second"):
        r = subprocess.run([sys.executable, "-c", script, which], cwd=ROOT, env=env, capture_output=True, text=True,
                           timeout=300)
        assert r.returncode == 0, r.stderr[-2000:]
        out.append(r.stdout.strip().splitlines()[-1])
    assert out[0] == out[1]
