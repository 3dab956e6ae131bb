"""``HipRuntime``: runs compiled eas kernels on an MI355X through ``easy_as_amd._hip``.

Replaces the reference's ``MetalRuntime`` (``eas/runtime/metal.py``):

* ``run`` maps the reference launch (programs for SPMD kernels, threadgroups or
  a 1-D thread count for thread kernels; ``metal.py:244-352``) onto HIP
  workgroups using the kernel's :class:`~easy_as_amd.codegen.hip.Geometry`,
  packs the arguments (``metal.py:142-242``) and launches;
* code objects are compiled once per source with hiprtc for gfx950 and cached
  in memory and on disk;
* ``benchmark`` times ``repeat`` launches between HIP events (the reference
  wall-clocks one command buffer, ``metal.py:362-506``).
"""

from __future__ import annotations

import hashlib
import os
import struct
from collections import deque
from pathlib import Path
from typing import Any, Mapping

import numpy as np

from ..ir import DType, IRModule
from .grid import grid_ndim, infer_grid, infer_nthreads
from .hip_ext import load_hip_ext

TARGET_ARCH = "gfx950"

COMPILE_OPTIONS = (
    f"--offload-arch={TARGET_ARCH}",
    "-O3",
    "-std=c++17",
    "-ffp-contract=off",
    # packed FP32 (v_pk_*_f32) is disabled for all HIP code of this project
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
)


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


_NP_DTYPES = {DType.F16: np.float16, DType.F32: np.float32}


class ScalarRangeError(struct.error, OverflowError):
    """A u32 scalar outside [0, 2^32).  The reference's ``struct.pack("<I", ...)`` raises
    ``struct.error`` for it (``metal.py:28-30``); this is both that and an ``OverflowError``."""


def pack_scalar(dtype: DType, value: Any) -> bytes:
    """Kernel-argument bytes of a scalar (reference ``metal.py:28-38``)."""
    if dtype == DType.U32:
        v = int(value)
        if not 0 <= v < (1 << 32):
            raise ScalarRangeError(f"u32 scalar out of range: {v}")
        return struct.pack("<I", v)
    if dtype == DType.F16:
        return np.float16(value).tobytes()
    if dtype == DType.F32:
        return struct.pack("<f", float(value))
    if dtype == DType.BOOL:
        return struct.pack("<?", bool(value))
    raise ValueError(f"unsupported scalar dtype: {dtype}")


def _cache_dir() -> Path:
    d = os.environ.get("EAS_HIP_CACHE_DIR")
    return Path(d) if d else Path.home() / ".cache" / "easy_as_amd"


def _compiler_tag(mod: Any) -> str:
    get = getattr(mod, "compiler_version", None)
    if get is None:
        return "unknown"
    major, minor, path = get()
    return f"hiprtc-{major}.{minor}:{path}"


def compile_code(mod: Any, src: str, entry: str, options: tuple[str, ...] = COMPILE_OPTIONS) -> bytes:
    """hiprtc-compile ``src`` to a gfx950 code object, through the on-disk cache.

    The cache key covers the source, entry, options, the extension's ABI version
    and the hiprtc version/path, so a different compiler never reuses old code."""
    key = hashlib.sha256("\0".join((src, entry, *options, str(getattr(mod, "ABI_VERSION", 0)),
                                     _compiler_tag(mod))).encode()).hexdigest()
    path = _cache_dir() / f"{key}.co"
    if os.environ.get("EAS_HIP_DISABLE_CACHE", "") not in ("", "0") or not path.exists():
        code = mod.compile_to_code(src, f"{entry}.hip", list(options))
        try:
            path.parent.mkdir(parents=True, exist_ok=True)
            tmp = path.with_suffix(f".{os.getpid()}.tmp")
            tmp.write_bytes(code)
            os.replace(tmp, path)
        except OSError:
            pass
        return code
    return path.read_bytes()


class LaunchPlan:
    """A concrete HIP dispatch: workgroup grid, block, hidden u32 arguments and the
    entry point to launch (``None``: the kernel's own)."""

    __slots__ = ("grid", "block", "hidden", "entry")

    def __init__(self, grid: tuple[int, int, int], block: tuple[int, int, int], hidden: tuple[int, ...],
                 entry: str | None = None) -> None:
        self.grid = grid
        self.block = block
        self.hidden = hidden
        self.entry = entry


def plan_launch(
    ck: Any,
    runtime_args: Mapping[str, Any],
    *,
    nthreads: int | None = None,
    grid: tuple[int, int, int] | None = None,
    tptg: tuple[int, int, int] | None = None,
    shape: tuple[int, ...] | None = None,
    compute_units: int = 256,
) -> LaunchPlan | None:
    """Reference launch semantics -> HIP dispatch (``None`` when nothing runs).

    Reference rules (``metal.py:256-326``): ``_tptg`` must equal (BLOCK,1,1) in
    thread mode and (1,1,1) in SPMD; without ``_grid`` a 2-D/3-D grid is
    inferred from ``_shape``/H/W/D, else a 1-D extent from ``_nthreads``/N
    (thread mode: that many threads; SPMD: ceil(N/BLOCK) programs); any zero
    extent launches nothing.
    """
    ir: IRModule = ck.ir
    block = int(ck.block_size)
    mode = str(ck.launch_mode)
    expected = (block, 1, 1) if mode == "thread" else (1, 1, 1)
    if tptg is not None and tuple(int(x) for x in tptg) != expected:
        raise ValueError(f"tptg must match kernel launch mode: expected {expected}, got {tuple(tptg)}")
    live_x: int | None = None
    if grid is None:
        inferred = infer_grid(ir, runtime_args, block, shape=shape)
        if inferred is None:
            n = infer_nthreads(runtime_args, nthreads=nthreads)
            if n == 0:
                return None
            groups = (_cdiv(n, block), 1, 1)
            live_x = n if mode == "thread" else None
        else:
            groups = tuple(int(g) for g in inferred)  # type: ignore[assignment]
    else:
        groups = tuple(int(g) for g in grid)  # type: ignore[assignment]
        if any(g < 0 for g in groups):
            raise ValueError("grid dims must be >= 0")
    if any(g == 0 for g in groups):
        return None
    geo = ck.geometry
    if geo.kind == "spmd":
        nblocks = _cdiv(groups[0], geo.programs_per_wg * geo.unroll) * geo.split
        if nblocks * geo.wg_size >= 1 << 32:
            raise ValueError(f"spmd launch of {groups[0]} programs exceeds 2^32 threads along x")
        return LaunchPlan((nblocks, groups[1], groups[2]), (geo.wg_size, 1, 1), (groups[0],))
    if geo.kind == "thread":
        # one workgroup per threadgroup, or (a kernel emitted as lanes) the SPMD mapping of one
        # program per threadgroup; the hidden extent is the live thread count either way
        live = live_x if live_x is not None else groups[0] * block
        nblocks = _cdiv(groups[0], geo.programs_per_wg * geo.unroll) * geo.split
        return LaunchPlan((nblocks, groups[1], groups[2]), (geo.wg_size, 1, 1), (live,))
    if geo.kind == "gemm":
        from ..codegen.gemm_lift import plan_gemm

        return plan_gemm(geo, groups, runtime_args, live_x, compute_units)
    raise ValueError(f"unknown kernel geometry: {geo.kind!r}")


def _is_eas_tensor(v: Any) -> bool:
    return bool(getattr(v, "__eas_tensor__", False))


class HipRuntime:
    """Process-wide HIP runtime (one per process, like the reference's MetalRuntime)."""

    def __init__(self, ext: Any | None = None) -> None:
        self._hip = ext
        self._available: bool | None = None if ext is None else True
        self._kernels: dict[tuple[str, str], Any] = {}
        self._pending: deque[Any] = deque()
        self._max_in_flight: int | None = None
        self._torch: Any = None
        self._torch_probed = False
        self._raw_stream: Any = None
        self._arg_specs: dict[int, tuple[IRModule, frozenset[str], tuple[tuple[str, bool, DType, bool], ...]]] = {}
        self._arch_checked = ext is not None
        self._cus = 256
        self._plans: dict[tuple[Any, ...], tuple[Any, LaunchPlan | None, list[bytes]]] = {}

    # -- plumbing ------------------------------------------------------------
    def is_available(self) -> bool:
        if self._available is None:
            mod = load_hip_ext(require=False)
            try:
                self._available = bool(mod is not None and mod.is_available())
            except Exception:
                self._available = False
        return bool(self._available)

    def _mod(self) -> Any:
        if self._hip is None:
            self._hip = load_hip_ext(require=True)
        if not self._arch_checked:
            props = self._hip.device_props()
            if props["arch"] != TARGET_ARCH:
                raise RuntimeError(f"this backend targets {TARGET_ARCH} (MI355X); the current device is {props['arch']}")
            self._cus = int(props["compute_units"])
            self._arch_checked = True
        return self._hip

    def _torch_mod(self) -> Any:
        if not self._torch_probed:
            self._torch_probed = True
            try:
                import torch  # type: ignore

                self._torch = torch
                self._torch_dtypes = {DType.F32: torch.float32, DType.F16: torch.float16, DType.BF16: torch.bfloat16}
            except Exception:
                self._torch = None
        return self._torch

    def _max_pending(self) -> int:
        if self._max_in_flight is None:
            try:
                self._max_in_flight = max(0, int(os.environ.get("EAS_MAX_IN_FLIGHT", "256").strip() or 256))
            except ValueError:
                self._max_in_flight = 256
        return self._max_in_flight

    def kernel_handle(self, ck: Any, entry: str | None = None) -> Any:
        """Loaded kernel ``entry`` (default: the kernel's own) of ``ck``'s source, which is
        compiled once (disk-cached) for all of its entry points."""
        main = ck.geometry.entry if ck.geometry is not None else ck.ir.name
        entry = entry or main
        key = (ck.src, entry)
        k = self._kernels.get(key)
        if k is None:
            mod = self._mod()
            if callable(getattr(mod, "compile_to_code", None)) and callable(getattr(mod, "load", None)):
                # the source's eas-launch line gives the kernel its launch shape and argument size
                k = mod.load(compile_code(mod, ck.src, main), entry, src=ck.src)
            else:
                k = mod.compile(ck.src, entry)
            self._kernels[key] = k
        return k

    # -- arguments ---------------------------------------------------------------
    def build_argv(self, ir: IRModule, runtime_args: Mapping[str, Any], writes: frozenset[str]) -> tuple[list, list, list, Any]:
        """Argument list for ``_hip.launch`` plus host copy-backs and the stream to use."""
        mod = self._mod()
        torch = self._torch_mod()
        argv: list[Any] = []
        writable: list[bool] = []
        copy_back: list[tuple[Any, np.ndarray]] = []
        # host arrays staged into device buffers, by id: the same array passed twice is staged
        # once.  The arrays are held here because an id is only unique while its object lives
        # (the NumPy views made of torch host tensors below are temporaries).
        staged: dict[int, tuple[Any, np.ndarray]] = {}
        cuda_index = None
        tensor_t = torch.Tensor if torch is not None else ()
        for name, scalar, dtype, w in self._arg_spec(ir, writes):
            v = runtime_args[name]
            if scalar:
                argv.append(pack_scalar(dtype, v))
                writable.append(False)
                continue
            want = None
            if isinstance(v, tensor_t):
                if v.dtype != self._torch_dtypes[dtype]:
                    raise TypeError(f"{name!r} must be {dtype.value}, got {v.dtype}")
                if v.is_cuda:
                    if not v.is_contiguous():
                        raise ValueError(f"{name!r} must be contiguous")
                    # a non-owning view of the tensor's memory that keeps the tensor alive
                    argv.append(mod.wrap_pointer(v.data_ptr(), v.nbytes, v))
                    writable.append(w)
                    cuda_index = v.get_device()
                    continue
                if v.device.type != "cpu":
                    raise TypeError(f"unsupported torch device for {name!r}: {v.device}")
                if dtype == DType.BF16:
                    # NumPy has no bfloat16: stage the raw 16-bit patterns (same memory)
                    v = v.detach().contiguous().view(torch.int16).numpy()
                    want = np.int16
                else:
                    v = v.detach().contiguous().numpy()
            if want is None:
                want = _NP_DTYPES.get(dtype)
            if _is_eas_tensor(v):
                if v.device == "hip":
                    if np.dtype(v.dtype) != np.dtype(want):
                        raise TypeError(f"{name!r} dtype mismatch: expected {np.dtype(want)}, got {v.dtype}")
                    argv.append(v._hip_buffer())
                    writable.append(w)
                    continue
                v = v.numpy()
            if isinstance(v, np.ndarray):
                if v.dtype != want:
                    raise TypeError(f"{name!r} must be {np.dtype(want).name}, got {v.dtype}")
                if not v.flags.c_contiguous:
                    raise ValueError(f"{name!r} must be C-contiguous")
                hit = staged.get(id(v))
                if hit is None:
                    buf = mod.alloc_buffer(max(int(v.nbytes), 1), "private")
                    if v.nbytes:
                        mod.copy_from_host(buf, v)
                    staged[id(v)] = (buf, v)
                else:
                    buf = hit[0]
                # an array passed twice is copied back once if either use writes it
                if w and v.nbytes and not any(b is buf for b, _ in copy_back):
                    copy_back.append((buf, v))
                argv.append(buf)
                writable.append(w)
                continue
            raise TypeError(f"expected numpy.ndarray, eas.Tensor or torch.Tensor for {name!r}, got {type(v)!r}")
        # launches with torch GPU tensors go on torch's current stream, ordered with torch's own work
        stream = None if cuda_index is None else self._current_stream(cuda_index)
        return argv, writable, copy_back, stream

    def _arg_spec(self, ir: IRModule, writes: frozenset[str]) -> tuple[tuple[str, bool, DType, bool], ...]:
        """Per-argument (name, is scalar, dtype, written) of a kernel, built once per IR."""
        hit = self._arg_specs.get(id(ir))
        if hit is not None and hit[0] is ir and hit[1] == writes:
            return hit[2]
        spec = tuple((a.name, a.kind == "scalar", a.dtype, a.name in writes) for a in ir.args)
        self._arg_specs[id(ir)] = (ir, writes, spec)  # holding ir keeps its id unique
        return spec

    def _stream_getter(self) -> Any:
        """device index -> torch's current stream on it, as a raw hipStream_t address."""
        raw = self._raw_stream
        if raw is None:
            torch = self._torch_mod()
            raw = getattr(torch._C, "_cuda_getCurrentRawStream", None) or (
                lambda i: torch.cuda.current_stream(i).cuda_stream)
            self._raw_stream = raw
        return raw

    def _current_stream(self, device_index: int) -> int:
        """torch's current stream on a device, as a raw hipStream_t address."""
        return int(self._stream_getter()(device_index))

    def fast_launcher(self, ck: Any, names: tuple[str, ...], args: tuple[Any, ...], sync: bool) -> Any:
        """A one-native-call launch of ``ck`` for later calls shaped like ``args`` (the call memo's
        hit path), or None when this specialisation does not take one.  It takes SPMD and
        thread-mode kernels sized by their u32 argument ``N`` (1-D launches) whose arguments are
        torch GPU tensors, eas.Tensors on the GPU and int, float or bool scalars, passed
        positionally in the kernel's argument order.  The returned callable launches what ``run(ck, ...)`` would launch for
        ``args`` (same dispatch, kernel arguments, stream and completion batching, and the
        EAS_MAX_IN_FLIGHT bound) and returns None, or returns NotImplemented without launching
        when an argument does not match (another type, dtype or device kind, a non-contiguous
        tensor, a scalar out of range): the caller then takes the full path."""
        from ..tensor import Tensor as EasTensor

        torch = self._torch_mod()
        geo = ck.geometry
        if geo is None or geo.kind not in ("spmd", "thread") or grid_ndim(ck.ir) > 1:
            return None
        mod = self._mod()
        if not callable(getattr(mod, "fast_make", None)) or tuple(a.name for a in ck.ir.args) != tuple(names):
            return None
        scalar_kinds = {DType.U32: (1, int), DType.F32: (2, float), DType.BOOL: (3, bool)}
        specs, n_index = [], None
        for i, (a, v) in enumerate(zip(ck.ir.args, args)):
            if a.kind == "buffer":
                if type(v) is EasTensor:
                    want = _NP_DTYPES.get(a.dtype)
                    if v.device != "hip" or want is None or v.dtype != np.dtype(want):
                        return None
                    specs.append((4, v.dtype))
                    continue
                if torch is None or type(v) is not torch.Tensor or not v.is_cuda \
                        or v.dtype != self._torch_dtypes.get(a.dtype):
                    return None
                specs.append((0, v.dtype))
                continue
            kind = scalar_kinds.get(a.dtype)
            if kind is None or type(v) is not kind[1]:
                return None
            specs.append(kind)
            if a.name == "N" and kind[0] == 1:
                n_index = i
        if n_index is None:
            return None
        limit = self._max_pending()
        # without torch every buffer is an eas.Tensor, and the launch goes on the default stream
        tensor_type, streams = (torch.Tensor, self._stream_getter()) if torch is not None else (type(None), id)
        fast = mod.fast_make(self.kernel_handle(ck), specs, n_index, bool(sync), min(16, limit) if limit else 16,
                             tensor_type, streams, EasTensor)
        call, pending, synchronize = mod.fast_call, self._pending, mod.synchronize

        def launch(call_args: tuple[Any, ...]) -> Any:
            p = call(fast, call_args)
            if p is None or p is NotImplemented:
                return p
            pending.append(p)
            while limit and len(pending) > limit:
                synchronize(pending.popleft())
            return None

        return launch

    # -- launching ------------------------------------------------------------------
    def run(
        self,
        ck: Any,
        runtime_args: Mapping[str, Any],
        meta: Mapping[str, Any],
        *,
        sync: bool = True,
        nthreads: int | None = None,
        grid: tuple[int, int, int] | None = None,
        tptg: tuple[int, int, int] | None = None,
        shape: tuple[int, ...] | None = None,
    ) -> None:
        _ = meta
        mod = self._mod()
        plan, hidden = self._plan(ck, runtime_args, nthreads, grid, tptg, shape)
        if plan is None:
            return
        argv, writable, copy_back, stream = self.build_argv(ck.ir, runtime_args, ck.writes)
        argv += hidden
        writable += [False] * len(hidden)
        kernel = self.kernel_handle(ck, plan.entry)
        if sync or copy_back:
            mod.launch_groups(kernel, argv, writable, plan.grid, plan.block, stream=stream)
            for buf, arr in copy_back:
                mod.copy_to_host(buf, arr)
            return
        limit = self._max_pending()
        # launches share a completion event per batch; with a bound, a batch holds at most `limit`
        # launches, so waiting on the oldest pending launch leaves the later batches in flight
        batch = min(16, limit) if limit else 16
        self._pending.append(mod.launch_groups_async(kernel, argv, writable, plan.grid, plan.block, stream=stream,
                                                     batch=batch))
        while limit and len(self._pending) > limit:
            mod.synchronize(self._pending.popleft())

    def _plan(self, ck: Any, runtime_args: Mapping[str, Any], nthreads: int | None, grid: Any, tptg: Any,
              shape: Any) -> tuple[LaunchPlan | None, list[bytes]]:
        """The launch plan and its packed hidden arguments.  An SPMD or thread-mode plan
        depends only on the kernel, the launch options and the scalars that size the grid
        (``N``, ``H``, ``W``, ``D``), so it is cached on those; a lifted GEMM's plan also
        checks its buffers' sizes and addresses and is made afresh each time."""
        geo = ck.geometry
        key = None
        if geo is not None and geo.kind != "gemm":
            key = (id(ck), nthreads, grid, tptg, shape, runtime_args.get("N"), runtime_args.get("H"),
                   runtime_args.get("W"), runtime_args.get("D"))
            try:
                hit = self._plans.get(key)
            except TypeError:  # an unhashable value: plan without the cache
                key, hit = None, None
            if hit is not None and hit[0] is ck:
                return hit[1], hit[2]
        plan = plan_launch(ck, runtime_args, nthreads=nthreads, grid=grid, tptg=tptg, shape=shape,
                           compute_units=self._cus)
        hidden = [] if plan is None else [struct.pack("<I", h) for h in plan.hidden]
        if key is not None:
            if len(self._plans) >= 4096:
                self._plans.clear()
            self._plans[key] = (ck, plan, hidden)  # holding ck keeps its id unique
        return plan, hidden

    def synchronize(self) -> None:
        mod = self._hip
        while self._pending:
            mod.synchronize(self._pending.popleft())

    def benchmark(
        self,
        ck: Any,
        runtime_args: Mapping[str, Any],
        meta: Mapping[str, Any],
        *,
        repeat: int,
        warmup: int = 0,
        nthreads: int | None = None,
        grid: tuple[int, int, int] | None = None,
        tptg: tuple[int, int, int] | None = None,
        shape: tuple[int, ...] | None = None,
        **_: Any,
    ) -> float:
        """Seconds per launch: ``warmup`` untimed launches, then ``repeat`` launches
        between HIP events on the launch stream."""
        _ = meta
        if repeat <= 0:
            raise ValueError("repeat must be > 0")
        if warmup < 0:
            raise ValueError("warmup must be >= 0")
        self.synchronize()
        self._mod()
        plan = plan_launch(ck, runtime_args, nthreads=nthreads, grid=grid, tptg=tptg, shape=shape,
                           compute_units=self._cus)
        if plan is None:
            return 0.0
        argv, writable, copy_back, stream = self.build_argv(ck.ir, runtime_args, ck.writes)
        if copy_back:
            raise ValueError("benchmark() with numpy outputs is not supported; use eas.Tensor(device='hip') or "
                             "torch GPU tensors for device-resident timing")
        argv += [struct.pack("<I", h) for h in plan.hidden]
        writable += [False] * len(plan.hidden)
        ms = self._mod().launch_timed(self.kernel_handle(ck, plan.entry), argv, writable, plan.grid, plan.block,
                                      repeat=int(repeat), warmup=int(warmup), stream=stream)
        return float(ms) * 1e-3
