"""``@eas.kernel``: argument binding, constexpr split, specialisation cache, launch.

Public behaviour follows the reference launcher (``eas/kernel.py:13-332``):

* parameters annotated ``eas.constexpr`` are meta params (trace-time literals);
* ``_sync``, ``_grid`` (int, tuple or ``callable(meta, runtime_args)``),
  ``_tptg``, ``_shape`` and ``_nthreads`` are per-call launch options;
* a specialisation is cached on ``(sorted meta, runtime-arg signature)``;
  scalar argument *values* never trigger a recompile;
* with an ``@eas.autotune`` spec every config is benchmarked once per key.
"""

from __future__ import annotations

import inspect
from typing import Any, Callable, Mapping

import numpy as np

from .autotune import AutotuneSpec, Config
from .compiler import CompiledKernel, _arg_key, _torch, compile as _compile
from .meta import constexpr
from .runtime import get_runtime
from .tensor import Tensor

_OPTION_NAMES = ("_sync", "_shape", "_grid", "_tptg", "_nthreads")
_MEMO_LIMIT = 64


def _light_key(v: Any) -> Any:
    """A call-memo key of one positional argument: its exact type, and for arrays and tensors
    their dtype (and whether a tensor is on the GPU).  Finer than the compile key of
    ``_arg_key``, so equal light keys imply the same specialisation.  Other types raise
    TypeError (the call then takes the full path)."""
    t = type(v)
    if t is int or t is float or t is bool:
        return t
    if t is np.ndarray:
        return (t, v.dtype)
    if t is Tensor:  # an eas.Tensor's dtype and device are fixed when it is made
        return (t, v.dtype, v.device)
    torch = _torch()
    if torch is not None and t is torch.Tensor:
        return (t, v.dtype, v.is_cuda)
    raise TypeError("no light key")


def _dims(value: Any, what: str, *, lo: int, max_dims: int, pad: bool) -> tuple[int, ...]:
    if isinstance(value, int):
        dims = [int(value)]
    elif isinstance(value, (tuple, list)):
        dims = [int(x) for x in value]
    else:
        kinds = "int/tuple/list or callable" if what == "_grid" else "int or tuple/list of ints"
        raise TypeError(f"{what} must be {kinds}, got {type(value)!r}")
    if not 1 <= len(dims) <= max_dims:
        raise ValueError(f"{what} must have 1..{max_dims} dims" if max_dims == 3 else f"{what} must have >= 1 dim")
    if any(d < lo for d in dims):
        raise ValueError(f"{what} dims must be {'> 0' if lo == 1 else '>= 0'}")
    if pad:
        dims += [1] * (3 - len(dims))
    return tuple(dims)


class Kernel:
    def __init__(self, fn: Callable[..., Any]):
        self.fn = fn
        self.name = fn.__name__
        self.sig = inspect.signature(fn)
        annotations = inspect.get_annotations(fn, eval_str=True)
        self.meta_params = {
            name for name, p in self.sig.parameters.items() if annotations.get(name, p.annotation) is constexpr
        }
        # plain signatures (every parameter positional-or-keyword) bind without inspect
        params = list(self.sig.parameters.values())
        self._plain = all(p.kind is inspect.Parameter.POSITIONAL_OR_KEYWORD for p in params)
        self._names = tuple(p.name for p in params)
        self._name_set = frozenset(self._names)
        self._defaults = {p.name: p.default for p in params if p.default is not inspect.Parameter.empty}
        self._cache: dict[tuple[Any, Any], CompiledKernel] = {}
        self._autotune_spec: AutotuneSpec | None = None
        self._tuned_cache: dict[tuple[Any, ...], Config] = {}
        # call memo for repeated launches: runtime parameters first and passed positionally,
        # keyword arguments only meta parameters and _sync (their values are part of the key)
        lead = 0
        while lead < len(params) and params[lead].name not in self.meta_params:
            lead += 1
        self._memo_ok = self._plain and lead == len(params) - len(self.meta_params)
        self._n_lead = lead
        self._memo_kw = frozenset(self.meta_params) | {"_sync"}
        self._memo: dict[Any, tuple[CompiledKernel, dict[str, Any], bool]] = {}
        # the runtime's one-native-call launch of a memoized specialisation, by keyword items
        self._fast: dict[Any, Callable[[tuple[Any, ...]], Any]] = {}

    def _set_autotune_spec(self, spec: AutotuneSpec) -> None:
        self._autotune_spec = spec

    # -- options ----------------------------------------------------------------
    @staticmethod
    def _extract_runtime_options(kwargs: dict[str, Any]) -> dict[str, Any]:
        """Pop the ``_``-prefixed launch options out of the call's kwargs."""
        sync = kwargs.pop("_sync", True)
        if not isinstance(sync, bool):
            raise TypeError(f"_sync must be bool, got {type(sync)!r}")
        nthreads = kwargs.pop("_nthreads", None)
        if nthreads is not None:
            try:
                nthreads = int(nthreads)
            except Exception as e:
                raise TypeError(f"_nthreads must be an int-like value, got {type(nthreads)!r}") from e
            if nthreads < 0:
                raise ValueError("_nthreads must be >= 0")
        return {
            "sync": sync,
            "nthreads": nthreads,
            "grid": kwargs.pop("_grid", None),
            "shape": kwargs.pop("_shape", None),
            "tptg": kwargs.pop("_tptg", None),
        }

    @staticmethod
    def _normalize_runtime_options(raw: dict[str, Any], meta: dict[str, Any], runtime_args: dict[str, Any]) -> dict[str, Any]:
        """Validate options and bring grid/tptg to 3-tuples (a callable grid is evaluated)."""
        shape = raw.get("shape")
        grid = raw.get("grid")
        if callable(grid):
            grid = grid(meta, runtime_args)
        tptg = raw.get("tptg")
        return {
            "sync": bool(raw["sync"]),
            "nthreads": raw["nthreads"],
            "grid": None if grid is None else _dims(grid, "_grid", lo=0, max_dims=3, pad=True),
            "shape": None if shape is None else _dims(shape, "_shape", lo=0, max_dims=1 << 30, pad=False),
            "tptg": None if tptg is None else _dims(tptg, "_tptg", lo=1, max_dims=3, pad=True),
        }

    @staticmethod
    def _check_tptg(ck: CompiledKernel, tptg: tuple[int, ...] | None) -> None:
        """``_tptg`` must equal the threadgroup shape the kernel was compiled for."""
        if tptg is None:
            return
        expected = (int(ck.block_size), 1, 1) if ck.launch_mode == "thread" else (1, 1, 1)
        if tuple(int(x) for x in tptg) != expected:
            raise ValueError(f"_tptg must match kernel launch mode: expected {expected}, got {tuple(tptg)}")

    # -- binding / specialisation --------------------------------------------------
    def _bind_and_split(self, /, *args: Any, **kwargs: Any) -> tuple[dict[str, Any], dict[str, Any]]:
        bound = self._bind_plain(args, kwargs) if self._plain else None
        if bound is None:  # not a plain signature, or a binding error that inspect reports
            b = self.sig.bind(*args, **kwargs)
            b.apply_defaults()
            bound = b.arguments
        meta = {k: v for k, v in bound.items() if k in self.meta_params}
        return meta, {k: v for k, v in bound.items() if k not in self.meta_params}

    def _bind_plain(self, args: tuple[Any, ...], kwargs: dict[str, Any]) -> dict[str, Any] | None:
        """``Signature.bind`` + ``apply_defaults`` for positional-or-keyword parameters, in
        parameter order; None when the call does not bind (inspect then raises its TypeError)."""
        names = self._names
        if len(args) > len(names) or any(k not in self._name_set for k in kwargs):
            return None
        given = dict(zip(names, args))
        for k, v in kwargs.items():
            if k in given:
                return None
            given[k] = v
        bound = {}
        for name in names:
            if name in given:
                bound[name] = given[name]
            elif name in self._defaults:
                bound[name] = self._defaults[name]
            else:
                return None
        return bound

    def _compile_from_split(self, meta: dict[str, Any], runtime_args: dict[str, Any]) -> CompiledKernel:
        # runtime_args come from the binding in parameter order, so the per-argument keys need no
        # sorting here (runtime_arg_signature sorts by name for callers with other orders)
        key = (tuple(sorted(meta.items())), tuple(map(_arg_key, runtime_args.values())))
        ck = self._cache.get(key)
        if ck is None:
            ck = _compile(self.fn, runtime_args, meta)
            self._cache[key] = ck
        return ck

    # -- autotune ------------------------------------------------------------------
    @staticmethod
    def _autotune_key(spec: AutotuneSpec, meta: Mapping[str, Any], runtime_args: Mapping[str, Any]) -> tuple[Any, ...]:
        def norm(v: Any) -> Any:
            if isinstance(v, (bool, int, float, str, type(None))):
                return v
            if isinstance(v, (tuple, list)):
                return tuple(norm(x) for x in v)
            if isinstance(v, dict):
                return tuple(sorted((str(k), norm(x)) for k, x in v.items()))
            for cast in (int, float):
                try:
                    return cast(v)
                except Exception:
                    pass
            shape = getattr(v, "shape", None)
            if shape is not None:
                try:
                    return ("shape", tuple(int(d) for d in shape))
                except Exception:
                    pass
            raise TypeError(f"autotune key value must be hashable/normalizable, got {type(v)!r}")

        key = []
        for name in spec.key:
            if name in meta:
                key.append(norm(meta[name]))
            elif name in runtime_args:
                key.append(norm(runtime_args[name]))
            else:
                raise KeyError(f"autotune key {name!r} not found in args/meta")
        return tuple(key)

    def _autotune_select(self, spec: AutotuneSpec, meta: dict[str, Any], runtime_args: dict[str, Any],
                         raw_opts: dict[str, Any]) -> tuple[dict[str, Any], dict[str, Any]]:
        key = self._autotune_key(spec, meta, runtime_args)
        best = self._tuned_cache.get(key)
        if best is None:
            bench = getattr(get_runtime(), "benchmark", None)
            if not callable(bench):
                raise RuntimeError("autotune requires a runtime with benchmark(); use the HIP runtime (EAS_BACKEND=auto|hip)")
            best_t: float | None = None
            for cfg in spec.configs:
                m = {**meta, **dict(cfg.meta)}
                opts = self._normalize_runtime_options(raw_opts, m, runtime_args)
                ck = self._compile_from_split(m, runtime_args)
                t = float(bench(ck, runtime_args, m, repeat=spec.repeat, warmup=spec.warmup,
                                nthreads=opts["nthreads"], grid=opts["grid"], tptg=opts["tptg"], shape=opts["shape"]))
                if best_t is None or t < best_t:
                    best_t, best = t, cfg
            assert best is not None
            self._tuned_cache[key] = best
        meta_best = {**meta, **dict(best.meta)}
        return meta_best, self._normalize_runtime_options(raw_opts, meta_best, runtime_args)

    # -- public ------------------------------------------------------------------
    def _prepare(self, args: tuple[Any, ...], kwargs: dict[str, Any]) -> tuple[CompiledKernel, dict, dict, dict, dict]:
        raw = self._extract_runtime_options(kwargs)
        meta, runtime_args = self._bind_and_split(*args, **kwargs)
        spec = self._autotune_spec
        if spec is not None:
            meta, opts = self._autotune_select(spec, meta, runtime_args, raw)
        else:
            opts = self._normalize_runtime_options(raw, meta, runtime_args)
        ck = self._compile_from_split(meta, runtime_args)
        if raw.get("tptg") is not None:
            self._check_tptg(ck, opts["tptg"])
        return ck, meta, runtime_args, opts, raw

    def compile(self, /, *args: Any, **kwargs: Any) -> CompiledKernel:
        return self._prepare(args, dict(kwargs))[0]

    def __call__(self, /, *args: Any, **kwargs: Any) -> None:
        key = None
        if self._memo_ok and len(args) == self._n_lead and self._autotune_spec is None:
            try:
                kw = tuple(kwargs.items())
                fast = self._fast.get(kw)
            except TypeError:  # a keyword value the memo does not key
                kw = fast = None
            if fast is not None and fast(args) is not NotImplemented:
                return
            try:
                key = (kw, tuple(map(_light_key, args)))
                hit = self._memo.get(key)
            except TypeError:  # an argument or keyword value the memo does not key
                key = hit = None
            if hit is not None:
                ck, meta, sync = hit
                get_runtime().run(ck, dict(zip(self._names, args)), meta, sync=sync)
                return
        ck, meta, runtime_args, opts, raw = self._prepare(args, dict(kwargs))
        rt = get_runtime()
        rt.run(ck, runtime_args, meta, **opts)
        if key is not None and kwargs.keys() <= self._memo_kw and all(
                raw[o] is None for o in ("nthreads", "grid", "shape", "tptg")):
            if len(self._memo) >= _MEMO_LIMIT:
                self._memo.clear()
            self._memo[key] = (ck, meta, opts["sync"])
            make = getattr(rt, "fast_launcher", None)
            if key[0] not in self._fast and callable(make):
                fast = make(ck, self._names[:self._n_lead], args, opts["sync"])
                if fast is not None:
                    if len(self._fast) >= _MEMO_LIMIT:
                        self._fast.clear()
                    self._fast[key[0]] = fast

    def to_hip(self, /, *args: Any, **kwargs: Any) -> str:
        """The generated gfx950 HIP C++ source for this specialisation (reference: ``to_msl``)."""
        return self.compile(*args, **kwargs).src


def kernel(fn: Callable[..., Any]) -> Kernel:
    k = Kernel(fn)
    spec = getattr(fn, "__eas_autotune_spec__", None)
    if isinstance(spec, AutotuneSpec):
        k._set_autotune_spec(spec)
    return k
