"""``@eas.autotune``: benchmark candidate meta configs per key and keep the best.

Semantics follow ``eas/autotune.py:9-57`` and ``eas/kernel.py:31-127`` of the
reference: the spec is attached to the kernel; on a call the key values are
normalised, each config is compiled and timed once with
``runtime.benchmark``, and the fastest config is cached for that key.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Callable, Mapping, Sequence


@dataclass(frozen=True, slots=True)
class Config:
    meta: Mapping[str, Any]


@dataclass(frozen=True, slots=True)
class AutotuneSpec:
    configs: tuple[Config, ...]
    key: tuple[str, ...]
    warmup: int
    repeat: int


def autotune(
    *,
    configs: Sequence[Config],
    key: Sequence[str],
    warmup: int = 5,
    repeat: int = 25,
) -> Callable[[Any], Any]:
    if not configs:
        raise ValueError("autotune(configs=...) must be non-empty")
    if not key:
        raise ValueError("autotune(key=...) must be non-empty")
    if warmup < 0:
        raise ValueError("autotune(warmup=...) must be >= 0")
    if repeat <= 0:
        raise ValueError("autotune(repeat=...) must be > 0")
    spec = AutotuneSpec(tuple(configs), tuple(str(k) for k in key), int(warmup), int(repeat))

    def decorate(obj: Any) -> Any:
        setter = getattr(obj, "_set_autotune_spec", None)
        if callable(setter):
            setter(spec)
        elif callable(obj):
            # Applied below @eas.kernel: the Kernel picks the spec up when it wraps fn.
            obj.__eas_autotune_spec__ = spec
        else:
            raise TypeError(f"@eas.autotune expects a callable or Kernel, got {type(obj)!r}")
        return obj

    return decorate
