"""``eas``: the import name user kernels use (``import eas``; ``from eas import mk``).

It is the ``easy_as_amd`` package under its reference name: this module
replaces itself in ``sys.modules`` with ``easy_as_amd`` and registers every
submodule under the ``eas.`` prefix as the *same* module object, so
``eas.kernel``, ``eas.runtime.grid``, ``eas.compiler`` ... are the backend's
own modules (patching one patches the other).
"""

from __future__ import annotations

import importlib
import importlib.abc
import importlib.util
import sys

import easy_as_amd as _impl

_PREFIX = "eas."
_TARGET = "easy_as_amd."


class _AliasLoader(importlib.abc.Loader):
    def __init__(self, target: str) -> None:
        self.target = target

    def create_module(self, spec):  # type: ignore[override]
        return importlib.import_module(self.target)

    def exec_module(self, module) -> None:  # type: ignore[override]
        pass


class _AliasFinder(importlib.abc.MetaPathFinder):
    def find_spec(self, fullname, path=None, target=None):  # type: ignore[override]
        if not fullname.startswith(_PREFIX):
            return None
        real = _TARGET + fullname[len(_PREFIX):]
        if importlib.util.find_spec(real) is None:
            return None
        return importlib.util.spec_from_loader(fullname, _AliasLoader(real), is_package=hasattr(importlib.import_module(real), "__path__"))


if not any(isinstance(f, _AliasFinder) for f in sys.meta_path):
    sys.meta_path.insert(0, _AliasFinder())

for _name, _mod in list(sys.modules.items()):
    if _name.startswith(_TARGET):
        sys.modules.setdefault(_PREFIX + _name[len(_TARGET):], _mod)

sys.modules[__name__] = _impl
