"""easy_as_amd — the MI355X (gfx950) backend of the eas kernel DSL.

The public surface is the reference's (``eas/__init__.py:5-30``): write kernels
with ``@eas.kernel`` and the ``mk`` DSL; they trace to eas IR, lower to gfx950
HIP C++ and run through the C-ABI runtime in ``easy_as_amd._hip`` /
``libeas_hip.so``.  ``import eas`` resolves to this package.
"""

from __future__ import annotations

from . import mk  # noqa: F401
from .autotune import Config, autotune
from .dlpack import from_dlpack, to_dlpack
from .kernel import Kernel, kernel
from .meta import constexpr
from .tensor import Tensor, empty, empty_like, tensor
from .torch import from_torch, to_torch

__all__ = [
    "Config",
    "Kernel",
    "Tensor",
    "autotune",
    "constexpr",
    "from_dlpack",
    "empty",
    "empty_like",
    "from_torch",
    "kernel",
    "mk",
    "tensor",
    "to_dlpack",
    "to_torch",
]
