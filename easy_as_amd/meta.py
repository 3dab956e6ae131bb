"""Compile-time meta parameter marker (reference: ``eas/meta.py:5-10``)."""

from __future__ import annotations


class constexpr:
    """Annotation for kernel parameters that are compile-time constants.

    A parameter annotated ``eas.constexpr`` is bound as a Python literal while
    the kernel is traced (it specialises the generated code and is part of the
    compile-cache key); it is never passed to the GPU as a kernel argument.
    """
