"""Code generation: eas IR -> gfx950 HIP C++."""

from .hip import Geometry, Lowered, ir_to_hip

__all__ = ["Geometry", "Lowered", "ir_to_hip"]
