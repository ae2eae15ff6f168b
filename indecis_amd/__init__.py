"""indecis_amd — MI355X (gfx950) int8 ModernBERT encoder forward pass of
indecis, behind a C ABI (include/indecis_hip.h). The Python modules mirror
the reference's internal/modernbert and linalg interfaces over that ABI.
"""
from . import _lib  # noqa: F401
from .modernbert import BASE, SMALL, Config, Model, Weights  # noqa: F401
