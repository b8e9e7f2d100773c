"""Compatibility module name: the reference's callers import the soft-reset kernels as
``from lifscan import triton_soft as S`` (or ``TS``); this re-exports the HIP implementation.
No Triton."""
from .hip_soft import *  # noqa: F401,F403
from .hip_soft import _soft_backward  # noqa: F401
from . import hip_lif as L  # noqa: F401  (the reference module exposes triton_lif as L)
