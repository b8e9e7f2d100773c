"""Compatibility module name: the reference's callers import the affine-reset kernels as
``from lifscan import triton_affine as A``; this re-exports the HIP implementation.  No Triton."""
from .hip_affine import *  # noqa: F401,F403
from .hip_affine import _aff_backward, last_aff_run  # noqa: F401
from . import hip_lif as L  # noqa: F401  (the reference module exposes triton_lif as L)
