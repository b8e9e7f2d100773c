"""Compatibility module name: the reference's callers import the ALIF kernels as
``from lifscan import triton_alif as A``; this re-exports the HIP implementation.  No Triton."""
from .hip_alif import *  # noqa: F401,F403
from .hip_alif import _rho_pow_c, last_alif_run  # noqa: F401
from . import hip_lif as L  # noqa: F401  (the reference module exposes triton_lif as L)
