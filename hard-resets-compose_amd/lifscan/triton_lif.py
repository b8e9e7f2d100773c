"""Compatibility module name.  The reference's callers import the LIF kernels as
``from . import triton_lif as L`` (shdnet.py, fit.py) or ``from lifscan import triton_lif``;
this module re-exports the HIP implementation under that name.  Nothing here uses Triton."""
from .hip_lif import *  # noqa: F401,F403
from .hip_lif import _pick_C, last_scan_run, last_fused_counters  # noqa: F401
