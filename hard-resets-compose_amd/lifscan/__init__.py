"""lifscan — MI355X-native (gfx950) exact hard-reset LIF / ALIF scans.

Drop-in for the reference package of the same name: ``from lifscan import triton_lif as L``
and ``from lifscan import triton_alif as A`` resolve to the HIP implementation
(``hip_lif`` / ``hip_alif``), which runs hand-written HIP kernels through the C ABI of
``liblifscan_hip.so`` (see include/lifscan_hip.h).  Put the directory that contains this
package on ``sys.path``.
"""
