"""The C-ABI library loads and exports every entry point declared in include/*.h, and its
host-side argument checks behave (no kernel is launched here: the container has no GPU)."""
import ctypes
import os
import re

import pytest

from tests.conftest import REPO


def _declared():
    names = set()
    inc = os.path.join(REPO, "include")
    for f in os.listdir(inc):
        if f.endswith(".h"):
            txt = open(os.path.join(inc, f)).read()
            names |= set(re.findall(r"^[A-Za-z_][\w \*]*?\b(lsh_\w+)\s*\(", txt, re.M))
    return names


def test_header_declares_entry_points():
    names = _declared()
    assert "lsh_lif_scan_v3_fwd" in names and "lsh_lif_serial_fwd" in names


def test_library_exports_every_declared_symbol():
    from lifscan import _native
    L = _native.lib()
    for name in sorted(_declared()):
        assert hasattr(L, name), name
        assert name in _native.SIGNATURES, f"{name} has no ctypes signature"


def test_identity_and_status_strings():
    from lifscan import _native
    L = _native.lib()
    assert L.lsh_abi_version() == 4
    assert L.lsh_arch() == b"gfx950"
    for rc in (0, -1, -2, -3, -4, -5):
        assert len(L.lsh_status_string(rc)) > 0


def test_workspace_queries_and_shape_checks():
    from lifscan import _native
    L = _native.lib()
    assert L.lsh_lif_scan_v3_workspace(4096, 65536, 128, 8) > 0
    assert L.lsh_lif_scan_v3_workspace(4095, 65536, 128, 8) == 0  # T % C
    assert L.lsh_lif_scan_v3_workspace(4096, 65536, 128, 65) == 0  # K too large
    assert L.lsh_lif_scan_bwd_workspace(4096, 65536, 128) > 0
    lay = _native.V3Layout()
    assert L.lsh_lif_scan_v3_layout(4096, 1000, 64, 16, ctypes.byref(lay)) == 0
    assert lay.total == L.lsh_lif_scan_v3_workspace(4096, 1000, 64, 16)
    offs = [getattr(lay, f) for f, _ in _native.V3Layout._fields_ if f != "total"]
    assert all(o % 256 == 0 for o in offs) and offs == sorted(offs)
    assert L.lsh_lif_scan_v3_layout(100, 1000, 64, 16, ctypes.byref(lay)) == -3


def test_pieces_workspace_and_checks():
    """The converged scan in pieces: P pieces of the v3 layout of T/P steps, each 256-byte
    aligned; T % (C*P) != 0, P < 1 and P > 64 are refused (host-side checks, no GPU)."""
    from lifscan import _native
    L = _native.lib()
    T, N, C, K = 2 ** 20, 1024, 2048, 32
    for P in (1, 2, 4, 8):
        piece = L.lsh_lif_scan_v3_workspace(T // P, N, C, K)
        assert piece > 0
        assert L.lsh_lif_scan_v3_pieces_workspace(T, N, C, K, P) == P * ((piece + 255) // 256 * 256)
    assert L.lsh_lif_scan_v3_pieces_workspace(T, N, C, K, 3) == 0    # 512 chunks: 3 does not divide
    assert L.lsh_lif_scan_v3_pieces_workspace(T, N, C, K, 0) == 0
    assert L.lsh_lif_scan_v3_pieces_workspace(T, N, C, K, 65) == 0
    rc = L.lsh_lif_scan_v3_pieces_fwd(None, None, None, None, T, N, 0.9, 1.0, 0.0, C, K, 4, None, 0,
                                      None)
    assert rc == -1


def test_null_pointer_rejected_before_launch():
    from lifscan import _native
    L = _native.lib()
    rc = L.lsh_lif_serial_fwd(None, None, None, None, 16, 16, 0.9, 1.0, 0.0, None)
    assert rc == -1
    rc = L.lsh_lif_scan_v3_fwd(None, None, None, None, 16, 16, 0.9, 1.0, 0.0, 8, 4, 0, None, 0,
                               None)
    assert rc == -1


def test_affine_reset_host_checks():
    """Affine-reset entry points: workspace and layout queries, and arguments rejected before
    any launch (gamma outside [0, 1], null pointers)."""
    from lifscan import _native
    L = _native.lib()
    assert L.lsh_aff_scan_workspace(8192, 200, 128, 32) > 0
    assert L.lsh_aff_scan_workspace(8191, 200, 128, 32) == 0  # T % C
    assert L.lsh_aff_scan_workspace(8192, 200, 128, 33) == 0  # K > 32
    assert L.lsh_aff_scan_workspace(8192, 200, 128, 0) == 0
    lay = _native.AffLayout()
    assert L.lsh_aff_scan_layout(8192, 200, 128, 32, ctypes.byref(lay)) == 0
    assert lay.total == L.lsh_aff_scan_workspace(8192, 200, 128, 32)
    offs = [getattr(lay, f) for f, _ in _native.AffLayout._fields_ if f != "total"]
    assert all(o % 256 == 0 for o in offs) and offs == sorted(offs)
    # pieces: [M, N, K] float4
    assert lay.NP - lay.PIECES >= 64 * 200 * 32 * 16
    fake = ctypes.c_void_p(256)  # never dereferenced: the checks fail first
    assert L.lsh_aff_serial_fwd(fake, fake, fake, fake, 16, 16, 0.9, 1.0, 1.5, 0.0, None) == -1
    assert L.lsh_aff_serial_fwd(None, fake, fake, fake, 16, 16, 0.9, 1.0, 0.5, 0.0, None) == -1
    assert L.lsh_aff_scan_fwd(fake, fake, fake, fake, 16, 16, 0.9, 1.0, -0.1, 0.0, 0.0, 8, 8, 0,
                              fake, 1 << 20, None) == -1
    assert L.lsh_aff_bwd(fake, fake, fake, fake, fake, fake, fake, 16, 16, 0.9, 1.0, 2.0, 4.0, 0, 1,
                         None, 0, None) == -1
    assert L.lsh_reverse_affine_scan(None, fake, fake, 4, 4, None) == -1
