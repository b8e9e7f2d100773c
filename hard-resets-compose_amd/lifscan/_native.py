"""ctypes binding of liblifscan_hip.so (the C ABI declared in include/lifscan_hip.h).

torch is imported first so that the HIP runtime it loads (SONAME libamdhip64.so.7) is the
one the library binds to: streams and device pointers handed over by torch are then valid
in the library.  There is no fallback: if the library is missing, every call raises.
"""
import contextlib
import ctypes
import os

import torch

from . import _build

_LIB = None

# LSH_ABI_VERSION of include/lifscan_hip.h that these signatures bind
ABI_VERSION = 4

LSH_OK = 0
LSH_ERR_ARG = -1
LSH_ERR_SHAPE = -2
LSH_ERR_DIVISIBILITY = -3
LSH_ERR_WORKSPACE = -4
LSH_ERR_HIP = -5
LSH_ERR_SCRATCH = -6

c_p = ctypes.c_void_p
c_i64 = ctypes.c_int64
c_f = ctypes.c_float
c_i = ctypes.c_int
c_sz = ctypes.c_size_t


class ScanStats(ctypes.Structure):
    _fields_ = [
        ("repair_iters", ctypes.c_int64),
        ("overflow_frac", ctypes.c_double),
        ("mean_pieces", ctypes.c_double),
        ("max_pieces", ctypes.c_int64),
        ("super_overflow_frac", ctypes.c_double),
        ("super_mean_pieces", ctypes.c_double),
        ("super_max_pieces", ctypes.c_int64),
        ("miss_frac", ctypes.c_double),
        ("mean_lines", ctypes.c_double),
        ("fused_fixups", ctypes.c_int64),
        ("fused_unknown", ctypes.c_int64),
        ("spin_timeouts", ctypes.c_int64),
    ]


class V3Layout(ctypes.Structure):
    _fields_ = [(n, ctypes.c_size_t) for n in (
        "EC", "EA", "EB", "MA", "MB", "CNT", "OVFRAW", "MX", "MC", "LO", "MN", "OVF", "STARTS",
        "ENDS", "LIST0", "LIST1", "total")]


class V4Layout(ctypes.Structure):
    _fields_ = [("v3", V3Layout)] + [(n, ctypes.c_size_t) for n in (
        "SA", "SB", "SN", "SOVF", "SX", "SC", "SSTARTS", "XT", "CT", "total")]


class AffLayout(ctypes.Structure):
    _fields_ = [(n, ctypes.c_size_t) for n in (
        "EC", "EA", "EB", "HC", "HA", "HB", "LO", "HI", "PIECES", "NP", "OVF", "STARTS", "ENDS",
        "LIST0", "LIST1", "total")]


class ALIFLayout(ctypes.Structure):
    _fields_ = [(n, ctypes.c_size_t) for n in (
        "EC", "EA", "EB", "LU", "HU", "LW", "HW", "MA", "MB", "NL", "NP", "OVF", "LS", "LC", "LX",
        "POWN", "PXL", "PXR", "PU", "PA", "POF", "SU", "SW", "EU", "EW", "MISS", "MSTAR", "LIST0",
        "LIST1", "total")]


# name -> (restype, argtypes); mirrors include/lifscan_hip.h
SIGNATURES = {
    "lsh_abi_version": (c_i, []),
    "lsh_arch": (ctypes.c_char_p, []),
    "lsh_status_string": (ctypes.c_char_p, [c_i]),
    "lsh_lif_serial_fwd": (c_i, [c_p, c_p, c_p, c_p, c_i64, c_i64, c_f, c_f, c_f, c_p]),
    "lsh_lif_serial_bwd": (c_i, [c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_i64, c_i64, c_f, c_f, c_f,
                                 c_f, c_i, c_p]),
    "lsh_lif_scan_v3_workspace": (c_sz, [c_i64, c_i64, c_i, c_i]),
    "lsh_lif_scan_v3_fwd": (c_i, [c_p, c_p, c_p, c_p, c_i64, c_i64, c_f, c_f, c_f, c_i, c_i, c_i64,
                                  c_p, c_sz, c_p]),
    "lsh_lif_scan_v3_pieces_workspace": (c_sz, [c_i64, c_i64, c_i, c_i, c_i]),
    "lsh_lif_scan_v3_pieces_fwd": (c_i, [c_p, c_p, c_p, c_p, c_i64, c_i64, c_f, c_f, c_f, c_i, c_i,
                                         c_i, c_p, c_sz, c_p]),
    "lsh_lif_scan_v3_assoc_workspace": (c_sz, [c_i64, c_i64, c_i, c_i]),
    "lsh_lif_scan_v3_assoc_fwd": (c_i, [c_p, c_p, c_p, c_p, c_i64, c_i64, c_f, c_f, c_f, c_i, c_i,
                                        c_i64, c_p, c_sz, c_p]),
    "lsh_lif_scan_warm_workspace": (c_sz, [c_i64, c_i64, c_i]),
    "lsh_lif_scan_warm_fwd": (c_i, [c_p, c_p, c_p, c_p, c_i64, c_i64, c_f, c_f, c_f, c_i, c_i, c_p,
                                    c_sz, c_p]),
    "lsh_lif_scan_lo_fwd": (c_i, [c_p, c_p, c_p, c_p, c_p, c_i64, c_i64, c_f, c_f, c_f, c_i, c_i,
                                  c_i64, c_p, c_sz, c_p]),
    "lsh_scan_stats_read": (c_i, [c_p, c_i64, c_i64, c_i, ctypes.POINTER(ScanStats), c_p]),
    "lsh_lif_scan_v3_layout": (c_i, [c_i64, c_i64, c_i, c_i, ctypes.POINTER(V3Layout)]),
    "lsh_lif_scan_exact_workspace": (c_sz, []),
    "lsh_lif_scan_exact_fwd": (c_i, [c_p, c_p, c_p, c_p, c_i64, c_i64, c_f, c_f, c_f, c_i, c_i, c_p,
                                     c_sz, c_p]),
    "lsh_lif_chunked_serial_fwd": (c_i, [c_p, c_p, c_p, c_p, c_i64, c_i64, c_f, c_f, c_f, c_i, c_p,
                                         c_sz, c_p]),
    "lsh_lif_scan_fused_bwd": (c_i, [c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_i64, c_i64, c_f, c_f, c_f,
                                     c_f, c_i, c_i, c_p]),
    "lsh_lif_scan_exact_fwd_starts": (c_i, [c_p, c_p, c_p, c_p, c_i64, c_i64, c_f, c_f, c_f, c_i, c_p,
                                            c_sz, c_p]),
    "lsh_lif_scan_fused_bwd_starts": (c_i, [c_p, c_p, c_p, c_p, c_p, c_i64, c_i64, c_f, c_f, c_f, c_f,
                                            c_i, c_p]),
    "lsh_lif_scan_v4_workspace": (c_sz, [c_i64, c_i64, c_i, c_i, c_i, c_i]),
    "lsh_lif_scan_v4_layout": (c_i, [c_i64, c_i64, c_i, c_i, c_i, c_i, ctypes.POINTER(V4Layout)]),
    "lsh_lif_scan_v4_fwd": (c_i, [c_p, c_p, c_p, c_p, c_i64, c_i64, c_f, c_f, c_f, c_i, c_i, c_i, c_i,
                                  c_i, c_i64, c_p, c_sz, c_p]),
    "lsh_alif_serial_fwd": (c_i, [c_p, c_p, c_p, c_p, c_p, c_p, c_i64, c_i64, c_f, c_f, c_f, c_f, c_f,
                                  c_p]),
    "lsh_alif_serial_fwd_dparams": (c_i, [c_p, c_p, c_p, c_p, c_p, c_p, c_i64, c_i64, c_p, c_f, c_p]),
    "lsh_alif_warm_predict": (c_i, [c_p, c_p, c_p, c_p, c_p, c_p, c_i64, c_i64, c_i, c_i, c_f, c_f,
                                    c_f, c_f, c_f, c_f, c_f, c_p]),
    "lsh_alif_scan_workspace": (c_sz, [c_i64, c_i64, c_i, c_i, c_i]),
    "lsh_alif_scan_layout": (c_i, [c_i64, c_i64, c_i, c_i, c_i, ctypes.POINTER(ALIFLayout)]),
    "lsh_alif_scan_fwd": (c_i, [c_p, c_p, c_p, c_p, c_f, c_p, c_p, c_p, c_i64, c_i64, c_f, c_f, c_f,
                                c_f, c_f, c_f, c_i, c_i, c_i, c_i, c_i64, c_p, c_sz,
                                ctypes.POINTER(c_p), c_p]),
    "lsh_alif_bwd_workspace": (c_sz, [c_i64, c_i64, c_i]),
    "lsh_alif_bwd_partials": (c_i64, [c_i64, c_i64, c_i, c_i]),
    "lsh_alif_bwd_lookback_workspace": (c_sz, [c_i64, c_i64]),
    "lsh_lif_param_partials": (c_i64, [c_i64, c_i64, c_i, c_i]),
    "lsh_lif_scan_lookback_bwd_workspace": (c_sz, [c_i64, c_i64]),
    "lsh_lif_scan_lookback_bwd": (c_i, [c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_i64, c_i64, c_f, c_f, c_f,
                                        c_f, c_i, c_i, c_p, c_sz, c_p]),
    "lsh_lif_scan_lookback_bwd_noalloc": (c_i, [c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_i64, c_i64, c_f,
                                                c_f, c_f, c_f, c_i, c_i, c_p]),
    "lsh_lif_param_bwd": (c_i, [c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_i64, c_i64, c_f, c_f, c_f, c_f,
                                c_i, c_i, c_p, c_sz, c_p]),
    "lsh_alif_bwd": (c_i, [c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_i64, c_i64, c_f,
                           c_f, c_f, c_f, c_f, c_i, c_i, c_p, c_sz, c_p]),
    "lsh_alif_bwd_dparams": (c_i, [c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_i64,
                                   c_i64, c_p, c_f, c_i, c_i, c_p, c_sz, c_p]),
    "lsh_alif_bwd_recompute": (c_i, [c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_i64, c_i64,
                                     c_p, c_f, c_f, c_f, c_f, c_f, c_f, c_i, c_i, c_p, c_sz, c_p]),
    "lsh_aff_serial_fwd": (c_i, [c_p, c_p, c_p, c_p, c_i64, c_i64, c_f, c_f, c_f, c_f, c_p]),
    "lsh_aff_scan_workspace": (c_sz, [c_i64, c_i64, c_i, c_i]),
    "lsh_aff_scan_layout": (c_i, [c_i64, c_i64, c_i, c_i, ctypes.POINTER(AffLayout)]),
    "lsh_aff_scan_fwd": (c_i, [c_p, c_p, c_p, c_p, c_i64, c_i64, c_f, c_f, c_f, c_f, c_f, c_i, c_i,
                               c_i64, c_p, c_sz, c_p]),
    "lsh_aff_bwd": (c_i, [c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_i64, c_i64, c_f, c_f, c_f, c_f, c_i,
                          c_i, c_p, c_sz, c_p]),
    "lsh_reverse_affine_scan": (c_i, [c_p, c_p, c_p, c_i64, c_i64, c_p]),
    "lsh_soft_bwd_workspace": (c_sz, [c_i64, c_i64, c_i]),
    "lsh_soft_bwd_partials": (c_i64, [c_i64, c_i64, c_i]),
    "lsh_soft_bwd": (c_i, [c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_i64, c_i64, ctypes.c_double, c_f, c_f,
                           c_i, c_p, c_sz, c_p]),
    "lsh_lif_scan_bwd_workspace": (c_sz, [c_i64, c_i64, c_i]),
    "lsh_lif_scan_bwd": (c_i, [c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_i64, c_i64, c_f, c_f, c_f, c_f,
                               c_i, c_i, c_p, c_sz, c_p]),
}


def lib_path():
    """The in-tree build, or the library named by LIFSCAN_HIP_LIB (another build of the same
    sources, e.g. with other tile constants)."""
    return os.environ.get("LIFSCAN_HIP_LIB") or _build.LIB_PATH


def lib():
    """Load (once) and return the ctypes handle of liblifscan_hip.so."""
    global _LIB
    if _LIB is None:
        path = lib_path()
        if not os.path.exists(path):
            raise RuntimeError(
                f"HIP extension not built ({path} missing): run `python -c \"import "
                f"__graft_entry__ as g; g.build()\"` or `python {_build.__file__}`")
        L = ctypes.CDLL(path)
        L.lsh_abi_version.restype = c_i
        if L.lsh_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{path} has C ABI version {L.lsh_abi_version()}, this binding "
                               f"needs {ABI_VERSION}: rebuild the library")
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _LIB = L
    return _LIB


_OPS = None


def ops():
    """The C++ autograd module of lif_tuned's recomputing pair (lifscan/_ops.cpp, built in-tree
    by build()) with the library's entry points handed over, or None when it is not built (the
    layer then runs the same kernels through its Python autograd function)."""
    global _OPS
    if _OPS is None:
        if not os.path.exists(_build.OPS_PATH):
            return None
        import importlib.util
        spec = importlib.util.spec_from_file_location(_build.OPS_NAME, _build.OPS_PATH)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        L = lib()
        addr = lambda f: ctypes.cast(f, ctypes.c_void_p).value
        mod.set_entry_points(addr(L.lsh_lif_scan_exact_fwd_starts),
                             addr(L.lsh_lif_scan_fused_bwd_starts), addr(L.lsh_status_string))
        _OPS = mod
    return _OPS


def check(rc, what):
    if rc == LSH_OK:
        return
    msg = f"{what}: {lib().lsh_status_string(rc).decode()} (status {rc})"
    if rc in (LSH_ERR_ARG, LSH_ERR_SHAPE, LSH_ERR_DIVISIBILITY, LSH_ERR_SCRATCH):
        raise ValueError(msg)
    raise RuntimeError(msg)


def ptr(t):
    """Device address of t (NULL for None) for a c_void_p argument: ctypes converts the plain
    int itself, which costs less per call than building a c_void_p."""
    return t.data_ptr() if t is not None else None


def stream_of(t):
    """torch's current stream on t's device as a raw hipStream_t (an int, as ptr)."""
    return torch._C._cuda_getCurrentRawStream(t.device.index)


def on_device(t):
    """Context making t's device the current one; a no-op when it already is (the common
    case, which then costs no device exchange on the host)."""
    idx = t.device.index
    if idx == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(idx)


def workspace(nbytes, device):
    """Caller-owned workspace (the library never allocates); 256-byte aligned by torch."""
    ws = torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)
    assert ws.data_ptr() % 256 == 0
    return ws


def read_stats(ws, chunk_neurons, super_neurons=0, alif=False):
    """alif: False (LIF), True (ALIF) or 2 (affine reset)."""
    st = ScanStats()
    check(lib().lsh_scan_stats_read(ptr(ws), int(chunk_neurons), int(super_neurons), int(alif),
                                    ctypes.byref(st), stream_of(ws)), "lsh_scan_stats_read")
    return st
