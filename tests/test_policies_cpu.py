"""CPU: the MI355X dispatch policies (no GPU needed): auto_modes thresholds, the chunk of the
three-kernel adjoint, and the reference's chunk policy kept verbatim."""
import pytest


def test_auto_modes_follow_mi355x_measurements():
    from lifscan import hip_lif as L
    assert L.auto_modes(1024, 65536) == ("scan", "scan")
    assert L.auto_modes(4096, 65536) == ("serial", "scan")
    assert L.auto_modes(65536, 4096) == ("serial", "scan")
    assert L.auto_modes(1024, 4096) == ("serial", "scan")
    assert L.auto_modes(65536, 128) == ("serial", "serial")
    # the grid of the reference's experiments/e11_auto.py: the serial adjoint below 16384
    # neurons up to T = 1024, the scan from T = 2048, and from 16384 neurons from T = 256
    assert L.auto_modes(1024, 1024) == ("serial", "serial")
    assert L.auto_modes(8192, 1024) == ("serial", "serial")
    assert L.auto_modes(8192, 2048) == ("serial", "scan")
    assert L.auto_modes(32768, 1024) == ("serial", "scan")
    assert L.auto_modes(16384, 256) == ("serial", "scan")


def test_chunked_bwd_chunk_choice():
    from lifscan import hip_lif as L
    assert L.chunked_bwd_C(2 ** 20, 1024) == 512        # 2048 chunks x 16 blocks
    assert L.chunked_bwd_C(65536, 1024) == 512          # 128 x 16 = 2048
    assert L.chunked_bwd_C(16384, 4096) == 512          # 32 chunks x 64 blocks = 2048
    assert L.chunked_bwd_C(1000, 64, C=8) == 8          # nothing gives 2048 blocks: the given C
    with pytest.raises(ValueError):
        L._pick_C(1001, D=2)


def test_alif_scan_adjoint_dispatch():
    """ALIF adjoint "scan": the single pass from 8192 neurons, else the look-back single pass when
    T is a multiple of 128, else the chunked passes at the power-of-two chunk nearest sqrt(T/4)."""
    from lifscan import hip_alif as H
    assert H.alif_chunked_C(4096) == 32
    assert H.alif_chunked_C(65536) == 128
    assert H.alif_chunked_C(2 ** 20) == 512
    assert H.alif_chunked_C(1000, C=8) == 8          # no power of two in 16..512 divides T
    assert H._bwd_mode("scan", 65536, 1024, 64) == (3, 16)   # look-back single pass
    assert H._bwd_mode("scan", 16384, 4096, 64) == (3, 16)
    assert H._bwd_mode("scan", 4096, 16384, 64) == (2, 16)
    assert H._bwd_mode("scan", 4160, 1024, 64) == (1, 32)    # T % 128 != 0: chunked
    assert H._bwd_mode("chunked", 65536, 1024, 128) == (1, 128)
    assert H._bwd_mode("serial", 4096, 16, 64) == (0, 64)
    with pytest.raises(ValueError):
        H._bwd_mode("chunked", 100, 8, 64)


def test_long_sequence_plan():
    """The converged long-chunk forward: unsplit below 2^30 neuron-steps, else half the long
    chunk in LONG_PIECES pieces (the measured optimum at N = 1024, T = 2^20)."""
    from lifscan import hip_lif as L
    assert L.long_sequence_C(2 ** 20, 1024) == 4096
    assert L.long_sequence_plan(2 ** 20, 1024) == (2048, L.LONG_PIECES)
    assert L.long_sequence_plan(2 ** 18, 1024) == (4096, 1)
    assert L.long_sequence_plan(2 ** 19, 512) == (4096, 1)
    assert L.long_sequence_plan(65536, 1000) == (1024, 1)
    assert L.long_sequence_plan(4096, 65536) == (0, 1)             # single pass


def test_auto_policies_accept_lengths_the_chunk_policy_rejects():
    """lif_auto / lif_param(mode="auto") run for every T: a pass whose chunk policy has no
    chunk for T stays serial, and the recomputing-pair test answers False instead of raising
    (T = 1000 and 1032 have no chunk divisible by 16; T = 1002 none divisible by 2 either)."""
    from lifscan import hip_lif as L
    for T in (1000, 1032, 257, 1002):
        assert L._recompute_ok(T, 65536, 16, 10 ** 6) is False
        assert L._recompute_ok(T, 4096, 16, T) is False
    assert L.auto_modes(16384, 1000) == ("serial", "scan")
    assert L.auto_modes(16384, 1032) == ("serial", "scan")
    assert L.auto_modes(16384, 1002) == ("serial", "serial")
    assert L.auto_modes(1024, 16386) == ("serial", "serial")   # 16386 = 2 * 8193
    assert L.auto_modes(1024, 16392) == ("serial", "scan")     # chunk 8 for the adjoint only
    assert L._recompute_ok(4096, 65536, 16, 10 ** 6) is True


def test_warm_plan():
    """The warm-started converged forward: W = 24/(1 - |beta|) rounded up to 256 (256..8192).
    Up to 4096 neurons and from T = 4W: the power-of-two chunk (>= 256, >= 4 chunks) whose
    (chunk, block) waves come nearest 512 (1024 from 2^29 neuron-steps), the longer on a tie.
    Above: the longest chunk >= 3W dividing T with >= 1024 waves, else the shortest; none above
    8192 neurons."""
    from lifscan import hip_lif as L
    assert L.warm_plan(2 ** 20, 1024, 0.99) == (16384, 2560)   # cfg4: 16 blocks x 64 chunks
    assert L.warm_plan(2 ** 20, 1024, 0.9) == (16384, 256)
    assert L.warm_plan(2 ** 18, 256, 0.99) == (2048, 2560)     # 4 blocks x 128 chunks
    assert L.warm_plan(65536, 4096, 0.99) == (8192, 2560)      # 64 blocks x 8 chunks
    assert L.warm_plan(16384, 1024, 0.99) == (512, 2560)       # 16 blocks x 32 chunks
    assert L.warm_plan(16384, 128, 0.99) == (256, 2560)        # as many waves as chunks of 256 give
    assert L.warm_plan(8192, 128, 0.99) is None                # T < 4W: a serial sweep
    assert L.warm_plan(16384, 4096, 0.9) == (2048, 256)
    assert L.warm_plan(65536, 8192, 0.99) == (8192, 2560)      # above 4096 neurons: the 3W rule
    assert L.warm_plan(16384, 8192, 0.99) is None
    assert L.warm_plan(4096, 65536, 0.9) is None               # N > 8192: single pass
    assert L.warm_plan(1000, 64, 0.9) is None                  # no power-of-two chunk
    assert L.warm_plan(2 ** 20, 64, 1.0)[1] == 8192
    assert L.warm_plan(0, 64, 0.9) is None and L.warm_plan(4096, 0, 0.9) is None
