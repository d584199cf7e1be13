"""bench.py's host-side pieces without a GPU: the amd-smi reading parser and summary of the
power phase, and the warm-up count it derives from a workload's time per launch."""
import bench

# `amd-smi metric -p -c -g 0` as printed on an MI355X box (trimmed to two XCDs)
AMD_SMI_TEXT = """GPU: 0
    POWER:
        SOCKET_POWER: 1396 W
        GFX_VOLTAGE: N/A
        THROTTLE_STATUS: N/A
    CLOCK:
        GFX_0:
            CLK: 1642 MHz
            MIN_CLK: 500 MHz
            MAX_CLK: 2400 MHz
            CLK_LOCKED: DISABLED
            DEEP_SLEEP: ENABLED
        GFX_1:
            CLK: 1650 MHz
            MIN_CLK: 500 MHz
            MAX_CLK: 2400 MHz
        MEM_0:
            CLK: 2000 MHz
            MIN_CLK: 2000 MHz
            MAX_CLK: 2000 MHz
        VCLK_0:
            CLK: 59 MHz
"""


def test_parse_power_and_gfx_clocks_only():
    watts, mhz = bench.PowerSampler.parse(AMD_SMI_TEXT)
    assert watts == 1396.0
    # the mean of the GFX_n clocks; the memory and video clocks are not graphics clocks
    assert mhz == (1642.0 + 1650.0) / 2


def test_parse_without_readings():
    assert bench.PowerSampler.parse("") == (None, None)
    assert bench.PowerSampler.parse("GPU: 0\n    POWER:\n        SOCKET_POWER: N/A\n") == (None, None)


def test_summary_skips_the_ramp_and_takes_medians():
    s = bench.PowerSampler(skip=2)
    s.samples = [(0.0, 250.0, 100.0), (0.4, 900.0, 1300.0)] + [(0.8 + 0.4 * i, w, c) for i, (w, c) in enumerate(
        [(1390.0, 1660.0), (1400.0, 1640.0), (1398.0, 1650.0)])]
    p = s.summary()
    assert p["samples"] == 3
    assert p["socket_w_median"] == 1398.0 and p["socket_w_min"] == 1390.0 and p["socket_w_max"] == 1400.0
    assert p["gfx_mhz_median"] == 1650 and p["seconds"] == 0.8


def test_summary_without_samples_says_so():
    p = bench.PowerSampler().summary()
    assert p["samples"] == 0 and "note" in p


def test_power_phase_covers_the_headline_and_the_mfma_workloads():
    assert bench.POWER_WORKLOADS[0] == bench.HEADLINE
    for key in bench.POWER_WORKLOADS[1:]:
        assert bench.WORKLOADS[key]().bound == "mfma"
