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


def _stub_result(w, ms: float) -> dict:
    """What bench.measure returns, for a workload timed at ``ms`` per launch (no GPU)."""
    return {"workload": w.name, "ms_per_step": ms, "kernel_ms": ms, "ms_min": ms * 0.99, "ms_max": ms * 1.013,
            "value": w.value(ms / 1e3), "unit": w.unit, "rate": w.rate(ms / 1e3), "bound": w.bound,
            "config": {"workload": w.name}, "replays": 20, "warmup_launches": 123456, "warmup_s": 1.0,
            "timing": "median of 20 hip-graph replays of 20 launches",
            "vendor": {"value": 1.0, "this_over_vendor": 1.093}}


def _stub_cpu(unit: str) -> dict:
    return {"value": 12.3456789, "unit": unit, "cores": 128, "kind": "port",
            "expression": "torch.softmax(x, dim=1) (python/test/asc2/kernels/test_softmax.py:43)",
            "sample": "the full 4096x4096 fp32 workload; 1234 timed call(s) after 1 warm-up, mean (10.0 s of CPU work)",
            "seconds_per_call": 0.0123456789, "host": {}}


class _Args:
    steps, warmup = 20, 5


def _full_line():
    import math
    suite = {}
    for i, key in enumerate(bench.SUITE):
        w = bench.WORKLOADS[key]()
        w.sets = w.xs = [None] * 3  # config() reads the rotation count
        r = _stub_result(w, 0.0123456789 * (i + 1) * math.pi)
        r["roofline"] = bench.roofline(w, r)
        r["roofline"]["traffic"] = 1234567890
        suite[key] = bench.compact_entry(r, r["roofline"], _stub_cpu(w.unit))
    head = bench.WORKLOADS[bench.HEADLINE]()  # not set up: the line takes the config measure() recorded
    res = _stub_result(head, 0.0230456)
    res["config"] = {"workload": head.name, "rows": 4096, "cols": 4096, "tile_size": 4096, "grid": 16,
                     "input": "randn*2 (N(0,4)), seed 1", "rotating_sets": 5}
    power = {k: {"value": 1234.5678, "w": 1391.0, "mhz": 1932, "frac_at_clock": 0.5702} for k in bench.POWER_WORKLOADS}
    extra = {"power": power, "launch_latency_us": {"asc2": 9.87, "asc2_always_compile": 31.2, "kernel_api": 6.5},
             "reference_published_us": {"asc1_vadd_8192_f32": [2.1, 3.6],
                                        "asc1_matmul_256_f32_bias_leakyrelu": [9.9, 25.5]}}
    return bench.build_line(_Args, head, res, _stub_cpu("GB/s"), suite, extra)


def test_stdout_line_is_compact_and_parses():
    import io
    import json
    text = bench.serialize_line(_full_line())
    assert len(text) < 8192, len(text)
    # what a reader of the run's stdout sees: progress on stderr, the line last on stdout
    out = io.StringIO("some earlier output\n" + text + "\n")
    line = json.loads(out.getvalue().strip().splitlines()[-1])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in line, key
    assert set(line["roofline"]) >= {"bound", "achieved", "peak", "unit", "frac", "traffic"}
    assert set(line["cpu_baseline"]) >= {"value", "unit", "cores", "kind", "sample"}
    assert line["steps"] == 20 and line["warmup"] == 5 and line["n_gpus"] == 1
    assert set(line["suite"]) == set(bench.SUITE)
    for key, e in line["suite"].items():
        assert set(e["roofline"]) == {"frac", "achieved", "traffic"}, key
        assert set(e["cpu_baseline"]) == {"value", "unit", "cores", "seconds_per_call"}, key
        assert e["ms_min"] <= e["ms_per_step"] <= e["ms_max"], key
    assert "power" in line and "host" in line


def test_serialize_trims_optional_parts_before_the_suite():
    line = _full_line()
    line["power"] = {f"k{i}": "x" * 100 for i in range(100)}  # 10 KB of padding
    text = bench.serialize_line(line)
    import json
    parsed = json.loads(text)
    assert len(text) < 8192 and "power" not in parsed
    assert all("cpu_baseline" in e for e in parsed["suite"].values())


def test_median_of_replays():
    assert bench._median([3.0, 1.0, 2.0]) == 2.0
    assert bench._median([4.0, 1.0, 2.0, 3.0]) == 2.5
    assert bench._sig(1234.5678, 4) == 1235 and bench._sig(0.000123456, 3) == 0.000123


def test_main_end_to_end_with_stubbed_gpu_legs(monkeypatch, capsys, tmp_path):
    # bench.main's control flow on the CPU: every GPU leg replaced by a stub of the same
    # return shape, the CPU baselines too; the last stdout line must be the parsed line
    import json
    import sys
    import torch
    from pyasc_amd import _native

    def fake_measure(w, steps, warmup, dev, graph=True, sampler=None, warmup_s=1.0, replays=7):
        r = _stub_result(w, 0.5)
        r["config"] = {"workload": w.name, "input": "stub"}
        return r

    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a: None)
    monkeypatch.setattr(torch.cuda, "empty_cache", lambda *a: None)
    monkeypatch.setattr(_native, "load_library", lambda *a, **k: None)
    monkeypatch.setattr(_native, "device_info", lambda *a: {"name": "stub"})
    monkeypatch.setattr(bench, "measure", fake_measure)
    monkeypatch.setattr(bench, "vendor", lambda w, steps, res: None)
    monkeypatch.setattr(bench, "launch_latency", lambda dev: {"asc2_cached_us": 9.0, "asc2_always_compile_us": 30.0,
                                                              "kernel_api_us": 6.0})
    monkeypatch.setattr(bench, "reference_durations", lambda dev: {
        "asc1_vadd_8192_f32": {"us_per_launch": 2.0, "reference_task_duration_us": 3.6}})
    monkeypatch.setattr(bench, "power_phase", lambda dev, keys, steps: {
        k: {"value": 1.0, "socket_w_median": 1400.0, "gfx_mhz_median": 1600, "frac_at_clock": 0.7} for k in keys})
    for cls in {type(bench.WORKLOADS[k]()) for k in bench.WORKLOADS}:
        monkeypatch.setattr(cls, "cpu_baseline", lambda self, min_total_s=2.0: _stub_cpu(self.unit))
    detail = tmp_path / "detail.json"
    monkeypatch.setattr(sys, "argv", ["bench.py", "--steps", "20", "--warmup", "5", "--detail", str(detail)])
    assert bench.main() == 0
    out = capsys.readouterr().out.strip().splitlines()
    assert len(out) == 1 and len(out[0]) < 8192
    line = json.loads(out[-1])
    assert line["steps"] == 20 and line["warmup"] == 5 and set(line["suite"]) == set(bench.SUITE) - {bench.HEADLINE}
    assert line["config"] == {"workload": "softmax_4096x4096_f32"}
    assert line["cpu_baseline"]["unit"] == "GB/s" and set(line["power"]) == set(bench.POWER_WORKLOADS)
    assert json.loads(detail.read_text())["line"] == line


def test_more_than_one_gpu_is_refused(monkeypatch, capsys):
    import sys
    monkeypatch.setattr(sys, "argv", ["bench.py", "--gpus", "8"])
    assert bench.main() == 2
    assert "one GPU only" in capsys.readouterr().err
