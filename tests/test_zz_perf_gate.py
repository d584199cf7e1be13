"""Performance regression gate on the MI355X, in the manner of the reference's presmoke gate.

The reference times its kernels under msprof and fails a run whose task duration exceeds
the golden by more than 10% (test/run_presmoke_npu_test.sh, test/collect_profiling_data.py,
goldens in test/all_task_durations_golden.csv).  Here:

- the two kernels with published reference durations (asc1 vadd 8192 fp32 on 16 cores,
  3.6 us; asc1 matmul 256^3 fp32 + bias + leaky relu, 25.5 us) must stay within the
  reference's rule, duration <= 1.1 x golden;
- every bench configuration of the asc2 hot path must stay above a floor set well below
  the lowest figure measured across boxes (the MFMA kernels run at the clock the board's
  1.4 kW limit allows, and boxes differ by up to about 20% on the int8 GEMM), so the gate
  catches a kernel that lost its fast path or its launch shape, not box-to-box spread.

Each figure is bench.py's own measurement (launches captured into a HIP graph, one timed
replay between HIP events), with fewer steps than the bench."""
import pytest

import bench

pytestmark = pytest.mark.gpu

# workload key -> (floor, unit): lowest figures measured (bench runs, and this gate's shorter
# warm-up) 5613 GB/s (softmax), 6074 (vadd), 1215 TFLOP/s, 1624 TOPS, 1095 and 880 TFLOP/s
FLOORS = {
    "softmax_4096x4096": (4500.0, "GB/s"),
    "softmax_16384x1024": (4500.0, "GB/s"),
    "vadd_268435456": (4800.0, "GB/s"),
    "matmul_bf16_8192": (950.0, "TFLOP/s"),
    "matmul_i8_4096x11008x4096": (1200.0, "TOPS"),
    "fa_fwd_noncausal": (820.0, "TFLOP/s"),
    "fa_fwd_causal": (680.0, "TFLOP/s"),
    "rms_norm_4096x4096": (4300.0, "GB/s"),
}


@pytest.mark.parametrize("key", sorted(FLOORS))
def test_hot_path_floor(device, key):
    floor, unit = FLOORS[key]
    w = bench.WORKLOADS[key]()
    res = bench.measure(w, steps=10, warmup=5, dev=device)
    assert w.unit == unit
    print(f"{w.name}: {res['value']:.1f} {unit} (floor {floor})")
    assert res["value"] >= floor, f"{w.name}: {res['value']:.1f} {unit} below the regression floor {floor}"


def test_reference_published_durations(device):
    # bench.reference_durations runs the two asc1 kernels through the launch surface (200
    # launches per graph replay) and checks their outputs against torch
    out = bench.reference_durations(device, steps=200)
    for name, r in out.items():
        print(f"{name}: {r['us_per_launch']} us (reference golden {r['reference_task_duration_us']} us)")
        assert r["us_per_launch"] <= 1.1 * r["reference_task_duration_us"], name
