"""Socket power and graphics clock of the bench workloads on one MI355X -> profiles/power_clock.md.

    python profile_power.py [--out profiles/power_clock.md]

Needs the GPU and ``amd-smi``.  Two parts, both sampled with bench.PowerSampler
(``amd-smi metric -p -c -g 0`` about every 0.4 s; median of the samples after the first
two):

1. Each workload below runs through ``bench.measure`` with four seconds of warm-up
   (graph replays of its timed launches); the sampler covers the warm-up and the timed
   replays.  Energy per
   operation = median socket power x time per launch / operations per launch.
2. The same GEMM kernels on one round of 128 output tiles (half of the 256 CUs busy) and
   on one round of 256 tiles (all CUs), launched back to back for three seconds each:
   whether a round's time follows the clock the card settles at.
"""
from __future__ import annotations

import argparse
import os
import sys
import time

import bench

REPO = os.path.dirname(os.path.abspath(__file__))

WORKLOADS = ["matmul_bf16_8192", "matmul_i8_4096x11008x4096", "fa_fwd_noncausal", "fa_fwd_causal",
             "softmax_4096x4096", "vadd_268435456"]
WARMUP_S = 4.0
ROUNDS = [  # (dtype, M, N, K): 128 tiles of 256x256 (half the CUs), then 256 (all)
    ("int8", 2048, 4096, 4096), ("int8", 4096, 4096, 4096),
    ("int8", 2048, 4096, 16384), ("int8", 4096, 4096, 16384),
    ("bf16", 2048, 4096, 8192), ("bf16", 4096, 4096, 8192),
]


def _fmt(v, nd=1):
    return "-" if v is None else f"{v:.{nd}f}"


def workloads(dev) -> list:
    rows = []
    for name in WORKLOADS:
        w = bench.WORKLOADS[name]()
        s = bench.PowerSampler()
        r = bench.measure(w, 20, 10, dev, sampler=s, warmup_s=WARMUP_S)
        p = s.summary()
        watts, mhz = p.get("socket_w_median"), p.get("gfx_mhz_median")
        row = {"name": w.name, "value": r["value"], "unit": w.unit, "bound": w.bound, "power": p,
               "kernel_ms": r["kernel_ms"], "peak": w.peak}
        if watts is not None and w.bound == "mfma":
            row["pj_per_op"] = watts * r["kernel_ms"] * 1e-3 / w.work() * 1e12
            row["peak_at_clock"] = w.peak * mhz / 2400.0
        elif watts is not None:
            row["pj_per_byte"] = watts * r["kernel_ms"] * 1e-3 / w.work() * 1e12
        rows.append(row)
        print(f"power: {w.name} {r['value']:.1f} {w.unit} {watts} W {mhz} MHz", file=sys.stderr, flush=True)
        del w
    return rows


def rounds(dev, secs: float = 3.0) -> list:
    import torch
    from pyasc_amd import kernels
    g = torch.Generator(device=dev).manual_seed(3)
    rows = []
    for dtype, M, N, K in ROUNDS:
        if dtype == "int8":
            a = torch.randint(-127, 128, (M, K), dtype=torch.int8, device=dev, generator=g)
            b = torch.randint(-127, 128, (K, N), dtype=torch.int8, device=dev, generator=g)
            scale = torch.rand(N, device=dev, generator=g) * 0.009 + 0.001
            c = torch.empty(M, N, dtype=torch.float16, device=dev)

            def fn():
                kernels.matmul_i8(a, b, c, scale=scale)
        else:
            a = (torch.randn(M, K, device=dev, generator=g) / K ** 0.5).bfloat16()
            b = (torch.randn(K, N, device=dev, generator=g) / K ** 0.5).bfloat16()
            c = torch.empty(M, N, dtype=torch.bfloat16, device=dev)

            def fn():
                kernels.matmul(a, b, c)
        for _ in range(5):
            fn()
        torch.cuda.synchronize()
        s = bench.PowerSampler()
        s.start()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        n, t_end = 0, time.time() + secs
        e0.record()
        while time.time() < t_end:
            for _ in range(50):
                fn()
            n += 50
            torch.cuda.synchronize()
        e1.record()
        torch.cuda.synchronize()
        s.stop()
        p = s.summary()
        us = e0.elapsed_time(e1) * 1e3 / n
        mhz = p.get("gfx_mhz_median")
        k_tiles = K // (64 if dtype == "int8" else 32)
        rows.append({"dtype": dtype, "M": M, "N": N, "K": K, "tiles": (M // 256) * (N // 256), "us": us,
                     "watts": p.get("socket_w_median"), "mhz": mhz,
                     "cycles_per_ktile": None if mhz is None else us * mhz / k_tiles})
        print(f"power: {dtype} {M}x{N}x{K} {us:.1f} us {p.get('socket_w_median')} W {mhz} MHz", file=sys.stderr,
              flush=True)
        del a, b, c
    return rows


def write(path: str, wl: list, rd: list) -> None:
    cmd = "python profile_power.py"
    lines = [
        "# Socket power and graphics clock under the bench workloads (amd-smi), one MI355X", "",
        f"Made by `{cmd}` (repository root, one GPU call).  `bench.PowerSampler` samples "
        "`amd-smi metric -p -c -g 0` about every 0.4 s and reports the median after the first two samples; "
        "the clock is the mean of the eight GFX_n (XCD) readings of a sample.  MAX_CLK is 2400 MHz.", "",
        "## 1. Bench workloads (about 4 s of launches each)", "",
        "| Workload | bench value | socket W (median, min-max) | GFX MHz | samples | dense peak at this clock "
        "| value / peak at this clock | energy |",
        "|---|---|---|---:|---:|---:|---:|---:|",
    ]
    for r in wl:
        p = r["power"]
        if "pj_per_op" in r:
            extra = (f"{r['peak_at_clock']:.0f} {r['unit']} | {r['value'] / r['peak_at_clock']:.3f} | "
                     f"{r['pj_per_op']:.2f} pJ/op")
        elif "pj_per_byte" in r:
            extra = f"(HBM-bound) | | {r['pj_per_byte']:.0f} pJ/byte"
        else:
            extra = " | | "
        lines.append(f"| {r['name']} | {r['value']:.1f} {r['unit']} | {_fmt(p.get('socket_w_median'), 0)} "
                     f"({_fmt(p.get('socket_w_min'), 0)}-{_fmt(p.get('socket_w_max'), 0)}) | "
                     f"{_fmt(p.get('gfx_mhz_median'), 0)} | {p.get('samples', 0)} | {extra} |")
    lines += [
        "", "Dense peak at a clock f = MI355X dense peak x f / 2400 MHz (bf16 2.5 PFLOP/s, int8 5.0 POPS).  "
        "Energy = median socket power x time per launch / algorithmic operations (or bytes) per launch.", "",
        "## 2. One round of GEMM tiles on half and on all of the CUs", "",
        "256x256 output tiles, one workgroup per CU: 128 tiles leave half of the 256 CUs idle, 256 tiles fill "
        "them.  Cycles per k-tile = time per launch x clock / k-tiles per tile (the MFMA work of a k-tile is "
        "1024 cycles per SIMD: 32 MFMAs of 32 cycles).", "",
        "| GEMM | M x N x K | tiles | us per launch | socket W | GFX MHz | cycles per k-tile |",
        "|---|---|---:|---:|---:|---:|---:|",
    ]
    for r in rd:
        lines.append(f"| {r['dtype']} | {r['M']}x{r['N']}x{r['K']} | {r['tiles']} | {r['us']:.1f} | "
                     f"{_fmt(r['watts'], 0)} | {_fmt(r['mhz'], 0)} | {_fmt(r['cycles_per_ktile'], 0)} |")
    lines.append("")
    with open(path, "w") as f:
        f.write("\n".join(lines))


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--out", default=os.path.join(REPO, "profiles", "power_clock.md"))
    args = ap.parse_args()
    import torch
    from pyasc_amd import _native
    if not torch.cuda.is_available():
        print("profile_power.py needs the MI355X", file=sys.stderr)
        return 1
    _native.load_library()
    dev = torch.device("cuda", 0)
    wl = workloads(dev)
    rd = rounds(dev)
    write(args.out, wl, rd)
    print(f"wrote {args.out}", file=sys.stderr)
    return 0


if __name__ == "__main__":
    sys.exit(main())
