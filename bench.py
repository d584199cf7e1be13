"""Benchmark of the asc2 hot-path kernels on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--no-suite] [--no-cpu] [--no-power]

A "step" is one launch of the headline kernel over one batch of synthetic,
device-resident input.  The headline workload is BASELINE.json's configs[1],
row softmax of a 4096x4096 fp32 matrix (HBM-bound; metric HBM GB/s).  The
other configurations (the asc2 vadd_kernel[16] of configs[0], the vadd
bandwidth shape, softmax 16384x1024, bf16/fp16 matmul 8192^3, int8 matmul
4096x11008x4096 + dequant, flash-attention forward causal and not) and the
kernels of the adjacent rows are measured the same way and reported under
"suite", with a plain streaming copy of the same sizes as the bandwidth
reference of the HBM-bound kernels.

Timing (steady state, in the manner of the reference's median-with-skip,
python/asc/lib/profiling/result.py:33-47): per workload, W untimed eager launches,
then the K timed launches captured into one HIP graph and replayed back to back
for at least WARMUP_S seconds (clocks and caches settle), then REPLAYS replays of
exactly K launches, each between its own pair of HIP events on the replay stream;
the figure is the median replay / K, with the fastest and slowest replay beside
it.  --no-graph times each launch with its own event pair instead.  HBM-bound
workloads rotate through enough input/output sets (> 512 MiB) that the 256 MiB
Infinity Cache cannot serve them; so do the MFMA workloads.  Every GPU leg runs
before any CPU baseline.  The CPU baseline of every workload is the reference
test's torch CPU golden expression (oracle/cpu_golden.py), timed on the host cores
on the full workload (the int8 product on a quarter of A's rows), repeated to at
least 2 s of CPU work (10 s for the headline); the line names the host (thread
count, os.cpu_count(), CPU model) once.

With the suite, a power phase follows the suite: the headline and each MFMA
workload are measured again after 3 s of warm-up while amd-smi samples socket
power and graphics clock ("power" in the line; for the MFMA workloads also the
fraction of the dense peak at the sampled clock).

`roofline.traffic` comes from profiles/traffic.json (rocprofv3 FETCH_SIZE /
WRITE_SIZE passes summarised by profile_summary.py).  Each entry is stamped with
a hash of the kernel sources it was measured on; when the sources have changed
since, the bench reports null instead of a stale figure.

Prints ONE JSON line of under 8 KB (the headline in full, a compact entry per suite
workload); --detail FILE writes every figure in full.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import math
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP16_PEAK_TFLOPS = 2500.0
INT8_PEAK_TOPS = 5000.0
METRIC = "HBM GB/s (vadd, softmax); TFLOP/s or TOPS (matmul, FA-fwd); % of MI355X peak"
ROTATE_BYTES = 640 << 20  # > 2x the 256 MiB Infinity Cache
SMALL_SET_BYTES = 4 << 20  # below this a workload is latency-bound and is not rotated
CSRC = os.path.join(REPO, "pyasc_amd", "csrc")
CPU_MIN_S = 2.0  # timed CPU work per suite baseline (the full workload, repeated to at least this long)
CPU_HEADLINE_S = 10.0  # the same for the headline's baseline
WARMUP_S = 1.0  # least warm-up per workload: graph replays of its timed launches (clocks and caches settle)
REPLAYS = 20  # timed graph replays per workload (60 for the us-scale launch); the figure is their median
LINE_LIMIT = 8192  # the stdout line stays below this many bytes (longer lines are not read back)


class Workload:
    """One benchmarked kernel configuration."""
    name = ""
    bound = "hbm"       # "hbm" | "mfma" | "latency"
    unit = "GB/s"
    dtype = "f32"
    peak = HBM_PEAK_GBS
    kernel_hint = ""    # substring of the HIP kernel's name in rocprof traces
    sources = ("common.h",)  # csrc files the kernel is built from (stamps its traffic measurement)

    def setup(self, dev):
        raise NotImplementedError

    def launch(self, i: int) -> None:
        raise NotImplementedError

    def work(self) -> float:
        """Algorithmic bytes (hbm) or operations (mfma) of one launch."""
        raise NotImplementedError

    def rate(self, seconds: float) -> float:
        scale = 1e9 if self.bound != "mfma" else 1e12
        return self.work() / seconds / scale

    def value(self, seconds: float) -> float:
        """The figure the line reports: the rate, or microseconds for a latency-bound launch."""
        return seconds * 1e6 if self.bound == "latency" else self.rate(seconds)

    def config(self) -> dict:
        return {"workload": self.name}

    def cpu_baseline(self):
        return None

    # The same operation through the ROCm library torch calls for it (None: no such
    # library kernel), launched by vendor_launch on the workload's own inputs.
    vendor_expression = None

    def vendor_launch(self, i: int) -> None:
        raise NotImplementedError


def _sets_for(bytes_per_set: int) -> int:
    if bytes_per_set < SMALL_SET_BYTES:
        return 1
    return max(1, math.ceil(ROTATE_BYTES / bytes_per_set))


def sources_hash(files) -> str:
    """SHA-256 (first 16 hex digits) of the named csrc files, in order."""
    h = hashlib.sha256()
    for f in files:
        with open(os.path.join(CSRC, f), "rb") as fh:
            h.update(f.encode() + b"\0" + fh.read())
    return h.hexdigest()[:16]


_HOST = None


def host_info() -> dict:
    """The host the CPU baselines ran on."""
    global _HOST
    if _HOST is None:
        import torch
        model = ""
        try:
            with open("/proc/cpuinfo") as f:
                for line in f:
                    if line.startswith("model name"):
                        model = line.split(":", 1)[1].strip()
                        break
        except OSError:
            pass
        try:
            affinity = len(os.sched_getaffinity(0))
        except (AttributeError, OSError):
            affinity = None
        _HOST = {"torch_threads": torch.get_num_threads(), "os_cpu_count": os.cpu_count(),
                 "affinity_cpus": affinity, "cpu_model": model}
    return _HOST


def _time_cpu(fn, min_total_s: float = CPU_MIN_S):
    """(seconds per call, calls timed): one warm-up call (kept as the sample when it alone
    takes over a second), then calls until ``min_total_s`` of timed work; the mean."""
    t0 = time.perf_counter()
    fn()
    first = time.perf_counter() - t0
    if first > 1.0 and first >= min_total_s:
        return first, 1
    calls, start = 0, time.perf_counter()
    while True:
        fn()
        calls += 1
        elapsed = time.perf_counter() - start
        if elapsed >= min_total_s:
            return elapsed / calls, calls


def _cpu(work: float, scale: float, unit: str, expression: str, sample: str, timing) -> dict:
    """A cpu_baseline object: ``work`` units per call timed as ``timing`` = (seconds per
    call, calls); value = work / seconds / scale (or microseconds for unit "us")."""
    import torch
    secs, calls = timing
    value = secs * 1e6 if unit == "us" else work / secs / scale
    return {"value": round(value, 5), "unit": unit, "cores": torch.get_num_threads(), "kind": "port",
            "expression": expression,
            "sample": f"{sample}; {calls} timed call(s) after 1 warm-up, mean ({secs * calls:.1f} s of CPU work)",
            "seconds_per_call": secs, "host": host_info()}


class Softmax(Workload):
    bound, unit, dtype, kernel_hint = "hbm", "GB/s", "f32", "softmax"
    sources = ("softmax.hip", "softmax_kernels.h", "rows.h", "numeric.h", "common.h")
    vendor_expression = "torch.softmax(x, dim=1) (PyTorch's ROCm softmax kernel)"

    def vendor_launch(self, i: int) -> None:
        import torch
        torch.softmax(self.xs[i % len(self.xs)], dim=1)

    def __init__(self, rows: int, cols: int):
        self.rows, self.cols = rows, cols
        self.name = f"softmax_{rows}x{cols}_f32"

    def setup(self, dev):
        import torch
        n_sets = _sets_for(8 * self.rows * self.cols)
        g = torch.Generator(device=dev).manual_seed(1)
        self.xs = [torch.randn(self.rows, self.cols, device=dev, generator=g) * 2.0 for _ in range(n_sets)]
        self.outs = [torch.empty_like(x) for x in self.xs]

    def launch(self, i: int) -> None:
        from pyasc_amd import kernels
        j = i % len(self.xs)
        kernels.softmax_rows(self.xs[j], self.outs[j], self.rows, self.cols, self.cols, 16)

    def work(self) -> float:
        return 2.0 * 4 * self.rows * self.cols

    def config(self) -> dict:
        return {"workload": self.name, "rows": self.rows, "cols": self.cols, "tile_size": self.cols, "grid": 16,
                "input": "randn*2 (N(0,4)), seed 1", "rotating_sets": len(self.xs)}

    def cpu_baseline(self, min_total_s: float = CPU_MIN_S):
        import torch
        from oracle import cpu_golden
        x = torch.randn(self.rows, self.cols, generator=torch.Generator().manual_seed(1)) * 2.0
        return _cpu(self.work(), 1e9, "GB/s", "torch.softmax(x, dim=1) (python/test/asc2/kernels/test_softmax.py:43)",
                    f"the full {self.rows}x{self.cols} fp32 workload",
                    _time_cpu(lambda: cpu_golden.softmax(x), min_total_s))


class Copy(Workload):
    """The bandwidth reference: a plain non-temporal 16-byte streaming copy (asc_copy_bytes)
    moving the same bytes per launch as the HBM-bound kernel it stands beside."""
    bound, unit, dtype, kernel_hint = "hbm", "GB/s", "u8", "copy_vec_kernel"
    sources = ("vadd.hip", "numeric.h", "common.h")

    def __init__(self, n_bytes: int, label: str):
        self.n = n_bytes  # bytes read (and written) per launch
        self.name = f"copy_{label}"

    def setup(self, dev):
        import torch
        g = torch.Generator(device=dev).manual_seed(0)
        self.sets = []
        for _ in range(_sets_for(2 * self.n)):
            src = torch.empty(self.n, dtype=torch.uint8, device=dev)
            src.random_(0, 256, generator=g)
            self.sets.append((src, torch.empty(self.n, dtype=torch.uint8, device=dev)))

    def launch(self, i: int) -> None:
        import torch
        from pyasc_amd import _native
        src, dst = self.sets[i % len(self.sets)]
        _native.call("asc_copy_bytes", src.data_ptr(), dst.data_ptr(), self.n,
                     int(torch.cuda.current_stream().cuda_stream))

    def work(self) -> float:
        return 2.0 * self.n

    def config(self) -> dict:
        return {"workload": self.name, "bytes_read": self.n, "bytes_written": self.n,
                "kernel": "asc_copy_bytes (non-temporal 16-byte vectors, 4 per thread)",
                "rotating_sets": len(self.sets)}

    def cpu_baseline(self, min_total_s: float = CPU_MIN_S):
        import torch
        src = torch.randint(0, 256, (self.n,), dtype=torch.uint8, generator=torch.Generator().manual_seed(0))
        dst = torch.empty_like(src)
        return _cpu(self.work(), 1e9, "GB/s", "dst.copy_(src) (torch host copy)", f"the full {self.n}-byte copy",
                    _time_cpu(lambda: dst.copy_(src), min_total_s))


class Vadd(Workload):
    bound, unit, dtype, kernel_hint = "hbm", "GB/s", "f32", "vadd"
    sources = ("vadd.hip", "vadd_kernels.h", "numeric.h", "common.h")
    vendor_expression = "torch.add(x, y, out=out) (PyTorch's ROCm elementwise kernel)"

    def vendor_launch(self, i: int) -> None:
        import torch
        x, y, out = self.sets[i % len(self.sets)]
        torch.add(x, y, out=out)

    def __init__(self, n: int):
        self.n = n
        self.name = f"vadd_{n}_f32"

    def setup(self, dev):
        import torch
        n_sets = _sets_for(12 * self.n)
        g = torch.Generator(device=dev).manual_seed(0)
        self.sets = []
        for _ in range(n_sets):
            self.sets.append((torch.rand(self.n, device=dev, generator=g), torch.rand(self.n, device=dev, generator=g),
                              torch.empty(self.n, device=dev)))
        num_tiles = (self.n + 127) // 128
        self.tpb = (num_tiles + 15) // 16  # vadd_launch's tile_per_block (test_vadd.py:31-38)

    def launch(self, i: int) -> None:
        from pyasc_amd import kernels
        x, y, out = self.sets[i % len(self.sets)]
        kernels.vadd(x, y, out, self.n, 128, self.tpb, 16)

    def work(self) -> float:
        return 12.0 * self.n

    def config(self) -> dict:
        return {"workload": self.name, "size": self.n, "tile_size": 128, "tile_per_block": self.tpb, "grid": 16,
                "input": "torch.rand (uniform [0,1)), seed 0", "rotating_sets": len(self.sets)}

    def cpu_baseline(self, min_total_s: float = CPU_MIN_S):
        import torch
        from oracle import cpu_golden
        g = torch.Generator().manual_seed(0)
        x, y = torch.rand(self.n, generator=g), torch.rand(self.n, generator=g)
        return _cpu(self.work(), 1e9, "GB/s", "x + y (README.md:53; test_vadd.py:48)",
                    f"the full workload, {self.n} fp32 elements", _time_cpu(lambda: cpu_golden.vadd(x, y), min_total_s))


class Asc2VaddPlumbing(Workload):
    """the asc2 vadd_kernel launched as written in the reference test,
    vadd_kernel[16](x, y, out, 8192, 128, 4) (python/test/asc2/kernels/test_vadd.py:31-38), on
    device tensors through the drop-in surface (JIT dispatch, launch cache, C ABI).  The figure
    is device time per launch in microseconds; the launches are captured in a HIP graph, so host
    launch cost is not in it (launch_latency reports that)."""
    bound, unit, dtype, kernel_hint = "latency", "us", "f32", "vadd"
    sources = ("vadd.hip", "vadd_kernels.h", "numeric.h", "common.h")
    name = "asc2_vadd_kernel_8192_grid16"

    def setup(self, dev):
        import torch
        import pyasc_amd
        pyasc_amd.install_aliases()
        import asc
        import asc2

        @asc2.jit
        def vadd_kernel(x_ptr: asc.GlobalAddress, y_ptr: asc.GlobalAddress, out_ptr: asc.GlobalAddress, size: int,
                        tile_size: asc.ConstExpr[int], tile_per_block: asc.ConstExpr[int]):
            ...  # declaration: binds the registered native kernel by signature

        self.kernel = vadd_kernel
        g = torch.Generator(device=dev).manual_seed(0)
        self.x, self.y = torch.rand(8192, device=dev, generator=g), torch.rand(8192, device=dev, generator=g)
        self.out = torch.empty(8192, device=dev)

    def launch(self, i: int) -> None:
        self.kernel[16](self.x, self.y, self.out, 8192, 128, 4)

    def work(self) -> float:
        return 12.0 * 8192

    def config(self) -> dict:
        return {"workload": self.name, "call": "vadd_kernel[16](x, y, out, 8192, 128, 4)", "size": 8192,
                "tile_size": 128, "tile_per_block": 4, "grid": 16, "input": "torch.rand (uniform [0,1)), seed 0",
                "note": "latency-bound (96 KiB per launch): value is device microseconds per launch, "
                        "not rotated (the inputs stay in L2 as in the reference test)"}

    def cpu_baseline(self, min_total_s: float = CPU_MIN_S):
        import torch
        from oracle import cpu_golden
        g = torch.Generator().manual_seed(0)
        x, y = torch.rand(8192, generator=g), torch.rand(8192, generator=g)
        return _cpu(self.work(), 1e9, "us", "x + y (README.md:53; test_vadd.py:48)",
                    "the full workload, 8192 fp32 elements (microseconds per call)",
                    _time_cpu(lambda: cpu_golden.vadd(x, y), min_total_s))


class LeakyRelu(Workload):
    """test_leaky_relu.py's kernel at a bandwidth size: bf16, alpha a 0-dim bf16 tensor (0.1)."""
    bound, unit, dtype, kernel_hint = "hbm", "GB/s", "bf16", "leaky_relu_vec"
    sources = ("elementwise.hip", "elementwise_kernels.h", "numeric.h", "common.h")

    def __init__(self, n: int):
        self.n = n
        self.name = f"leaky_relu_{n}_bf16"

    def setup(self, dev):
        import torch
        g = torch.Generator(device=dev).manual_seed(0)
        self.sets = [((torch.rand(self.n, device=dev, generator=g) * 10.0 - 5.0).to(torch.bfloat16),
                      torch.empty(self.n, device=dev, dtype=torch.bfloat16)) for _ in range(_sets_for(4 * self.n))]
        self.alpha = float(torch.tensor(0.1, dtype=torch.bfloat16).item())
        self.tpb = ((self.n + 127) // 128 + 15) // 16  # leaky_relu_launch (test_leaky_relu.py:29-37)

    def launch(self, i: int) -> None:
        from pyasc_amd import kernels
        x, out = self.sets[i % len(self.sets)]
        kernels.leaky_relu(x, self.alpha, out, self.n, 128, self.tpb, 16)

    def work(self) -> float:
        return 4.0 * self.n

    def config(self) -> dict:
        return {"workload": self.name, "size": self.n, "tile_size": 128, "tile_per_block": self.tpb, "grid": 16,
                "alpha": "bf16 0.1", "input": "rand*10-5 bf16", "rotating_sets": len(self.sets)}

    def cpu_baseline(self, min_total_s: float = CPU_MIN_S):
        import torch
        from oracle import cpu_golden
        x = torch.rand(self.n, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16) * 10.0 - 5.0
        alpha = torch.tensor(0.1, dtype=torch.bfloat16)
        return _cpu(self.work(), 1e9, "GB/s", "torch.where(x >= 0, x, x * alpha) (test_leaky_relu.py:47)",
                    f"the full workload, {self.n} bf16 elements",
                    _time_cpu(lambda: cpu_golden.leaky_relu(x, alpha), min_total_s))


class VMulAdd(Workload):
    """test_vmuladd.py's kernel at a bandwidth size (fp32, tile 32 as in vmuladd_launch)."""
    bound, unit, dtype, kernel_hint = "hbm", "GB/s", "f32", "vmuladd_vec"
    sources = ("elementwise.hip", "elementwise_kernels.h", "numeric.h", "common.h")

    def __init__(self, n: int):
        self.n = n
        self.name = f"vmuladd_{n}_f32"

    def setup(self, dev):
        import torch
        g = torch.Generator(device=dev).manual_seed(0)
        self.sets = [tuple(torch.rand(self.n, device=dev, generator=g) * 10 for _ in range(3)) +
                     (torch.empty(self.n, device=dev),) for _ in range(_sets_for(16 * self.n))]
        self.tpb = ((self.n + 31) // 32 + 15) // 16  # vmuladd_launch (test_vmuladd.py:34-40)

    def launch(self, i: int) -> None:
        from pyasc_amd import kernels
        x, y, z, out = self.sets[i % len(self.sets)]
        kernels.vmuladd(x, y, z, out, self.n, 32, self.tpb, 16)

    def work(self) -> float:
        return 16.0 * self.n

    def config(self) -> dict:
        return {"workload": self.name, "size": self.n, "tile_size": 32, "tile_per_block": self.tpb, "grid": 16,
                "input": "rand*10 fp32, seed 0", "rotating_sets": len(self.sets)}

    def cpu_baseline(self, min_total_s: float = CPU_MIN_S):
        import torch
        from oracle import cpu_golden
        g = torch.Generator().manual_seed(0)
        x, y, z = (torch.rand(self.n, generator=g) * 10 for _ in range(3))
        return _cpu(self.work(), 1e9, "GB/s",
                    "x * y + z, unfused (test_vmuladd.py:52's numpy golden, evaluated with torch)",
                    f"the full workload, {self.n} fp32 elements",
                    _time_cpu(lambda: cpu_golden.vmuladd(x, y, z), min_total_s))


class Gelu(Workload):
    """test_gelu.py's kernel at softmax's second shape (fp32 rows, tile = row length)."""
    bound, unit, dtype, kernel_hint = "hbm", "GB/s", "f32", "gelu_rows_f32"
    sources = ("elementwise.hip", "elementwise_kernels.h", "numeric.h", "common.h")

    def __init__(self, rows: int, cols: int, approximate: bool):
        self.rows, self.cols, self.approximate = rows, cols, approximate
        self.name = f"gelu_{'tanh' if approximate else 'erf'}_{rows}x{cols}_f32"

    def setup(self, dev):
        import torch
        g = torch.Generator(device=dev).manual_seed(1)
        self.sets = [(torch.randn(self.rows, self.cols, device=dev, generator=g) * 2.0,
                      torch.empty(self.rows, self.cols, device=dev))
                     for _ in range(_sets_for(8 * self.rows * self.cols))]

    def launch(self, i: int) -> None:
        from pyasc_amd import kernels
        x, out = self.sets[i % len(self.sets)]
        kernels.gelu_rows(x, out, self.rows, self.cols, self.cols, self.approximate, 16)

    def work(self) -> float:
        return 8.0 * self.rows * self.cols

    def config(self) -> dict:
        return {"workload": self.name, "rows": self.rows, "cols": self.cols, "tile_size": self.cols, "grid": 16,
                "approximate": self.approximate, "input": "randn*2 fp32", "rotating_sets": len(self.sets)}

    def cpu_baseline(self, min_total_s: float = CPU_MIN_S):
        import torch
        from oracle import cpu_golden
        x = torch.randn(self.rows, self.cols, generator=torch.Generator().manual_seed(1)) * 2.0
        return _cpu(self.work(), 1e9, "GB/s", "test_gelu.py:44-48 golden",
                    f"the full {self.rows}x{self.cols} workload",
                    _time_cpu(lambda: cpu_golden.gelu(x, self.approximate), min_total_s))


class RmsNorm(Workload):
    """asc2.rms_norm rows (build-defined rms_norm_kernel) at softmax's headline shape."""
    bound, unit, dtype, kernel_hint = "hbm", "GB/s", "f32", "rms_norm"
    sources = ("reduce.hip", "rows.h", "numeric.h", "common.h")

    def __init__(self, rows: int, cols: int):
        self.rows, self.cols = rows, cols
        self.name = f"rms_norm_{rows}x{cols}_f32"

    def setup(self, dev):
        import torch
        g = torch.Generator(device=dev).manual_seed(1)
        self.gamma = torch.rand(self.cols, device=dev, generator=g) + 0.5
        self.sets = [(torch.randn(self.rows, self.cols, device=dev, generator=g) * 2.0,
                      torch.empty(self.rows, self.cols, device=dev))
                     for _ in range(_sets_for(8 * self.rows * self.cols))]

    def launch(self, i: int) -> None:
        from pyasc_amd import kernels
        x, out = self.sets[i % len(self.sets)]
        kernels.rms_norm(x, self.gamma, out, self.rows, self.cols, 1e-6)

    def work(self) -> float:
        return 8.0 * self.rows * self.cols + 4.0 * self.cols

    def config(self) -> dict:
        return {"workload": self.name, "rows": self.rows, "cols": self.cols, "epsilon": 1e-6,
                "input": "randn*2 fp32, gamma rand+0.5", "rotating_sets": len(self.sets)}

    def cpu_baseline(self, min_total_s: float = CPU_MIN_S):
        import torch
        g = torch.Generator().manual_seed(1)
        x = torch.randn(self.rows, self.cols, generator=g) * 2.0
        gamma = torch.rand(self.cols, generator=g) + 0.5
        return _cpu(self.work(), 1e9, "GB/s", "torch.nn.functional.rms_norm(x, [C], gamma, 1e-6)",
                    f"the full {self.rows}x{self.cols} workload",
                    _time_cpu(lambda: torch.nn.functional.rms_norm(x, [self.cols], gamma, eps=1e-6), min_total_s))


class ReduceRows(Workload):
    """asc2.reduce_sum along dim 1 (test_reduce_ops.py's kernel) at a bandwidth size."""
    bound, unit, dtype, kernel_hint = "hbm", "GB/s", "f32", "reduce_rows"
    sources = ("reduce.hip", "rows.h", "numeric.h", "common.h")

    def __init__(self, rows: int, cols: int):
        self.rows, self.cols = rows, cols
        self.name = f"reduce_sum_dim1_{rows}x{cols}_f32"

    def setup(self, dev):
        import torch
        g = torch.Generator(device=dev).manual_seed(1)
        self.sets = [(torch.randn(self.rows, self.cols, device=dev, generator=g) * 2.0,
                      torch.empty(self.rows, device=dev)) for _ in range(_sets_for(4 * self.rows * self.cols))]

    def launch(self, i: int) -> None:
        from pyasc_amd import kernels
        x, out = self.sets[i % len(self.sets)]
        kernels.reduce_f32(x, out, "sum", 1)

    def work(self) -> float:
        return 4.0 * self.rows * self.cols + 4.0 * self.rows

    def config(self) -> dict:
        return {"workload": self.name, "rows": self.rows, "cols": self.cols, "op": "sum", "dim": 1,
                "input": "randn*2 fp32", "rotating_sets": len(self.sets)}

    def cpu_baseline(self, min_total_s: float = CPU_MIN_S):
        import torch
        x = torch.randn(self.rows, self.cols, generator=torch.Generator().manual_seed(1)) * 2.0
        return _cpu(self.work(), 1e9, "GB/s", "torch.sum(x, 1) (test_reduce_ops.py golden)",
                    f"the full {self.rows}x{self.cols} workload", _time_cpu(lambda: torch.sum(x, 1), min_total_s))


class Matmul(Workload):
    bound, unit, kernel_hint = "mfma", "TFLOP/s", "mm_mfma"
    sources = ("matmul.hip", "matmul_kernels.h", "gemm_direct.h", "gemm_core.h", "gemm_common.h", "numeric.h",
               "common.h")

    def __init__(self, n: int, dtype: str, bias_leaky: bool = False):
        self.n, self.dt, self.bias_leaky = n, dtype, bias_leaky
        self.dtype = {"bfloat16": "bf16", "float16": "f16"}[dtype]
        self.peak = BF16_PEAK_TFLOPS if dtype == "bfloat16" else FP16_PEAK_TFLOPS
        # the 05_matmul_leakyrelu tutorial's epilogue: fp32 C = leaky_relu(A B + bias, 0.001)
        self.name = f"matmul_{n}x{n}x{n}_{self.dtype}" + ("_bias_leakyrelu_f32out" if bias_leaky else "")

    def setup(self, dev):
        import torch
        td = getattr(torch, self.dt)
        g = torch.Generator(device=dev).manual_seed(2)
        c_bytes = 4 if self.bias_leaky else 2
        self.sets = []
        for _ in range(_sets_for(self.n * self.n * (4 + c_bytes))):
            a = (torch.randn(self.n, self.n, device=dev, generator=g) / math.sqrt(self.n)).to(td)
            b = (torch.randn(self.n, self.n, device=dev, generator=g) / math.sqrt(self.n)).to(td)
            c = torch.empty(self.n, self.n, device=dev, dtype=torch.float32 if self.bias_leaky else td)
            self.sets.append((a, b, c))
        self.bias = torch.randn(self.n, device=dev, generator=g) if self.bias_leaky else None

    def launch(self, i: int) -> None:
        from pyasc_amd import kernels
        a, b, c = self.sets[i % len(self.sets)]
        if self.bias_leaky:
            kernels.matmul(a, b, c, bias=self.bias, leaky_alpha=0.001)
        else:
            kernels.matmul(a, b, c)

    def work(self) -> float:
        return 2.0 * self.n ** 3

    @property
    def vendor_expression(self):
        # the plain product only: torch has no fused bias + leaky-relu GEMM
        return None if self.bias_leaky else "torch.matmul(a, b, out=c) (hipBLASLt)"

    def vendor_launch(self, i: int) -> None:
        import torch
        a, b, c = self.sets[i % len(self.sets)]
        torch.matmul(a, b, out=c)

    def config(self) -> dict:
        cfg = {"workload": self.name, "M": self.n, "N": self.n, "K": self.n, "layout": "A row-major, B row-major",
               "input": "randn/sqrt(K), seed 2", "accumulate": "fp32", "out": self.dtype,
               "rotating_sets": len(self.sets)}
        if self.bias_leaky:
            cfg.update({"out": "f32", "epilogue": "leaky_relu(acc + bias[n], 0.001)"})
        return cfg

    def cpu_baseline(self, min_total_s: float = CPU_MIN_S):
        import torch
        from oracle import cpu_golden
        td = getattr(torch, self.dt)
        g = torch.Generator().manual_seed(2)
        a = (torch.randn(self.n, self.n, generator=g) / math.sqrt(self.n)).to(td)
        b = (torch.randn(self.n, self.n, generator=g) / math.sqrt(self.n)).to(td)
        if self.bias_leaky:
            bias = torch.randn(self.n, generator=g)

            def run():
                r = cpu_golden.matmul(a, b) + bias
                return torch.where(r >= 0, r, r * 0.001)
            expr = "leaky_relu(a.float() @ b.float() + bias, 0.001) (05_matmul_leakyrelu golden)"
        else:
            def run():
                return cpu_golden.matmul(a, b)
            expr = "a.to(float32) @ b.to(float32) (python/test/asc2/kernels/test_matmul_tiled.py:49)"
        return _cpu(self.work(), 1e12, "TFLOP/s", expr, f"the full {self.n}^3 workload", _time_cpu(run, min_total_s))


class MatmulI8(Workload):
    bound, unit, dtype, kernel_hint = "mfma", "TOPS", "int8", "gemm_i8"
    peak = INT8_PEAK_TOPS
    sources = ("matmul_i8.hip", "matmul_i8_kernels.h", "gemm_direct.h", "gemm_core.h", "gemm_common.h", "numeric.h",
               "common.h")

    def __init__(self, M: int, N: int, K: int):
        self.M, self.N, self.K = M, N, K
        self.name = f"matmul_i8_dequant_{M}x{N}x{K}"

    def setup(self, dev):
        import torch
        g = torch.Generator(device=dev).manual_seed(3)
        self.sets = []
        for _ in range(_sets_for(self.M * self.K + self.K * self.N + 2 * self.M * self.N)):
            a = torch.randint(-127, 128, (self.M, self.K), dtype=torch.int8, device=dev, generator=g)
            b = torch.randint(-127, 128, (self.K, self.N), dtype=torch.int8, device=dev, generator=g)
            s = torch.rand(self.N, device=dev, generator=g) * 0.009 + 0.001
            c = torch.empty(self.M, self.N, dtype=torch.float16, device=dev)
            self.sets.append((a, b, s, c))

    def launch(self, i: int) -> None:
        from pyasc_amd import kernels
        a, b, s, c = self.sets[i % len(self.sets)]
        kernels.matmul_i8(a, b, c, scale=s)

    def work(self) -> float:
        return 2.0 * self.M * self.N * self.K

    # int8 GEMM with int32 output and no dequant: less epilogue work than this kernel's
    vendor_expression = "torch._int_mm(a, b) (hipBLASLt int8, int32 C, no dequant)"

    def vendor_launch(self, i: int) -> None:
        import torch
        a, b, _, _ = self.sets[i % len(self.sets)]
        torch._int_mm(a, b)

    def config(self) -> dict:
        return {"workload": self.name, "M": self.M, "N": self.N, "K": self.K, "accumulate": "int32 (exact)",
                "epilogue": "fp16(fp32(acc) * scale[n])", "input": "int8 uniform[-127,127], seed 3",
                "rotating_sets": len(self.sets)}

    def cpu_baseline(self, min_total_s: float = CPU_MIN_S):
        import torch
        from oracle import cpu_golden
        g = torch.Generator().manual_seed(3)
        a = torch.randint(-127, 128, (self.M, self.K), dtype=torch.int8, generator=g)
        b = torch.randint(-127, 128, (self.K, self.N), dtype=torch.int8, generator=g)
        scale = torch.rand(self.N, generator=g) * 0.009 + 0.001
        # torch's int32 CPU product runs at some 20-40 GOPS: a quarter of A's rows keeps the
        # sample to a few seconds; the rate is per operation, so it scales to the full shape
        rows = min(self.M, 1024)
        a = a[:rows].contiguous()
        return _cpu(2.0 * rows * self.N * self.K, 1e12, "TOPS",
                    "(a.to(int32) @ b.to(int32)) then (acc.float() * scale).half() "
                    "(test_matmul_iterate_all.py:116; dequant of test_matmul_quant.py)",
                    f"the first {rows} of {self.M} rows of A ({rows}x{self.N}x{self.K}), same B and scale",
                    _time_cpu(lambda: cpu_golden.dequant(cpu_golden.matmul_i8(a, b), scale), min_total_s))


class FlashAttention(Workload):
    bound, unit, dtype, kernel_hint = "mfma", "TFLOP/s", "bf16", "fa_fwd"
    peak = BF16_PEAK_TFLOPS
    sources = ("flash_attn.hip", "flash_attn_kernels.h", "numeric.h", "common.h")

    def __init__(self, B: int, H: int, S: int, D: int, causal: bool):
        self.B, self.H, self.S, self.D, self.causal = B, H, S, D, causal
        self.name = f"flash_attn_fwd_b{B}h{H}s{S}d{D}_{'causal' if causal else 'noncausal'}"

    def setup(self, dev):
        import torch
        g = torch.Generator(device=dev).manual_seed(4)
        shape = (self.B, self.H, self.S, self.D)
        self.sets = []
        for _ in range(_sets_for(4 * 2 * self.B * self.H * self.S * self.D)):
            q, k, v = [torch.randn(*shape, device=dev, generator=g).to(torch.bfloat16) for _ in range(3)]
            self.sets.append((q, k, v, torch.empty_like(q)))

    def launch(self, i: int) -> None:
        from pyasc_amd import kernels
        q, k, v, o = self.sets[i % len(self.sets)]
        kernels.flash_attention_fwd(q, k, v, o, 1 / math.sqrt(self.D), self.causal)

    vendor_expression = "torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=causal) (ROCm SDPA)"

    def vendor_launch(self, i: int) -> None:
        import torch
        q, k, v, _ = self.sets[i % len(self.sets)]
        torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=self.causal)

    def work(self) -> float:
        full = 4.0 * self.B * self.H * self.S * self.S * self.D
        return full / 2 if self.causal else full  # causal counted as half of the dense work

    def config(self) -> dict:
        return {"workload": self.name, "batch": self.B, "heads": self.H, "seq_len": self.S, "head_dim": self.D,
                "causal": self.causal, "sm_scale": 1 / math.sqrt(self.D), "input": "bf16 randn, seed 4",
                "flop_convention": "4*B*H*S^2*D, halved for causal", "rotating_sets": len(self.sets)}

    def cpu_baseline(self, min_total_s: float = CPU_MIN_S):
        import torch
        from oracle import cpu_golden
        g = torch.Generator().manual_seed(4)
        shape = (self.B * self.H, self.S, self.D)
        q, k, v = [torch.randn(*shape, generator=g).to(torch.bfloat16) for _ in range(3)]
        scale = 1 / math.sqrt(self.D)

        def run():
            for i in range(shape[0]):
                cpu_golden.attention(q[i], k[i], v[i], scale, self.causal)

        return _cpu(self.work(), 1e12, "TFLOP/s",
                    "fp32 softmax((q @ k.T) * scale [+ causal mask]) @ v per (batch, head) slice",
                    f"the full workload, {shape[0]} (batch, head) slices of S={self.S}, D={self.D}, "
                    "same FLOP convention", _time_cpu(run, min_total_s))


WORKLOADS = {
    "softmax_4096x4096": lambda: Softmax(4096, 4096),
    "softmax_16384x1024": lambda: Softmax(16384, 1024),
    "asc2_vadd_8192": Asc2VaddPlumbing,
    "vadd_268435456": lambda: Vadd(1 << 28),
    "copy_128MiB": lambda: Copy(64 << 20, "128MiB"),
    "copy_3GiB": lambda: Copy(3 << 29, "3GiB"),
    "matmul_bf16_8192": lambda: Matmul(8192, "bfloat16"),
    "matmul_f16_8192": lambda: Matmul(8192, "float16"),
    "matmul_f16_8192_bias_leakyrelu": lambda: Matmul(8192, "float16", bias_leaky=True),
    "matmul_i8_4096x11008x4096": lambda: MatmulI8(4096, 11008, 4096),
    "fa_fwd_noncausal": lambda: FlashAttention(4, 32, 4096, 128, False),
    "fa_fwd_causal": lambda: FlashAttention(4, 32, 4096, 128, True),
    "leaky_relu_268435456": lambda: LeakyRelu(1 << 28),
    "vmuladd_268435456": lambda: VMulAdd(1 << 28),
    "gelu_tanh_16384x1024": lambda: Gelu(16384, 1024, True),
    "gelu_erf_16384x1024": lambda: Gelu(16384, 1024, False),
    "rms_norm_4096x4096": lambda: RmsNorm(4096, 4096),
    "reduce_sum_dim1_16384x4096": lambda: ReduceRows(16384, 4096),
}
HEADLINE = "softmax_4096x4096"
SUITE = ["asc2_vadd_8192", "softmax_16384x1024", "copy_128MiB", "vadd_268435456", "copy_3GiB", "matmul_bf16_8192",
         "matmul_f16_8192", "matmul_i8_4096x11008x4096", "matmul_f16_8192_bias_leakyrelu", "fa_fwd_noncausal",
         "fa_fwd_causal", "leaky_relu_268435456", "vmuladd_268435456", "gelu_tanh_16384x1024",
         "gelu_erf_16384x1024", "rms_norm_4096x4096", "reduce_sum_dim1_16384x4096"]


class PowerSampler:
    """Samples the board's socket power and the graphics clock with ``amd-smi metric -p -c``
    in a background thread (each call takes about 0.4 s) from ``start()`` to ``stop()``.
    ``summary()`` drops the first ``skip`` samples (the clock ramps up as the launches
    begin) and reports the median, minimum and maximum of the rest; the clock is the mean
    over the XCDs' GFX_n domains of one sample."""

    def __init__(self, skip: int = 2):
        import threading
        self.skip = skip
        self.samples = []  # (seconds since start, watts, MHz)
        self._stop = threading.Event()
        self._thread = threading.Thread(target=self._run, daemon=True)
        self._t0 = 0.0

    @staticmethod
    def parse(text: str):
        watts, mhz, in_gfx = None, [], False
        for line in text.splitlines():
            s = line.strip()
            if s.startswith("SOCKET_POWER:"):
                try:
                    watts = float(s.split()[1])
                except (IndexError, ValueError):
                    pass
            elif s.startswith("GFX_") and s.endswith(":"):
                in_gfx = True
            elif s.endswith(":") and not s.startswith("GFX_"):
                in_gfx = False
            elif in_gfx and s.startswith("CLK:"):
                try:
                    mhz.append(float(s.split()[1]))
                except (IndexError, ValueError):
                    pass
        return watts, (sum(mhz) / len(mhz) if mhz else None)

    def _run(self):
        import subprocess
        while not self._stop.is_set():
            try:
                out = subprocess.run(["amd-smi", "metric", "-p", "-c", "-g", "0"], capture_output=True, text=True,
                                     timeout=10).stdout
            except (OSError, subprocess.SubprocessError):
                return
            watts, mhz = self.parse(out)
            if watts is not None and mhz is not None:
                self.samples.append((time.perf_counter() - self._t0, watts, mhz))
            self._stop.wait(0.2)

    def start(self):
        self._t0 = time.perf_counter()
        self._thread.start()

    def stop(self):
        self._stop.set()
        self._thread.join(timeout=15)

    def summary(self) -> dict:
        kept = self.samples[self.skip:]
        if not kept:
            return {"samples": 0, "note": "amd-smi gave no reading (run a longer --warmup)"}

        def med(v):
            v = sorted(v)
            return v[len(v) // 2]
        w = [s[1] for s in kept]
        c = [s[2] for s in kept]
        return {"samples": len(kept), "seconds": round(kept[-1][0] - kept[0][0], 2),
                "socket_w_median": med(w), "socket_w_min": min(w), "socket_w_max": max(w),
                "gfx_mhz_median": round(med(c)), "gfx_mhz_min": round(min(c)), "gfx_mhz_max": round(max(c)),
                "source": "amd-smi metric -p -c -g 0 (SOCKET_POWER; mean of the GFX_n CLK readings)"}


def _median(v):
    v = sorted(v)
    n = len(v)
    return v[n // 2] if n % 2 else 0.5 * (v[n // 2 - 1] + v[n // 2])


def measure(w: Workload, steps: int, warmup: int, dev, graph: bool = True, sampler: PowerSampler = None,
            warmup_s: float = WARMUP_S, replays: int = REPLAYS) -> dict:
    """Times ``steps`` launches on the launch stream with HIP events, ``replays`` times.

    Warm-up: ``warmup`` eager launches, then the timed launches themselves (captured once
    into a HIP graph) replayed back to back until at least ``warmup_s`` seconds have
    passed, so the clocks and caches are in the state the timed replays run in.
    Timed region: ``replays`` graph replays, each of exactly ``steps`` launches and each
    between its own pair of events recorded on the replay stream, issued without a host
    synchronisation in between (the device stays busy); ``kernel_ms`` is the median replay
    time / ``steps``, with the fastest and slowest replay beside it.  ``graph=False`` times
    each launch with its own event pair instead and reports the median launch."""
    import torch
    w.setup(dev)
    if sampler is not None:
        sampler.start()
    for i in range(warmup):
        w.launch(i)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    warm_launches = warmup
    if graph:
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(stream)
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                for i in range(steps):
                    w.launch(warmup + i)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        while True:  # the first replay also uploads the graph
            g.replay()
            torch.cuda.synchronize()
            warm_launches += steps
            if time.perf_counter() - t0 >= warmup_s:
                break
        warm_seconds = time.perf_counter() - t0
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(replays)]
        for a, b in ev:
            a.record(stream)
            g.replay()
            b.record(stream)
        torch.cuda.synchronize()
        per_step = [a.elapsed_time(b) / steps for a, b in ev]
        del g
    else:
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < warmup_s:
            for i in range(steps):
                w.launch(warmup + i)
            torch.cuda.synchronize()
            warm_launches += steps
        warm_seconds = time.perf_counter() - t0
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        for i in range(steps):
            ev[i][0].record(stream)
            w.launch(warmup + i)
            ev[i][1].record(stream)
        torch.cuda.synchronize()
        per_step = [a.elapsed_time(b) for a, b in ev]
    if sampler is not None:
        sampler.stop()
    kernel_ms = _median(per_step)
    value = w.value(kernel_ms / 1e3)
    return {"workload": w.name, "ms_per_step": kernel_ms, "kernel_ms": kernel_ms, "ms_min": min(per_step),
            "ms_max": max(per_step), "value": value, "unit": w.unit, "rate": w.rate(kernel_ms / 1e3),
            "bound": w.bound, "config": w.config(), "replays": len(per_step) if graph else 0,
            "warmup_launches": warm_launches, "warmup_s": round(warm_seconds, 2),
            "timing": (f"median of {replays} hip-graph replays of {steps} launches" if graph
                       else f"median of {steps} per-launch event pairs")}


def vendor(w: Workload, steps: int, res: dict):
    """The workload's operation through torch's ROCm library kernel on the same inputs
    (after ``measure``, which set them up), timed with one event pair per launch; None
    when there is no library equivalent.  ``this_over_vendor`` = this build's rate / the
    library's."""
    if w.vendor_expression is None:
        return None
    import torch
    try:
        for i in range(3):
            w.vendor_launch(i)
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        for i in range(steps):
            ev[i][0].record(stream)
            w.vendor_launch(3 + i)
            ev[i][1].record(stream)
        torch.cuda.synchronize()
    except RuntimeError as e:  # the library refuses the shape or dtype
        return {"expression": w.vendor_expression, "error": str(e).splitlines()[0][:200]}
    ms = sum(a.elapsed_time(b) for a, b in ev) / steps
    value = w.value(ms / 1e3)
    return {"value": round(value, 3), "unit": w.unit, "ms_per_launch": ms, "expression": w.vendor_expression,
            "timing": "per-launch events", "this_over_vendor": round(res["value"] / value, 3)}


def roofline(w: Workload, res: dict) -> dict:
    """The roofline object of one workload: achieved algorithmic rate against the MI355X peak."""
    if w.bound == "latency":
        return {"bound": "latency", "achieved": round(res["rate"], 3), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(res["rate"] / HBM_PEAK_GBS, 6), "traffic": traffic_for(w),
                "note": "launch-latency-bound: the HBM fraction is not a target here"}
    return {"bound": w.bound, "achieved": round(res["value"], 3), "peak": w.peak, "unit": w.unit,
            "frac": round(res["value"] / w.peak, 4), "traffic": traffic_for(w)}


POWER_WORKLOADS = ["softmax_4096x4096", "matmul_bf16_8192", "matmul_i8_4096x11008x4096", "fa_fwd_noncausal",
                   "fa_fwd_causal"]
POWER_SECONDS = 3.0


def power_phase(dev, keys, steps: int) -> dict:
    """Socket power and graphics clock while each of ``keys`` (of POWER_WORKLOADS) is
    measured again with POWER_SECONDS of warm-up, sampled with PowerSampler.  For an MFMA
    workload the entry also gives the dense peak at the sampled clock (peak x MHz / 2400)
    and the fraction of it this run reached: the MFMA kernels hold the board at its power
    limit, which sets the clock."""
    import torch
    out = {}
    for key in keys:
        w = WORKLOADS[key]()
        sampler = PowerSampler()
        r = measure(w, steps, 10, dev, sampler=sampler, warmup_s=POWER_SECONDS)
        entry = {"value": round(r["value"], 3), "unit": w.unit, "warmup_s": r["warmup_s"], **sampler.summary()}
        mhz = entry.get("gfx_mhz_median")
        if mhz and w.bound == "mfma":
            peak = w.peak * mhz / 2400.0
            entry["dense_peak_at_clock"] = round(peak, 1)
            entry["frac_at_clock"] = round(r["value"] / peak, 4)
        out[key] = entry
        print(f"bench: power {w.name} {r['value']:.1f} {w.unit}, {entry.get('socket_w_median')} W, "
              f"{mhz} MHz", file=sys.stderr, flush=True)
        del w
        torch.cuda.empty_cache()
    return out


def launch_latency(dev, n: int = 2000) -> dict:
    """Host time per launch of the reference-size vadd (8192 fp32, grid 16, tile 128,
    tpb 4; test_vadd.py:31-38) on device tensors, through the asc2 surface with the
    kernel cache, with always_compile=True (re-resolved every call), and through the
    kernel API.  Wall time over ``n`` back-to-back launches / n: the GPU work (a few
    microseconds) overlaps the host work, so this is the host-side launch cost."""
    import torch
    import pyasc_amd
    from pyasc_amd import kernels
    pyasc_amd.install_aliases()
    import asc
    import asc2

    def make(**options):
        @asc2.jit(**options)
        def vadd_kernel(x_ptr: asc.GlobalAddress, y_ptr: asc.GlobalAddress, out_ptr: asc.GlobalAddress, size: int,
                        tile_size: asc.ConstExpr[int], tile_per_block: asc.ConstExpr[int]):
            ...  # declaration: binds the registered native kernel by signature

        return vadd_kernel

    x, y = torch.rand(8192, device=dev), torch.rand(8192, device=dev)
    out = torch.empty(8192, device=dev)

    def per_launch(fn) -> float:
        for _ in range(50):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n * 1e6

    cached, fresh = make(), make(always_compile=True)
    res = {
        "workload": "vadd 8192 fp32, grid 16, tile 128, tpb 4, device tensors",
        "asc2_cached_us": per_launch(lambda: cached[16](x, y, out, 8192, 128, 4)),
        "asc2_always_compile_us": per_launch(lambda: fresh[16](x, y, out, 8192, 128, 4)),
        "kernel_api_us": per_launch(lambda: kernels.vadd(x, y, out, 8192, 128, 4, 16)),
    }
    assert torch.equal(out, x + y)
    return {k: (round(v, 2) if isinstance(v, float) else v) for k, v in res.items()}


def reference_durations(dev, steps: int = 200) -> dict:
    """The reference's only published timings are NPU task durations of two asc1 kernels
    (test/all_task_durations_golden.csv: python/test/kernels/test_vadd.py at 8192 fp32 on 16
    cores, 3.6 us; python/test/kernels/test_matmul.py, 256^3 fp32 + bias + leaky relu, 25.5 us).
    Here the same kernels run through the same launch surface on device-resident tensors;
    ``steps`` launches are captured into a HIP graph and one replay is timed, so each figure
    is the per-launch device time including the dispatch gap between back-to-back kernels."""
    import numpy as np
    import torch
    import pyasc_amd
    pyasc_amd.install_aliases()
    import asc

    @asc.jit
    def vadd_kernel(x: asc.GlobalAddress, y: asc.GlobalAddress, z: asc.GlobalAddress,
                    BLOCK_LENGTH: asc.ConstExpr[int], BUFFER_NUM: asc.ConstExpr[int],
                    TILE_LENGTH: asc.ConstExpr[int], TILE_NUM: asc.ConstExpr[int]):
        ...  # declaration: binds the registered native kernel by signature

    @asc.jit
    def matmul_kernel(a: asc.GlobalAddress, b: asc.GlobalAddress, c: asc.GlobalAddress, alpha: float,
                      tiling: asc.adv.TCubeTiling, bias: asc.GlobalAddress, workspace: asc.GlobalAddress):
        ...  # declaration: binds the registered native kernel by signature

    rng = np.random.default_rng(seed=2025)
    x, y = (torch.from_numpy(rng.random(8192, dtype=np.float32)).to(dev) for _ in range(2))
    z = torch.zeros_like(x)
    m = k = n = 256
    a, b = (torch.from_numpy((rng.random((m, k), dtype=np.float32) - .5) * 10).to(dev) for _ in range(2))
    bias = torch.from_numpy((rng.random((1, n), dtype=np.float32) - .5) * 10).to(dev)
    c = torch.empty(m, n, device=dev)
    tiling = asc.adv.TCubeTiling(used_core_num=16, m=m, k_a=k, k_b=k, n=n, base_m=64, base_k=64, base_n=64,
                                 single_core_m=64, single_core_k=k, single_core_n=64, depth_a1=1, depth_b1=1,
                                 step_m=1, step_n=1, share_mode=0, is_bias=1)
    workspace = torch.zeros(16 << 20, dtype=torch.uint8, device=dev)
    cases = {
        "asc1_vadd_8192_f32": (lambda: vadd_kernel[16](x, y, z, 512, 1, 64, 8), 3.6,
                               "python/test/kernels/test_vadd.py: 8192 fp32, 16 cores, TILE_NUM 8, BUFFER_NUM 1"),
        "asc1_matmul_256_f32_bias_leakyrelu": (
            lambda: matmul_kernel[16](a, b, c, 0.01, tiling, bias, workspace), 25.5,
            "python/test/kernels/test_matmul.py: 256x256x256 fp32, bias, leaky relu 0.01, 16 cores"),
    }
    out = {}
    for name, (fn, ref_us, what) in cases.items():
        for _ in range(20):
            fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                for _ in range(steps):
                    fn()
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / steps
        out[name] = {"us_per_launch": round(us, 2), "reference_task_duration_us": ref_us,
                     "reference_over_this": round(ref_us / us, 2), "kernel": what,
                     "reference_source": "test/all_task_durations_golden.csv (Ascend NPU, model unstated)"}
        del g
    ref = a.cpu() @ b.cpu() + bias.cpu()
    assert torch.equal(z, x + y) and torch.allclose(c.cpu(), torch.where(ref >= 0, ref, ref * 0.01), atol=1e-3)
    return out


TRAFFIC_FILE = os.path.join(REPO, "profiles", "traffic.json")


def traffic_for(w: Workload):
    """HBM bytes per launch measured for ``w`` (profiles/traffic.json), or None when no
    measurement exists or the kernel sources changed since it was taken."""
    try:
        with open(TRAFFIC_FILE) as f:
            entry = json.load(f).get("workloads", {}).get(w.name)
    except (OSError, ValueError):
        return None
    if not entry or entry.get("sources_hash") != sources_hash(w.sources):
        return None
    return entry.get("bytes")


def _sig(x, digits: int = 4):
    """``x`` rounded to ``digits`` significant digits (None stays None)."""
    if x is None or x == 0:
        return x
    return round(x, max(0, digits - 1 - int(math.floor(math.log10(abs(x))))))


def compact_roofline(r: dict) -> dict:
    return {"frac": r["frac"], "achieved": _sig(r["achieved"], 5), "traffic": r.get("traffic")}


def compact_cpu(c):
    if not c:
        return None
    return {"value": _sig(c["value"], 4), "unit": c["unit"], "cores": c["cores"],
            "seconds_per_call": _sig(c["seconds_per_call"], 4)}


def compact_entry(res: dict, roof: dict, cpu) -> dict:
    """One suite entry of the stdout line."""
    return {"value": _sig(res["value"], 5), "unit": res["unit"], "ms_per_step": _sig(res["ms_per_step"], 5),
            "ms_min": _sig(res["ms_min"], 5), "ms_max": _sig(res["ms_max"], 5),
            "roofline": compact_roofline(roof), "cpu_baseline": compact_cpu(cpu),
            **({"vs_vendor": res["vendor"]["this_over_vendor"]} if (res.get("vendor") or {}).get("value") else {})}


def build_line(args, head, res: dict, cpu, suite: dict, extra: dict) -> dict:
    """The ONE stdout line: the headline's figures, roofline and CPU baseline in full, and
    for every suite workload its value, median/min/max time per step, roofline fraction,
    achieved rate and traffic, and CPU baseline (``suite``: key -> compact_entry).  The
    host block appears once.  ``extra`` holds short summaries (power, launch latency, the
    reference's published durations)."""
    roof = roofline(head, res)
    head_cpu = None
    if cpu:
        head_cpu = {"value": _sig(cpu["value"], 5), "unit": cpu["unit"], "cores": cpu["cores"], "kind": cpu["kind"],
                    "sample": cpu["sample"], "expression": cpu["expression"],
                    "seconds_per_call": _sig(cpu["seconds_per_call"], 5)}
    line = {
        "metric": METRIC,
        "value": round(res["value"], 3),
        "unit": head.unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": res["ms_per_step"],
        "higher_is_better": head.bound != "latency",
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": head.dtype,
        "data": "synthetic (seeded torch generator on the device; distribution of BASELINE.json's config)",
        "config": {k: v for k, v in res["config"].items() if k != "input"},
        "roofline": roof,
        "cpu_baseline": head_cpu,
        "timing": {"method": res["timing"], "ms_min": _sig(res["ms_min"], 5), "ms_max": _sig(res["ms_max"], 5),
                   "warmup_s": res["warmup_s"], "warmup_launches": res["warmup_launches"],
                   "cpu_after_gpu": True},
        "host": host_info() if cpu or any(e.get("cpu_baseline") for e in suite.values()) else None,
        "suite": suite,
    }
    line.update(extra)
    return line


def serialize_line(line: dict) -> str:
    """The line as compact JSON below LINE_LIMIT bytes: should it be longer, the optional
    summaries go first, then the suite's CPU baselines (both stay in --detail)."""
    text = json.dumps(line, separators=(",", ":"))
    for trim in ("power", "launch_latency_us", "reference_published_us", "suite_cpu"):
        if len(text) < LINE_LIMIT:
            break
        if trim == "suite_cpu":
            for e in line["suite"].values():
                e.pop("cpu_baseline", None)
        else:
            line.pop(trim, None)
        print(f"bench: line over {LINE_LIMIT} bytes; dropped {trim}", file=sys.stderr, flush=True)
        text = json.dumps(line, separators=(",", ":"))
    return text


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default=HEADLINE, choices=sorted(WORKLOADS))
    ap.add_argument("--no-suite", action="store_true")
    ap.add_argument("--no-cpu", action="store_true", help="skip every CPU baseline")
    ap.add_argument("--no-graph", action="store_true", help="time with per-launch event pairs, no HIP graph")
    ap.add_argument("--no-vendor", action="store_true", help="skip the ROCm library comparisons")
    ap.add_argument("--cpu-all", action="store_true", help=argparse.SUPPRESS)  # the default now
    ap.add_argument("--no-power", action="store_true",
                    help="skip the power phase (with the suite: socket power and graphics clock sampled with "
                         "amd-smi during about 3 s of launches of the headline and of each MFMA workload)")
    ap.add_argument("--warmup-s", type=float, default=WARMUP_S,
                    help="least seconds of warm-up replays per workload (default %(default)s; 0 for profiler runs)")
    ap.add_argument("--detail", metavar="FILE",
                    help="also write every figure in full (configs, CPU samples, vendor comparisons, power "
                         "readings, launch latency) to FILE as JSON")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run torch's device copy of 256 MiB 5 times (the known-size kernel that scales "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); every kernel here runs on a single "
              "MI355X and no multi-GPU figure is produced.", file=sys.stderr)
        return 2

    import torch
    from pyasc_amd import _native
    if not torch.cuda.is_available():
        print("bench.py needs the MI355X (no HIP device visible)", file=sys.stderr)
        return 1
    _native.load_library()
    dev = torch.device("cuda", 0)

    # GPU legs first, back to back: the headline, the suite, the power phase, launch costs
    head = WORKLOADS[args.workload]()
    res = measure(head, args.steps, args.warmup, dev, graph=not args.no_graph, warmup_s=args.warmup_s)
    head_vendor = None if args.no_vendor else vendor(head, args.steps, res)
    print(f"bench: {head.name} {res['value']:.2f} {head.unit} (replays {res['ms_min'] * 1e3:.2f}-"
          f"{res['ms_max'] * 1e3:.2f} us/step)", file=sys.stderr, flush=True)
    del head
    torch.cuda.empty_cache()
    head = WORKLOADS[args.workload]()
    suite_res = {}
    keys = [] if args.no_suite else [k for k in SUITE if k != args.workload]
    for key in keys:
        w = WORKLOADS[key]()
        r = measure(w, args.steps, args.warmup, dev, graph=not args.no_graph, warmup_s=args.warmup_s,
                    replays=REPLAYS if w.bound != "latency" else 3 * REPLAYS)
        r["roofline"] = roofline(w, r)
        r["vendor"] = None if args.no_vendor else vendor(w, args.steps, r)
        suite_res[key] = r
        v = r["vendor"]
        print(f"bench: {w.name} {r['value']:.2f} {w.unit} [{r['ms_min'] * 1e3:.2f}-{r['ms_max'] * 1e3:.2f} us]" +
              (f" (vendor {v['value']:.2f})" if v and "value" in v else ""), file=sys.stderr, flush=True)
        del w
        torch.cuda.empty_cache()
    latency = published = power = None
    if not args.no_suite:
        latency = launch_latency(dev)
        published = reference_durations(dev)
        if not args.no_power:
            power = power_phase(dev, [k for k in POWER_WORKLOADS if k == args.workload or k in suite_res],
                                args.steps)
    if args.copy_calibration:
        src = torch.empty((256 << 20) // 4, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    torch.cuda.synchronize()

    # CPU baselines after every GPU leg (they leave the GPU idle)
    cpu = None
    cpu_suite = {}
    if not args.no_cpu:
        cpu = head.cpu_baseline(CPU_HEADLINE_S)
        print(f"bench: cpu {head.name} {cpu['value']:.4g} {cpu['unit']}", file=sys.stderr, flush=True)
        for key in suite_res:
            c = WORKLOADS[key]().cpu_baseline()
            cpu_suite[key] = c
            print(f"bench: cpu {key} {c['value']:.4g} {c['unit']}", file=sys.stderr, flush=True)

    suite = {k: compact_entry(r, r["roofline"], cpu_suite.get(k)) for k, r in suite_res.items()}
    extra = {}
    if power:
        extra["power"] = {k: {"value": _sig(p["value"], 5), "w": p.get("socket_w_median"),
                              "mhz": p.get("gfx_mhz_median"), "frac_at_clock": p.get("frac_at_clock")}
                          for k, p in power.items()}
    if latency:
        extra["launch_latency_us"] = {"asc2": latency["asc2_cached_us"],
                                      "asc2_always_compile": latency["asc2_always_compile_us"],
                                      "kernel_api": latency["kernel_api_us"]}
    if published:
        extra["reference_published_us"] = {k: [v["us_per_launch"], v["reference_task_duration_us"]]
                                           for k, v in published.items()}
    line = build_line(args, head, res, cpu, suite, extra)
    text = serialize_line(line)
    if args.detail:
        detail = {"line": line, "headline": {**res, "vendor": head_vendor, "cpu_baseline": cpu},
                  "suite": {k: {**r, "cpu_baseline": cpu_suite.get(k)} for k, r in suite_res.items()},
                  "power": power, "launch_latency": latency, "reference_published": published,
                  "device": _native.device_info(0), "host": host_info()}
        os.makedirs(os.path.dirname(os.path.abspath(args.detail)), exist_ok=True)
        with open(args.detail, "w") as f:
            json.dump(detail, f, indent=1, default=str)
    print(text, flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
