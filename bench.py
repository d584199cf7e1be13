"""Benchmark of the asc2 hot-path kernels on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--no-suite] [--no-cpu]

A "step" is one launch of the headline kernel over one batch of synthetic,
device-resident input.  The headline workload is BASELINE.json's configs[1],
row softmax of a 4096x4096 fp32 matrix (HBM-bound; metric HBM GB/s).  The
other configurations (vadd bandwidth shape, softmax 16384x1024, bf16/fp16
matmul 8192^3, int8 matmul 4096x11008x4096 + dequant, flash-attention forward)
are measured the same way and reported under "suite".

Timing: W untimed warm-up steps, then exactly K steps bracketed by
torch.cuda.synchronize().  The K launches are captured into one HIP graph and
one replay is timed with HIP events on the replay stream (the kernels run back
to back, without host launch overhead); --no-graph times each launch with its
own event pair instead.  HBM-bound workloads rotate
through enough input/output sets (> 512 MiB) that the 256 MiB Infinity Cache
cannot serve them.  The CPU baseline is the reference test's torch CPU golden
expression (oracle/cpu_golden.py), timed on the host cores on a bounded sample.

Prints ONE JSON line.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
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
COPY_BYTES = 256 << 20    # calibration copy: reads and writes exactly this many bytes


class Workload:
    """One benchmarked kernel configuration."""
    name = ""
    bound = "hbm"       # "hbm" | "mfma"
    unit = "GB/s"
    dtype = "f32"
    peak = HBM_PEAK_GBS
    kernel_hint = ""    # substring of the HIP kernel's name in rocprof traces

    def setup(self, dev):
        raise NotImplementedError

    def launch(self, i: int) -> None:
        raise NotImplementedError

    def work(self) -> float:
        """Algorithmic bytes (hbm) or operations (mfma) of one launch."""
        raise NotImplementedError

    def rate(self, seconds: float) -> float:
        scale = 1e9 if self.bound == "hbm" else 1e12
        return self.work() / seconds / scale

    def config(self) -> dict:
        return {"workload": self.name}

    def cpu_baseline(self):
        return None


def _sets_for(bytes_per_set: int) -> int:
    return max(1, math.ceil(ROTATE_BYTES / bytes_per_set))


class Softmax(Workload):
    bound, unit, dtype, kernel_hint = "hbm", "GB/s", "f32", "softmax"

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

    def cpu_baseline(self):
        import torch
        from oracle import cpu_golden
        x = torch.randn(self.rows, self.cols, generator=torch.Generator().manual_seed(1)) * 2.0
        secs = _time_cpu(lambda: cpu_golden.softmax(x), budget_s=20.0)
        return {"value": round(self.work() / secs / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
                "kind": "port",
                "sample": f"torch.softmax(x, dim=1) on the full {self.rows}x{self.cols} fp32 input (the reference "
                          "test's golden, python/test/asc2/kernels/test_softmax.py:43), median of up to 5 runs "
                          "after 1 warm-up", "seconds_per_call": secs}


class Vadd(Workload):
    bound, unit, dtype, kernel_hint = "hbm", "GB/s", "f32", "vadd"

    def __init__(self, n: int):
        self.n = n
        self.name = f"vadd_{n}_f32"

    def setup(self, dev):
        import torch
        n_sets = _sets_for(12 * self.n)
        self.sets = []
        for _ in range(n_sets):
            self.sets.append((torch.rand(self.n, device=dev), torch.rand(self.n, device=dev),
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
                "rotating_sets": len(self.sets)}

    def cpu_baseline(self):
        import torch
        from oracle import cpu_golden
        n = min(self.n, 1 << 26)
        x, y = torch.rand(n), torch.rand(n)
        secs = _time_cpu(lambda: cpu_golden.vadd(x, y), budget_s=10.0)
        return {"value": round(12.0 * n / secs / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
                "kind": "port", "sample": f"x + y on {n} fp32 elements (README.md:53)", "seconds_per_call": secs}


class LeakyRelu(Workload):
    """test_leaky_relu.py's kernel at a bandwidth size: bf16, alpha a 0-dim bf16 tensor (0.1)."""
    bound, unit, dtype, kernel_hint = "hbm", "GB/s", "bf16", "map_vec_kernel"

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

    def cpu_baseline(self):
        import torch
        from oracle import cpu_golden
        n = min(self.n, 1 << 26)
        x = torch.rand(n).to(torch.bfloat16) * 10.0 - 5.0
        alpha = torch.tensor(0.1, dtype=torch.bfloat16)
        secs = _time_cpu(lambda: cpu_golden.leaky_relu(x, alpha), budget_s=10.0)
        return {"value": round(4.0 * n / secs / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
                "kind": "port", "sample": f"torch.where(x >= 0, x, x * alpha) on {n} bf16 elements "
                "(test_leaky_relu.py:47)", "seconds_per_call": secs}


class VMulAdd(Workload):
    """test_vmuladd.py's kernel at a bandwidth size (fp32, tile 32 as in vmuladd_launch)."""
    bound, unit, dtype, kernel_hint = "hbm", "GB/s", "f32", "map_vec_kernel"

    def __init__(self, n: int):
        self.n = n
        self.name = f"vmuladd_{n}_f32"

    def setup(self, dev):
        import torch
        self.sets = [tuple(torch.rand(self.n, device=dev) * 10 for _ in range(3)) + (torch.empty(self.n, device=dev),)
                     for _ in range(_sets_for(16 * self.n))]
        self.tpb = ((self.n + 31) // 32 + 15) // 16  # vmuladd_launch (test_vmuladd.py:34-40)

    def launch(self, i: int) -> None:
        from pyasc_amd import kernels
        x, y, z, out = self.sets[i % len(self.sets)]
        kernels.vmuladd(x, y, z, out, self.n, 32, self.tpb, 16)

    def work(self) -> float:
        return 16.0 * self.n

    def config(self) -> dict:
        return {"workload": self.name, "size": self.n, "tile_size": 32, "tile_per_block": self.tpb, "grid": 16,
                "input": "rand*10 fp32", "rotating_sets": len(self.sets)}

    def cpu_baseline(self):
        import numpy as np
        import torch
        from oracle import cpu_golden
        n = min(self.n, 1 << 25)
        rng = np.random.default_rng(seed=2026)
        x, y, z = (rng.random(n, dtype=np.float32) * 10 for _ in range(3))
        secs = _time_cpu(lambda: cpu_golden.vmuladd(x, y, z), budget_s=10.0)
        return {"value": round(16.0 * n / secs / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
                "sample": f"numpy x * y + z on {n} fp32 elements (test_vmuladd.py:52)", "seconds_per_call": secs}


class Gelu(Workload):
    """test_gelu.py's kernel at softmax's second shape (fp32 rows, tile = row length)."""
    bound, unit, dtype, kernel_hint = "hbm", "GB/s", "f32", "gelu_rows_kernel"

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

    def cpu_baseline(self):
        import torch
        from oracle import cpu_golden
        x = torch.randn(self.rows, self.cols) * 2.0
        secs = _time_cpu(lambda: cpu_golden.gelu(x, self.approximate), budget_s=10.0)
        return {"value": round(self.work() / secs / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
                "kind": "port", "sample": f"test_gelu.py:44-48 golden on the full {self.rows}x{self.cols} input",
                "seconds_per_call": secs}


class RmsNorm(Workload):
    """asc2.rms_norm rows (build-defined rms_norm_kernel) at softmax's headline shape."""
    bound, unit, dtype, kernel_hint = "hbm", "GB/s", "f32", "rms_norm"

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

    def cpu_baseline(self):
        import torch
        x = torch.randn(self.rows, self.cols) * 2.0
        gamma = torch.rand(self.cols) + 0.5
        secs = _time_cpu(lambda: torch.nn.functional.rms_norm(x, [self.cols], gamma, eps=1e-6), budget_s=10.0)
        return {"value": round(self.work() / secs / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
                "kind": "port", "sample": f"torch.nn.functional.rms_norm on the full {self.rows}x{self.cols} input",
                "seconds_per_call": secs}


class ReduceRows(Workload):
    """asc2.reduce_sum along dim 1 (test_reduce_ops.py's kernel) at a bandwidth size."""
    bound, unit, dtype, kernel_hint = "hbm", "GB/s", "f32", "reduce_rows"

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

    def cpu_baseline(self):
        import torch
        x = torch.randn(self.rows, self.cols) * 2.0
        secs = _time_cpu(lambda: torch.sum(x, 1), budget_s=10.0)
        return {"value": round(self.work() / secs / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
                "kind": "port", "sample": f"torch.sum(x, 1) on the full {self.rows}x{self.cols} input",
                "seconds_per_call": secs}


class Matmul(Workload):
    bound, unit, kernel_hint = "mfma", "TFLOP/s", "gemm_mfma"

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
        self.a = (torch.randn(self.n, self.n, device=dev, generator=g) / math.sqrt(self.n)).to(td)
        self.b = (torch.randn(self.n, self.n, device=dev, generator=g) / math.sqrt(self.n)).to(td)
        self.c = torch.empty(self.n, self.n, device=dev, dtype=torch.float32 if self.bias_leaky else td)
        self.bias = torch.randn(self.n, device=dev, generator=g) if self.bias_leaky else None

    def launch(self, i: int) -> None:
        from pyasc_amd import kernels
        if self.bias_leaky:
            kernels.matmul(self.a, self.b, self.c, bias=self.bias, leaky_alpha=0.001)
        else:
            kernels.matmul(self.a, self.b, self.c)

    def work(self) -> float:
        return 2.0 * self.n ** 3

    def config(self) -> dict:
        cfg = {"workload": self.name, "M": self.n, "N": self.n, "K": self.n, "layout": "A row-major, B row-major",
               "input": "randn/sqrt(K), seed 2", "accumulate": "fp32", "out": self.dtype}
        if self.bias_leaky:
            cfg.update({"out": "f32", "epilogue": "leaky_relu(acc + bias[n], 0.001)"})
        return cfg

    def cpu_baseline(self):
        import torch
        from oracle import cpu_golden
        rows = 1024  # a row band of A against all of B: 1/8 of the FLOPs of the full product
        td = getattr(torch, self.dt)
        g = torch.Generator().manual_seed(2)
        a = (torch.randn(rows, self.n, generator=g) / math.sqrt(self.n)).to(td)
        b = (torch.randn(self.n, self.n, generator=g) / math.sqrt(self.n)).to(td)
        secs = _time_cpu(lambda: cpu_golden.matmul(a, b), budget_s=20.0)
        return {"value": round(2.0 * rows * self.n * self.n / secs / 1e12, 4), "unit": "TFLOP/s",
                "cores": torch.get_num_threads(), "kind": "port",
                "sample": f"a.to(float32) @ b.to(float32) (python/test/asc2/kernels/test_matmul_tiled.py:49) on "
                          f"rows 0..{rows - 1} of A ({rows}x{self.n}x{self.n}), median of up to 5 runs after 1 "
                          "warm-up", "seconds_per_call": secs}


class MatmulI8(Workload):
    bound, unit, dtype, kernel_hint = "mfma", "TOPS", "int8", "gemm_i8"
    peak = INT8_PEAK_TOPS

    def __init__(self, M: int, N: int, K: int):
        self.M, self.N, self.K = M, N, K
        self.name = f"matmul_i8_dequant_{M}x{N}x{K}"

    def setup(self, dev):
        import torch
        g = torch.Generator(device=dev).manual_seed(3)
        self.a = torch.randint(-127, 128, (self.M, self.K), dtype=torch.int8, device=dev, generator=g)
        self.b = torch.randint(-127, 128, (self.K, self.N), dtype=torch.int8, device=dev, generator=g)
        self.s = torch.rand(self.N, device=dev, generator=g) * 0.009 + 0.001
        self.c = torch.empty(self.M, self.N, dtype=torch.float16, device=dev)

    def launch(self, i: int) -> None:
        from pyasc_amd import kernels
        kernels.matmul_i8(self.a, self.b, self.c, scale=self.s)

    def work(self) -> float:
        return 2.0 * self.M * self.N * self.K

    def config(self) -> dict:
        return {"workload": self.name, "M": self.M, "N": self.N, "K": self.K, "accumulate": "int32 (exact)",
                "epilogue": "fp16(fp32(acc) * scale[n])", "input": "int8 uniform[-127,127], seed 3"}

    def cpu_baseline(self):
        import torch
        from oracle import cpu_golden
        rows = 128  # a row band: 1/32 of the full product's operations
        g = torch.Generator().manual_seed(3)
        a = torch.randint(-127, 128, (rows, self.K), dtype=torch.int8, generator=g)
        b = torch.randint(-127, 128, (self.K, self.N), dtype=torch.int8, generator=g)
        scale = torch.rand(self.N, generator=g) * 0.009 + 0.001
        secs = _time_cpu(lambda: cpu_golden.dequant(cpu_golden.matmul_i8(a, b), scale), budget_s=20.0)
        return {"value": round(2.0 * rows * self.N * self.K / secs / 1e12, 4), "unit": "TOPS",
                "cores": torch.get_num_threads(), "kind": "port",
                "sample": f"(a.to(int32) @ b.to(int32)) then (acc.float() * scale).half() "
                          f"(test_matmul_iterate_all.py:116, test_matmul_quant.py dequant) on rows 0..{rows - 1} "
                          f"of A ({rows}x{self.N}x{self.K}), median of up to 5 runs after 1 warm-up",
                "seconds_per_call": secs}


class FlashAttention(Workload):
    bound, unit, dtype, kernel_hint = "mfma", "TFLOP/s", "bf16", "fa_fwd"
    peak = BF16_PEAK_TFLOPS

    def __init__(self, B: int, H: int, S: int, D: int, causal: bool):
        self.B, self.H, self.S, self.D, self.causal = B, H, S, D, causal
        self.name = f"flash_attn_fwd_b{B}h{H}s{S}d{D}_{'causal' if causal else 'noncausal'}"

    def setup(self, dev):
        import torch
        g = torch.Generator(device=dev).manual_seed(4)
        shape = (self.B, self.H, self.S, self.D)
        self.q, self.k, self.v = [torch.randn(*shape, device=dev, generator=g).to(torch.bfloat16) for _ in range(3)]
        self.o = torch.empty_like(self.q)

    def launch(self, i: int) -> None:
        from pyasc_amd import kernels
        kernels.flash_attention_fwd(self.q, self.k, self.v, self.o, 1 / math.sqrt(self.D), self.causal)

    def work(self) -> float:
        full = 4.0 * self.B * self.H * self.S * self.S * self.D
        return full / 2 if self.causal else full  # causal counted as half of the dense work

    def config(self) -> dict:
        return {"workload": self.name, "batch": self.B, "heads": self.H, "seq_len": self.S, "head_dim": self.D,
                "causal": self.causal, "sm_scale": 1 / math.sqrt(self.D), "input": "bf16 randn, seed 4",
                "flop_convention": "4*B*H*S^2*D, halved for causal"}

    def cpu_baseline(self):
        import torch
        from oracle import cpu_golden
        heads = 2  # (batch, head) slices, each the full S x S problem
        g = torch.Generator().manual_seed(4)
        q, k, v = [torch.randn(heads, self.S, self.D, generator=g).to(torch.bfloat16) for _ in range(3)]
        scale = 1 / math.sqrt(self.D)

        def run():
            for i in range(heads):
                cpu_golden.attention(q[i], k[i], v[i], scale, self.causal)

        secs = _time_cpu(run, budget_s=20.0)
        work = heads * 4.0 * self.S * self.S * self.D * (0.5 if self.causal else 1.0)
        return {"value": round(work / secs / 1e12, 4), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
                "kind": "port",
                "sample": f"fp32 softmax((q @ k.T) * scale [+ causal mask]) @ v per (batch, head) slice on {heads} "
                          f"slices of S={self.S}, D={self.D}, same FLOP convention, median of up to 5 runs after 1 "
                          "warm-up", "seconds_per_call": secs}


WORKLOADS = {
    "softmax_4096x4096": lambda: Softmax(4096, 4096),
    "softmax_16384x1024": lambda: Softmax(16384, 1024),
    "vadd_268435456": lambda: Vadd(1 << 28),
    "vadd_8192": lambda: Vadd(8192),
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
SUITE = ["softmax_16384x1024", "vadd_268435456", "matmul_bf16_8192", "matmul_f16_8192", "matmul_i8_4096x11008x4096",
         "matmul_f16_8192_bias_leakyrelu", "fa_fwd_noncausal", "fa_fwd_causal", "leaky_relu_268435456",
         "vmuladd_268435456", "gelu_tanh_16384x1024", "gelu_erf_16384x1024", "rms_norm_4096x4096",
         "reduce_sum_dim1_16384x4096"]


def _time_cpu(fn, budget_s: float) -> float:
    fn()  # warm-up
    times = []
    start = time.perf_counter()
    for _ in range(5):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - start > budget_s:
            break
    return statistics.median(times)


def measure(w: Workload, steps: int, warmup: int, dev, graph: bool = True) -> dict:
    """Times exactly ``steps`` launches on the launch stream with HIP events.

    Default: the ``steps`` launches are captured once into a HIP graph and the
    graph is replayed between two events, so the kernels run back to back with
    no host launch overhead in the timed region (``kernel_ms`` = region / steps).
    ``graph=False``: each launch is bracketed by its own event pair instead and
    ``kernel_ms`` is their mean (adds about 2 us of event overhead per launch)."""
    import torch
    w.setup(dev)
    for i in range(warmup):
        w.launch(i)
    torch.cuda.synchronize()
    if graph:
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                for i in range(steps):
                    w.launch(warmup + i)
        torch.cuda.synchronize()
        g.replay()  # untimed: first replay uploads the graph
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        g.replay()
        end.record(stream)
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / steps
        kernel_ms = ms
        del g
    else:
        stream = torch.cuda.current_stream()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        torch.cuda.synchronize()
        for i in range(steps):
            ev[i][0].record(stream)
            w.launch(warmup + i)
            ev[i][1].record(stream)
        torch.cuda.synchronize()
        ms = ev[0][0].elapsed_time(ev[-1][1]) / steps
        kernel_ms = sum(a.elapsed_time(b) for a, b in ev) / steps
    rate = w.rate(kernel_ms / 1e3)
    return {"workload": w.name, "ms_per_step": ms, "kernel_ms": kernel_ms, "value": rate, "unit": w.unit,
            "frac_of_peak": rate / w.peak, "bound": w.bound, "config": w.config(),
            "timing": "hip-graph replay" if graph else "per-launch events"}


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
            raise AssertionError("kernel bodies are not executed")

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
        raise AssertionError("kernel bodies are not executed")

    @asc.jit
    def matmul_kernel(a: asc.GlobalAddress, b: asc.GlobalAddress, c: asc.GlobalAddress, alpha: float,
                      tiling: asc.adv.TCubeTiling, bias: asc.GlobalAddress, workspace: asc.GlobalAddress):
        raise AssertionError("kernel bodies are not executed")

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


def traffic_for(name: str):
    path = os.path.join(REPO, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(name)
    except (OSError, ValueError):
        return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default=HEADLINE, choices=sorted(WORKLOADS))
    ap.add_argument("--no-suite", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="time with per-launch event pairs, no HIP graph")
    ap.add_argument("--cpu-all", action="store_true",
                    help="also time the CPU baseline of every suite workload (adds a few minutes)")
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

    head = WORKLOADS[args.workload]()
    res = measure(head, args.steps, args.warmup, dev, graph=not args.no_graph)
    suite = {}
    if not args.no_suite:
        for name in SUITE:
            if name == args.workload:
                continue
            w = WORKLOADS[name]()
            r = measure(w, max(5, args.steps // 2), max(2, args.warmup // 2), dev, graph=not args.no_graph)
            r["roofline"] = {"bound": w.bound, "achieved": r["value"], "peak": w.peak, "unit": w.unit,
                             "frac": r["value"] / w.peak, "traffic": traffic_for(w.name)}
            if args.cpu_all and not args.no_cpu:
                r["cpu_baseline"] = w.cpu_baseline()
            suite[name] = r
            del w
            torch.cuda.empty_cache()
    latency = None if args.no_suite else launch_latency(dev)
    published = None if args.no_suite else reference_durations(dev)
    if args.copy_calibration:
        src = torch.empty(COPY_BYTES // 4, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    cpu = None if args.no_cpu else head.cpu_baseline()
    line = {
        "metric": METRIC,
        "value": round(res["value"], 3),
        "unit": head.unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": res["ms_per_step"],
        "kernel_ms": res["kernel_ms"],
        "timing": res["timing"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": head.dtype,
        "data": "synthetic (seeded torch generator on the device; distribution of BASELINE.json's config)",
        "config": head.config(),
        "roofline": {"bound": head.bound, "achieved": round(res["value"], 3), "peak": head.peak, "unit": head.unit,
                     "frac": round(res["value"] / head.peak, 4), "traffic": traffic_for(head.name)},
        "cpu_baseline": cpu,
        "device": _native.device_info(0),
        "suite": suite,
        "launch_latency": latency,
        "reference_published": published,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
