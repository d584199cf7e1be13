"""Summarises rocprofv3 output of bench.py runs into profiles/ (no GPU needed).

    python profile_summary.py traffic DIR   # FETCH_SIZE / WRITE_SIZE passes -> profiles/traffic.json + hbm_traffic.md
    python profile_summary.py mfma DIR      # MFMA-busy / clock passes -> profiles/mfma_counters.md
    python profile_summary.py trace DIR     # kernel traces -> profiles/kernel_trace_suite.md
    python profile_summary.py ea DIR        # L2 read-miss requests by destination -> profiles/l2_miss_destinations.md
    python profile_summary.py lds DIR       # LDS / VALU / MFMA instruction and LDS-busy passes -> profiles/lds_valu_counters.md

DIR holds one rocprofv3 output folder per pass, written with ``-f csv -o run`` by
the commands the summaries print:

  traffic: DIR/<workload>_FETCH_SIZE and DIR/<workload>_WRITE_SIZE, from
      rocprofv3 --pmc FETCH_SIZE -f csv -d DIR/<workload>_FETCH_SIZE -o run -- \
          python3 bench.py --workload <workload> --no-suite --no-cpu --no-vendor --steps 5 --warmup 1 --warmup-s 0 --copy-calibration
  trace: DIR/<workload>_TRACE and the bench's output in DIR/<workload>_TRACE.log, from
      rocprofv3 --kernel-trace --stats -f csv -d DIR/<workload>_TRACE -o run -- \
          python3 bench.py --workload <workload> --no-suite --no-cpu --no-vendor --steps 20 --warmup 3 > DIR/<workload>_TRACE.log
  mfma: DIR/<workload>_MFMA, from
      rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CU_CYCLES GRBM_GUI_ACTIVE --kernel-trace -f csv \
          -d DIR/<workload>_MFMA -o run -- python3 bench.py --workload <workload> --no-suite --no-cpu --no-vendor --steps 5 \
          --warmup 1 --warmup-s 0
  ea: DIR/<workload>_EA, from
      rocprofv3 --pmc TCC_EA0_RDREQ_sum TCC_EA0_RDREQ_DRAM_sum TCC_EA0_RDREQ_32B_sum -f csv -d DIR/<workload>_EA \
          -o run -- python3 bench.py --workload <workload> --no-suite --no-cpu --no-vendor --steps 5 --warmup 1 \
          --warmup-s 0 --copy-calibration
  lds: DIR/<workload>_LDS, from
      rocprofv3 --pmc SQ_LDS_IDX_ACTIVE SQ_LDS_BANK_CONFLICT SQ_INSTS_LDS SQ_INSTS_VALU SQ_INSTS_MFMA \
          SQ_INSTS_VALU_TRANS_F32 GRBM_GUI_ACTIVE --kernel-trace -f csv -d DIR/<workload>_LDS -o run -- \
          python3 bench.py --workload <workload> --no-suite --no-cpu --no-vendor --steps 5 --warmup 1 --warmup-s 0

FETCH_SIZE and WRITE_SIZE are KiB per dispatch past the L2.  ``--copy-calibration``
adds five torch device copies of exactly 256 MiB; their readings give the factor that
turns each counter into bytes (factor = 262144 KiB / reading).
"""
from __future__ import annotations

import collections
import csv
import glob
import json
import os
import sys

import bench

REPO = os.path.dirname(os.path.abspath(__file__))
PROFILES = os.path.join(REPO, "profiles")
COPY_KIB = 262144.0
SIMDS_PER_CU = 4


def _rows(folder: str):
    files = glob.glob(os.path.join(folder, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise FileNotFoundError(f"no counter_collection.csv under {folder}")
    for path in files:
        with open(path, newline="") as f:
            yield from csv.DictReader(f)


def _short(kernel: str) -> str:
    name = kernel.replace("void (anonymous namespace)::", "").replace("(anonymous namespace)::", "")
    depth, out = 0, []
    for ch in name:  # keep the template arguments, drop the parameter list
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            break
        out.append(ch)
    return "".join(out).strip()


def _is_library_kernel(kernel: str) -> bool:
    return "at::native" not in kernel and not kernel.startswith("__amd") and "elementwise_kernel" not in kernel


def _per_kernel(folder: str, counter: str):
    """counter values per dispatch, keyed by kernel name."""
    vals = collections.defaultdict(list)
    for r in _rows(folder):
        if r["Counter_Name"] == counter:
            vals[r["Kernel_Name"]].append(float(r["Counter_Value"]))
    return vals


def traffic(folder: str) -> int:
    path = os.path.join(PROFILES, "traffic.json")
    try:
        with open(path) as f:
            table = json.load(f)
    except (OSError, ValueError):
        table = {}
    table.setdefault("workloads", {})
    table["format"] = ("bytes per launch past the L2 (FETCH_SIZE + WRITE_SIZE, KiB per dispatch, each scaled by "
                       "the reading of a 256 MiB device copy), stamped with the hash of the kernel sources")
    for key, make in bench.WORKLOADS.items():
        fetch_dir = os.path.join(folder, f"{key}_FETCH_SIZE")
        write_dir = os.path.join(folder, f"{key}_WRITE_SIZE")
        if not (os.path.isdir(fetch_dir) and os.path.isdir(write_dir)):
            continue
        w = make()
        row = {}
        for counter, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
            vals = _per_kernel(d, counter)
            # the calibration copies run as the runtime's blit kernel (__amd_rocclr_copyBuffer)
            copy = [v for k, v in vals.items() if "copyBuffer" in k]
            if len(copy) != 1:
                raise RuntimeError(f"{d}: no calibration copy dispatches (run with --copy-calibration)")
            lib = {k: v for k, v in vals.items() if _is_library_kernel(k) and w.kernel_hint in k}
            if len(lib) != 1:
                raise RuntimeError(f"{d}: expected one library kernel matching {w.kernel_hint!r}, got {list(lib)}")
            (kname, kvals), = lib.items()
            row["kernel"] = _short(kname)
            row[counter.lower() + "_kib"] = round(sum(kvals) / len(kvals), 1)
            row["copy_" + counter.lower() + "_kib"] = round(sum(copy[0]) / len(copy[0]), 1)
        ff = COPY_KIB / row["copy_fetch_size_kib"]
        wf = COPY_KIB / row["copy_write_size_kib"]
        row.update({"fetch_factor": round(ff, 3), "write_factor": round(wf, 3),
                    "bytes": int(round((row["fetch_size_kib"] * ff + row["write_size_kib"] * wf) * 1024)),
                    "algorithmic_bytes": int(_algorithmic_bytes(w)),
                    "sources_hash": bench.sources_hash(w.sources)})
        table["workloads"][w.name] = row
        print(f"{w.name}: {row['kernel']} {row['bytes'] / 1e6:.1f} MB "
              f"({row['bytes'] / row['algorithmic_bytes']:.2f}x algorithmic)")
    table["workloads"] = dict(sorted(table["workloads"].items()))
    with open(path, "w") as f:
        json.dump(table, f, indent=1)
        f.write("\n")
    _write_traffic_md(table)
    return 0


def _algorithmic_bytes(w) -> float:
    """Minimum HBM bytes of one launch: every operand read once, every result written once."""
    if w.bound in ("hbm", "latency"):
        return w.work()
    if isinstance(w, bench.Matmul):
        return w.n * w.n * (2 + 2 + (4 if w.bias_leaky else 2)) + (4 * w.n if w.bias_leaky else 0)
    if isinstance(w, bench.MatmulI8):
        return w.M * w.K + w.K * w.N + 2 * w.M * w.N + 4 * w.N
    if isinstance(w, bench.FlashAttention):
        return 4 * 2 * w.B * w.H * w.S * w.D
    raise TypeError(type(w).__name__)


def _write_traffic_md(table: dict) -> None:
    lines = [
        "# HBM traffic per launch (rocprofv3 PMC), one MI355X", "",
        "Generated by `python profile_summary.py traffic DIR` from two rocprofv3 passes per workload "
        "(repository root on the GPU box, `TMPDIR=/tmp`, `W` a bench workload key):", "",
        "```",
        "rocprofv3 --pmc FETCH_SIZE -f csv -d gpurun_out/pmc/${W}_FETCH_SIZE -o run -- python3 bench.py "
        "--workload $W --no-suite --no-cpu --no-vendor --steps 5 --warmup 1 --warmup-s 0 --copy-calibration",
        "rocprofv3 --pmc WRITE_SIZE -f csv -d gpurun_out/pmc/${W}_WRITE_SIZE -o run -- python3 bench.py "
        "--workload $W --no-suite --no-cpu --no-vendor --steps 5 --warmup 1 --warmup-s 0 --copy-calibration",
        "```", "",
        "`FETCH_SIZE` and `WRITE_SIZE` count the bytes that pass the L2 (misses and write-backs, including "
        "those the 256 MiB MALL then serves), so for kernels with operand reuse (the GEMMs) they bound HBM "
        "traffic from above; for streaming kernels they equal it.  `--copy-calibration` adds five device "
        "copies of exactly 256 MiB (read 262144 KiB, written 262144 KiB); factor = 262144 / the copy's "
        "reading.  Values are KiB per dispatch, averaged over the library kernel's dispatches.  Each row "
        "is stamped with the hash of the kernel sources it was measured on; bench.py reports "
        "`roofline.traffic` only while the sources still match.", "",
        "| Workload | Kernel | FETCH KiB | WRITE KiB | fetch factor | write factor | traffic MB | algorithmic MB "
        "| ratio | sources |",
        "|---|---|---:|---:|---:|---:|---:|---:|---:|---|",
    ]
    for name, r in table["workloads"].items():
        lines.append(f"| `{name}` | `{r['kernel']}` | {r['fetch_size_kib']:.0f} | {r['write_size_kib']:.0f} | "
                     f"{r['fetch_factor']:.3f} | {r['write_factor']:.3f} | {r['bytes'] / 1e6:.1f} | "
                     f"{r['algorithmic_bytes'] / 1e6:.1f} | {r['bytes'] / r['algorithmic_bytes']:.2f} | "
                     f"`{r['sources_hash']}` |")
    with open(os.path.join(PROFILES, "hbm_traffic.md"), "w") as f:
        f.write("\n".join(lines) + "\n")


def mfma(folder: str) -> int:
    """MFMA utilisation and clock of the MFMA kernels from one counter pass each.

    SQ_VALU_MFMA_BUSY_CYCLES is summed over every SIMD; GRBM_GUI_ACTIVE is summed over
    the XCDs (each counts the GPU-active cycles of its own clock).  So
      cycles per XCD   = GRBM_GUI_ACTIVE / XCDs
      clock            = cycles per XCD / kernel duration
      MFMA busy        = SQ_VALU_MFMA_BUSY_CYCLES / (cycles per XCD x CUs x 4 SIMDs)
    and the achieved rate at 100 % busy is the MFMA peak scaled by clock / 2.4 GHz."""
    cus, xcds, info = device_shape(folder)
    lines = [
        "# MFMA utilisation and shader clock (rocprofv3 PMC), one MI355X", "",
        "Generated by `python profile_summary.py mfma DIR` from one counter pass per workload "
        "(repository root on the GPU box, `TMPDIR=/tmp`, `W` a bench workload key):", "",
        "```",
        "rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CU_CYCLES GRBM_GUI_ACTIVE --kernel-trace -f csv "
        "-d gpurun_out/pmc/${W}_MFMA -o run -- python3 bench.py --workload $W --no-suite --no-cpu --no-vendor --steps 5 "
        "--warmup 1 --warmup-s 0",
        "```", "",
        f"Device: {info}.  `SQ_VALU_MFMA_BUSY_CYCLES` is summed over all SIMDs; `GRBM_GUI_ACTIVE` over the "
        "XCDs, so cycles per XCD = GRBM_GUI_ACTIVE / XCDs.  clock = cycles per XCD / dispatch duration "
        "(Start/End timestamps of the counter pass); MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (cycles per XCD "
        "x CUs x 4).  A `v_mfma_f32_32x32x16_bf16` (or `_i32_32x32x32_i8`) keeps a SIMD's MFMA unit busy 32 "
        "cycles (8 passes of 4), so 100 % busy is the dense peak at that clock: peak x clock / 2.4 GHz.  "
        "Durations here are under counter collection (serialised dispatches) and are a few percent above "
        "the unprofiled bench times.", "",
        "| Workload | Kernel | dispatches | duration us | clock GHz | MFMA busy % | CU busy % | "
        "peak at this clock | achieved (bench FLOP / duration) | achieved / peak at this clock |",
        "|---|---|---:|---:|---:|---:|---:|---:|---:|---:|",
    ]
    for key, make in bench.WORKLOADS.items():
        d = os.path.join(folder, f"{key}_MFMA")
        if not os.path.isdir(d):
            continue
        w = make()
        per = collections.defaultdict(dict)
        for r in _rows(d):
            if not (_is_library_kernel(r["Kernel_Name"]) and w.kernel_hint in r["Kernel_Name"]):
                continue
            e = per[r["Dispatch_Id"]]
            e["kernel"] = _short(r["Kernel_Name"])
            e[r["Counter_Name"]] = float(r["Counter_Value"])
            e["dur"] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-9
        disp = [e for e in per.values() if "SQ_VALU_MFMA_BUSY_CYCLES" in e and "GRBM_GUI_ACTIVE" in e]
        if not disp:
            raise RuntimeError(f"{d}: no dispatch of a kernel matching {w.kernel_hint!r}")
        n = len(disp)
        dur = sum(e["dur"] for e in disp) / n
        gui = sum(e["GRBM_GUI_ACTIVE"] for e in disp) / n / xcds
        busy = sum(e["SQ_VALU_MFMA_BUSY_CYCLES"] for e in disp) / n
        cu_busy = sum(e.get("SQ_BUSY_CU_CYCLES", 0.0) for e in disp) / n
        clock = gui / dur / 1e9
        util = busy / (gui * cus * SIMDS_PER_CU)
        peak_at_clock = w.peak * clock / 2.4
        achieved = w.work() / dur / 1e12
        lines.append(f"| `{w.name}` | `{disp[0]['kernel']}` | {n} | {dur * 1e6:.1f} | {clock:.3f} | "
                     f"{100 * util:.1f} | {100 * cu_busy / (gui * cus):.1f} | {peak_at_clock:.0f} {w.unit} | "
                     f"{achieved:.0f} {w.unit} | {achieved / peak_at_clock:.3f} |")
        print(lines[-1])
    with open(os.path.join(PROFILES, "mfma_counters.md"), "w") as f:
        f.write("\n".join(lines) + "\n")
    return 0


def trace(folder: str) -> int:
    """Traced kernel durations of each workload's timed replay beside the bench's own
    HIP-event figure for the same replay (the last ``steps`` dispatches of the
    workload's kernel are the timed replay: warm-up launches and the untimed first
    replay come before it)."""
    lines = [
        "# Kernel trace: the bench workloads on one MI355X", "",
        "Generated by `python profile_summary.py trace DIR` from one traced bench run per workload "
        "(repository root on the GPU box, `TMPDIR=/tmp`, `W` a bench workload key):", "",
        "```",
        "rocprofv3 --kernel-trace --stats -f csv -d gpurun_out/prof/${W}_TRACE -o run -- python3 bench.py "
        "--workload $W --no-suite --no-cpu --no-vendor --steps 20 --warmup 3 > gpurun_out/prof/${W}_TRACE.log",
        "```", "",
        "Durations in microseconds: average, minimum and maximum of the last timed replay's dispatches "
        "(Start/End timestamps), the bench's figure (HIP events around each graph replay on the launch "
        "stream, the median of its timed replays divided by the launches) and the bench's value "
        "computed from it.", "",
        "| Workload | Kernel | timed dispatches | avg us | min | max | bench events us | trace / events | "
        "bench value |",
        "|---|---|---:|---:|---:|---:|---:|---:|---:|",
    ]
    for key, make in bench.WORKLOADS.items():
        d = os.path.join(folder, f"{key}_TRACE")
        log = d + ".log"
        if not (os.path.isdir(d) and os.path.exists(log)):
            continue
        w = make()
        with open(log) as f:
            res = json.loads([ln for ln in f if ln.startswith("{")][-1])
        files = glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True)
        if not files:
            raise FileNotFoundError(f"no kernel_trace.csv under {d}")
        rows = []
        for path in files:
            with open(path, newline="") as f:
                rows += [r for r in csv.DictReader(f)
                         if _is_library_kernel(r["Kernel_Name"]) and w.kernel_hint in r["Kernel_Name"]]
        rows.sort(key=lambda r: int(r["Start_Timestamp"]))
        steps = int(res["steps"])
        launches = getattr(w, "launches_per_step", 1)
        timed = rows[-steps * launches:]
        if len(timed) < steps * launches:
            raise RuntimeError(f"{d}: {len(timed)} dispatches of {w.kernel_hint!r}, expected {steps * launches}")
        durs = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in timed]
        names = sorted({_short(r["Kernel_Name"]) for r in timed})
        per_step = sum(durs) / steps
        ev = res.get("kernel_ms", res["ms_per_step"]) * 1e3  # the bench's median replay / launches
        lines.append(f"| `{w.name}` | {', '.join(f'`{n}`' for n in names)} | {len(durs)} | {per_step:.2f} | "
                     f"{min(durs):.2f} | {max(durs):.2f} | {ev:.2f} | {per_step / ev:.3f} | "
                     f"{res['value']:.4g} {res['unit']} |")
        print(lines[-1])
    with open(os.path.join(PROFILES, "kernel_trace_suite.md"), "w") as f:
        f.write("\n".join(lines) + "\n")
    return 0


def ea(folder: str) -> int:
    """L2 read misses by destination for the MFMA workloads: TCC_EA0_RDREQ (every read
    request the L2s send out) against TCC_EA0_RDREQ_DRAM (those destined for DRAM, i.e.
    the memory controllers, in front of which the MALL sits), with the 256 MiB
    calibration copies giving the bytes per request; and the floor the GEMMs' tile walk
    sets on those reads."""
    lines = [
        "# L2 read misses by destination (rocprofv3 PMC), one MI355X", "",
        "Generated by `python profile_summary.py ea DIR` from one counter pass per workload "
        "(repository root on the GPU box, `TMPDIR=/tmp`, `W` a bench workload key):", "",
        "```",
        "rocprofv3 --pmc TCC_EA0_RDREQ_sum TCC_EA0_RDREQ_DRAM_sum TCC_EA0_RDREQ_32B_sum -f csv "
        "-d gpurun_out/pmc/${W}_EA -o run -- python3 bench.py --workload $W --no-suite --no-cpu --no-vendor "
        "--steps 5 --warmup 1 --warmup-s 0 --copy-calibration",
        "```", "",
        "`TCC_EA0_RDREQ_sum` counts the read requests the L2s send to the data fabric, "
        "`TCC_EA0_RDREQ_DRAM_sum` those destined for DRAM (the memory controllers; the 256 MiB MALL, AMD "
        "Infinity Cache, sits in front of them on the memory side), `TCC_EA0_RDREQ_32B_sum` the 32-byte "
        "ones.  The calibration copy reads exactly 256 MiB; its request count gives the bytes per "
        "request.  `rocprofv3 --list-avail` on this image offers no MALL or memory-controller counter, so "
        "reads the MALL serves and reads that reach HBM cannot be told apart: every L2 read miss is "
        "destined for DRAM, and the MALL's share is not observable here.", "",
        "The floor column is what the GEMMs' tile walk cannot go below: each XCD runs 32 workgroups of "
        "256x256 output tiles at once, in groups of 8 tile-rows x 4 tile-columns, so every round streams "
        "8 A panels and 4 B panels (256 rows or columns x K) through that XCD's 4 MB L2 once; a panel "
        "(4 MiB for bf16 at K = 8192, 1 MiB for int8 at K = 4096) does not fit the L2 twice over, so no "
        "round reuses the previous one's panels.  Any 32 tiles need at least 12 distinct panels (r + c "
        "with r x c = 32).  Floor = XCDs x rounds x 12 panels.", "",
        "| Workload | Kernel | RDREQ | RDREQ_DRAM | 32B | bytes per request (copy) | L2 read misses MB | "
        "A+B MB | misses / (A+B) | tile-walk floor MB |",
        "|---|---|---:|---:|---:|---:|---:|---:|---:|---:|",
    ]
    for key, make in bench.WORKLOADS.items():
        d = os.path.join(folder, f"{key}_EA")
        if not os.path.isdir(d):
            continue
        w = make()
        vals = {c: _per_kernel(d, c) for c in ("TCC_EA0_RDREQ_sum", "TCC_EA0_RDREQ_DRAM_sum",
                                              "TCC_EA0_RDREQ_32B_sum")}
        avg = {}
        for c, per in vals.items():
            lib = {k: v for k, v in per.items() if _is_library_kernel(k) and w.kernel_hint in k}
            copy = [v for k, v in per.items() if "copyBuffer" in k]
            if len(lib) != 1 or len(copy) != 1:
                raise RuntimeError(f"{d}: expected one library kernel and the calibration copy for {c}")
            (kname, kv), = lib.items()
            avg[c] = (sum(kv) / len(kv), sum(copy[0]) / len(copy[0]), _short(kname))
        req, copy_req, kname = avg["TCC_EA0_RDREQ_sum"]
        per_req = COPY_KIB * 1024 / copy_req
        miss = req * per_req
        if isinstance(w, bench.Matmul):
            ab, panel, tiles = 2 * 2 * w.n * w.n, 256 * w.n * 2, (w.n // 256) ** 2
        elif isinstance(w, bench.MatmulI8):
            ab, panel, tiles = w.M * w.K + w.K * w.N, 256 * w.K, (w.M // 256) * (w.N // 256)
        else:
            ab, panel, tiles = 3 * w.B * w.H * w.S * w.D * 2, None, None
        floor = f"{8 * (tiles / 256) * 12 * panel / 1e6:.0f}" if panel else "-"
        lines.append(f"| `{w.name}` | `{kname}` | {req:.0f} | {avg['TCC_EA0_RDREQ_DRAM_sum'][0]:.0f} | "
                     f"{avg['TCC_EA0_RDREQ_32B_sum'][0]:.0f} | {per_req:.0f} | {miss / 1e6:.1f} | {ab / 1e6:.1f} | "
                     f"{miss / ab:.2f} | {floor} |")
        print(lines[-1])
    with open(os.path.join(PROFILES, "l2_miss_destinations.md"), "w") as f:
        f.write("\n".join(lines) + "\n")
    return 0


def _gpu_agent(folder: str) -> dict:
    """The GPU row of rocprofv3's agent_info.csv under ``folder``."""
    for path in glob.glob(os.path.join(folder, "**", "*agent_info.csv"), recursive=True):
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                if r.get("Agent_Type") == "GPU":
                    return r
    return {}


def lds(folder: str) -> int:
    """LDS and VALU activity of the MFMA kernels from one counter pass each.

    SQ_LDS_IDX_ACTIVE and SQ_LDS_BANK_CONFLICT count LDS cycles (indexed accesses, and
    the cycles of those stalled by bank conflicts), summed over the CUs; the SQ_INSTS_*
    counters count wave instructions issued, summed over the SIMDs.  So
      LDS busy          = SQ_LDS_IDX_ACTIVE / (cycles per XCD x CUs)
      conflict share    = SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE
    and the instruction counts are given per MFMA instruction."""
    cus, xcds, info = device_shape(folder)
    lines = [
        "# LDS, VALU and MFMA activity (rocprofv3 PMC), one MI355X", "",
        "Generated by `python profile_summary.py lds DIR` from one counter pass per workload "
        "(repository root on the GPU box, `TMPDIR=/tmp`, `W` a bench workload key):", "",
        "```",
        "rocprofv3 --pmc SQ_LDS_IDX_ACTIVE SQ_LDS_BANK_CONFLICT SQ_INSTS_LDS SQ_INSTS_VALU SQ_INSTS_MFMA "
        "SQ_INSTS_VALU_TRANS_F32 GRBM_GUI_ACTIVE --kernel-trace -f csv -d gpurun_out/pmc/${W}_LDS -o run -- "
        "python3 bench.py --workload $W --no-suite --no-cpu --no-vendor --steps 5 --warmup 1 --warmup-s 0",
        "```", "",
        f"Device: {info}.  LDS busy = SQ_LDS_IDX_ACTIVE / (GRBM_GUI_ACTIVE / XCDs x CUs), the share of "
        "each CU's cycles in which its LDS serves indexed reads or writes (the direct-to-LDS loads are "
        "not indexed accesses); bank conflicts = SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE.  The "
        "instruction columns are wave instructions issued per MFMA instruction (`SQ_INSTS_VALU` counts "
        "every VALU-issued instruction, the MFMAs included; `TRANS` counts fp32 transcendentals, here "
        "`v_exp_f32`).", "",
        "| Workload | Kernel | dispatches | duration us | LDS busy % | bank conflicts % of LDS busy | "
        "LDS instr / MFMA | VALU instr / MFMA | TRANS / MFMA |",
        "|---|---|---:|---:|---:|---:|---:|---:|---:|",
    ]
    for key, make in bench.WORKLOADS.items():
        d = os.path.join(folder, f"{key}_LDS")
        if not os.path.isdir(d):
            continue
        w = make()
        per = collections.defaultdict(dict)
        for r in _rows(d):
            if not (_is_library_kernel(r["Kernel_Name"]) and w.kernel_hint in r["Kernel_Name"]):
                continue
            e = per[r["Dispatch_Id"]]
            e["kernel"] = _short(r["Kernel_Name"])
            e[r["Counter_Name"]] = e.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
            e["dur"] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-9
        need = ("SQ_LDS_IDX_ACTIVE", "SQ_INSTS_MFMA", "GRBM_GUI_ACTIVE")
        disp = [e for e in per.values() if all(k in e for k in need)]
        if not disp:
            raise RuntimeError(f"{d}: no dispatch of a kernel matching {w.kernel_hint!r}")
        n = len(disp)

        def avg(k):
            return sum(e.get(k, 0.0) for e in disp) / n
        gui = avg("GRBM_GUI_ACTIVE") / xcds
        lds_active, mfma = avg("SQ_LDS_IDX_ACTIVE"), avg("SQ_INSTS_MFMA")
        lines.append(f"| `{w.name}` | `{disp[0]['kernel']}` | {n} | {avg('dur') * 1e6:.1f} | "
                     f"{100 * lds_active / (gui * cus):.1f} | "
                     f"{100 * avg('SQ_LDS_BANK_CONFLICT') / max(lds_active, 1.0):.2f} | "
                     f"{avg('SQ_INSTS_LDS') / mfma:.3f} | {avg('SQ_INSTS_VALU') / mfma:.3f} | "
                     f"{avg('SQ_INSTS_VALU_TRANS_F32') / mfma:.3f} |")
        print(lines[-1])
    with open(os.path.join(PROFILES, "lds_valu_counters.md"), "w") as f:
        f.write("\n".join(lines) + "\n")
    return 0


def device_shape(folder: str):
    """(CUs, XCDs, description) of the profiled GPU (256, 8 for MI355X)."""
    for d in sorted(glob.glob(os.path.join(folder, "*"))):
        r = _gpu_agent(d)
        if r:
            cus, xcds = int(r.get("Cu_Count") or 256), int(r.get("Num_Xcc") or 8)
            return cus, xcds, (f"{r.get('Name') or 'gfx950'}, {cus} CUs in {xcds} XCDs, max engine clock "
                               f"{r.get('Max_Engine_Clk_Fcompute', '?')} MHz")
    return 256, 8, "gfx950, 256 CUs in 8 XCDs"


def main(argv) -> int:
    modes = {"traffic": traffic, "mfma": mfma, "trace": trace, "ea": ea, "lds": lds}
    if len(argv) != 3 or argv[1] not in modes:
        print(__doc__, file=sys.stderr)
        return 2
    return modes[argv[1]](argv[2])


if __name__ == "__main__":
    sys.exit(main(sys.argv))
