"""Summaries of rocprofv3 hardware-counter runs (``--pmc``, CSV output).

    python -m rl_project_amd.counters KERNEL ELEMENTS DIR [DIR ...]
    python -m rl_project_amd.counters --traffic KERNEL ALG_BYTES FETCH_DIR WRITE_DIR CAL_FETCH_DIR CAL_WRITE_DIR
    python -m rl_project_amd.counters --traffic-step STEP_KERNEL ALG_BYTES FETCH_DIR WRITE_DIR CAL_FETCH_DIR
                                      CAL_WRITE_DIR KERNEL [KERNEL ...]

reads every ``*counter_collection.csv`` under the directories (one
directory per counter pass: a pass may hold at most 8 SQ, 4 TCC, 2 TA/TD and
2 GRBM counters), keeps the dispatches whose kernel name contains ``KERNEL``,
drops the first quarter of them (warm-up), and prints the per-dispatch
median of each counter plus the ratios used to explain a kernel's time:

* instructions per wave and, per element of the launch (``ELEMENTS``: logits
  read by one dispatch), VALU / LDS lane-instructions;
* the share of wave-cycles spent issuing VALU, LDS and memory instructions
  and waiting (``SQ_WAIT_INST_ANY``, ``SQ_WAIT_INST_LDS``);
* LDS bank conflicts per active LDS cycle;
* DRAM read bytes from the request-size counters
  (32 / 64 / 128-byte ``TCC_EA0_RDREQ``), next to ``FETCH_SIZE``.

The SQ cycle counters count in units of four cycles on CDNA; only their
ratios are used."""

from __future__ import annotations

import csv
import glob
import os
import statistics
import sys
from collections import defaultdict
from typing import Dict, List


def load(dirs: List[str], kernel: str) -> Dict[str, List[float]]:
    """counter name -> per-dispatch values (summed over the rows a dispatch
    has for that counter), in dispatch order, warm-up quarter dropped."""
    per: Dict[str, Dict[int, float]] = defaultdict(dict)
    for d in dirs:
        for path in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            with open(path, newline="") as f:
                for row in csv.DictReader(f):
                    if kernel not in row["Kernel_Name"]:
                        continue
                    name = row["Counter_Name"]
                    disp = int(row["Dispatch_Id"])
                    per[name][disp] = per[name].get(disp, 0.0) + float(row["Counter_Value"])
    out: Dict[str, List[float]] = {}
    for name, by_disp in per.items():
        vals = [by_disp[k] for k in sorted(by_disp)]
        out[name] = vals[len(vals) // 4:]
    return out


def summarise(kernel: str, elements: float, dirs: List[str]) -> str:
    c = load(dirs, kernel)
    if not c:
        return f"no dispatch of a kernel matching {kernel!r} under {dirs}"
    med = {k: statistics.median(v) for k, v in c.items() if v}
    lines = [f"kernel: {kernel}", f"dispatches per counter (after warm-up): "
             f"{min(len(v) for v in c.values())}..{max(len(v) for v in c.values())}", "counters (median per dispatch):"]
    for k in sorted(med):
        lines.append(f"  {k:32s} {med[k]:.6g}")
    g = med.get
    lines.append("derived:")

    def put(label, value, fmt="{:.4g}"):
        if value is not None:
            lines.append(f"  {label:44s} " + fmt.format(value))

    waves = g("SQ_WAVES")
    if waves:
        for k in ("SQ_INSTS_VALU", "SQ_INSTS_SALU", "SQ_INSTS_LDS", "SQ_INSTS_VMEM_RD", "SQ_INSTS_SMEM"):
            if g(k) is not None:
                put(f"{k} per wave", g(k) / waves, "{:.1f}")
    if elements:
        for k in ("SQ_INSTS_VALU", "SQ_INSTS_LDS", "SQ_INSTS_LDS_ATOMIC"):
            if g(k) is not None:
                put(f"{k} lane-instructions per element", g(k) * 64.0 / elements, "{:.2f}")
    wc = g("SQ_WAVE_CYCLES")
    if wc:
        for k in ("SQ_ACTIVE_INST_VALU", "SQ_ACTIVE_INST_LDS", "SQ_ACTIVE_INST_VMEM", "SQ_WAIT_INST_ANY",
                  "SQ_WAIT_INST_LDS", "SQ_WAIT_ANY", "SQ_INST_CYCLES_VMEM_RD"):
            if g(k) is not None:
                put(f"{k} / SQ_WAVE_CYCLES", g(k) / wc, "{:.3f}")
    if g("SQ_LDS_BANK_CONFLICT") is not None and g("SQ_LDS_IDX_ACTIVE"):
        put("SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE", g("SQ_LDS_BANK_CONFLICT") / g("SQ_LDS_IDX_ACTIVE"), "{:.3f}")
    if g("SQ_LDS_ADDR_CONFLICT") is not None and g("SQ_LDS_IDX_ACTIVE"):
        put("SQ_LDS_ADDR_CONFLICT / SQ_LDS_IDX_ACTIVE", g("SQ_LDS_ADDR_CONFLICT") / g("SQ_LDS_IDX_ACTIVE"), "{:.3f}")
    if wc and waves:
        # SQ_*_CYCLES and SQ_ACTIVE_INST_* count in units of 4 cycles, summed over waves
        put("mean wave lifetime, cycles", 4.0 * wc / waves, "{:.0f}")
        for k in ("SQ_ACTIVE_INST_VALU", "SQ_ACTIVE_INST_LDS"):
            if g(k) is not None:
                put(f"{k} cycles per SIMD (1024 SIMDs)", 4.0 * g(k) / 1024.0, "{:.0f}")
    r32, r64, r128 = g("TCC_EA0_RDREQ_32B_sum"), g("TCC_EA0_RDREQ_64B_sum"), g("TCC_EA0_RDREQ_128B_sum")
    if None not in (r32, r64, r128):
        by_size = 32.0 * r32 + 64.0 * r64 + 128.0 * r128
        put("DRAM read bytes from request sizes", by_size, "{:.6g}")
        if g("TCC_EA0_RDREQ_sum"):
            put("requests counted by size / TCC_EA0_RDREQ_sum", (r32 + r64 + r128) / g("TCC_EA0_RDREQ_sum"), "{:.4f}")
            put("share of 128-byte read requests", r128 / g("TCC_EA0_RDREQ_sum"), "{:.4f}")
    if g("FETCH_SIZE") is not None:
        put("FETCH_SIZE bytes", g("FETCH_SIZE") * 1024.0, "{:.6g}")
        if None not in (r32, r64, r128) and g("FETCH_SIZE"):
            put("request-size bytes / FETCH_SIZE bytes", (32.0 * r32 + 64.0 * r64 + 128.0 * r128) /
                (g("FETCH_SIZE") * 1024.0), "{:.4f}")
    return "\n".join(lines)


def traffic(kernel: str, alg_bytes: float, fetch_dir: str, write_dir: str, cal_fetch_dir: str, cal_write_dir: str,
            cal_kernel: str = "neg_kernel", cal_bytes: float = 256.0 * (1 << 20)) -> str:
    """HBM bytes per dispatch of ``kernel`` from one FETCH_SIZE run and one
    WRITE_SIZE run (KiB per dispatch, median after the warm-up quarter), each
    scaled by the same counter's reading for a copy kernel of known size
    (``cal_kernel`` reads and writes ``cal_bytes`` per dispatch)."""
    med = lambda d, k, n: statistics.median(load([d], k)[n])  # noqa: E731
    cf, cw = med(cal_fetch_dir, cal_kernel, "FETCH_SIZE"), med(cal_write_dir, cal_kernel, "WRITE_SIZE")
    fs, ws = cal_bytes / 1024.0 / cf, cal_bytes / 1024.0 / cw
    kf_all, kw = load([fetch_dir], kernel)["FETCH_SIZE"], med(write_dir, kernel, "WRITE_SIZE")
    kf = statistics.median(kf_all)
    t = 1024.0 * (kf * fs + kw * ws)
    return "\n".join([
        f"calib_fetch_kib_median: {cf:.1f}", f"calib_write_kib_median: {cw:.1f}",
        f"fetch_scale: {fs:.5f}", f"write_scale: {ws:.5f}",
        f"kernel_fetch_kib_median: {kf:.1f}   (launches: {len(kf_all)} after the warm-up quarter)",
        f"kernel_write_kib_median: {kw:.1f}",
        f"algorithmic_bytes_per_launch: {alg_bytes:.0f}",
        f"traffic_bytes_per_launch: {t:.0f}",
        f"traffic_over_algorithmic: {t / alg_bytes:.3f}"])


def traffic_step(step_kernel: str, alg_bytes: float, fetch_dir: str, write_dir: str, cal_fetch_dir: str,
                 cal_write_dir: str, kernels: List[str], cal_kernel: str = "neg_kernel",
                 cal_bytes: float = 256.0 * (1 << 20)) -> str:
    """HBM bytes per step of a workload made of several kernels: for each
    kernel name fragment in ``kernels``, its median FETCH_SIZE / WRITE_SIZE
    per dispatch (scaled as in ``traffic``) times its dispatches per step, a
    step being one dispatch of ``step_kernel``."""
    med = lambda d, k, n: statistics.median(load([d], k)[n])  # noqa: E731
    fs = cal_bytes / 1024.0 / med(cal_fetch_dir, cal_kernel, "FETCH_SIZE")
    ws = cal_bytes / 1024.0 / med(cal_write_dir, cal_kernel, "WRITE_SIZE")
    steps = len(load([fetch_dir], step_kernel)["FETCH_SIZE"])
    lines, total = [f"fetch_scale: {fs:.5f}", f"write_scale: {ws:.5f}"], 0.0
    for k in kernels:
        fv, wv = load([fetch_dir], k)["FETCH_SIZE"], load([write_dir], k)["WRITE_SIZE"]
        per_step = len(fv) / steps
        b = 1024.0 * (statistics.median(fv) * fs + statistics.median(wv) * ws) * per_step
        total += b
        lines.append(f"{k}: fetch_kib_median {statistics.median(fv):.1f} write_kib_median {statistics.median(wv):.1f} "
                     f"launches_per_step {per_step:.2f} bytes_per_step {b:.0f}")
    lines += [f"algorithmic_bytes_per_step: {alg_bytes:.0f}", f"traffic_bytes_per_step: {total:.0f}",
              f"traffic_over_algorithmic: {total / alg_bytes:.3f}"]
    return "\n".join(lines)


def main(argv: List[str]) -> int:
    if argv and argv[0] == "--traffic-step" and len(argv) >= 9:
        print(traffic_step(argv[1], float(argv[2]), *argv[3:7], kernels=argv[7:]))
        return 0
    if argv and argv[0] == "--traffic" and len(argv) == 7:
        print(traffic(argv[1], float(argv[2]), *argv[3:7]))
        return 0
    if len(argv) < 3:
        print(__doc__, file=sys.stderr)
        return 2
    print(summarise(argv[0], float(argv[1]), argv[2:]))
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
