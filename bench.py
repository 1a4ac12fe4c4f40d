"""Benchmark: 40-step Joint-CFG RF sampling of a 750-frame latent (the headline workload) on
one MI355X through libirodori_hip, plus the roofline of the dominant kernel and the CPU
oracle timed on the host's cores.

A bench "step" is one whole RF run (40 Euler steps, each one B=2 DiT forward + CFG
combine + Euler update), with its inputs already resident in HBM.  Prints one JSON line.

    python bench.py [--steps K] [--warmup W] [--no-cpu-baseline] [--cpu-threads N]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "irodori-tts-burn_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "RF ms per 40 steps @750 frames, B=2 joint CFG; attn/MLP MFMA util %"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_FP8_TFLOPS = 5000.0    # MI355X dense fp8 MFMA
PEAK_HBM_GBS = 8000.0


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "rf_config4_hbm_traffic.txt")
CODEC_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "codec_decode_hbm_traffic.txt")
CODEC_KERNELS = ("gemm_kernel", "codec_in_kernel", "codec_head_kernel", "zero_halo_kernel")
TRACE_FILE = os.path.join(ROOT, "profiles", "rf_config4_kernel_trace.md")
MFMA_FILE = os.path.join(ROOT, "profiles", "rf_config4_mfma_busy.txt")
COPY_BYTES = 1 << 30  # the --copy-calibration copy: reads and writes 1 GiB
SIMDS, SHADER_ENGINES, CLOCK_GHZ = 1024, 32, 2.4  # MI355X: 256 CUs x 4 SIMDs, 8 XCDs x 4 SEs, peak clock
EPI_NAMES = {0: "STORE", 1: "RESID", 2: "SWIGLU", 3: "QKVG", 4: "CTXKV", 5: "ADD", 6: "SNAKE", 7: "RESUNIT"}
# The block's hot kernels, keyed as the bench line's kernel_us / mfma_util: GEMMs by epilogue.
EPI_KEYS = {2: "w13_gemm", 3: "qkvg_gemm", 1: "resid_gemm"}


def kernel_info(name):
    """(key, label) of a kernel name from a rocprofv3 CSV: key is one of w13_gemm, qkvg_gemm,
    resid_gemm (W_o and W2 share the EPI_RESID instantiation), attention, or None."""
    import re
    m = re.search(r"gemm_kernelI(DF16b|DF16_|f)Li(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELb(\d)ELb(\d)E", name)
    if m:
        t = {"DF16b": "bf16", "DF16_": "f16", "f": "f32"}[m.group(1)]
        bm, bn, wm, wn, st, epi, f8, conv = (int(g) for g in m.groups()[1:])
        label = "gemm_kernel<%s%s, %dx%d, %dx%d waves, %d stages, EPI_%s%s>" % (
            t, " fp8" if f8 else "", bm, bn, wm, wn, st, EPI_NAMES.get(epi, str(epi)), ", conv" if conv else "")
        return (EPI_KEYS.get(epi) if t == "bf16" and not f8 and not conv else None), label
    m = re.search(r"attn32_kernelI(DF16b|DF16_)Li(\d+)ELi(\d+)E", name)
    if m:
        return ("attention" if m.group(1) == "DF16b" else None), "attn32_kernel<%s, %s,%s>" % (
            "bf16" if m.group(1) == "DF16b" else "f16", m.group(2), m.group(3))
    if "attn32_kernel<" in name:
        # rocprofv3 prints this instantiation's name demangled but garbled ("bool _Accum" for
        # the element type, the integer arguments dropped); the benchmark workloads run the
        # bf16 instantiation only.
        return "attention", "attn32_kernel<bf16, 2,2> (name as printed: garbled by the demangler)"
    short = name.replace("_ZN7irodori12_GLOBAL__N_1", "").replace("irodori::(anonymous namespace)::", "")
    return None, (short if len(short) <= 90 else short[:87] + "...")


def trace_summary(trace_csv, M=750, D=1024, F=2816, w13_frac=True):
    """Markdown summary of a rocprofv3 --kernel-trace CSV of this script: per kernel and grid,
    calls / total / avg / min / max; then the hot kernels' average durations, the per-dispatch
    floor (the average of scale_copy_kernel in the same trace: one pass over the 24k-float
    initial state per RF run, a launch with next to no work) and the SwiGLU
    up-projection's fraction of the bf16 peak at M rows, raw and floor-corrected."""
    import csv
    agg, names = {}, {}
    rows = list(csv.DictReader(open(trace_csv)))
    for r in rows:
        d = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0
        key = (r["Kernel_Name"], r["Grid_Size_X"], r["Workgroup_Size_X"])
        agg.setdefault(key, []).append(d)
    total = sum(sum(v) for v in agg.values())
    lines = ["| kernel | grid x | wg | calls | total ms | avg us | min us | max us | % |",
             "|---|---|---|---|---|---|---|---|---|"]
    per_key = {}
    for (n, g, wg), v in sorted(agg.items(), key=lambda kv: -sum(kv[1])):
        key, label = kernel_info(n)
        if key:
            per_key.setdefault(key, []).extend(v)
        if sum(v) >= 0.001 * total:
            lines.append("| %s | %s | %s | %d | %.2f | %.2f | %.2f | %.2f | %.2f |" % (
                label, g, wg, len(v), sum(v) / 1e3, sum(v) / len(v), min(v), max(v), 100 * sum(v) / total))
    floor = [d for (n, g, wg), v in agg.items() if "scale_copy_kernel" in n for d in v]
    lines.append("")
    for key in ("w13_gemm", "qkvg_gemm", "resid_gemm", "attention"):
        v = per_key.get(key, [])
        if v:
            lines.append("avg_us.%s: %.3f  (%d dispatches)" % (key, sum(v) / len(v), len(v)))
    fl = sum(floor) / len(floor) if floor else 0.0
    lines.append("floor_us.scale_copy_kernel: %.3f" % fl)
    # irodori_profile_layer's phase: its back-to-back launches of one kernel (the runs of at
    # least 8 identical consecutive dispatches; the RF graphs never repeat a kernel).  In
    # launch order: QKVG, attention, W_o, W13, W2 (W_o and W2 share the EPI_RESID kernel).
    runs = []
    for r in sorted(rows, key=lambda r: int(r["Start_Timestamp"])):
        d = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0
        if runs and runs[-1][0] == r["Kernel_Name"]:
            runs[-1][1].append(d)
        else:
            runs.append((r["Kernel_Name"], [d]))
    prof = {}
    for n, v in runs:
        key = kernel_info(n)[0]
        if key and len(v) >= 8:
            if key == "resid_gemm":
                key = "wo_gemm" if "wo_gemm" not in prof else "w2_gemm"
            prof.setdefault(key, v)
    flops = {"qkvg_gemm": 2.0 * M * D * 4 * D, "wo_gemm": 2.0 * M * D * D, "w13_gemm": 2.0 * M * D * 2 * F,
             "w2_gemm": 2.0 * M * F * D, "attention": 4.0 * 16 * M * (M + 256 + 375) * 64}
    if prof:
        lines.append("")
        lines.append("irodori_profile_layer phase (back-to-back launches, one kernel at a time%s):"
                     % (", M = %d" % M if w13_frac else ""))
        for key in ("qkvg_gemm", "attention", "wo_gemm", "w13_gemm", "w2_gemm"):
            v = prof.get(key)
            if v:
                avg = sum(v) / len(v)
                frac = ("; %.4f of the bf16 peak" % (flops[key] / (avg * 1e-6) / (PEAK_BF16_TFLOPS * 1e12))
                        if w13_frac else "")
                lines.append("profile_avg_us.%s: %.3f  (%d launches%s)" % (key, avg, len(v), frac))
        if w13_frac and prof.get("wo_gemm") and prof.get("w2_gemm"):
            t = sum(prof["wo_gemm"]) / len(prof["wo_gemm"]) + sum(prof["w2_gemm"]) / len(prof["w2_gemm"])
            lines.append("resid_frac_at_M%d: %.4f  (W_o + W2 algorithmic FLOPs over their summed averages)"
                         % (M, (flops["wo_gemm"] + flops["w2_gemm"]) / (t * 1e-6) / (PEAK_BF16_TFLOPS * 1e12)))
    if w13_frac and per_key.get("w13_gemm"):
        v = per_key["w13_gemm"]
        avg = sum(v) / len(v)
        fl_ = 2.0 * M * D * 2 * F / 1e12 / PEAK_BF16_TFLOPS
        lines.append("w13_frac_at_M%d: %.4f" % (M, fl_ / (avg * 1e-6)))
        lines.append("w13_frac_at_M%d_floor_corrected: %.4f" % (M, fl_ / ((avg - fl) * 1e-6)))
    return "\n".join(lines)


def mfma_summary(pmc_csv, M=750, D=1024, F=2816, H=16, Dh=64, T=1381):
    """MFMA busy figures from a rocprofv3 --pmc run of this script collecting
    SQ_VALU_MFMA_BUSY_CYCLES (per SIMD, summed), SQ_BUSY_CYCLES (per shader engine, summed),
    SQ_INSTS_VALU_MFMA_MOPS_BF16 (bf16 MFMA FLOPs / 512) and GRBM_GUI_ACTIVE: per hot kernel,
    busy = MFMA busy SIMD-cycles / (SIMDs x the shader engines' mean active cycles), i.e. the
    fraction of the time with waves resident that the matrix cores are busy; and the counted
    MFMA FLOPs per dispatch beside the algorithmic ones at M rows."""
    import csv
    per = {}
    for r in csv.DictReader(open(pmc_csv)):
        key, _ = kernel_info(r["Kernel_Name"])
        if not key:
            continue
        d = per.setdefault(key, {}).setdefault(r["Dispatch_Id"], {})
        d[r["Counter_Name"]] = float(r["Counter_Value"])
        d["ns"] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
    algo = {"w13_gemm": 2.0 * M * D * 2 * F, "qkvg_gemm": 2.0 * M * D * 4 * D,
            "resid_gemm": None, "attention": 4.0 * H * M * T * Dh}
    lines = ["%-11s %6s %16s %14s %14s %8s %14s %14s" % (
        "kernel", "disp", "MFMA busy/disp", "SE active cyc", "GUI active cyc", "busy", "MFMA GFLOP", "algo GFLOP")]
    out = []
    for key in ("w13_gemm", "qkvg_gemm", "resid_gemm", "attention"):
        ds = [d for d in per.get(key, {}).values() if "SQ_VALU_MFMA_BUSY_CYCLES" in d and "SQ_BUSY_CYCLES" in d]
        if not ds:
            continue
        n = len(ds)
        busy = sum(d["SQ_VALU_MFMA_BUSY_CYCLES"] for d in ds) / n
        se = sum(d["SQ_BUSY_CYCLES"] for d in ds) / n / SHADER_ENGINES
        gui = sum(d.get("GRBM_GUI_ACTIVE", 0.0) for d in ds) / n
        mops = sum(d.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", 0.0) for d in ds) / n * 512
        ratio = busy / (SIMDS * se) if se else 0.0
        a = algo[key]
        lines.append("%-11s %6d %16.0f %14.0f %14.0f %8.4f %14.3f %14s" % (
            key, n, busy, se, gui, ratio, mops / 1e9, "%.3f" % (a / 1e9) if a else "W_o|W2"))
        out.append("mfma_busy.%s: %.4f" % (key, ratio))
    return "\n".join(lines + [""] + out)


def stall_summary(*pmc_csvs):
    """Where the hot kernels' waves spend their resident time, from rocprofv3 --pmc runs of
    this script (any split of SQ_WAVE_CYCLES, SQ_WAIT_ANY, SQ_WAIT_INST_ANY,
    SQ_ACTIVE_INST_ANY, SQ_WAVES, SQ_INSTS_{VALU,SALU,MFMA,LDS,VMEM_RD},
    SQ_LDS_BANK_CONFLICT, SQ_VALU_MFMA_COEXEC_CYCLES over the passes).  The wait and active
    counters are wave-cycles (quad-cycle units, like SQ_WAVE_CYCLES), so their ratios to
    SQ_WAVE_CYCLES are fractions of the waves' resident time: WAIT_ANY = waiting on a
    dependency (s_waitcnt on memory or LDS, s_barrier), WAIT_INST_ANY = ready but not issued
    (issue port or matrix core busy).  Instruction counts are per wave."""
    import csv
    per = {}
    for path in pmc_csvs:
        for r in csv.DictReader(open(path)):
            key, _ = kernel_info(r["Kernel_Name"])
            if not key:
                continue
            acc = per.setdefault(key, {})
            tot = acc.setdefault(r["Counter_Name"], [0.0, set()])
            tot[0] += float(r["Counter_Value"])
            tot[1].add((path, r["Dispatch_Id"]))
    def avg(acc, c):
        v = acc.get(c)
        return v[0] / len(v[1]) if v and v[1] else None
    cols = ("wait dep", "wait issue", "active", "VALU/wave", "SALU/wave", "MFMA/wave", "LDS/wave",
            "VMEM rd/wave", "LDS bank confl.")
    lines = ["| kernel | " + " | ".join(cols) + " |", "|---|" + "---|" * len(cols)]
    for key in ("w13_gemm", "qkvg_gemm", "resid_gemm", "attention"):
        acc = per.get(key)
        if not acc:
            continue
        wc, waves = avg(acc, "SQ_WAVE_CYCLES"), avg(acc, "SQ_WAVES")
        def frac(c):
            v = avg(acc, c)
            return "%.2f" % (v / wc) if v is not None and wc else "-"
        def pw(c):
            v = avg(acc, c)
            return "%.0f" % (v / waves) if v is not None and waves else "-"
        bank = avg(acc, "SQ_LDS_BANK_CONFLICT")
        lines.append("| %s | %s | %s | %s | %s | %s | %s | %s | %s | %s |" % (
            key, frac("SQ_WAIT_ANY"), frac("SQ_WAIT_INST_ANY"), frac("SQ_ACTIVE_INST_ANY"),
            pw("SQ_INSTS_VALU"), pw("SQ_INSTS_SALU"), pw("SQ_INSTS_MFMA"), pw("SQ_INSTS_LDS"),
            pw("SQ_INSTS_VMEM_RD"), "-" if bank is None else "%.0f" % bank))
    return "\n".join(lines)


def marker_summary(marker_csv):
    """Per-range host durations of a rocprofv3 --marker-trace CSV of this script run with
    IRODORI_ROCTX=1 (the library's ranges carry the reference's NVTX names,
    src/profiling.rs:29-92).  Ranges bracket host work: graph capture for the per-block ranges,
    the per-evaluation graph launch for the sampler's."""
    import collections
    import csv
    dur = collections.defaultdict(list)
    first = {}
    with open(marker_csv) as f:
        for i, r in enumerate(csv.DictReader(f)):
            name = r["Function"]
            dur[name].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
            first.setdefault(name, (int(r["Start_Timestamp"]), i))
    lines = ["| range | count | avg us | min us | max us |", "|---|---|---|---|---|"]
    for name in sorted(dur, key=lambda n: first[n]):
        v = dur[name]
        lines.append("| %s | %d | %.1f | %.1f | %.1f |" % (name, len(v), sum(v) / len(v), min(v), max(v)))
    return "\n".join(lines)


def read_profile_value(path, key):
    """The number after `key:` in a committed profile summary, or None."""
    try:
        for line in open(path):
            if line.startswith(key + ":"):
                return float(line.split(":", 1)[1].split()[0])
    except OSError:
        pass
    return None


def log(msg):
    print("[bench] " + msg, file=sys.stderr, flush=True)


def pmc_summary(fetch_csv, write_csv):
    """Text summary of two rocprofv3 --pmc runs of this script (FETCH_SIZE, then
    WRITE_SIZE, with --copy-calibration): per-kernel KiB per dispatch, the scale factors
    that make the 1 GiB copy read 1 GiB and write 1 GiB, and the calibrated HBM bytes per
    launch of the SwiGLU up-projection GEMM."""
    import csv
    per = {}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        for r in csv.DictReader(open(path)):
            if r["Counter_Name"] != counter:
                continue
            per.setdefault(counter, {}).setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
    lines, factor = [], {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        copies = per[counter].get("__amd_rocclr_copyBuffer", [])
        kib = max(copies) if copies else 0.0
        if kib < 0.25 * COPY_BYTES / 1024:
            raise SystemExit("no 1 GiB calibration copy in %s (run with --copy-calibration)" % counter)
        factor[counter] = COPY_BYTES / (kib * 1024.0)
        lines.append("%s calibration: the 1 GiB copy counts %.1f KiB -> factor %.4f bytes per counted byte"
                     % (counter, kib, factor[counter]))
    lines.append("")
    lines.append("%-72s %6s %14s %14s %12s" % ("kernel", "calls", "FETCH KiB/disp", "WRITE KiB/disp", "MB/disp cal."))
    names = sorted(set(per["FETCH_SIZE"]) | set(per["WRITE_SIZE"]),
                   key=lambda n: -sum(per["FETCH_SIZE"].get(n, [0.0])) / max(len(per["FETCH_SIZE"].get(n, [1])), 1))
    w13 = None
    hot = {}
    for n in names:
        f = per["FETCH_SIZE"].get(n, [0.0])
        wv = per["WRITE_SIZE"].get(n, [0.0])
        fa, wa = sum(f) / len(f), sum(wv) / len(wv)
        cal = (fa * factor["FETCH_SIZE"] + wa * factor["WRITE_SIZE"]) * 1024.0
        short = n.replace("_ZN7irodori12_GLOBAL__N_1", "").replace("irodori::(anonymous namespace)::", "")
        short = short if len(short) <= 72 else short[:69] + "..."
        lines.append("%-72s %6d %14.1f %14.1f %12.2f" % (short, len(f), fa, wa, cal / 1e6))
        key = kernel_info(n)[0]
        if key:
            hot[key] = (fa * factor["FETCH_SIZE"] * 1024.0, wa * factor["WRITE_SIZE"] * 1024.0)
    if "resid_gemm" not in hot:
        raise SystemExit("no bf16 EPI_RESID GEMM kernel in the counter files")
    lines.append("")
    for key in ("qkvg_gemm", "attention", "resid_gemm", "w13_gemm"):
        if key in hot:
            lines.append("traffic_bytes.%s: %d  (fetch %d + write %d per launch)"
                         % (key, round(sum(hot[key])), round(hot[key][0]), round(hot[key][1])))
    lines.append("traffic_bytes_per_launch: %d" % round(sum(hot["resid_gemm"])))
    return "\n".join(lines)


def pmc_codec_summary(fetch_csv, write_csv, rows=2):
    """Whole-decode HBM traffic from two rocprofv3 --pmc runs of `--workload codec
    --copy-calibration` (FETCH_SIZE, then WRITE_SIZE): the calibrated bytes of every decode
    kernel (convolution GEMMs, out_proj, halo clears, head), per decode of `rows` rows."""
    import csv
    per = {}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        for r in csv.DictReader(open(path)):
            if r["Counter_Name"] == counter:
                per.setdefault(counter, {}).setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
    lines, factor = [], {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        copies = per[counter].get("__amd_rocclr_copyBuffer", [])
        kib = max(copies) if copies else 0.0
        if kib < 0.25 * COPY_BYTES / 1024:
            raise SystemExit("no 1 GiB calibration copy in %s (run with --copy-calibration)" % counter)
        factor[counter] = COPY_BYTES / (kib * 1024.0)
        lines.append("%s calibration: the 1 GiB copy counts %.1f KiB -> factor %.4f bytes per counted byte"
                     % (counter, kib, factor[counter]))
    heads = [n for n in per["FETCH_SIZE"] if "codec_head_kernel" in n]
    if not heads:
        raise SystemExit("no codec_head_kernel dispatch in the counter files")
    decodes = len(per["FETCH_SIZE"][heads[0]]) / rows
    lines.append("decodes in the run: %g (%d rows each)" % (decodes, rows))
    lines.append("")
    lines.append("%-72s %6s %14s %14s" % ("kernel (decode kernels only)", "calls", "read MB/decode", "write MB/decode"))
    tot_r = tot_w = 0.0
    for n in sorted(per["FETCH_SIZE"], key=lambda n: -sum(per["FETCH_SIZE"][n])):
        if not any(k in n for k in CODEC_KERNELS):
            continue
        rd = sum(per["FETCH_SIZE"][n]) * 1024.0 * factor["FETCH_SIZE"] / decodes
        wr = sum(per["WRITE_SIZE"].get(n, [0.0])) * 1024.0 * factor["WRITE_SIZE"] / decodes
        tot_r += rd
        tot_w += wr
        short = n.replace("_ZN7irodori12_GLOBAL__N_1", "")
        short = short if len(short) <= 72 else short[:69] + "..."
        lines.append("%-72s %6d %14.1f %14.1f" % (short, len(per["FETCH_SIZE"][n]), rd / 1e6, wr / 1e6))
    lines.append("")
    lines.append("decode_read_bytes: %d" % round(tot_r))
    lines.append("decode_write_bytes: %d" % round(tot_w))
    lines.append("traffic_bytes_per_decode: %d" % round(tot_r + tot_w))
    return "\n".join(lines)


def read_traffic(path=TRAFFIC_FILE, key="traffic_bytes_per_launch:"):
    """Calibrated HBM bytes from a committed PMC summary (per w13 launch by default), or None."""
    try:
        for line in open(path):
            if line.startswith(key):
                return int(line.split(":", 1)[1].split()[0])
    except OSError:
        pass
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--cpu-steps", type=int, default=6,
                    help="Euler steps of the CPU oracle timed after one warm-up step (at least 2)")
    ap.add_argument("--profile-iters", type=int, default=50)
    ap.add_argument("--cfg5-dtype", choices=["fp8", "bf16"], default="fp8",
                    help="compute mode of --workload cfg5 (config 5 names fp8 weights)")
    ap.add_argument("--workload", choices=["cfg4", "cfg2", "cfg3", "cfg5", "encode", "codec", "a6000"],
                    default="cfg4",
                    help="cfg4 (default): the headline B=2 Joint-CFG RF run; cfg2: the isolated joint "
                         "attention operator; cfg3: the isolated SwiGLU MLP half of a block; cfg5: batched "
                         "throughput, 16 utterances x 2 CFG rows, lengths U[200,750] padded; "
                         "encode: per-request conditioning; codec: DACVAE decode of config 4's "
                         "two 750-frame latents; a6000: the published RTX A6000 benchmark's "
                         "request (500M-v2 shape, Independent CFG, encoders included) as context")
    ap.add_argument("--codec-dtype", choices=["bf16", "f32"], default="bf16",
                    help="compute mode of --workload codec")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run one 1 GiB device-to-device copy (the known-size kernel that "
                         "scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings; 32x the L2, so "
                         "cache residency does not skew it)")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="print the calibrated traffic summary of two rocprofv3 --pmc "
                         "counter_collection.csv files of this script and exit")
    ap.add_argument("--trace-summary", metavar="KERNEL_TRACE_CSV",
                    help="print the summary of a rocprofv3 --kernel-trace CSV of this script and exit")
    ap.add_argument("--stall-summary", nargs="+", metavar="COUNTER_CSV",
                    help="print the wave stall / instruction-mix summary of rocprofv3 --pmc CSVs of "
                         "this script and exit")
    ap.add_argument("--marker-summary", metavar="MARKER_API_TRACE_CSV",
                    help="print the roctx range summary of a rocprofv3 --marker-trace CSV of this "
                         "script (run with IRODORI_ROCTX=1) and exit")
    ap.add_argument("--mfma-summary", metavar="COUNTER_CSV",
                    help="print the MFMA-busy summary of a rocprofv3 --pmc CSV of this script "
                         "(SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CYCLES SQ_INSTS_VALU_MFMA_MOPS_BF16 "
                         "GRBM_GUI_ACTIVE) and exit")
    args = ap.parse_args()
    if args.pmc_summary:
        print(pmc_codec_summary(*args.pmc_summary) if args.workload == "codec" else pmc_summary(*args.pmc_summary))
        return
    if args.trace_summary:
        # The W13 fraction lines are the headline's (config 4, one CFG row per launch).
        print(trace_summary(args.trace_summary, w13_frac=args.workload == "cfg4"))
        return
    if args.mfma_summary:
        print(mfma_summary(args.mfma_summary))
        return
    if args.stall_summary:
        print(stall_summary(*args.stall_summary))
        return
    if args.marker_summary:
        print(marker_summary(args.marker_summary))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the RF step of one model instance "
              "runs on one MI355X; multi-GPU sharding is by utterance and is not part of this "
              "build). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import irodori_hip as ih

    if args.workload == "cfg5":
        print(json.dumps(run_cfg5(args, np, torch, ih)), flush=True)
        return
    if args.workload in ("cfg2", "cfg3"):
        print(json.dumps(run_isolated(args, np, torch, ih)), flush=True)
        return
    if args.workload == "encode":
        print(json.dumps(run_encode(args, np, torch, ih)), flush=True)
        return
    if args.workload == "codec":
        print(json.dumps(run_codec(args, np, torch, ih)), flush=True)
        return
    if args.workload == "a6000":
        print(json.dumps(run_a6000(args, np, torch, ih)), flush=True)
        return

    cfg = ih.cfg_full_rf()
    U, S, Tt, Ts, N, SCALE = 1, 750, 256, 375, 40, 3.0
    log("generating seeded random-init weights (12 x d1024) and inputs")
    w = ih.DitWeights.random(cfg, 0)
    ctx = ih.make_context_kv(cfg, U, Tt, Ts, seed=1)
    x0 = ih.make_noise(U, S, cfg.latent_dim, 2)
    g = ih.GuidanceConfig(mode=ih.CfgGuidanceMode.JOINT, scale_text=SCALE, scale_speaker=SCALE,
                          min_t=0.0, max_t=1.0)
    params = ih.SamplerParams(num_steps=N, guidance=g)

    log("creating HIP context and ingesting weights")
    eng = ih.HipInferenceEngine(cfg, ih.InferenceBackendKind.HIP_BF16, max_rows=2 * U,
                                max_seq=S, max_ctx=Tt + Ts)
    eng.load_weights(w)
    eng.set_context_kv(ctx)
    d_x0 = torch.from_numpy(x0).to("cuda")
    d_out = torch.empty_like(d_x0)
    torch.cuda.synchronize()

    for i in range(args.warmup):
        eng.sample_device(d_x0.data_ptr(), d_out.data_ptr(), U, S, params)
    torch.cuda.synchronize()
    log("warmup done (%d runs); timing %d runs" % (args.warmup, args.steps))
    times = []
    for i in range(args.steps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        eng.sample_device(d_x0.data_ptr(), d_out.data_ptr(), U, S, params)
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t0) * 1e3)
    ms = float(np.mean(times))
    log("RF run: mean %.2f ms, p50 %.2f ms, min %.2f ms" % (ms, float(np.median(times)), min(times)))
    out = d_out.cpu().numpy()
    assert np.all(np.isfinite(out)), "non-finite sampler output"

    # Per-kernel device time (HIP events on the context's stream) at the RF graph's launch
    # shape: one CFG row per role chain (M = S), weights cycling through the 12 layers.
    kt = eng.profile_layer(U, S, args.profile_iters)
    if args.copy_calibration:
        src = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    log("kernel us: " + ", ".join("%s=%.1f" % (k, v) for k, v in kt.items()))
    M, D, F, H, Dh = U * S, cfg.model_dim, cfg.mlp_hidden, cfg.num_heads, cfg.head_dim
    flops = {
        "qkvg_gemm": 2.0 * M * D * 4 * D,
        "wo_gemm": 2.0 * M * D * D,
        "w13_gemm": 2.0 * M * D * 2 * F,
        "w2_gemm": 2.0 * M * F * D,
        # the conditioned row (the profiled chain): every latent and context key
        "attention": 4.0 * U * H * S * (S + Tt + Ts) * Dh,
    }
    util = {k: flops[k] / (kt[k + "_us"] * 1e-6) / (PEAK_BF16_TFLOPS * 1e12) for k in flops}
    mlp_util = (flops["w13_gemm"] + flops["w2_gemm"]) / (
        (kt["w13_gemm_us"] + kt["w2_gemm_us"]) * 1e-6) / (PEAK_BF16_TFLOPS * 1e12)
    # The roofline kernel is the one with the largest share of the step's kernel time: the
    # EPI_RESID GEMM, launched twice per block and chain (W_o and W2).  Its achieved rate is
    # the two launches' FLOPs over their summed event times.
    dom_flops = flops["wo_gemm"] + flops["w2_gemm"]
    dom_us = kt["wo_gemm_us"] + kt["w2_gemm_us"]
    achieved = dom_flops / (dom_us * 1e-6) / 1e12
    T = Tt + Ts
    # Minimum HBM bytes per launch: operands, weights and outputs once each (bf16 unless
    # noted; the residual x f32 read and written; Hn the next norm's operand, rstat its row
    # partial sums).
    alg = {
        "qkvg_gemm": 2 * (M * D + 4 * D * D + 3 * M * D + H * Dh * ((M + 63) // 64 * 64)) + M * (D // 32) * 4,
        "attention": 2 * (M * D * 3 + H * Dh * ((M + 63) // 64 * 64) + 2 * H * T * Dh + M * D),
        "wo_gemm": 2 * (M * D + D * D) + 8 * M * D + 2 * M * D + 4 * M * (D // 32),
        "w13_gemm": 2 * (M * D + 2 * F * D + M * F),
        "w2_gemm": 2 * (M * F + F * D) + 8 * M * D + 2 * M * D + 4 * M * (D // 32),
    }
    alg["resid_gemm"] = (alg["wo_gemm"] + alg["w2_gemm"]) // 2  # per launch, the two alternating
    norm_bytes = M * D * 4 + M * D * 2  # read x f32, write h bf16
    norm_gbs = norm_bytes / (kt["norm_mod_us"] * 1e-6) / 1e9
    peak_meas = achievable_bf16_peak(torch)
    log("achievable dense bf16 (large square GEMM): %.0f TFLOP/s = %.3f of the published peak"
        % (peak_meas["tflops"], peak_meas["frac_of_peak"]))

    # Every hot kernel at the RF launch shape: event time (this run), the committed trace's
    # average over the same back-to-back launches, both as fractions of the bf16 peak, and
    # the committed HBM traffic against the algorithmic bytes.
    hot = {}
    for k in ("qkvg_gemm", "attention", "wo_gemm", "w13_gemm", "w2_gemm"):
        tr_us = read_profile_value(TRACE_FILE, "profile_avg_us." + k)
        pk = "resid_gemm" if k in ("wo_gemm", "w2_gemm") else k
        traffic = read_traffic(key="traffic_bytes.%s:" % pk)
        ab = alg[pk]
        hot[k] = {"events_us": round(kt[k + "_us"], 2), "trace_us": tr_us,
                  "frac_events": round(flops[k] / (kt[k + "_us"] * 1e-6) / (PEAK_BF16_TFLOPS * 1e12), 4),
                  "frac_trace": round(flops[k] / (tr_us * 1e-6) / (PEAK_BF16_TFLOPS * 1e12), 4) if tr_us else None,
                  "traffic_bytes": traffic, "algorithmic_bytes": alg[k],
                  "traffic_ratio": round(traffic / ab, 3) if traffic else None,
                  "mfma_busy": read_profile_value(MFMA_FILE, "mfma_busy." + pk)}

    cpu = None
    if not args.no_cpu_baseline:
        from oracle.oracle import Oracle, get_threads, set_threads
        if args.cpu_threads:
            set_threads(args.cpu_threads)
        c, u = ctx.rows([0]), ctx.rows([1])
        orc = Oracle("f32")
        K = max(2, args.cpu_steps)
        log("timing the CPU oracle (f32, %d threads): 1 warm-up step, then %d of 40 Euler steps"
            % (get_threads(), K))
        orc.sample_joint_cfg(cfg, w, x0, (c.k, c.v, c.mask), (u.k, u.v, u.mask), N, SCALE, 0.0,
                             1.0, max_steps_run=1)
        t0 = time.perf_counter()
        _, ran = orc.sample_joint_cfg(cfg, w, x0, (c.k, c.v, c.mask), (u.k, u.v, u.mask), N,
                                      SCALE, 0.0, 1.0, max_steps_run=K)
        total_s = time.perf_counter() - t0
        assert ran == K, "oracle ran %d steps, expected %d" % (ran, K)
        step_s = total_s / K
        cpu = {"value": round(step_s * N * 1e3, 1), "unit": "ms (extrapolated 40-step RF run)",
               "cores": get_threads(), "kind": "port", "cpu_model": cpu_model(),
               "sample": "%d of 40 Joint-CFG Euler steps at config 4 (cond + uncond forward, B=1 "
                         "each, f32 C oracle, OpenMP) after one untimed warm-up step: %.2f s, "
                         "%.3f s per step, x40" % (K, total_s, step_s)}
        log("CPU oracle: %.2f s per step -> %.0f ms per RF run" % (step_s, step_s * N * 1e3))

    rec = {
        "metric": METRIC,
        "value": round(ms, 3),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded random-init DiT (all Linear N(0,0.02)), N(0,1) noise and "
                "context K/V, text valid length U[32,256]",
        "config": {"workload": "BASELINE config 4: 12-layer d1024 DiT, 16x64 heads, SwiGLU 2816, "
                               "latent 32; B=2 Joint CFG (scale 3, min_t 0), 750 frames, 256 "
                               "text + 375 speaker context keys, 40 Euler steps, hipGraph step",
                   "global_batch": 2, "seq_len": S, "rf_steps": N, "parallelism": "none"},
        "tokens_per_s": round(S * N * 2 / (ms * 1e-3), 1),
        "latent_frames_per_s": round(S * N / (ms * 1e-3), 1),
        "mfma_util": {"attention": round(util["attention"], 4), "mlp": round(mlp_util, 4),
                      "qkvg_gemm": round(util["qkvg_gemm"], 4), "wo_gemm": round(util["wo_gemm"], 4),
                      "w13_gemm": round(util["w13_gemm"], 4), "w2_gemm": round(util["w2_gemm"], 4)},
        "kernel_us": {k: round(v, 2) for k, v in kt.items()},
        "mfma_busy": {k: read_profile_value(MFMA_FILE, "mfma_busy." + k)
                      for k in ("attention", "qkvg_gemm", "resid_gemm", "w13_gemm")},
        "mfma_busy_note": "SQ_VALU_MFMA_BUSY_CYCLES / (1024 SIMDs x mean shader-engine active cycles) per "
                          "dispatch, from the committed rocprofv3 --pmc summary; resid_gemm = W_o and W2",
        "norm_mod_hbm_gbs": round(norm_gbs, 1),
        "norm_mod_note": "unfused adaLN kernel (the bf16 RF chains fold it into their GEMMs), x f32 read + "
                         "h bf16 write, each launch on its own buffers from a >= 640 MB pool (cold HBM)",
        "roofline": {"kernel": "gemm_kernel<bf16, EPI_RESID>: W_o (%dx1024x1024) and W2 (%dx2816x1024), the "
                               "largest share of the step's kernel time; one CFG row per launch as the RF "
                               "graph launches it" % (M, M), "bound": "mfma",
                     "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": read_traffic(),
                     "traffic_unit": "bytes per launch, the W_o / W2 average (rocprofv3 FETCH_SIZE + "
                                     "WRITE_SIZE, copy-calibrated; profiles/rf_config4_hbm_traffic.txt)",
                     "algorithmic_bytes": alg["resid_gemm"],
                     "rocprof": {"avg_us_wo": read_profile_value(TRACE_FILE, "profile_avg_us.wo_gemm"),
                                 "avg_us_w2": read_profile_value(TRACE_FILE, "profile_avg_us.w2_gemm"),
                                 "frac": read_profile_value(TRACE_FILE, "resid_frac_at_M750"),
                                 "source": "profiles/rf_config4_kernel_trace.md (rocprofv3 kernel trace of this "
                                           "script, its irodori_profile_layer phase: the same back-to-back "
                                           "launches the event figures time)"},
                     "hot_kernels": hot,
                     "achievable_peak": peak_meas},
        "cpu_baseline": cpu,
    }
    eng.close()
    print(json.dumps(rec), flush=True)


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo) and logical CPU count."""
    name = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    name = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return "%s (%d logical CPUs visible)" % (name, os.cpu_count() or 0)


def time_on_stream(torch, fn, warmup, steps):
    """Average ms per call of fn(stream_handle), HIP events on a default-priority torch stream
    (the one the calls are enqueued on)."""
    st = torch.cuda.Stream()
    torch.cuda.synchronize()
    for _ in range(warmup):
        fn(st.cuda_stream)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(steps):
        fn(st.cuda_stream)
    e1.record(st)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def achievable_bf16_peak(torch, n=8192, reps=10):
    """The dense bf16 rate a large square GEMM reaches on this GPU: torch.matmul (the ROCm
    BLAS library) on contiguous n x n bf16 operands, HIP events over reps calls after two
    warm-up calls.  A reference point for the roofline fractions (they stay against the
    published peak); not part of the timed RF run."""
    a = torch.randn((n, n), device="cuda", dtype=torch.bfloat16)
    b = torch.randn((n, n), device="cuda", dtype=torch.bfloat16)
    c = torch.empty((n, n), device="cuda", dtype=torch.bfloat16)
    for _ in range(2):
        torch.matmul(a, b, out=c)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()  # torch's current stream, the one the products run on
    for _ in range(reps):
        torch.matmul(a, b, out=c)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    tflops = 2.0 * n ** 3 / (ms * 1e-3) / 1e12
    del a, b, c
    return {"gemm": "torch.matmul bf16 %dx%dx%d (ROCm BLAS), contiguous operands" % (n, n, n),
            "ms": round(ms, 3), "tflops": round(tflops, 1), "frac_of_peak": round(tflops / PEAK_BF16_TFLOPS, 4)}


def run_isolated(args, np, torch, ih):
    """The block's hot kernels alone at the isolated-kernel configurations, on a one-layer
    d1024 context (bf16): cfg2 = irodori_op_joint_attention (B = 2, 16 x 64 heads, 750 latent
    queries; keys 750 latent + 256 text (valid U[32, 256]) + 375 speaker; Q/K/V ~ N(0, 1); RoPE
    on the latent keys; sigmoid gate), cfg3 = irodori_op_swiglu_mlp (1500 tokens = 2 x 750,
    1024 -> 2816 -> 1024, weights N(0, 0.02), x ~ N(0, 1), shift / scale / gate ~ N(0, 0.1) per
    row, eps 1e-6).  value = us per operator call, inputs resident in HBM."""
    import dataclasses
    cfg2 = args.workload == "cfg2"
    cfg = dataclasses.replace(ih.cfg_full_rf(), num_layers=1, norm_eps=1e-5 if cfg2 else 1e-6)
    B, S, H, Dh, D, F = 2, 750, cfg.num_heads, cfg.head_dim, cfg.model_dim, cfg.mlp_hidden
    w = ih.DitWeights.random(cfg, 7 if cfg2 else 3, norm_jitter=0.1 if cfg2 else 0.0)
    rng = np.random.default_rng(9 if cfg2 else 4)
    Tt, Ts = 256, 375
    eng = ih.HipInferenceEngine(cfg, ih.InferenceBackendKind.HIP_BF16, max_rows=B, max_seq=S,
                                max_ctx=Tt + Ts if cfg2 else 1)
    eng.load_weights(w)

    def cuda(a):
        return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to("cuda")

    if cfg2:
        ctx = ih.make_role_context(cfg, B, Tt, Ts, ["cond"], seed=8)
        eng.set_context_kv(ctx)
        q, k, v = (cuda(rng.standard_normal((B, S, H, Dh)).astype(np.float32)) for _ in range(3))
        g = cuda(rng.standard_normal((B, S, H * Dh)).astype(np.float32))
        out = torch.empty((B, S, H * Dh), dtype=torch.float32, device="cuda")
        fn = lambda st: eng.joint_attention(0, B, S, q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(),
                                            out.data_ptr(), st)
        ms = time_on_stream(torch, fn, args.warmup, args.steps)
        valid = int(ctx.mask.sum())
        flops = 4.0 * B * H * S * (S + Tt + Ts) * Dh  # every key, as the workload counts them
        useful = 4.0 * H * S * Dh * (B * S + valid)
        kernel = "joint attention operator (staging + attn32 + f32 store), B=2 x 16 heads x 750 queries x 1381 keys"
        metric = "isolated joint attention us per call (B=2, 16x64 heads, 750 q, 750+256+375 keys)"
        extra = {"valid_context_keys": valid, "useful_tflops": round(useful / (ms * 1e-3) / 1e12, 1)}
        algo_bytes = 2 * B * H * Dh * 4 * (3 * S) + B * S * H * Dh * 4 * 2  # q,k,v,gate in, out (f32)
    else:
        x = cuda(rng.standard_normal((B, S, D)).astype(np.float32))
        shift, scale, gate = (cuda((0.1 * rng.standard_normal((B, D))).astype(np.float32)) for _ in range(3))
        fn = lambda st: eng.swiglu_mlp(0, B, S, x.data_ptr(), shift.data_ptr(), scale.data_ptr(), gate.data_ptr(),
                                       st)
        ms = time_on_stream(torch, fn, args.warmup, args.steps)
        flops = 2.0 * B * S * D * 2 * F + 2.0 * B * S * F * D
        kernel = "SwiGLU MLP half (fused adaLN operand + W1|W3 + W2 gated residual, one launch set per row)"
        metric = "isolated SwiGLU MLP + adaLN us per call (1500 tokens, 1024 -> 2816 -> 1024)"
        extra = {}
        algo_bytes = 2 * (2 * F * D + F * D) + B * S * D * 4 * 2 + B * S * D * 2  # weights, x r/w, h
    eng.close()
    achieved = flops / (ms * 1e-3) / 1e12
    log("%s: %.2f us per call, %.1f TFLOP/s" % (args.workload, ms * 1e3, achieved))
    rec = {
        "metric": metric, "value": round(ms * 1e3, 2), "unit": "us", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: seeded N(0,1) activations, N(0,0.02) weights" + (
            ", N(0,1) context K/V" if cfg2 else ", N(0,0.1) modulation vectors"),
        "config": {"workload": metric, "global_batch": B, "seq_len": S, "parallelism": "none"},
        "roofline": {"kernel": kernel, "bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": None,
                     "algorithmic_bytes": int(algo_bytes)},
        "cpu_baseline": None,
    }
    rec.update(extra)
    return rec


def run_cfg5(args, np, torch, ih):
    """Batched throughput: 16 utterances x Joint CFG = 32 rows of the 12-layer d1024 DiT, latent
    lengths U[200,750] padded to 750 with the latent key mask, text valid lengths U[32,256],
    40 Euler steps; fp8 (e4m3 weights with per-output-channel f32 scales, GEMM inputs with
    power-of-two scales per 32 values, bf16 attention) or bf16.  Aggregate latent
    frames/s = sum(lengths) / RF-run seconds."""
    fp8 = args.cfg5_dtype == "fp8"
    cfg = ih.cfg_full_rf()
    U, S, Tt, Ts, N, SCALE = 16, 750, 256, 375, 40, 3.0
    rng = np.random.default_rng(5)
    lengths = rng.integers(200, S + 1, U).astype(np.int32)
    log("config 5: generating weights and inputs; lengths sum %d" % int(lengths.sum()))
    w = ih.DitWeights.random(cfg, 0)
    ctx = ih.make_context_kv(cfg, U, Tt, Ts, seed=1)
    x0 = ih.make_noise(U, S, cfg.latent_dim, 2)
    g = ih.GuidanceConfig(mode=ih.CfgGuidanceMode.JOINT, scale_text=SCALE, scale_speaker=SCALE,
                          min_t=0.0, max_t=1.0)
    params = ih.SamplerParams(num_steps=N, guidance=g)
    kind = ih.InferenceBackendKind.HIP_FP8 if fp8 else ih.InferenceBackendKind.HIP_BF16
    eng = ih.HipInferenceEngine(cfg, kind, max_rows=2 * U, max_seq=S, max_ctx=Tt + Ts)
    eng.load_weights(w)
    eng.set_context_kv(ctx)
    d_x0 = torch.from_numpy(x0).to("cuda")
    d_out = torch.empty_like(d_x0)
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        eng.sample_device(d_x0.data_ptr(), d_out.data_ptr(), U, S, params, lengths=lengths)
    torch.cuda.synchronize()
    log("warmup done (%d runs); timing %d runs" % (args.warmup, args.steps))
    times = []
    for _ in range(args.steps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        eng.sample_device(d_x0.data_ptr(), d_out.data_ptr(), U, S, params, lengths=lengths)
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t0) * 1e3)
    ms = float(np.mean(times))
    out = d_out.cpu().numpy()
    assert all(np.all(np.isfinite(out[u, :n])) for u, n in enumerate(lengths)), "non-finite output"
    log("RF run: mean %.2f ms, min %.2f ms" % (ms, min(times)))
    kt = eng.profile_layer(2 * U, S, max(5, args.profile_iters // 5))
    log("kernel us (B=32): " + ", ".join("%s=%.1f" % (k, v) for k, v in kt.items()))
    eng.close()
    M, D, F = 2 * U * S, cfg.model_dim, cfg.mlp_hidden
    w13_flops = 2.0 * M * D * 2 * F
    achieved = w13_flops / (kt["w13_gemm_us"] * 1e-6) / 1e12
    peak = PEAK_FP8_TFLOPS if fp8 else PEAK_BF16_TFLOPS
    frames = int(lengths.sum())
    H, Dh, T = cfg.num_heads, cfg.head_dim, Tt + Ts
    per_tok = 2.0 * D * (4 * D + D + 2 * F) + 2.0 * F * D  # GEMM FLOP per token per block
    useful = N * 2 * cfg.num_layers * sum(
        n * per_tok + 4.0 * H * Dh * n * (n + T) for n in lengths)  # both CFG rows, valid frames
    return {
        "metric": "RF aggregate latent frames/s, 16 utterances x 2 CFG (BASELINE config 5)",
        "value": round(frames / (ms * 1e-3), 1),
        "unit": "latent frames/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp8 (e4m3 block GEMMs; bf16 attention)" if fp8 else "bf16",
        "data": "synthetic: seeded random-init DiT (all Linear N(0,0.02)), N(0,1) noise and "
                "context K/V, latent lengths U[200,750] (seed 5), text valid length U[32,256]",
        "config": {"workload": "BASELINE config 5%s: 12-layer d1024 DiT, 16 utterances x Joint "
                               "CFG = 32 rows padded to 750 frames with the latent key mask, 256 "
                               "text + 375 speaker keys, 40 Euler steps"
                               % ("" if fp8 else " shape in bf16"),
                   "global_batch": 2 * U, "seq_len": S, "rf_steps": N, "parallelism": "none",
                   "lengths_sum": frames},
        "useful_tflops": round(useful / (ms * 1e-3) / 1e12, 1),
        "kernel_us": {k: round(v, 2) for k, v in kt.items()},
        "roofline": {"kernel": "w13_gemm (SwiGLU up-projection, %dx1024x5632)" % M,
                     "bound": "mfma", "achieved": round(achieved, 2), "peak": peak,
                     "unit": "TFLOP/s", "frac": round(achieved / peak, 4),
                     "traffic": None},
        "cpu_baseline": None,
    }


A6000_LIBTORCH_BF16_MS = 987.0  # docs/benchmarks/rtx-a6000.md:44 (RTX A6000, Rust/burn LibTorch bf16)


def run_a6000(args, np, torch, ih):
    """The reference's published full-inference benchmark request (bench_realmodel.rs:219-246,
    docs/benchmarks/rtx-a6000.md:13-36) at the 500M-v2 shape: d 1280, 12 layers, 20 x 64 heads,
    SwiGLU 3680; text and speaker encoders 1280 wide, 14 layers, 10 heads, SwiGLU 3328.  One
    request = text encoder over 4 tokens + speaker encoder over 8 reference frames (+ the mean
    token) + the context-KV build of the three Independent-CFG rows (conditioned, text dropped,
    speaker dropped: the dropped signal's keys masked out, euler_sampler.rs:41-67) + 40 Euler
    steps over 750 frames (text scale 3, speaker scale 5, CFG on the steps with t >= 0.5) + the
    latent read back to the host, as the reference times sample_euler_rf_cfg and into_data.
    The initial noise is made once and stays resident.  Random-init weights (no checkpoint)."""
    cfg = ih.cfg_published_500m()
    te, se = ih.enc_text_default(), ih.enc_speaker_default(cfg.latent_dim)
    te.vocab_size = 4096  # the embedding table's size does not change the work per token
    Tt, Tr, S, N = 4, 8, 750, 40
    log("a6000: generating random-init weights (DiT 12 x d1280; encoders 14 x 1280 each)")
    w = ih.DitWeights.random(cfg, 0)
    tw, sw = ih.EncoderWeights.random(te, 1), ih.EncoderWeights.random(se, 2)
    proj = ih.CtxProjWeights.random(cfg, te.dim, se.dim, seed=3)
    g = ih.GuidanceConfig(mode=ih.CfgGuidanceMode.INDEPENDENT, scale_text=3.0, scale_speaker=5.0,
                          min_t=0.5, max_t=1.0)
    params = ih.SamplerParams(num_steps=N, guidance=g)
    roles = params.cfg_roles(has_speaker=True)
    assert roles == ["cond", "no_text", "no_aux"]
    ids = np.zeros((1, Tt), np.int32)  # the reference's request: token ids 0, reference latent 0
    lat = np.zeros((1, Tr, se.in_dim), np.float32)
    tm, rm = np.ones((1, Tt), np.uint8), np.ones((1, Tr), np.uint8)
    tenc = ih.HipEncoder(te, ih.InferenceBackendKind.HIP_BF16, max_rows=1, max_seq=Tt)
    senc = ih.HipEncoder(se, ih.InferenceBackendKind.HIP_BF16, max_rows=1, max_seq=Tr)
    tenc.load_weights(tw)
    senc.load_weights(sw)
    eng = ih.HipInferenceEngine(cfg, ih.InferenceBackendKind.HIP_BF16, max_rows=len(roles), max_seq=S,
                                max_ctx=Tt + Tr + 1)
    eng.load_weights(w)
    eng.load_ctx_proj_weights(proj)
    del w, tw, sw, proj
    d_x0 = torch.from_numpy(ih.make_noise(1, S, cfg.latent_dim, 2)).to("cuda")
    d_out = torch.empty_like(d_x0)
    torch.cuda.synchronize()

    def request():
        ts, tmo = tenc.forward(tm, ids=ids)
        ss, smo = senc.forward(rm, latent=lat)
        none_t, none_s = np.zeros_like(tmo[0]), np.zeros_like(smo[0])
        eng.build_context_kv(0, ts[0], tmo[0], ss[0], smo[0])       # conditioned
        eng.build_context_kv(1, ts[0], none_t, ss[0], smo[0])       # text dropped
        eng.build_context_kv(2, ts[0], tmo[0], ss[0], none_s)       # speaker dropped
        eng.sample_device(d_x0.data_ptr(), d_out.data_ptr(), 1, S, params, has_speaker=True,
                          ctx_aux_start=Tt)
        return d_out.cpu().numpy()

    for _ in range(max(args.warmup, 2)):
        request()
    torch.cuda.synchronize()
    times = []
    for _ in range(args.steps):
        t0 = time.perf_counter()
        out = request()
        times.append((time.perf_counter() - t0) * 1e3)
    assert np.all(np.isfinite(out)), "non-finite sampler output"
    ms = float(np.mean(times))
    log("a6000 request: mean %.2f ms, p50 %.2f ms, min %.2f ms" % (ms, float(np.median(times)), min(times)))
    kt = eng.profile_layer(1, S, args.profile_iters)
    log("kernel us (M=750): " + ", ".join("%s=%.1f" % (k, v) for k, v in kt.items()))
    tenc.close()
    senc.close()
    eng.close()
    M, D, F = S, cfg.model_dim, cfg.mlp_hidden
    w13_flops = 2.0 * M * D * 2 * F
    achieved = w13_flops / (kt["w13_gemm_us"] * 1e-6) / 1e12
    return {
        "metric": "full-inference request ms at the published 500M-v2 shape (RTX A6000 benchmark "
                  "configuration; context, not the headline)",
        "value": round(ms, 3), "unit": "ms", "n_gpus": 1, "steps": args.steps,
        "warmup": max(args.warmup, 2), "ms_per_step": round(ms, 3), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": round(ms / A6000_LIBTORCH_BF16_MS, 4),
        "vs_baseline_note": "value / 987 ms, the reference's Rust/burn LibTorch bf16 mean on an RTX "
                            "A6000 (docs/benchmarks/rtx-a6000.md:44): other hardware, published",
        "dtype": "bf16",
        "data": "synthetic: random-init DiT, encoders and context projections (N(0,0.02)); token ids 0, "
                "reference latent 0 (as the reference's request); N(0,1) initial noise",
        "config": {"workload": "500M-v2 shape (d1280, 12 layers, 20x64 heads, SwiGLU 3680 padded to 3712, "
                               "latent 32); text encoder 4 tokens + speaker encoder 8 frames (+mean "
                               "token); Independent CFG 3 rows (text 3, speaker 5, min_t 0.5); 750 "
                               "frames; 40 Euler steps; latent read back",
                   "global_batch": 1, "seq_len": S, "rf_steps": N, "parallelism": "none"},
        "p50_ms": round(float(np.median(times)), 3), "min_ms": round(min(times), 3),
        "kernel_us": {k: round(v, 2) for k, v in kt.items()},
        "roofline": {"kernel": "w13_gemm (SwiGLU up-projection, 750x1280x7424)", "bound": "mfma",
                     "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": None},
        "cpu_baseline": None,
    }


def run_encode(args, np, torch, ih):
    """Per-request conditioning on the GPU at config 4's sizes: the reference-width text
    encoder over 256 tokens, the speaker encoder over 375 reference frames (plus its mean
    token), and the context-KV build of the 12-layer d1024 DiT from both states (one CFG row;
    the unconditioned row is zeros).  value = ms per request (encoders + context build)."""
    cfg = ih.cfg_full_rf()
    te, se = ih.enc_text_default(), ih.enc_speaker_default(cfg.latent_dim)
    te.vocab_size = 4096  # the embedding table's size does not change the work per token
    log("encode: generating weights (text and speaker encoders, 14 x 1280 each; DiT)")
    tw, sw = ih.EncoderWeights.random(te, 1), ih.EncoderWeights.random(se, 2)
    w = ih.DitWeights.random(cfg, 0)
    proj = ih.CtxProjWeights.random(cfg, te.dim, se.dim, seed=3)
    rng = np.random.default_rng(4)
    Tt, Ts = 256, 375
    ids = rng.integers(0, te.vocab_size, (1, Tt)).astype(np.int32)
    lat = rng.standard_normal((1, Ts, se.in_dim)).astype(np.float32)
    tm, sm = np.ones((1, Tt), np.uint8), np.ones((1, Ts), np.uint8)
    tenc = ih.HipEncoder(te, ih.InferenceBackendKind.HIP_BF16, max_rows=1, max_seq=Tt)
    senc = ih.HipEncoder(se, ih.InferenceBackendKind.HIP_BF16, max_rows=1, max_seq=Ts)
    tenc.load_weights(tw)
    senc.load_weights(sw)
    eng = ih.HipInferenceEngine(cfg, ih.InferenceBackendKind.HIP_BF16, max_rows=2, max_seq=750,
                                max_ctx=Tt + Ts + 1)
    eng.load_weights(w)
    eng.load_ctx_proj_weights(proj)

    import threading

    def request():
        # The two encoders are independent and own a stream each: the speaker encoder runs
        # on a second host thread (the C calls release the GIL), so their kernels overlap.
        out = {}

        def speaker():
            t = time.perf_counter()
            out["s"] = senc.forward(sm, latent=lat)
            out["s_ms"] = (time.perf_counter() - t) * 1e3

        t0 = time.perf_counter()
        th = threading.Thread(target=speaker)
        th.start()
        ts, tmo = tenc.forward(tm, ids=ids)
        te = (time.perf_counter() - t0) * 1e3
        th.join()
        t1 = time.perf_counter()
        ss, smo = out["s"]
        eng.build_context_kv(0, ts[0], tmo[0], ss[0], smo[0])
        t2 = time.perf_counter()
        return (t1 - t0) * 1e3, (t2 - t1) * 1e3, te, out["s_ms"]

    for _ in range(args.warmup):
        request()
    parts = np.array([request() for _ in range(args.steps)])
    ms = float(parts[:, :2].sum(1).mean())
    enc_ms, kv_ms, te_ms, se_ms = (float(v) for v in parts.mean(0))
    log("encode: encoders %.2f ms (text %.2f, speaker %.2f, overlapped), context build %.2f ms"
        % (enc_ms, te_ms, se_ms, kv_ms))
    # GEMM + attention FLOPs of an encoder over n tokens (TextBlock: [Wq|Wk|Wv|Wg], Wo, W1|W3, W2;
    # attention 4 n^2 E).
    def enc_flops(ec, n):
        E, F = ec.dim, ec.mlp_hidden
        return ec.num_layers * (2.0 * n * E * (4 * E + E + 2 * F) + 2.0 * n * F * E + 4.0 * n * n * E)
    kv_flops = cfg.num_layers * 2.0 * (Tt + Ts + 1) * 1280 * 2 * cfg.model_dim
    flops = enc_flops(te, Tt) + enc_flops(se, Ts) + kv_flops
    tenc.close()
    senc.close()
    eng.close()
    cpu = None
    if not args.no_cpu_baseline:
        from oracle.oracle import Oracle, get_threads, set_threads
        if args.cpu_threads:
            set_threads(args.cpu_threads)
        te1 = ih.EncoderConfig(dim=te.dim, num_layers=1, num_heads=te.num_heads, mlp_hidden=te.mlp_hidden,
                               vocab_size=te.vocab_size)
        tw1 = ih.EncoderWeights(tw.io, tw.blocks[:1])
        t0 = time.perf_counter()
        Oracle("f32").encoder_forward(te1, tw1, tm, ids=ids)
        layer_s = time.perf_counter() - t0
        cpu = {"value": round(layer_s * te.num_layers * 1e3, 1), "unit": "ms (text encoder, extrapolated)",
               "cores": get_threads(), "kind": "port",
               "sample": "1 of 14 text-encoder blocks over 256 tokens (f32 C oracle, OpenMP), measured "
                         "%.2f s, x14; the speaker encoder and context build not included" % layer_s}
    return {
        "metric": "per-request conditioning ms (text + speaker encoders + context-KV build, config 4 sizes)",
        "value": round(ms, 3), "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 3), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: random-init encoders (1280 wide, 14 blocks, 10 heads, SwiGLU 3328) and DiT, "
                "random token ids / N(0,1) reference latents",
        "config": {"workload": "text encoder 256 tokens + speaker encoder 375 frames (+ mean token), "
                               "run concurrently from two host threads, then the 12-layer context-KV "
                               "build, one CFG row; host pointers in and out",
                   "global_batch": 1, "seq_len": Tt + Ts, "parallelism": "none"},
        "parts_ms": {"encoders_overlapped": round(enc_ms, 3), "text_encoder": round(te_ms, 3),
                     "speaker_encoder": round(se_ms, 3), "context_build": round(kv_ms, 3)},
        "achieved_tflops": round(flops / (ms * 1e-3) / 1e12, 1),
        "roofline": None,
        "cpu_baseline": cpu,
    }


def codec_bytes(ccfg, T, es=2):
    """Compulsory HBM bytes of the decode's kernel sequence over T latent frames (each
    tensor read or written once per kernel that touches it; es-byte GEMM operands, f32
    residual stream): out_proj, the stem, per block the transposed convolution and three
    ResidualUnits (one kernel each: operand in, x in and out, next operand out; two kernels
    for streams wider than 192 channels: + the 1x1 operand out and in), the head."""
    b = T * ccfg.latent_dim * 4 + T * ccfg.proj_dim * es                       # out_proj
    b += T * ccfg.proj_dim * es + T * ccfg.decoder_dim * (4 + es)               # stem
    L = T
    for i, r in enumerate(ccfg.rates):
        C, O = ccfg.block_dims(i)
        b += L * C * es + L * r * O * (4 + es)                                  # transposed conv
        L *= r
        last = i == ccfg.num_blocks - 1
        for u in range(3):
            per = es + 8 + (0 if (last and u == 2) else es)
            if O > 192:
                per += 2 * es                                                   # the 1x1 operand
            b += L * O * per
    return b + L * ccfg.head_dim * 4 + L * 4                                    # head


def codec_flops(ccfg, T):
    """Algorithmic FLOPs of DacVaeCodec::decode over T latent frames (unpadded channels):
    out_proj, stem (k 7), per block the transposed convolution (two taps of C inputs per
    output frame) and three ResidualUnits (k 7 + k 1), the head (k 7 to one channel)."""
    f = 2.0 * T * ccfg.latent_dim * ccfg.proj_dim + 2.0 * T * ccfg.proj_dim * ccfg.decoder_dim * 7
    L = T
    for i, r in enumerate(ccfg.rates):
        C, O = ccfg.block_dims(i)
        L *= r
        f += 2.0 * L * O * 2 * C + 3 * (2.0 * L * O * O * 7 + 2.0 * L * O * O)
    return f + 2.0 * L * ccfg.head_dim * 7


def run_codec(args, np, torch, ih):
    """The DACVAE decode of config 4's output (codec/model.rs:60-65): two 750-frame latents
    -> two 1.44 M-sample waveforms (2 x 30 s at 48 kHz), latents already in HBM
    (irodori_codec_decode_device), timed with events on the codec's stream.
    value = ms per decode of both rows."""
    ccfg = ih.codec_default()
    backend = ih.InferenceBackendKind.HIP_BF16 if args.codec_dtype == "bf16" else ih.InferenceBackendKind.HIP_F32
    B, T = 2, 750
    log("codec: generating weights (DACVAE decoder, 1536 -> 96 over rates 12/10/8/2)")
    cw = ih.CodecWeights.random(ccfg, 1)
    codec = ih.HipDacVaeCodec(ccfg, backend, max_frames=T)
    codec.load_weights(cw)
    lat = np.random.default_rng(2).standard_normal((B, T, ccfg.latent_dim)).astype(np.float32)
    d_lat = torch.from_numpy(lat).cuda()
    d_wav = torch.empty((B, T * ccfg.hop_length), dtype=torch.float32, device="cuda")
    # A stream of its own (default priority): the events below must sit on the stream the
    # decode is enqueued on (handle 0, torch's default stream, would mean the codec's own).
    st = torch.cuda.Stream()
    torch.cuda.synchronize()
    if args.copy_calibration:  # the known-size kernel that scales the --pmc readings
        src = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    for _ in range(args.warmup):
        codec.decode_device(d_lat.data_ptr(), B, T, d_wav.data_ptr(), st.cuda_stream)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(st)
    for _ in range(args.steps):
        codec.decode_device(d_lat.data_ptr(), B, T, d_wav.data_ptr(), st.cuda_stream)
    e1.record(st)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / args.steps
    ms = e0.elapsed_time(e1) / args.steps
    flops = B * codec_flops(ccfg, T)
    samples = B * T * ccfg.hop_length
    log("codec: %.3f ms per decode (wall %.3f ms), %.1f TFLOP/s algorithmic, %.0fx real time"
        % (ms, wall, flops / (ms * 1e-3) / 1e12, samples / ccfg.sample_rate / (ms * 1e-3)))
    wav = d_wav.cpu().numpy()
    if not np.isfinite(wav).all():
        raise RuntimeError("codec produced non-finite samples")
    codec.close()
    cpu = None
    if not args.no_cpu_baseline:
        from oracle.oracle import Oracle, get_threads, set_threads
        if args.cpu_threads:
            set_threads(args.cpu_threads)
        n = 6
        t0 = time.perf_counter()
        Oracle("f32").codec_decode(ccfg, cw, lat[:1, :n])
        sec = time.perf_counter() - t0
        cpu = {"value": round(sec / n * T * B * 1e3, 1), "unit": "ms (extrapolated)",
               "cores": get_threads(), "kind": "port",
               "sample": "%d latent frames of one row (f32 C oracle, OpenMP), measured %.2f s, "
                         "scaled linearly to 2 x 750 frames" % (n, sec)}
    achieved = flops / (ms * 1e-3) / 1e12
    return {
        "metric": "DACVAE decode ms (2 x 750 latent frames -> 2 x 1.44 M samples at 48 kHz)",
        "value": round(ms, 3), "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 3), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": args.codec_dtype,
        "data": "synthetic: random-init DACVAE decoder (Snake alphas U(0.5, 2)), N(0,1) latents",
        "config": {"workload": "DACVAE decoder (out_proj 32->1024, stem 1024->1536 k7, 4 DecoderBlocks "
                               "rates 12/10/8/2 with 3 ResidualUnits each, watermark head), config 4's "
                               "two 750-frame rows; latents resident in HBM",
                   "global_batch": B, "seq_len": T, "parallelism": "none"},
        "realtime_factor": round(samples / ccfg.sample_rate / (ms * 1e-3), 1),
        "achieved_tflops": round(achieved, 1),
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS
                     if args.codec_dtype == "bf16" else 157.3, "unit": "TFLOP/s",
                     "frac": round(achieved / (PEAK_BF16_TFLOPS if args.codec_dtype == "bf16" else 157.3), 4),
                     "traffic": read_traffic(CODEC_TRAFFIC_FILE, "traffic_bytes_per_decode:"),
                     "traffic_unit": "HBM bytes per decode (rocprofv3 FETCH_SIZE + WRITE_SIZE over the decode "
                                     "kernels, copy-calibrated; profiles/codec_decode_hbm_traffic.txt)",
                     "algorithmic_bytes": B * codec_bytes(ccfg, T, 2 if args.codec_dtype == "bf16" else 4),
                     "scope": "whole decode: algorithmic convolution FLOPs (unpadded channels) over the "
                              "event-timed decode, element-wise passes included"},
        "cpu_baseline": cpu,
    }


if __name__ == "__main__":
    main()
