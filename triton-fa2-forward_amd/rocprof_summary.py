"""rocprofv3 CSV output -> the text summaries under profiles/ (counterpart of the reference's
bench/ncu_summary.py, which condenses its Nsight Compute exports).

    bash triton-fa2-forward_amd/profile_configs.sh gpurun_out/prof C3 C2 C4 C5   # on the GPU box
    python triton-fa2-forward_amd/rocprof_summary.py --root gpurun_out/prof --configs C3 C2 C4 C5

profile_configs.sh runs, per config, in runs of their own (one counter group per rocprofv3 run):
  <root>/<cfg>_trace   rocprofv3 --kernel-trace --stats  over bench.py --config <cfg>
  <root>/<cfg>_fetch   rocprofv3 --pmc FETCH_SIZE        over profile_target.py (3 launches + a
  <root>/<cfg>_write   rocprofv3 --pmc WRITE_SIZE         1 GiB device copy for the calibration)
  <root>/<cfg>_sq      rocprofv3 --pmc SQ_WAVES SQ_INSTS_MFMA ... GRBM_GUI_ACTIVE
  <root>/<cfg>_util    rocprofv3 --pmc SQ_LDS_IDX_ACTIVE SQ_ACTIVE_INST_VALU ... GRBM_GUI_ACTIVE
and this module writes, from those CSVs and the bench.py line in <root>/<cfg>_trace.log:
  profiles/attn_fwd_kernel_<cfg>_kernel_trace.md      per-kernel statistics and the timed steps
  profiles/attn_fwd_kernel_<cfg>_l2_miss_traffic.md   bytes that left L2 per launch
  profiles/attn_fwd_kernel_<cfg>_sq_counters.md       instruction mix, MFMA busy, bank conflicts
  profiles/attn_fwd_kernel_utilisation_counters.md    per-unit busy fractions, all configs
  profiles/l2_miss_traffic.json                        the traffic figures bench.py reports
and, from bench.py's JSON lines (--bench-log: `bench.py --all --sdpa --no-cpu-baseline` then
`bench.py --pack-short --no-cpu-baseline`, appended to one log), profiles/bench_all_configs.md.

L2-miss bytes: TCC FETCH_SIZE and WRITE_SIZE count, in KiB per dispatch, the requests that leave
the L2; a plain device copy of known size read by the same counters gives the factor that turns
the readings into bytes (on MI355X FETCH_SIZE reads half the copy's bytes, so it is scaled by 2).
Infinity Cache hits count as well, so the DRAM bytes are at most these figures.
"""

import argparse
import csv
import glob
import json
import os
import statistics

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
PROFILES = os.path.join(ROOT, "profiles")

ATTN = "attn_fwd_kernel"
KEY_NORM = "key_norm_kernel"
COPY = "copyBuffer"
COPY_KIB = 1 << 20   # profile_target.py --copy-mib 1024: 1 GiB read and 1 GiB written
PEAK_TFLOPS = 256 * 2.4e9 * 4096 / 1e12
HBM_GBS = 8000.0
SIMDS, XCDS, CUS = 1024, 8, 256

SQ_COUNTERS = ["SQ_WAVES", "SQ_INSTS_MFMA", "SQ_INSTS_VALU", "SQ_INSTS_LDS", "SQ_LDS_BANK_CONFLICT",
               "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_BUSY_CYCLES", "SQ_WAVE_CYCLES", "GRBM_GUI_ACTIVE"]
UTIL_COUNTERS = ["SQ_LDS_IDX_ACTIVE", "SQ_ACTIVE_INST_VALU", "SQ_VALU_MFMA_COEXEC_CYCLES",
                 "SQ_INSTS_VALU_TRANS_F32", "SQ_INST_CYCLES_SALU", "SQ_VALU_MFMA_BUSY_CYCLES",
                 "SQ_WAIT_INST_LDS", "GRBM_GUI_ACTIVE"]


def commands(root, cfg):
    """The rocprofv3 command lines profile_configs.sh runs for one config (quoted in the .md)."""
    target = (f"python3 triton-fa2-forward_amd/profile_target.py --config {cfg} --launches 3 "
              f"--copy-mib 1024")
    pmc = lambda tag, ctrs: (f"timeout -s KILL 90 rocprofv3 --pmc {' '.join(ctrs)} --output-format csv "  # noqa: E731
                             f"-d {root}/{cfg}_{tag} -o pmc -- {target}")
    return {
        "trace": (f"rocprofv3 --kernel-trace --stats --output-format csv -d {root}/{cfg}_trace -o trace "
                  f"-- python3 bench.py --config {cfg} --no-cpu-baseline --flush-iters 0"),
        "fetch": pmc("fetch", ["FETCH_SIZE"]),
        "write": pmc("write", ["WRITE_SIZE"]),
        "sq": pmc("sq", SQ_COUNTERS),
        "util": pmc("util", UTIL_COUNTERS),
    }


# ------------------------------------------------------------------------------------------
# CSV readers
# ------------------------------------------------------------------------------------------

def find_csv(directory, suffix):
    """The one rocprofv3 CSV named *<suffix> under `directory` (rocprofv3 may add a subfolder)."""
    hits = sorted(glob.glob(os.path.join(directory, "**", "*" + suffix), recursive=True))
    if not hits:
        raise FileNotFoundError(f"no *{suffix} under {directory}")
    return hits[0]


def read_rows(path):
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def kernel_stats(directory):
    """[(name, calls, average ns, min ns, max ns, percent)] from *kernel_stats.csv, as listed."""
    return [(r["Name"], int(r["Calls"]), float(r["AverageNs"]), float(r["MinNs"]), float(r["MaxNs"]),
             float(r["Percentage"])) for r in read_rows(find_csv(directory, "kernel_stats.csv"))]


def dispatches(directory, name_part):
    """[(start ns, end ns)] of the dispatches whose kernel name contains name_part, in time order,
    from *kernel_trace.csv."""
    rows = [r for r in read_rows(find_csv(directory, "kernel_trace.csv")) if name_part in r["Kernel_Name"]]
    out = [(int(r["Start_Timestamp"]), int(r["End_Timestamp"])) for r in rows]
    return sorted(out)


def pmc(directory):
    """{dispatch id: {"kernel": name, counter: value summed over the CSV's rows}} from
    *counter_collection.csv (rocprofv3 writes one row per dispatch and counter, or per
    dimension instance; the sum is the counter's value for the dispatch)."""
    out = {}
    for r in read_rows(find_csv(directory, "counter_collection.csv")):
        d = out.setdefault(int(r["Dispatch_Id"]), {"kernel": r["Kernel_Name"]})
        d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    return dict(sorted(out.items()))


def values(disp, name_part, counter):
    """The counter's value of every dispatch of a kernel, in dispatch order."""
    return [d[counter] for d in disp.values() if name_part in d["kernel"] and counter in d]


def bench_line(log_path):
    """The last bench.py JSON line of a log, or None."""
    try:
        lines = [ln for ln in open(log_path) if ln.startswith('{"metric"')]
    except OSError:
        return None
    return json.loads(lines[-1]) if lines else None


# ------------------------------------------------------------------------------------------
# derived figures
# ------------------------------------------------------------------------------------------

def copy_scales(fetch, write):
    """Scale factors of FETCH_SIZE and WRITE_SIZE from the calibration copy: its known 1 GiB each
    way (in KiB) against what each counter read for it (KiB as the counter reports them)."""
    cf, cw = values(fetch, COPY, "FETCH_SIZE"), values(write, COPY, "WRITE_SIZE")
    if not cf or not cw or cf[0] <= 0 or cw[0] <= 0:
        raise ValueError("the calibration copy (copyBuffer) is missing from the counter runs")
    return COPY_KIB / cf[0], COPY_KIB / cw[0]


def traffic(fetch, write):
    """Bytes per attention launch that left L2: mean FETCH_SIZE and WRITE_SIZE over its
    dispatches, each times the copy's factor. Returns a dict of the figures."""
    fs, ws = copy_scales(fetch, write)
    f_kib, w_kib = values(fetch, ATTN, "FETCH_SIZE"), values(write, ATTN, "WRITE_SIZE")
    if not f_kib or not w_kib:
        raise ValueError("no attention dispatch in the counter runs")
    fm, wm = statistics.fmean(f_kib), statistics.fmean(w_kib)
    return {"bytes": int(round(1024.0 * (fm * fs + wm * ws))), "fetch_kib": fm, "write_kib": wm,
            "fetch_scale": fs, "write_scale": ws, "fetch_kib_each": f_kib, "write_kib_each": w_kib}


def utilisation(c):
    """Per-unit busy fractions over the kernel's active time from one dispatch's counters
    (GRBM_GUI_ACTIVE summed over the XCDs; SQ_ACTIVE_INST_VALU, SQ_LDS_IDX_ACTIVE and
    SQ_INST_CYCLES_SALU are rocprofv3's VALUBusy, LdsUtil and SALUBusy inputs, quad-cycles
    summed over a CU's four SIMDs)."""
    active = c["GRBM_GUI_ACTIVE"] / XCDS
    return {
        "mfma_busy": c["SQ_VALU_MFMA_BUSY_CYCLES"] / SIMDS / active,
        # quad-cycles (x4) summed over a CU's four SIMDs (/4): per-SIMD busy cycles per CU
        "valu_busy": c["SQ_ACTIVE_INST_VALU"] / CUS / active,
        "mfma_with_valu": c["SQ_VALU_MFMA_COEXEC_CYCLES"] / c["SQ_VALU_MFMA_BUSY_CYCLES"],
        "lds_busy": c["SQ_LDS_IDX_ACTIVE"] / CUS / active,
        "salu_busy": c["SQ_INST_CYCLES_SALU"] / CUS / active,
        "exp_insts": c["SQ_INSTS_VALU_TRANS_F32"],
    }


def first_attn(disp):
    for d in disp.values():
        if ATTN in d["kernel"]:
            return d
    raise ValueError("no attention dispatch in the counter run")


# ------------------------------------------------------------------------------------------
# writers
# ------------------------------------------------------------------------------------------

def write_trace(root, cfg, out_dir):
    d = os.path.join(root, f"{cfg}_trace")
    stats = kernel_stats(d)
    b = bench_line(d + ".log")
    ours = [s for s in stats if ATTN in s[0]]
    lines = [f"# Kernel trace: fa2::attn_fwd_kernel on {cfg}"
             + (f" ({b['config']['workload']})" if b else ""), "",
             "Command (run from the repository root on the MI355X box, TMPDIR=/tmp):", "", "```",
             commands(root, cfg)["trace"], "```", "",
             "rocprofv3 kernel statistics (kernel_stats.csv, top rows):", "",
             "| Kernel | Calls | Average ns | Min ns | Max ns | % of GPU time |", "|---|---|---|---|---|---|"]
    for name, calls, avg, mn, mx, pct in stats[:5]:
        nm = name if len(name) < 72 else name[:69] + "..."
        lines.append(f"| `{nm}` | {calls} | {avg:.0f} | {mn:.0f} | {mx:.0f} | {pct:.1f} |")
    attn = dispatches(d, ATTN)
    kn = dispatches(d, KEY_NORM)
    if b and attn:
        K = int(b["steps"])
        # bench.py's order of launches: the gate, the settle, W warmups, the K timed steps, then
        # K steps with an event pair around each: the timed steps are the K before the last K
        timed = attn[-2 * K:-K] if len(attn) >= 2 * K else attn
        ktimed = kn[-2 * K:-K] if len(kn) >= 2 * K else []
        t_attn = statistics.fmean(e - s for s, e in timed)
        t_kn = statistics.fmean(e - s for s, e in ktimed) if ktimed else 0.0
        lines += ["", "The same run's bench.py line (under the profiler):", "",
                  f"* kernels per step: {b['roofline']['kernel']}.",
                  f"* HIP events over the {K} timed steps: {b['roofline']['avg_kernel_ms'] * 1e3:.1f} us per "
                  f"step; rocprofv3 over the same dispatches: "
                  + (f"key-norm pass {t_kn / 1e3:.1f} us + " if ktimed else "")
                  + f"attention kernel {t_attn / 1e3:.1f} us"
                  + (f" = {(t_kn + t_attn) / 1e3:.1f} us" if ktimed else "") + " per step.",
                  f"* attention kernel over all {len(attn)} dispatches (the gate, settle and warmups "
                  f"included): {ours[0][2] / 1e3:.1f} us average." if ours else "",
                  f"* value {b['value']} TFLOP/s; roofline.achieved {b['roofline']['achieved']} TFLOP/s = "
                  f"{b['config']['flops_per_step']:.6g} FLOP / HIP-event step time, frac {b['roofline']['frac']} "
                  f"of {PEAK_TFLOPS:.1f}.",
                  f"* from the trace alone: {b['config']['flops_per_step']:.6g} FLOP / {t_attn / 1e3:.1f} us = "
                  f"{b['config']['flops_per_step'] / (t_attn * 1e-9) / 1e12:.1f} TFLOP/s for the attention "
                  f"kernel, frac {b['config']['flops_per_step'] / (t_attn * 1e-9) / 1e12 / PEAK_TFLOPS:.4f}."]
    lines += ["", "Made by `python triton-fa2-forward_amd/rocprof_summary.py` from the run's CSVs.", ""]
    path = os.path.join(out_dir, f"attn_fwd_kernel_{cfg}_kernel_trace.md")
    with open(path, "w") as f:
        f.write("\n".join(lines))
    return path


def write_traffic(root, cfg, out_dir, json_path, label):
    fetch, write = pmc(os.path.join(root, f"{cfg}_fetch")), pmc(os.path.join(root, f"{cfg}_write"))
    t = traffic(fetch, write)
    b = bench_line(os.path.join(root, f"{cfg}_trace.log"))
    avg_ns = None
    try:
        avg_ns = statistics.fmean(e - s for s, e in dispatches(os.path.join(root, f"{cfg}_trace"), ATTN))
    except (FileNotFoundError, statistics.StatisticsError):
        pass
    cmd = commands(root, cfg)
    lines = [f"# L2-miss traffic: fa2::attn_fwd_kernel on {cfg}", "",
             "FETCH_SIZE and WRITE_SIZE count the bytes of requests that leave the L2 (TCC); Infinity "
             "Cache (MALL) hits count as well, so the DRAM traffic is at most these figures.", "",
             "Commands (each counter in its own run, TMPDIR=/tmp):", "", "```", cmd["fetch"], cmd["write"],
             "```", "", "| Dispatch | FETCH_SIZE KiB | WRITE_SIZE KiB |", "|---|---|---|"]
    for i, (fv, wv) in enumerate(zip(t["fetch_kib_each"], t["write_kib_each"])):
        lines.append(f"| attention launch {i + 1} | {fv:.0f} | {wv:.0f} |")
    for i, (fv, wv) in enumerate(zip(values(fetch, KEY_NORM, "FETCH_SIZE"), values(write, KEY_NORM, "WRITE_SIZE"))):
        lines.append(f"| key-norm pass {i + 1} (reads K once) | {fv:.0f} | {wv:.0f} |")
    lines.append(f"| 1 GiB device copy (calibration) | {values(fetch, COPY, 'FETCH_SIZE')[0]:.0f} | "
                 f"{values(write, COPY, 'WRITE_SIZE')[0]:.0f} |")
    minb = b["roofline"].get("algorithmic_bytes") if b else None
    lines += ["", f"Calibration: the copy moves {COPY_KIB} KiB each way, so FETCH_SIZE x {t['fetch_scale']:.3f} "
                  f"and WRITE_SIZE x {t['write_scale']:.3f} give bytes.",
              f"Attention launch: {t['fetch_kib'] * t['fetch_scale'] / 1024:.1f} MiB read + "
              f"{t['write_kib'] * t['write_scale'] / 1024:.1f} MiB written = {t['bytes'] / 2**20:.1f} MiB per launch "
              f"({t['bytes']} bytes)."
              + (f" Algorithmic minimum (q, k, v read once, out written once): {minb / 2**20:.1f} MiB "
                 f"({minb} bytes), so {t['bytes'] / minb:.2f}x." if minb else "")]
    if avg_ns:
        rate = t["bytes"] / (avg_ns * 1e-9) / 1e9
        lines.append(f"Rate past L2: {t['bytes']:.4g} bytes over the kernel's average duration in its trace "
                     f"({avg_ns / 1e3:.1f} us) = {rate:.0f} GB/s, {100 * rate / HBM_GBS:.1f}% of the 8 TB/s HBM peak "
                     f"even if every byte went to DRAM.")
    lines += ["", "Made by `python triton-fa2-forward_amd/rocprof_summary.py` from the run's CSVs.", ""]
    path = os.path.join(out_dir, f"attn_fwd_kernel_{cfg}_l2_miss_traffic.md")
    with open(path, "w") as f:
        f.write("\n".join(lines))
    j = {"about": "bytes per launch of fa2::attn_fwd_kernel that left L2 (rocprofv3 FETCH_SIZE + "
                  "WRITE_SIZE, copy-calibrated; Infinity Cache hits included)", "configs": {}}
    if os.path.exists(json_path):
        with open(json_path) as f:
            j = json.load(f)
    j["configs"][cfg] = {"bytes": t["bytes"], "fetch_kib": t["fetch_kib"], "write_kib": t["write_kib"],
                         "fetch_scale": t["fetch_scale"], "write_scale": t["write_scale"],
                         "kernel_build": label, "algorithmic_bytes": minb,
                         "summary": f"profiles/attn_fwd_kernel_{cfg}_l2_miss_traffic.md"}
    with open(json_path, "w") as f:
        json.dump(j, f, indent=1)
    return path, t


def write_sq(root, cfg, out_dir):
    first = first_attn(pmc(os.path.join(root, f"{cfg}_sq")))
    lines = [f"# SQ counters: fa2::attn_fwd_kernel on {cfg} (first profiled launch)", "",
             f"Kernel: `{first['kernel']}`", "", "```", commands(root, cfg)["sq"], "```", "",
             "| Counter | Value |", "|---|---|"]
    for n in SQ_COUNTERS:
        if n in first:
            lines.append(f"| {n} | {first[n]:.6g} |")
    busy = first["SQ_VALU_MFMA_BUSY_CYCLES"] / SIMDS
    active = first["GRBM_GUI_ACTIVE"] / XCDS
    lines += ["", "Readings:", "",
              f"* MFMA busy: SQ_VALU_MFMA_BUSY_CYCLES / {SIMDS} SIMDs = {busy:.4g} cycles per SIMD, against "
              f"GRBM_GUI_ACTIVE / {XCDS} XCDs = {active:.4g} cycles of kernel activity: the matrix cores are busy "
              f"{100 * busy / active:.1f}% of the kernel's time at the clock it ran at (roofline.frac uses the "
              f"2.4 GHz peak clock instead).",
              f"* SQ_INSTS_MFMA / SQ_WAVES = {first['SQ_INSTS_MFMA'] / first['SQ_WAVES']:.0f} MFMAs per wave; "
              f"SQ_INSTS_VALU / SQ_INSTS_MFMA = {first['SQ_INSTS_VALU'] / first['SQ_INSTS_MFMA']:.2f} VALU "
              f"instructions per MFMA; SQ_INSTS_LDS / SQ_INSTS_MFMA = "
              f"{first['SQ_INSTS_LDS'] / first['SQ_INSTS_MFMA']:.2f}.",
              f"* SQ_LDS_BANK_CONFLICT = {first['SQ_LDS_BANK_CONFLICT']:.0f}"
              + (": the XOR-swizzled K and V tiles are read without bank conflicts." if first['SQ_LDS_BANK_CONFLICT'] == 0
                 else " cycles of bank conflicts."),
              "", "Made by `python triton-fa2-forward_amd/rocprof_summary.py` from the run's CSVs.", ""]
    path = os.path.join(out_dir, f"attn_fwd_kernel_{cfg}_sq_counters.md")
    with open(path, "w") as f:
        f.write("\n".join(lines))
    return path


def write_util(root, cfgs, out_dir):
    firsts = {c: first_attn(pmc(os.path.join(root, f"{c}_util"))) for c in cfgs}
    u = {c: utilisation(firsts[c]) for c in cfgs}
    cmd = commands(root, "<config>")["util"]
    lines = [f"# Utilisation counters: fa2::attn_fwd_kernel on {', '.join(cfgs)} (first profiled launch)", "",
             f"One counter pass per config (`<config>` = {', '.join(cfgs)}):", "", "```", cmd, "```", "",
             "Kernel instances (from the runs): "
             + "; ".join(f"{c} `{firsts[c]['kernel']}`" for c in cfgs)
             + ". Template arguments: <dtype (0 fp16, 1 bf16), head_dim, waves, keys per tile, causal, "
               "variant>; variant 4 is the instance that reads the key-norm table.", "",
             "| Counter (sum over the GPU) | " + " | ".join(cfgs) + " |", "|---|" + "---|" * len(cfgs)]
    for n in ["GRBM_GUI_ACTIVE", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_VALU_MFMA_COEXEC_CYCLES", "SQ_ACTIVE_INST_VALU",
              "SQ_INSTS_VALU_TRANS_F32", "SQ_LDS_IDX_ACTIVE", "SQ_WAIT_INST_LDS", "SQ_INST_CYCLES_SALU"]:
        lines.append(f"| {n} | " + " | ".join(f"{firsts[c][n]:.4g}" for c in cfgs) + " |")
    lines += ["", f"Derived, per unit, over the kernel's active time (GRBM_GUI_ACTIVE / {XCDS} XCDs cycles; "
                  f"{CUS} CUs, {SIMDS} SIMDs):", "",
              "| Metric | " + " | ".join(cfgs) + " |", "|---|" + "---|" * len(cfgs)]
    rows = [("matrix cores busy (SQ_VALU_MFMA_BUSY_CYCLES / 1024 SIMDs)", "mfma_busy", True),
            ("VALU busy per SIMD (SQ_ACTIVE_INST_VALU / 256 CUs)", "valu_busy", True),
            ("share of MFMA cycles with VALU work beside them (COEXEC / MFMA_BUSY)", "mfma_with_valu", True),
            ("LDS busy (SQ_LDS_IDX_ACTIVE / 256 CUs)", "lds_busy", True),
            ("scalar ALU busy (SQ_INST_CYCLES_SALU / 256 CUs)", "salu_busy", True),
            ("transcendental (exp) instructions", "exp_insts", False)]
    for label, key, pct in rows:
        lines.append(f"| {label} | " + " | ".join(
            (f"{100 * u[c][key]:.1f}%" if pct else f"{u[c][key]:.4g}") for c in cfgs) + " |")
    lines += ["", "Made by `python triton-fa2-forward_amd/rocprof_summary.py` from the runs' CSVs.", ""]
    path = os.path.join(out_dir, "attn_fwd_kernel_utilisation_counters.md")
    with open(path, "w") as f:
        f.write("\n".join(lines))
    return path, u


def bench_lines(log_path):
    """Every bench.py JSON line of a log, in order."""
    out = []
    with open(log_path) as f:
        for ln in f:
            if ln.startswith('{"metric"'):
                out.append(json.loads(ln))
    return out


def write_bench(log_path, out_dir):
    """profiles/bench_all_configs.md from bench.py's lines: the configs' TFLOP/s, clock and
    roofline fractions, torch SDPA beside them, and the few-queries table."""
    lines_ = bench_lines(log_path)
    cfg = [b for b in lines_ if b.get("unit") == "TFLOP/s"]
    short = [b for b in lines_ if b.get("unit") == "TB/s"]
    env = cfg[0].get("env", {}) if cfg else {}
    L = ["# bench.py on every configuration, one box, current build", "",
         "Commands (from the repository root on the MI355X box):", "",
         "    python bench.py --all --sdpa --no-cpu-baseline",
         "    python bench.py --pack-short --no-cpu-baseline", "",
         f"Box: {env.get('gpu', '?')} ({env.get('arch', '?')}), ROCm {env.get('rocm', '?')}, torch {env.get('torch', '?')}. "
         "Each line is `bench.py`'s JSON line summarised: back-to-back steps after a 1 s clock "
         "settle (`value`), the sampled graphics clock over the timed steps, `roofline.frac` "
         "against the 2.4 GHz dense peak (2516.6 TFLOP/s) and at the sampled clock, the measured mix "
         "ceiling with the kernel's VGPR accumulators, the reference's flushed per-launch protocol, "
         "and torch's fused SDPA (AOTriton flash) on the same inputs, K/V expanded.", "",
         "| config | TFLOP/s | ms per step | frac of peak | sclk MHz | frac at sampled sclk | frac of mix "
         "ceiling (VGPR acc.) | reference protocol TFLOP/s | torch SDPA TFLOP/s |",
         "|---|---|---|---|---|---|---|---|---|"]
    for b in cfg:
        r = b["roofline"]
        sclk = b.get("clock", {}).get("timed_steps", {}).get("sclk_mhz_median")
        sd = b.get("sdpa_same_box") or {}
        ref = b.get("value_reference_protocol", {}).get("tflops")
        L.append(f"| {b['config']['workload']} | {b['value']} | {b['ms_per_step']:.4f} | {r['frac']} | "
                 f"{sclk if sclk else '-'} | {r.get('frac_at_sampled_sclk', '-')} | "
                 f"{r.get('frac_of_measured_mix_ceiling_vgpr_acc', '-')} | {ref if ref else '-'} | "
                 f"{sd.get('tflops', '-')} |")
    if short:
        L += ["", "Few queries against a long K/V (the reference's README.md:282-301 table; fp16, B 16, "
                  "H 32/8, N_kv 4096, D 128, non-causal; K + V = 256 MiB read once per call):", "",
              "| N_q | us per call | K/V read rate TB/s | frac of 8 TB/s | frac of a streaming read of the "
              "same size | splits | reference H100 us | speedup |",
              "|---|---|---|---|---|---|---|---|"]
        for b in short:
            r = b["roofline"]
            L.append(f"| {b['config']['n_q']} | {b['us_per_step']} | {b['value']} | {r['frac']} | "
                     f"{r.get('frac_of_measured_read_rate', '-')} | {b['config']['num_splits']} | "
                     f"{b.get('reference_h100_us', '-')} | {b.get('vs_reference_h100', '-')}x |")
    L += ["", "Made by `python triton-fa2-forward_amd/rocprof_summary.py --bench-log <log>` from the "
              "runs' JSON lines.", ""]
    path = os.path.join(out_dir, "bench_all_configs.md")
    with open(path, "w") as f:
        f.write("\n".join(L))
    return path


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--root", default="gpurun_out/prof", help="profile_configs.sh's output folder")
    ap.add_argument("--configs", nargs="+", default=["C3", "C2", "C4", "C5"])
    ap.add_argument("--out", default=PROFILES)
    ap.add_argument("--json", default=os.path.join(PROFILES, "l2_miss_traffic.json"))
    ap.add_argument("--label", default="current", help="kernel_build label in the JSON")
    ap.add_argument("--parts", nargs="+", default=["trace", "traffic", "sq", "util"],
                    choices=["trace", "traffic", "sq", "util"])
    ap.add_argument("--bench-log", default=None, help="also write bench_all_configs.md from it")
    args = ap.parse_args()
    if args.bench_log:
        print(write_bench(args.bench_log, args.out))
    os.makedirs(args.out, exist_ok=True)
    for cfg in args.configs:
        if "trace" in args.parts:
            print(write_trace(args.root, cfg, args.out))
        if "traffic" in args.parts:
            path, t = write_traffic(args.root, cfg, args.out, args.json, args.label)
            print(path, t["bytes"])
        if "sq" in args.parts:
            print(write_sq(args.root, cfg, args.out))
    if "util" in args.parts:
        print(write_util(args.root, args.configs, args.out)[0])


if __name__ == "__main__":
    main()
