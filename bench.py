#!/usr/bin/env python3
"""Headline benchmark: attention forward TFLOP/s and % of the dense bf16 MFMA peak, one MI355X.

    python bench.py [--steps K] [--warmup W] [--config C3] [--all] [--no-cpu-baseline]
    python bench.py --pack-short     # the reference's few-queries table (K/V read rate)
    python bench.py --all --sdpa     # also torch's own fused SDPA on the same inputs, for context
    python bench.py --seqlens 1024 4096 16384 --dtype bf16 [--batch --hq --hkv --head-dim
                    --kv-len --no-causal --iters --no-flush --providers --out]
                                     # the reference's sweep (bench/bench.py:226-307): a table of
                                     # median TFLOP/s per N and provider (fa2, fa2-nopack,
                                     # fa2-pack, sdpa), instead of the JSON line

Workload: BASELINE.json's target config C3 (bf16 causal GQA, B=1, H_q=32, H_kv=8, N=8192,
D=128), the shape the reference's own bench defaults to (bench/bench.py:228-235) and the one
its published 447.1 TFLOP/s (H100) is quoted on. A "step" is one fa2.kernel.attention call over
that batch; inputs are seeded synthetic data already resident in HBM.

Protocol (the reference's, bench/bench.py:51-92, restated for ROCm):
  * correctness gate before timing: max-abs vs torch SDPA <= 2e-2 (bench/bench.py:265-268);
  * an untimed settle phase (steps back to back for 1 s: the GPU's clocks ramp up over the
    first few dozen launches after the idle gate, and each process sees one 17-25 ms hold-up
    in its first half second of GPU work; reported as "settle"), then W untimed
    warmups, then exactly K (default 100) back-to-back steps bracketed by synchronize and by
    one pair of HIP events on the launch stream; `value` is K x FLOPs / the events' elapsed
    time, and that time / K is the average duration of one step's kernels (roofline.achieved;
    on long problems a step is the key-norm pass, ~1% of it, then the attention kernel);
    FLOPs = 4 B H_q pairs D with causal pairs N(N+1)/2. No event sits between the timed steps:
    a timed event between two launches adds a few microseconds of GPU-side gap (6.5 us per
    step on C3, 1.3%; 6 us on C5's 35 us kernel);
  * a second pass of K steps with events around every launch, the reference's own protocol,
    gives the median / IQR and the slowest steps (these per-launch times include that gap);
  * a second pass follows the reference's flush protocol exactly: a 1 GiB fill (larger than
    L2 + the 256 MB Infinity Cache) before every iteration, median of per-iteration events;
  * cpu_baseline: the oracle's blocked_attention (the reference's CPU path, fa2/reference.py:
    35-82, restated) timed on this host, one thread, on whole (batch, head) pairs of the
    workload until at least 10 s of CPU work, reported as its TFLOP/s;
  * roofline.traffic: bytes per launch that left L2 (TCC FETCH_SIZE + WRITE_SIZE, copy-calibrated;
    Infinity Cache hits count too, so DRAM traffic is at most this) from the committed rocprofv3
    summary (profiles/l2_miss_traffic.json), next to the algorithmic minimum (q, k, v read, out
    written);
  * clock: the graphics clock (mean over the XCDs) and socket power sampled with amdsmi during
    the timed steps and during 1 s of sustained steps; roofline.frac_at_sampled_sclk divides by
    the dense peak at that clock instead of at 2.4 GHz;
  * value_reference_protocol: the reference's own protocol (flush, events per launch, median)
    beside `value`;

Prints ONE JSON line. --gpus N with N > 1 exits: this build is one GPU per box.
"""

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "triton-fa2-forward_amd"), ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "attention fwd TFLOP/s and % of bf16 MFMA peak, 1 MI355X"
# MI355X dense fp16/bf16 MFMA peak: 256 CUs x 2.4 GHz x 4096 FLOP/clk/CU.
PEAK_TFLOPS = 256 * 2.4e9 * 4096 / 1e12
H100_C3_TFLOPS = 447.1   # the reference's published C3 number (bench/results/2026-10-04/bench-bf16.log:73)

# name: (dtype, causal, B, H_q, H_kv, N, D, input scale, k-row outliers)
WORKLOADS = {
    "C2": ("bf16", True, 4, 16, 16, 4096, 128, 1.0, False),
    "C3": ("bf16", True, 1, 32, 8, 8192, 128, 1.0, False),
    "C4": ("fp16", False, 2, 16, 16, 16384, 64, 0.5, False),
    "C5": ("bf16", True, 3, 28, 4, 1000, 128, 1.0, True),
}


def describe(name):
    dt, causal, B, hq, hkv, n, d, scale, outl = WORKLOADS[name]
    return (f"{name}: {dt} {'causal' if causal else 'full'} B={B} Hq={hq} Hkv={hkv} N={n} D={d}"
            + (f" x{scale}" if scale != 1.0 else "") + (" +1% k rows x8" if outl else ""))


def make_inputs(name, device):
    """The BASELINE.json recipe: CPU generator seed 0, randn fp32 for q, k, v in that order,
    perturb in fp32, cast, move to the device."""
    import torch

    dt, causal, B, hq, hkv, n, d, scale, outl = WORKLOADS[name]
    g = torch.Generator("cpu").manual_seed(0)
    q = torch.randn(B, hq, n, d, generator=g)
    k = torch.randn(B, hkv, n, d, generator=g)
    v = torch.randn(B, hkv, n, d, generator=g)
    if scale != 1.0:
        q, k, v = q * scale, k * scale, v * scale
    if outl:
        rows = B * hkv * n
        k.view(rows, d)[torch.randperm(rows, generator=g)[: rows // 100]] *= 8.0
    dtype = {"bf16": torch.bfloat16, "fp16": torch.float16}[dt]
    return q.to(dtype).to(device), k.to(dtype).to(device), v.to(dtype).to(device), causal


def attn_flops(B, H_q, N_q, N_kv, D, causal):
    pairs = N_q * (N_q + 1) / 2 if causal else N_q * N_kv
    return 4 * B * H_q * pairs * D


def correctness_gate(out, q, k, v, causal):
    """Max-abs against torch's fused SDPA (K/V expanded, no math backend)."""
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    group = q.shape[1] // k.shape[1]
    ke = k.repeat_interleave(group, dim=1).contiguous()
    ve = v.repeat_interleave(group, dim=1).contiguous()
    for name in ("FLASH_ATTENTION", "EFFICIENT_ATTENTION"):
        try:
            with sdpa_kernel(getattr(SDPBackend, name)):
                ref = F.scaled_dot_product_attention(q, ke, ve, is_causal=causal)
            err = (out.float() - ref.float()).abs().max().item()
            return err, name.lower()
        except RuntimeError:
            continue
    return None, "unavailable"


def sdpa_rate(q, k, v, causal, flops, steps=30):
    """torch's own fused SDPA on the same inputs (K/V expanded to MHA beforehand, untimed), timed
    like the headline: settle, then back-to-back steps between one event pair. Context only."""
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    group = q.shape[1] // k.shape[1]
    ke = k.repeat_interleave(group, dim=1).contiguous()
    ve = v.repeat_interleave(group, dim=1).contiguous()
    for name in ("FLASH_ATTENTION", "EFFICIENT_ATTENTION"):
        def fn(name=name):
            with sdpa_kernel(getattr(SDPBackend, name)):
                return F.scaled_dot_product_attention(q, ke, ve, is_causal=causal)
        try:
            fn()
            torch.cuda.synchronize()
        except RuntimeError:
            continue
        settle_clocks(fn, min_ms=300.0)
        total_ms, _ = time_steps(fn, steps, 3)
        ms = total_ms / steps
        return {"backend": name.lower(), "ms_per_step": round(ms, 5),
                "tflops": round(flops / (ms * 1e-3) / 1e12, 2),
                "note": "torch.nn.functional.scaled_dot_product_attention, K/V expanded to MHA"}
    return None


def settle_clocks(fn, min_ms=1000.0, max_steps=20000):
    """Run the step back to back until min_ms of wall time has passed (untimed).

    Two start-up effects on MI355X, measured per launch on C3: clocks ramp up over the first
    few dozen back-to-back launches after an idle phase (the correctness gate is one), which
    makes them 10-15% slower than the steady state; and once per process, within its first
    half second of GPU work, one launch is held up for 17-25 ms. Settling for a second first
    keeps both out of the timed steps, whatever W is."""
    import torch

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    n = 0
    while n < max_steps:
        for _ in range(10):
            fn()
        n += 10
        torch.cuda.synchronize()
        if (time.perf_counter() - t0) * 1e3 >= min_ms:
            break
    return {"steps": n, "ms": round((time.perf_counter() - t0) * 1e3, 1)}


def time_steps(fn, steps, warmup):
    """W untimed warmups, then `steps` back-to-back launches between one pair of HIP events
    on the launch stream, synchronized on both sides. Returns (elapsed ms of the events, host
    wall ms of the timed loop including the final synchronize)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    begin, finish = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    begin.record(stream)
    for _ in range(steps):
        fn()
    finish.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    return begin.elapsed_time(finish), wall_ms


def time_each(fn, steps):
    """The reference's per-iteration protocol (bench/bench.py:61-80): events around every
    launch; returns the per-launch ms (each includes the gap a timed event adds)."""
    import torch

    stream = torch.cuda.current_stream()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    torch.cuda.synchronize()
    for s, e in zip(starts, ends):
        s.record(stream)
        fn()
        e.record(stream)
    torch.cuda.synchronize()
    return [s.elapsed_time(e) for s, e in zip(starts, ends)]


def flushed_median(fn, iters):
    """bench/bench.py:54-80 with a 1 GiB flush (MI355X: 4 MB L2 per XCD + 256 MB Infinity Cache)."""
    import torch

    buf = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream()
    fn()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    for s, e in zip(starts, ends):
        buf.zero_()
        s.record(stream)
        fn()
        e.record(stream)
    torch.cuda.synchronize()
    ms = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    del buf
    q1, med, q3 = statistics.quantiles(ms, n=4, method="inclusive")
    return {"median_ms": med, "p25_ms": q1, "p75_ms": q3}


def cpu_baseline(name, q, k, v, causal, min_seconds=10.0):
    """The reference's CPU path (blocked_attention, restated in oracle/) on whole (b, h) pairs
    of the workload, single thread, on CPU copies of the same inputs, until at least
    `min_seconds` of CPU work; scaled to the whole job by per-head work (identical per head)."""
    import torch

    from oracle import reference as ref

    B, H_q, N, D = q.shape
    group = H_q // k.shape[1]
    threads = torch.get_num_threads()
    torch.set_num_threads(1)
    done, dt = 0, 0.0
    try:
        while dt < min_seconds and done < B * H_q:
            b, h = divmod(done, H_q)
            qs = q[b:b + 1, h:h + 1].cpu()
            ks = k[b:b + 1, h // group:h // group + 1].cpu()
            vs = v[b:b + 1, h // group:h // group + 1].cpu()
            t0 = time.perf_counter()
            ref.blocked_attention(qs, ks, vs, causal=causal)
            dt += time.perf_counter() - t0
            done += 1
    finally:
        torch.set_num_threads(threads)
    sample_flops = done * attn_flops(1, 1, N, k.shape[2], D, causal)
    return {
        "value": sample_flops / dt / 1e12,
        "unit": "TFLOP/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"oracle.blocked_attention (fa2/reference.py:35-82 restated; block 32x16, fp32 "
                   f"state) on {done} of {B * H_q} (batch, head) pairs of {name} (group {group}), "
                   f"{dt:.1f} s on 1 thread of {os.cpu_count()} host CPUs; per-head work is "
                   f"identical, so the rate holds for the whole job"),
        "seconds": dt,
        "est_full_job_s": dt * B * H_q / done,
    }


def measured_traffic(name):
    """Bytes per launch that left L2 for this workload, from the committed rocprofv3 counter
    summary (profiles/l2_miss_traffic.json: FETCH_SIZE and WRITE_SIZE per dispatch, each scaled by
    what the counter reads for a plain copy of known size), or None."""
    path = os.path.join(ROOT, "profiles", "l2_miss_traffic.json")
    try:
        with open(path) as f:
            entry = json.load(f)["configs"][name]
        return {"bytes": entry["bytes"], "source": f"profiles/l2_miss_traffic.json ({entry['kernel_build']})"}
    except (OSError, KeyError, ValueError):
        return None


def _read(path):
    try:
        with open(path) as f:
            return f.read().strip()
    except OSError:
        return None


def _sha256(path):
    import hashlib

    try:
        with open(path, "rb") as f:
            return hashlib.sha256(f.read()).hexdigest()
    except OSError:
        return None


def _hipcc_version():
    import shutil
    import subprocess

    cc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    try:
        out = subprocess.run([cc, "--version"], capture_output=True, text=True, timeout=30).stdout
    except (OSError, subprocess.SubprocessError):
        return None
    lines = [l.strip() for l in out.splitlines() if l.strip()]
    return " | ".join(lines[:2]) or None


def gpu_env():
    """The run environment (the reference records driver, versions and date with every result,
    bench/bench.py:196-219): GPU, ROCm, HIP, hipcc, torch, Python, the driver as amdsmi reports
    it, the SHA-256 of the library that ran, and the UTC date."""
    import datetime
    import platform

    import torch

    from fa2 import _lib

    props = torch.cuda.get_device_properties(0)
    env = {
        "gpu": props.name or getattr(props, "gcnArchName", ""),
        "arch": getattr(props, "gcnArchName", None),
        "cus": props.multi_processor_count,
        "rocm": _read("/opt/rocm/.info/version"),
        "hip_runtime": torch.version.hip,
        "hipcc": _hipcc_version(),
        "torch": torch.__version__,
        "python": platform.python_version(),
        "kernel": platform.release(),
        "library": _lib.LIB_PATH.replace(ROOT + os.sep, ""),
        "library_sha256": _sha256(_lib.LIB_PATH),
        "date_utc": datetime.datetime.now(datetime.timezone.utc).isoformat(timespec="seconds"),
        "host_cpus": os.cpu_count(),
    }
    try:
        import amdsmi

        amdsmi.amdsmi_init()
        try:
            h = amdsmi.amdsmi_get_processor_handles()[0]
            drv = amdsmi.amdsmi_get_gpu_driver_info(h)
            env["driver"] = f"{drv.get('driver_name')} {drv.get('driver_version')}"
            clk = amdsmi.amdsmi_get_clock_info(h, amdsmi.AmdSmiClkType.GFX)
            env["sclk_range_mhz"] = [clk.get("min_clk"), clk.get("max_clk")]
            pw = amdsmi.amdsmi_get_power_info(h)
            env["power_limit_w"] = (pw.get("power_limit") / 1e6 if isinstance(pw.get("power_limit"), (int, float))
                                    else pw.get("power_limit"))
        finally:
            amdsmi.amdsmi_shut_down()
    except Exception as e:  # noqa: BLE001 - the environment record is best effort
        env["driver"] = f"unavailable ({type(e).__name__})"
    return env


class ClockSampler:
    """Samples the GPU's graphics clock (every XCD's, MHz) and socket power (W) with amdsmi on a
    background thread while GPU work runs (the reference samples clock and power beside its runs,
    bench/results/2026-10-03/clock.py:7-8). One amdsmi call takes ~0.3 ms; the thread sleeps
    `period_s` between calls and takes no GIL while it sleeps, so the launches it runs beside
    are not held up. Device 0 is the only GPU of the box."""

    def __init__(self, period_s=0.002):
        self.period_s = period_s
        self.sclk, self.power, self.error = [], [], None
        self.per_xcd = []
        self._stop = None
        self._thread = None

    def __enter__(self):
        import threading

        self._stop = threading.Event()
        try:
            import amdsmi

            amdsmi.amdsmi_init()
            self._amdsmi = amdsmi
            self._h = amdsmi.amdsmi_get_processor_handles()[0]
        except Exception as e:  # noqa: BLE001
            self.error = f"amdsmi unavailable: {type(e).__name__}: {e}"
            return self
        self._thread = threading.Thread(target=self._run, daemon=True)
        self._thread.start()
        return self

    def _run(self):
        while not self._stop.is_set():
            try:
                m = self._amdsmi.amdsmi_get_gpu_metrics_info(self._h)
                clks = [c for c in m.get("current_gfxclks", []) if isinstance(c, (int, float))]
                if clks:
                    self.sclk.append(sum(clks) / len(clks))
                    self.per_xcd.append(clks)
                pw = m.get("current_socket_power")
                if isinstance(pw, (int, float)):
                    self.power.append(float(pw))
            except Exception as e:  # noqa: BLE001
                self.error = f"{type(e).__name__}: {e}"
                return
            self._stop.wait(self.period_s)

    def __exit__(self, *exc):
        if self._thread is not None:
            self._stop.set()
            self._thread.join()
            self._amdsmi.amdsmi_shut_down()
        return False

    def summary(self):
        if not self.sclk:
            return {"samples": 0, "error": self.error or "no samples"}
        return {"samples": len(self.sclk),
                "sclk_mhz_median": round(statistics.median(self.sclk), 1),
                "sclk_mhz_min": round(min(self.sclk), 1), "sclk_mhz_max": round(max(self.sclk), 1),
                "power_w_median": round(statistics.median(self.power), 1) if self.power else None,
                "power_w_max": round(max(self.power), 1) if self.power else None,
                "sclk_mhz_median_per_xcd": [round(statistics.median(c), 1) for c in zip(*self.per_xcd)]
                if self.per_xcd else None}


def sustained_clock(fn, seconds=1.0):
    """Steps back to back for `seconds` with the clock sampler running: the clock and power the
    kernel sustains (the timed steps of a short kernel last only a few milliseconds)."""
    import torch

    with ClockSampler() as smp:
        t0 = time.perf_counter()
        n = 0
        while time.perf_counter() - t0 < seconds:
            for _ in range(10):
                fn()
            n += 10
            torch.cuda.synchronize()
    out = smp.summary()
    out["steps"] = n
    return out


def tail_schedule_info(B, H_q, H_kv, N, D, causal):
    """The dynamic tail the library gives this launch (fa2_ablate_tail_schedule, a host-side
    policy query in the measurement library): programs run in the static order, programs dealt
    at run time and the workgroups that take them; None where the launch keeps the static order
    or the measurement library is not built."""
    import ctypes

    import ablation

    try:
        lib = ablation.ablate_lib()
    except RuntimeError:
        return None
    fn = lib.fa2_ablate_tail_schedule
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_int32] * 7 + [ctypes.POINTER(ctypes.c_int32)] * 3
    out = [ctypes.c_int32() for _ in range(3)]
    if fn(B, H_q, H_kv, N, D, int(causal), 1, *(ctypes.byref(o) for o in out)) != 0 or not out[1].value:
        return None
    return {"static_programs": out[0].value, "tail_programs": out[1].value,
            "tail_workgroups": out[2].value}


def measured_ceiling(seconds=1.0):
    """The MFMA rate this box sustains under its power limit (triton-fa2-forward_amd/ceiling.py,
    fa2_ablate_mfma_ceiling in the measurement library): bf16 MFMAs on random operands alone, and
    with the attention kernel's LDS operand reads and softmax vector work beside them, with the
    accumulators in AGPRs (the compiler's choice for the probe) and in VGPRs (where the attention
    kernel keeps them). The nominal peak assumes 2.4 GHz; on random data the chip holds its power
    by running lower."""
    try:
        import ceiling

        out = {m: ceiling.measure(m, seconds)
               for m in ("mfma", "mfma_lds_softmax", "mfma_lds_softmax_vacc")}
    except Exception as e:  # noqa: BLE001
        return {"error": f"{type(e).__name__}: {e}"}
    out["source"] = ("fa2_ablate_mfma_ceiling (libfa2_ablate.so, csrc/mfma_ceiling.hip), "
                     f"each mode alone for {seconds:g} s in this run")
    return out


def run(name, steps, warmup, with_cpu, flush_iters, with_sdpa=False, ceiling=None):
    import torch

    from fa2 import _lib
    from fa2.kernel import attention

    q, k, v, causal = make_inputs(name, "cuda")
    B, H_q, N, D = q.shape
    flops = attn_flops(B, H_q, N, k.shape[2], D, causal)
    fn = lambda: attention(q, k, v, causal=causal)  # noqa: E731

    out = fn()
    torch.cuda.synchronize()
    err, backend = correctness_gate(out, q, k, v, causal)
    if err is not None and not (math.isfinite(err) and err <= 2e-2):
        raise SystemExit(f"correctness gate failed on {name}: max-abs vs SDPA {err:.3e}")

    # kernels per step: the attention kernel, after the key-norm pass where attention() asks for
    # its table (long problems: fa2_workspace_bytes_for)
    H_kv, N_kv = k.shape[1], k.shape[2]
    key_norm = (_lib.workspace_bytes_for(B, H_q, H_kv, N, N_kv, D, q.dtype, causal, 1)
                > _lib.workspace_bytes(B, H_q, N, D, 1))
    kernels = (["fa2::key_norm_kernel"] if key_norm else []) + ["fa2::attn_fwd_kernel"]

    settle = settle_clocks(fn)
    with ClockSampler() as timed_clock:
        total_ms, wall_ms = time_steps(fn, steps, warmup)
    avg_kernel_ms = total_ms / steps   # one step: the kernels above, back to back
    clock = {"timed_steps": timed_clock.summary(), "sustained_1s": sustained_clock(fn)}
    per = time_each(fn, steps)
    q1, med, q3 = statistics.quantiles(per, n=4, method="inclusive") if len(per) > 1 else (per[0],) * 3
    value = flops * steps / (total_ms * 1e-3) / 1e12
    achieved = flops / (avg_kernel_ms * 1e-3) / 1e12
    traffic = measured_traffic(name)
    min_bytes = sum(t.numel() * t.element_size() for t in (q, k, v)) + out.numel() * out.element_size()
    fl = None
    if flush_iters:
        fl = flushed_median(fn, flush_iters)
        fl["tflops"] = round(flops / (fl["median_ms"] * 1e-3) / 1e12, 2)
    # the dense peak at the clock the kernel ran at: CUs x sampled sclk x 4096 FLOP/clk
    sclk = clock["timed_steps"].get("sclk_mhz_median") or clock["sustained_1s"].get("sclk_mhz_median")
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    peak_at_sclk = cus * sclk * 1e6 * 4096 / 1e12 if sclk else None
    res = {
        "metric": METRIC,
        "value": round(value, 2),
        "value_reference_protocol": {
            "tflops": fl["tflops"] if fl else None,
            "protocol": "the reference's (bench/bench.py:61-80): 1 GiB flush before every launch, "
                        "HIP events around each launch, median"},
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "settle": settle,
        "ms_per_step": round(total_ms / steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": WORKLOADS[name][0],
        "data": "synthetic (seeded randn, BASELINE.json recipe)",
        "config": {"workload": describe(name), "batch": B, "h_q": H_q, "h_kv": k.shape[1],
                   "seq_len": N, "head_dim": D, "causal": causal, "flops_per_step": flops,
                   "flops_rule": "4*B*H_q*pairs*D, causal pairs N(N+1)/2 (bench/bench.py:83-87)"},
        "dynamic_tail": tail_schedule_info(B, H_q, k.shape[1], N, D, causal),
        "pct_of_peak": round(100 * value / PEAK_TFLOPS, 2),
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": round(PEAK_TFLOPS, 1),
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_TFLOPS, 4),
                     "traffic": traffic["bytes"] if traffic else None,
                     "traffic_counts": "L2-miss bytes: TCC FETCH_SIZE + WRITE_SIZE, the requests that "
                                       "left L2 (Infinity Cache hits included, so DRAM bytes are at most "
                                       "this), copy-calibrated",
                     "traffic_source": traffic["source"] if traffic else None,
                     "algorithmic_bytes": min_bytes,
                     "kernel": " + ".join(kernels), "avg_kernel_ms": round(avg_kernel_ms, 5),
                     "peak_at_sampled_sclk": round(peak_at_sclk, 1) if peak_at_sclk else None,
                     "frac_at_sampled_sclk": round(achieved / peak_at_sclk, 4) if peak_at_sclk else None},
        "clock": clock,
        "per_launch_events": {"median_ms": round(med, 5), "p25_ms": round(q1, 5), "p75_ms": round(q3, 5),
                              "slowest_steps": [[i, round(per[i], 4)] for i in
                                                sorted(range(len(per)), key=per.__getitem__)[-3:]]},
        "host_wall_ms": round(wall_ms, 3),
        "vs_reference_h100_c3": round(value / H100_C3_TFLOPS, 3) if name == "C3" else None,
        "correctness_gate": {"max_abs_vs_sdpa": err, "sdpa_backend": backend},
        "env": gpu_env(),
        "library": _lib.lib().fa2_version().decode(),
    }
    if ceiling is not None:
        res["roofline"]["measured_ceiling"] = ceiling
        top = ceiling.get("mfma", {}).get("tflops")
        mix = ceiling.get("mfma_lds_softmax", {}).get("tflops")
        res["roofline"]["frac_of_measured_mfma_ceiling"] = round(achieved / top, 4) if top else None
        res["roofline"]["frac_of_measured_mix_ceiling"] = round(achieved / mix, 4) if mix else None
        vmix = ceiling.get("mfma_lds_softmax_vacc", {}).get("tflops")
        res["roofline"]["frac_of_measured_mix_ceiling_vgpr_acc"] = (
            round(achieved / vmix, 4) if vmix else None)
    if fl:
        res["flushed"] = fl
    if with_sdpa:
        res["sdpa_same_box"] = sdpa_rate(q, k, v, causal, flops)
    if with_cpu:
        res["cpu_baseline"] = cpu_baseline(name, q, k, v, causal)
    return res


# The reference's few-queries table (README.md:282-301, bench/gpu_session.sh:27-28): batch 16,
# H_q 32, H_kv 8, N_kv 4096, D 128, non-causal fp16; its default path's median us on H100
# (packed where should_pack_gqa packs: N_q <= 64; unpacked above).
PACK_SHORT = {"B": 16, "H_q": 32, "H_kv": 8, "N_kv": 4096, "D": 128}
PACK_SHORT_H100_US = {1: 106.5, 16: 105.5, 32: 107.6, 64: 151.2, 128: 307.9, 256: 642.5}
HBM_PEAK_GBS = 8000.0


def run_pack_short(n_q, steps, warmup):
    """One line of the few-queries regime: time per step (back to back) and the K/V read rate
    (bench/bench.py:90-92: bytes of K and V over the time, the bound when N_q is small)."""
    import torch

    from fa2 import _lib
    from fa2.kernel import _cu_count, attention, should_pack_gqa

    c = PACK_SHORT
    g = torch.Generator(device="cpu").manual_seed(0)
    q = torch.randn(c["B"], c["H_q"], n_q, c["D"], generator=g).half().cuda()
    k = torch.randn(c["B"], c["H_kv"], c["N_kv"], c["D"], generator=g).half().cuda()
    v = torch.randn(c["B"], c["H_kv"], c["N_kv"], c["D"], generator=g).half().cuda()
    fn = lambda: attention(q, k, v, causal=False)  # noqa: E731
    out = fn()
    torch.cuda.synchronize()
    err, backend = correctness_gate(out, q, k, v, False)
    if err is not None and not (math.isfinite(err) and err <= 2e-2):
        raise SystemExit(f"correctness gate failed on pack-short N_q={n_q}: max-abs vs SDPA {err:.3e}")
    settle = settle_clocks(fn)
    total_ms, _ = time_steps(fn, steps, warmup)
    step_ms = total_ms / steps          # one step: the attention launch (and the merge, if split)
    med = statistics.median(time_each(fn, steps))
    kv = 2 * k.numel() * k.element_size()
    rate_gbs = kv / (step_ms * 1e-3) / 1e9
    splits = _lib.num_splits(c["B"], c["H_q"], c["H_kv"], n_q, c["N_kv"], c["D"], False, 128, 64,
                             _cu_count(q.device))
    return {
        "metric": "K/V read rate, few queries against a long K/V (README.md:282-301)",
        "value": round(rate_gbs / 1e3, 3), "unit": "TB/s", "n_gpus": 1, "steps": steps,
        "warmup": warmup, "settle": settle, "higher_is_better": True, "dtype": "fp16",
        "data": "synthetic (seeded randn)",
        "config": {"workload": f"pack-short: fp16 full B={c['B']} Hq={c['H_q']} Hkv={c['H_kv']} "
                               f"N_q={n_q} N_kv={c['N_kv']} D={c['D']}",
                   "n_q": n_q, "pack_gqa": should_pack_gqa(n_q, c["H_q"] // c["H_kv"], 128),
                   "num_splits": splits},
        "us_per_step": round(step_ms * 1e3, 2),
        "per_launch_events_median_us": round(med * 1e3, 2),
        "reference_h100_us": PACK_SHORT_H100_US.get(n_q),
        "vs_reference_h100": (round(PACK_SHORT_H100_US[n_q] / (step_ms * 1e3), 3)
                              if n_q in PACK_SHORT_H100_US else None),
        "roofline": {"bound": "hbm", "achieved": round(rate_gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(rate_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "algorithmic_bytes": kv},
        "correctness_gate": {"max_abs_vs_sdpa": err, "sdpa_backend": backend},
    }


SWEEP_PROVIDERS = ("fa2", "fa2-nopack", "fa2-pack", "sdpa")


def sweep_provider(name, q, k, v, causal):
    """A zero-argument launch of `name` on (q, k, v), or None where it does not apply: fa2 is
    attention() with its own packing choice, fa2-nopack / fa2-pack force the GQA layout, sdpa is
    torch's fused SDPA (flash, else memory-efficient) on K/V expanded to MHA beforehand."""
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    from fa2.kernel import attention

    if name.startswith("fa2"):
        pack = {"fa2": None, "fa2-nopack": False, "fa2-pack": True}[name]
        return lambda: attention(q, k, v, causal=causal, pack_gqa=pack)
    group = q.shape[1] // k.shape[1]
    ke = k.repeat_interleave(group, dim=1).contiguous()
    ve = v.repeat_interleave(group, dim=1).contiguous()
    for backend in ("FLASH_ATTENTION", "EFFICIENT_ATTENTION"):
        def fn(backend=backend):
            with sdpa_kernel(getattr(SDPBackend, backend)):
                return F.scaled_dot_product_attention(q, ke, ve, is_causal=causal)
        try:
            fn()
            return fn
        except RuntimeError:
            continue
    return None


def run_seqlens(args):
    """The reference's sweep (bench/bench.py:226-307) on this GPU: for every N and provider, the
    correctness gate (max-abs vs SDPA <= 2e-2), then per-launch HIP events over --iters launches
    after --warmup, each after a 1 GiB flush unless --no-flush; median TFLOP/s and IQR. Prints a
    line per (N, provider) and the Markdown table; writes the rows as JSON to --out if given.
    One difference from the reference's loop: each provider first runs back to back for 0.3 s
    (settle_clocks), so that the first provider of every N is not timed on clocks still ramping
    up from idle (without it the first provider ran up to 4% slower than the same call later)."""
    import torch

    causal = not args.no_causal
    if causal and args.kv_len:
        raise SystemExit("--kv-len needs --no-causal (causal here assumes N_q == N_kv)")
    dtype = {"fp16": torch.float16, "bf16": torch.bfloat16}[args.dtype]
    env = gpu_env()
    rows = []
    for n in args.seqlens:
        n_kv = args.kv_len or n
        g = torch.Generator(device="cuda").manual_seed(0)
        q = torch.randn(args.batch, args.hq, n, args.head_dim, device="cuda", dtype=dtype, generator=g)
        k = torch.randn(args.batch, args.hkv, n_kv, args.head_dim, device="cuda", dtype=dtype, generator=g)
        v = torch.randn(args.batch, args.hkv, n_kv, args.head_dim, device="cuda", dtype=dtype, generator=g)
        flops = attn_flops(args.batch, args.hq, n, n_kv, args.head_dim, causal)
        kv_bytes = 2 * k.numel() * k.element_size()
        for name in args.providers:
            try:
                fn = sweep_provider(name, q, k, v, causal)
                if fn is None:
                    raise RuntimeError("no fused SDPA backend for this shape")
                err, _ = correctness_gate(fn(), q, k, v, causal)
                if err is None or not math.isfinite(err) or err > 2e-2:
                    raise RuntimeError(f"output vs SDPA: max-abs {err}")
                settle_clocks(fn, min_ms=300.0)
                for _ in range(args.warmup):
                    fn()
                torch.cuda.synchronize()
                if args.no_flush:
                    ms = time_each(fn, args.iters)
                    q1, med, q3 = statistics.quantiles(ms, n=4, method="inclusive")
                    st = {"median_ms": med, "p25_ms": q1, "p75_ms": q3}
                else:
                    st = flushed_median(fn, args.iters)
            except (RuntimeError, ValueError) as e:  # a provider that does not apply is skipped
                print(f"  skip {name:11s} N={n:6d}: {type(e).__name__}: {str(e)[:120]}", flush=True)
                continue
            row = {"provider": name, "seqlen": n, "kv_len": n_kv, "max_abs_err_vs_sdpa": err,
                   "median_ms": round(st["median_ms"], 5), "p25_ms": round(st["p25_ms"], 5),
                   "p75_ms": round(st["p75_ms"], 5),
                   "iqr_ms": round(st["p75_ms"] - st["p25_ms"], 5),
                   "tflops": round(flops / (st["median_ms"] * 1e-3) / 1e12, 2),
                   "kv_tbps": round(kv_bytes / (st["median_ms"] * 1e-3) / 1e12, 3)}
            rows.append(row)
            print(f"  {name:11s} N={n:6d}  {row['median_ms']:8.3f} ms [IQR {row['p25_ms']:.3f}-"
                  f"{row['p75_ms']:.3f}]  {row['tflops']:7.1f} TFLOP/s  K/V {row['kv_tbps']:5.2f} TB/s",
                  flush=True)
        del q, k, v
        torch.cuda.empty_cache()
    names = [p for p in args.providers if any(r["provider"] == p for r in rows)]
    kv = f" N_kv={args.kv_len}" if args.kv_len else ""
    print(f"\nB={args.batch} H_q={args.hq} H_kv={args.hkv} D={args.head_dim}{kv} {args.dtype} "
          f"causal={causal} {'' if args.no_flush else 'flushed '}| median TFLOP/s (IQR ms)\n")
    print("| N | " + " | ".join(names) + " |")
    print("|---|" + "---|" * len(names))
    for n in args.seqlens:
        cells = []
        for p in names:
            r = next((r for r in rows if r["provider"] == p and r["seqlen"] == n), None)
            cells.append(f"{r['tflops']:.1f} ({r['iqr_ms']:.3f})" if r else "-")
        print(f"| {n} | " + " | ".join(cells) + " |")
    if args.out:
        with open(args.out, "w") as f:
            json.dump({"env": env, "config": vars(args), "results": rows}, f, indent=1)
        print(f"\nwrote {args.out}")


def main():
    ap = argparse.ArgumentParser(description="MI355X FlashAttention-2 forward benchmark")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="C3", choices=sorted(WORKLOADS))
    ap.add_argument("--all", action="store_true", help="one line per GPU config C2..C5 (C3 first)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--pack-short", action="store_true",
                    help="instead of C3: the reference's few-queries table, one line per N_q")
    ap.add_argument("--flush-iters", type=int, default=10, help="iterations of the flushed pass (0: skip)")
    ap.add_argument("--no-ceiling", action="store_true",
                    help="skip the measured ceilings (fa2_ablate_mfma_ceiling, ~3 s; with "
                         "--pack-short fa2_ablate_hbm_read, ~5 s)")
    ap.add_argument("--sdpa", action="store_true",
                    help="also time torch's fused SDPA on the same inputs (sdpa_same_box, context)")
    sw = ap.add_argument_group("the reference's sequence-length sweep (bench/bench.py:226-307)")
    sw.add_argument("--seqlens", type=int, nargs="+", default=None,
                    help="N_q values (also N_kv unless --kv-len): print the sweep table instead")
    sw.add_argument("--kv-len", type=int, default=None, help="fixed N_kv (non-causal only)")
    sw.add_argument("--batch", type=int, default=1)
    sw.add_argument("--hq", type=int, default=32)
    sw.add_argument("--hkv", type=int, default=8)
    sw.add_argument("--head-dim", type=int, default=128)
    sw.add_argument("--dtype", choices=["fp16", "bf16"], default="fp16")
    sw.add_argument("--no-causal", action="store_true")
    sw.add_argument("--iters", type=int, default=20)
    sw.add_argument("--no-flush", action="store_true")
    sw.add_argument("--providers", nargs="+", default=list(SWEEP_PROVIDERS[:1]) + ["sdpa"],
                    choices=list(SWEEP_PROVIDERS))
    sw.add_argument("--out", default=None, help="also write the rows as JSON here")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus > 1 or world > 1:
        print(json.dumps({"metric": METRIC, "error": "single-GPU build: bench.py runs on one GPU; "
                          f"--gpus {args.gpus} (WORLD_SIZE {world}) is not supported",
                          "n_gpus": args.gpus}), flush=True)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs the GPU")
    if args.seqlens:
        run_seqlens(args)
        return
    if args.pack_short:
        hbm = None
        if not args.no_ceiling:
            try:
                import ceiling

                kv_mib = (2 * PACK_SHORT["B"] * PACK_SHORT["H_kv"] * PACK_SHORT["N_kv"]
                          * PACK_SHORT["D"] * 2) >> 20
                hbm = {"hbm_2gib": ceiling.measure_hbm_read(1.0, 2048),
                       "same_size_as_kv": ceiling.measure_hbm_read(1.0, kv_mib)}
                hbm["gbs"] = hbm["same_size_as_kv"]["gbs"]
                hbm["source"] = ("fa2_ablate_hbm_read (libfa2_ablate.so, csrc/mfma_ceiling.hip): a "
                                 "streaming read, back to back, best grid size, of a 2 GiB buffer "
                                 "(past the 256 MiB Infinity Cache: HBM) and of one the size of "
                                 f"K + V ({kv_mib} MiB, partly cache-resident when read back to back, "
                                 "as the attention's K/V are here); the fraction is against the "
                                 "latter")
            except Exception as e:  # noqa: BLE001
                hbm = {"error": f"{type(e).__name__}: {e}"}
        for n_q in sorted(PACK_SHORT_H100_US):
            res = run_pack_short(n_q, args.steps, args.warmup)
            if hbm is not None:
                res["roofline"]["measured_ceiling"] = hbm
                if hbm.get("gbs"):
                    res["roofline"]["frac_of_measured_read_rate"] = round(
                        res["roofline"]["achieved"] / hbm["gbs"], 4)
            print(json.dumps(res), flush=True)
        return
    names = ["C3", "C2", "C4", "C5"] if args.all else [args.config]
    ceil = None if args.no_ceiling else measured_ceiling()
    for i, name in enumerate(names):
        res = run(name, args.steps, args.warmup, with_cpu=(i == 0 and not args.no_cpu_baseline),
                  flush_iters=args.flush_iters, with_sdpa=args.sdpa, ceiling=ceil)
        print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
