"""What the matrix cores sustain on this chip (measurement tool; GPU only).

    python triton-fa2-forward_amd/ceiling.py [--seconds 2]

MI355X's dense bf16 peak (2516.6 TFLOP/s) is 256 CUs x 4096 FLOP per clock at 2.4 GHz. Under a
long MFMA load the chip holds its socket power near the limit by lowering the graphics clock, and
an MFMA's energy depends on its operands' bits, so what it sustains depends on the data and on
the other work beside the MFMAs. fa2_ablate_mfma_ceiling (include/fa2_ablate.h; the kernel is
csrc/mfma_ceiling.hip in the measurement library) issues bf16 32x32x16 MFMAs back to back in the
attention kernel's launch shape; each mode runs alone for --seconds after a short warm-up, with
amdsmi sampling the clock and the socket power:

  mfma              random operands in registers: the chip's MFMA ceiling on real data
  mfma_const        constant operands (1.0): the ceiling the data sheet's clock allows
  mfma_lds          random, plus one 1 KiB ds_read_b128 per MFMA (the K/V operand reads of the
                    attention kernel's 32-row waves)
  mfma_lds_softmax  that plus the softmax's vector work per MFMA (head_dim 128: one FMA and one
                    exp2 per score, half a bf16 pack, half a dot2 row sum), on independent data
  mfma_exp          random, registers, one exp2 per MFMA    } what one exp2 costs beside the
  mfma_fma2         random, registers, two FMAs per MFMA    } MFMAs, against two FMAs
  mfma_lds_softmax_vacc  mfma_lds_softmax with the accumulators in VGPRs, as the attention
                    kernel holds them (the compiler puts the other modes' in AGPRs)
  half_lds_softmax_vacc  that with one 1 KiB read per two MFMAs: the operand reads of 64-row
                    waves, whose K and V operands each feed two 32-row blocks' MFMAs (four
                    accumulators, as such a wave has at least that many tiles in flight)
  half_lds_softmax_vacc_1wave  the same at one wave per SIMD (128 KiB of LDS per workgroup,
                    one workgroup per CU), the occupancy of 64-row waves at head_dim 128
  lds_softmax64_vacc_3wave  mfma_lds_softmax_vacc with head_dim 64's softmax per MFMA (two FMAs,
                    two exp2, one pack, one dot2) at three waves per SIMD (48 KiB of LDS each)

Per mode: TFLOP/s, the median graphics clock and power, TFLOP/s per GHz (the issue efficiency,
whatever the clock: the peak is 1048.6 per GHz) and the fraction of the 2.4 GHz peak.

--hbm adds the memory-side ceiling (fa2_ablate_hbm_read): a streaming read, back to back, 16
bytes per lane per load, at a few grid sizes, against the 8 TB/s HBM peak, of a 2 GiB buffer (far
past the 256 MiB Infinity Cache: what HBM sustains) and of 256 and 64 MiB buffers (partly or
wholly cache-resident when read back to back).
"""

import argparse
import ctypes
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.dirname(HERE))

MODES = {"mfma": 0, "mfma_const": 1, "mfma_lds": 2, "mfma_lds_softmax": 3,  # FA2_ABLATE_CEIL_*
         "mfma_exp": 4, "mfma_fma2": 5, "mfma_lds_softmax_vacc": 6,
         "half_lds_softmax_vacc": 7, "half_lds_softmax_vacc_1wave": 8,
         "lds_softmax64_vacc_3wave": 9}
PEAK_TFLOPS = 2516.6            # 256 CUs x 4096 FLOP/clk x 2.4 GHz (dense bf16/fp16)
PEAK_MHZ = 2400.0
MFMA_FLOP = 32 * 32 * 16 * 2    # one v_mfma_f32_32x32x16_bf16
WORKGROUPS = 2048               # 8 per CU: four rounds of the two resident workgroups
# three resident workgroups per CU: 9 per CU, three whole rounds
WORKGROUPS_BY_MODE = {"lds_softmax64_vacc_3wave": 2304}
ITERS = 6000                    # 16 MFMAs each: ~10 ms per launch at ~1900 TFLOP/s


def _fn():
    import ablation

    lib = ablation.ablate_lib()
    fn = lib.fa2_ablate_mfma_ceiling
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p,
                   ctypes.c_int64, ctypes.c_void_p]
    return lib, fn


def launch_flops(workgroups=WORKGROUPS, iters=ITERS):
    return workgroups * 4 * iters * 16 * MFMA_FLOP


def measure(mode, seconds=2.0, warm_s=0.5, workgroups=WORKGROUPS, iters=ITERS):
    """Run `mode` back to back: `warm_s` untimed, then `seconds` timed with the clock sampler.
    Returns {tflops, sclk_mhz, power_w, tflops_per_ghz, frac_of_peak, launches}."""
    import torch

    import bench

    lib, fn = _fn()
    out = torch.empty(workgroups * 256, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream

    def launch():
        rc = fn(MODES[mode], workgroups, iters, out.data_ptr(), out.numel(), stream)
        if rc != 0:
            raise RuntimeError(lib.fa2_ablate_last_error().decode(errors="replace"))

    t0 = time.perf_counter()
    while time.perf_counter() - t0 < warm_s:
        launch()
        torch.cuda.synchronize()
    with bench.ClockSampler() as smp:
        t0 = time.perf_counter()
        n = 0
        while time.perf_counter() - t0 < seconds:
            for _ in range(4):
                launch()
            n += 4
            torch.cuda.synchronize()
        dt = time.perf_counter() - t0
    clk = smp.summary()
    tflops = launch_flops(workgroups, iters) * n / dt / 1e12
    sclk = clk.get("sclk_mhz_median")
    return {"tflops": round(tflops, 1), "sclk_mhz": sclk, "power_w": clk.get("power_w_median"),
            "tflops_per_ghz": round(tflops / (sclk / 1000.0), 1) if sclk else None,
            "frac_of_peak": round(tflops / PEAK_TFLOPS, 4), "launches": n,
            "seconds": round(dt, 2)}


HBM_PEAK_GBS = 8000.0


def measure_hbm_read(seconds=1.0, mib=2048, workgroups=(1024, 2048, 4096, 8192)):
    """Streaming read of a `mib` MiB buffer back to back for `seconds` per grid size: {workgroups:
    GB/s} and the best, in GB/s and as a fraction of the 8 TB/s peak."""
    import torch

    import ablation

    lib = ablation.ablate_lib()
    fn = lib.fa2_ablate_hbm_read
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32,
                   ctypes.c_void_p]
    nbytes = mib << 20
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").random_(0, 256)
    out = torch.empty(max(workgroups) * 256, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    rates = {}
    for wg in workgroups:
        def launch():
            rc = fn(src.data_ptr(), nbytes, out.data_ptr(), out.numel(), wg, stream)
            if rc != 0:
                raise RuntimeError(lib.fa2_ablate_last_error().decode(errors="replace"))
        for _ in range(3):
            launch()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        n = 0
        while time.perf_counter() - t0 < seconds:
            for _ in range(5):
                launch()
            n += 5
            torch.cuda.synchronize()
        rates[wg] = round(nbytes * n / (time.perf_counter() - t0) / 1e9, 1)
    best = max(rates.values())
    del src
    return {"gbs_by_workgroups": rates, "gbs": best, "frac_of_peak": round(best / HBM_PEAK_GBS, 4),
            "buffer_mib": mib}


def main():
    ap = argparse.ArgumentParser(description="sustained MFMA rate under the chip's power limit")
    ap.add_argument("--seconds", type=float, default=2.0)
    ap.add_argument("--modes", nargs="+", default=list(MODES), choices=list(MODES))
    ap.add_argument("--hbm", action="store_true", help="also the streaming HBM read rate")
    args = ap.parse_args()

    import torch

    if not torch.cuda.is_available():
        raise SystemExit("ceiling.py needs the GPU")
    print(f"{torch.cuda.get_device_name(0)}: bf16 32x32x16 MFMAs, {WORKGROUPS} workgroups of 256 "
          f"threads (two per CU), {ITERS} x 16 MFMAs per wave per launch; each mode alone for "
          f"{args.seconds:g} s after 0.5 s")
    print("| mode | TFLOP/s | sclk MHz (median) | power W (median) | TFLOP/s per GHz | % of 2516.6 |")
    print("|---|---|---|---|---|---|")
    rows = {}
    for m in args.modes:
        r = rows[m] = measure(m, args.seconds, workgroups=WORKGROUPS_BY_MODE.get(m, WORKGROUPS))
        print(f"| {m} | {r['tflops']:.0f} | {r['sclk_mhz']} | {r['power_w']} | "
              f"{r['tflops_per_ghz']} | {100 * r['frac_of_peak']:.1f} |", flush=True)
    if args.hbm:
        print()
        for mib in (2048, 256, 64):
            h = measure_hbm_read(args.seconds / 2, mib)
            print(f"streaming read of {h['buffer_mib']} MiB (fa2_ablate_hbm_read): "
                  + ", ".join(f"{wg} workgroups {gbs:.0f} GB/s" for wg, gbs in h["gbs_by_workgroups"].items())
                  + f"; best {h['gbs']:.0f} GB/s = {100 * h['frac_of_peak']:.1f}% of 8 TB/s", flush=True)
            rows[f"hbm_read_{mib}mib"] = h
    return rows


if __name__ == "__main__":
    main()
