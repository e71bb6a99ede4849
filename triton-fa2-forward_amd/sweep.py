"""Tile-configuration sweep on gfx950 (counterpart of the reference's bench/sweep.py:24-105).

    python triton-fa2-forward_amd/sweep.py --config C3 [--block-m 64 128 256] [--block-n 32 64 128]
                                           [--rounds 5] [--iters 10] [--sustained 2] [--json out.json]

Times every (block_m, block_n) pair on one BASELINE.json workload, interleaved over rounds so
that clock drift hits all variants alike (the reference's ablation protocol,
bench/ablation.py:252-255), after checking each variant's output against the default one
(max-abs within the 2e-2 bench gate). Prints one line per variant: median TFLOP/s, median ms,
and the compiled resources of the kernel instance that ran it, as the reference's sweep prints
registers, spills and shared memory (bench/sweep.py:95-100): VGPRs, AGPRs, SGPRs, VGPR and SGPR
spills, LDS per workgroup and waves per SIMD, from the compiler's own report of this build
(fa2/kernel_resources.json, written by csrc/build.py from -Rpass-analysis=kernel-resource-usage).
With --sustained S, each variant then also runs alone, back to back, for S seconds with the clock
and socket power sampled (ablation.sustained_run): the chip holds its power limit by lowering the
clock, so a configuration that stages fewer K/V bytes per FLOP (more rows per workgroup) can gain
clock that the interleaved rounds, which share one clock between all variants, do not show.
"""

import argparse
import json
import os
import statistics
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.dirname(HERE))


RESOURCES_PATH = os.path.join(HERE, "fa2", "kernel_resources.json")


def load_resources():
    try:
        with open(RESOURCES_PATH) as f:
            return json.load(f)["kernels"]
    except (OSError, KeyError, ValueError):
        return {}


def instance_name(dtype_code, head_dim, block_m, block_n, causal, key_table):
    """Mangled name of the attn_fwd_kernel instance a launch with these tiles runs (the C ABI's
    choice: block_m -> 1, 2, 4 or 8 waves of 32 rows, block_n -> 32, 64 or 128 keys; the key-norm
    instance, VARIANT 4, only at the default configuration when the table is in use)."""
    from fa2.kernel import _default_config

    waves = 1
    while waves * 32 < block_m:
        waves *= 2
    bn = 32 if block_n <= 32 else 64 if block_n <= 64 else 128
    default_bn = _default_config(head_dim, True)[1]
    variant = 4 if key_table and waves == 4 and bn == default_bn else 0
    return (f"_ZN3fa215attn_fwd_kernelILi{dtype_code}ELi{head_dim}ELi{waves}ELi{bn}"
            f"ELb{int(bool(causal))}ELi{variant}EEEvNS_6ParamsE")


def resource_text(res):
    if not res:
        return "(resources: build the library to get fa2/kernel_resources.json)"
    return (f"vgpr {res['vgprs']:3d} agpr {res['agprs']} sgpr {res['sgprs']:3d} "
            f"spill v{res['vgpr_spills']}/s{res['sgpr_spills']} lds {res['lds_bytes'] // 1024} KiB "
            f"{res['waves_per_simd']} waves/SIMD")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="C3")
    ap.add_argument("--block-m", type=int, nargs="+", default=[64, 128, 256])
    ap.add_argument("--block-n", type=int, nargs="+", default=[32, 64, 128])
    ap.add_argument("--rounds", type=int, default=5)
    ap.add_argument("--iters", type=int, default=10)
    ap.add_argument("--sustained", type=float, default=0.0,
                    help="also each variant alone for this many seconds: its rate, clock and power")
    ap.add_argument("--json", default=None)
    args = ap.parse_args()

    import torch

    import bench
    from fa2 import _lib
    from fa2.kernel import attention

    q, k, v, causal = bench.make_inputs(args.config, "cuda")
    B, H_q, N, D = q.shape
    flops = bench.attn_flops(B, H_q, N, k.shape[2], D, causal)
    ref = attention(q, k, v, causal=causal)
    variants = []
    for bm in args.block_m:
        for bn in args.block_n:
            try:
                out = attention(q, k, v, causal=causal, block_m=bm, block_n=bn)
                err = (out.float() - ref.float()).abs().max().item()
                if not err <= 2e-2:
                    raise RuntimeError(f"output differs from the default config: max-abs {err:.3e}")
                variants.append((bm, bn))
            except Exception as e:  # noqa: BLE001 - report and skip the variant
                print(f"skip block_m={bm} block_n={bn}: {e}", flush=True)
    stream = torch.cuda.current_stream()
    # settle the clocks first (bench.py's settle phase): otherwise the first rounds run in the
    # ramp after the idle correctness checks
    bench.settle_clocks(lambda: attention(q, k, v, causal=causal))
    samples = {vv: [] for vv in variants}
    for r in range(args.rounds):
        for bm, bn in variants:
            fn = lambda: attention(q, k, v, causal=causal, block_m=bm, block_n=bn)  # noqa: E731
            fn()
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            s.record(stream)
            for _ in range(args.iters):
                fn()
            e.record(stream)
            torch.cuda.synchronize()
            samples[(bm, bn)].append(s.elapsed_time(e) / args.iters)
        print(f"round {r + 1}/{args.rounds} done", flush=True)
    sustained = {}
    if args.sustained > 0:
        from ablation import sustained_run

        for bm, bn in variants:
            sustained[(bm, bn)] = sustained_run(
                lambda: attention(q, k, v, causal=causal, block_m=bm, block_n=bn), args.sustained,
                flops)
            print(f"sustained block_m={bm} block_n={bn} done", flush=True)
    resources = load_resources()
    key_table = (_lib.workspace_bytes_for(B, H_q, k.shape[1], N, k.shape[2], D, q.dtype, causal, 1)
                 > _lib.workspace_bytes(B, H_q, N, D, 1))
    rows = []
    for (bm, bn), ms in samples.items():
        med = statistics.median(ms)
        name = instance_name(_lib.DTYPE_CODE[q.dtype], D, bm, bn, causal, key_table)
        rows.append({"block_m": bm, "block_n": bn, "median_ms": med,
                     "tflops": flops / (med * 1e-3) / 1e12, "samples_ms": ms,
                     "kernel": name, "resources": resources.get(name),
                     **({"sustained": sustained[(bm, bn)]} if (bm, bn) in sustained else {})})
    rows.sort(key=lambda r: r["median_ms"])
    print(f"{bench.describe(args.config)}: median over {args.rounds} interleaved rounds of {args.iters}")
    for r in rows:
        su = r.get("sustained")
        alone = ""
        if su:
            ghz = (su["sclk_mhz"] or 0) / 1000.0
            alone = (f"  alone: {su['tflops']:7.1f} TFLOP/s at {su['sclk_mhz']} MHz, {su['power_w']} W"
                     + (f", {su['tflops'] / ghz:.1f} per GHz" if ghz else ""))
        print(f"  block_m={r['block_m']:4d} block_n={r['block_n']:4d}  {r['median_ms']:8.4f} ms  "
              f"{r['tflops']:7.1f} TFLOP/s  {resource_text(r['resources'])}{alone}", flush=True)
    if args.json:
        with open(args.json, "w") as f:
            json.dump({"config": args.config, "rows": rows}, f, indent=1)


if __name__ == "__main__":
    main()
