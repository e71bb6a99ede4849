"""Tile-configuration sweep on gfx950 (counterpart of the reference's bench/sweep.py:24-105).

    python triton-fa2-forward_amd/sweep.py --config C3 [--block-m 64 128 256] [--block-n 32 64 128]
                                           [--rounds 5] [--iters 10] [--json out.json]

Times every (block_m, block_n) pair on one BASELINE.json workload, interleaved over rounds so
that clock drift hits all variants alike (the reference's ablation protocol,
bench/ablation.py:252-255), after checking each variant's output against the default one
(max-abs within the 2e-2 bench gate). Prints one line per variant: median TFLOP/s, median ms,
and the kernel's register, LDS and occupancy figures the library was built with are in the
build log (hipcc -Rpass-analysis=kernel-resource-usage).
"""

import argparse
import json
import os
import statistics
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.dirname(HERE))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="C3")
    ap.add_argument("--block-m", type=int, nargs="+", default=[64, 128, 256])
    ap.add_argument("--block-n", type=int, nargs="+", default=[32, 64, 128])
    ap.add_argument("--rounds", type=int, default=5)
    ap.add_argument("--iters", type=int, default=10)
    ap.add_argument("--json", default=None)
    args = ap.parse_args()

    import torch

    import bench
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
    rows = []
    for (bm, bn), ms in samples.items():
        med = statistics.median(ms)
        rows.append({"block_m": bm, "block_n": bn, "median_ms": med,
                     "tflops": flops / (med * 1e-3) / 1e12, "samples_ms": ms})
    rows.sort(key=lambda r: r["median_ms"])
    print(f"{bench.describe(args.config)}: median over {args.rounds} interleaved rounds of {args.iters}")
    for r in rows:
        print(f"  block_m={r['block_m']:4d} block_n={r['block_n']:4d}  {r['median_ms']:8.4f} ms  "
              f"{r['tflops']:7.1f} TFLOP/s", flush=True)
    if args.json:
        with open(args.json, "w") as f:
            json.dump({"config": args.config, "rows": rows}, f, indent=1)


if __name__ == "__main__":
    main()
