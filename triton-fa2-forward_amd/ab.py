"""Same-box A/B timing of two or more builds of the product library, in interleaved rounds.

    python triton-fa2-forward_amd/csrc/build.py --variant tail0 -D FA2_TAIL_PRIVATE_PCT=0
    python triton-fa2-forward_amd/ab.py --libs cur=triton-fa2-forward_amd/fa2/libfa2_fwd.so \\
        tail0=triton-fa2-forward_amd/variants/tail0/libfa2_fwd.so --configs C3 C2 --rounds 8

Design decisions of a few percent (a schedule rule, a register budget, a tail policy) are made
by timing two builds of the same sources on the same box, in one process: clocks on MI355X move
by several percent between boxes and over minutes under the power limit, so numbers from two
runs do not compare. Each library is loaded from its own path (ctypes), called as attention()
calls the product (fa2_attn_fwd_ex with a workspace of fa2_workspace_bytes_for bytes: the
key-norm table where it pays, default tiles, no split-KV), and the outputs of all libraries are
compared bit for bit with the first one's before and after timing (a schedule change must not
change a result). Clocks are settled once (bench.settle_clocks); then, round after round, every
library runs W warmups and K launches back to back between one pair of HIP events
(bench.time_steps), in forward order on even rounds and reverse order on odd rounds, so that
drift within a round hits all libraries alike. The reference interleaves its variants the same
way (bench/ablation.py:252-255).

Workloads: the BASELINE configs by name (C2..C5), or X:B:Hq:Hkv:N:D:causal:dtype[:scale] for any
other shape (q, k, v from a CPU generator with seed 0, times scale); a ":nt" suffix gives no
workspace (no key-norm table), a ":kt" suffix a workspace with room for the table whatever the
library's policy says (the table then always runs). A library given as NAME=PATH@kt or @nt
takes that table mode on every workload, so that one build can be timed with and without the
table in the same rounds (outputs then need not be equal bit for bit: rows that skip the row max
round differently). A further @bmNNN suffix (after the table mode, if any) launches that library
with BLOCK_M NNN instead of 128 (256: 8-wave programs). With --sustained S, each library then also
runs alone, back to back, for S seconds with the clock and socket power sampled
(ablation.sustained_run): work that costs energy also costs clock under the chip's power limit,
which interleaved rounds, sharing one clock, do not show. Prints one line of JSON per workload,
and a table.
"""

import argparse
import ctypes
import json
import math
import os
import statistics
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.dirname(HERE))


def load(path):
    """One build of the product library, with the C ABI's signatures."""
    from fa2 import _lib

    h = ctypes.CDLL(os.path.abspath(path))
    for name, (rt, at) in _lib.SIGNATURES.items():
        f = getattr(h, name)
        f.restype = rt
        f.argtypes = at
    return h


def parse_lib_suffixes(path):
    """PATH[@kt|@nt][@bmNNN] -> (PATH, table mode or None, BLOCK_M)."""
    bm = 128
    head, sep, tail = path.rpartition("@bm")
    if sep and tail.isdigit():
        path, bm = head, int(tail)
    mode = None
    if path.endswith("@kt") or path.endswith("@nt"):
        path, mode = path[:-3], path[-2:]
    return path, mode, bm


def make_workload(spec):
    """(q, k, v, causal, table) for a config name or X:B:Hq:Hkv:N:D:causal:dtype[:scale], with an
    optional ':nt' (table False: no workspace) or ':kt' (table "force") suffix."""
    import torch

    import bench

    table = True
    if spec.endswith(":nt") or spec.endswith(":kt"):
        table = False if spec.endswith(":nt") else "force"
        spec = spec[:-3]
    base = spec
    if base.startswith("X:"):
        f = base.split(":")
        B, hq, hkv, n, d, c, dt = f[1:8]
        scale = float(f[8]) if len(f) > 8 else 1.0
        g = torch.Generator(device="cpu").manual_seed(0)
        dtype = {"bf16": torch.bfloat16, "fp16": torch.float16}[dt]
        q, k, v = ((torch.randn(int(B), int(h), int(n), int(d), generator=g) * scale).to(dtype).cuda()
                   for h in (hq, hkv, hkv))
        return q, k, v, c == "1", table
    q, k, v, causal = bench.make_inputs(base, "cuda")
    return q, k, v, causal, table


def make_call(h, q, k, v, out, causal, table, block_m=128):
    """A no-argument launch of library `h` on the current stream, as attention() calls it."""
    import torch

    from fa2 import _lib

    B, Hq, Nq, D = q.shape
    Hkv, Nkv = k.shape[1], k.shape[2]
    dt = _lib.DTYPE_CODE[q.dtype]
    if table == "force":   # room for the key-norm table: one float per (batch, kv head, 64 keys)
        nb = (B * Hkv * ((Nkv + 63) // 64) * 4 + 255) // 256 * 256
    else:
        nb = h.fa2_workspace_bytes_for(B, Hq, Hkv, Nq, Nkv, D, dt, int(causal), 1) if table else 0
    ws = torch.empty(max(nb, 1), dtype=torch.uint8, device="cuda")
    strides = [_lib._strides(t) for t in (q, k, v, out)]
    scale = 1.4426950408889634 / math.sqrt(D)
    stream = torch.cuda.current_stream().cuda_stream

    def fn():
        rc = h.fa2_attn_fwd_ex(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), *strides,
                               B, Hq, Hkv, Nq, Nkv, D, dt, int(causal), 1, block_m, 0, scale, None, 1,
                               ws.data_ptr() if nb else None, nb, stream)
        if rc:
            raise RuntimeError(h.fa2_last_error().decode())
    return fn


def ab(libs, spec, rounds, steps, warmup, sustained=0.0):
    """Interleaved rounds over the libraries on one workload; returns the result dict."""
    import torch

    import bench

    q, k, v, causal, table = make_workload(spec)
    B, Hq, N, D = q.shape
    flops = bench.attn_flops(B, Hq, N, k.shape[2], D, causal)
    outs = {n: torch.empty_like(q) for n in libs}
    modes = {"kt": "force", "nt": False, None: table}
    fns = {n: make_call(h, q, k, v, outs[n], causal, modes[mode], bm)
           for n, (h, mode, bm) in libs.items()}
    names = list(libs)
    first = names[0]

    def bit_equal():
        for n in names:
            outs[n].zero_()
            fns[n]()
        torch.cuda.synchronize()
        return {n: bool(torch.equal(outs[n], outs[first])) for n in names}

    same = bit_equal()
    bench.settle_clocks(fns[first])
    per = {n: [] for n in names}
    for r in range(rounds):
        for n in (names if r % 2 == 0 else names[::-1]):
            ms, _ = bench.time_steps(fns[n], steps, warmup)
            per[n].append(ms / steps)
    after = bit_equal()
    alone = {}
    if sustained > 0:
        from ablation import sustained_run

        for n in names:
            alone[n] = sustained_run(fns[n], sustained, flops)
    base = statistics.median(per[first])
    res = {}
    for n in names:
        med = statistics.median(per[n])
        res[n] = {"us": round(med * 1e3, 2), "min_us": round(min(per[n]) * 1e3, 2),
                  "max_us": round(max(per[n]) * 1e3, 2),
                  "tflops": round(flops / (med * 1e-3) / 1e12, 1),
                  "vs_first_pct": round(100.0 * (base / med - 1.0), 2),
                  "bit_equal_to_first": same[n] and after[n]}
        if n in alone:
            a = alone[n]
            res[n]["alone"] = {"tflops": round(a["tflops"], 1), "sclk_mhz": a["sclk_mhz"],
                               "power_w": a["power_w"]}
    del q, k, v, outs, fns
    torch.cuda.empty_cache()
    return res


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--libs", nargs="+", required=True, metavar="NAME=PATH")
    ap.add_argument("--configs", nargs="+", default=["C3"])
    ap.add_argument("--rounds", type=int, default=8)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--sustained", type=float, default=0.0,
                    help="also each build alone for this many seconds: its rate, clock and power")
    ap.add_argument("--out", default=None, help="also write the results as JSON here")
    args = ap.parse_args()

    import torch  # noqa: F401  (the HIP runtime before the libraries)

    libs = {}
    for spec in args.libs:
        name, path = spec.split("=", 1)
        path, mode, bm = parse_lib_suffixes(path)
        libs[name] = (load(path), mode, bm)
    results = {}
    for cfg in args.configs:
        print(f"ab: {cfg}, {len(libs)} builds, {args.rounds} rounds x {args.steps} steps", flush=True)
        res = ab(libs, cfg, args.rounds, args.steps, args.warmup, args.sustained)
        results[cfg] = res
        print(json.dumps({"workload": cfg, "builds": res}), flush=True)
        for n, r in res.items():
            print(f"  {cfg:24s} {n:12s} {r['us']:10.2f} us [{r['min_us']:.2f}-{r['max_us']:.2f}] "
                  f"{r['tflops']:8.1f} TFLOP/s {r['vs_first_pct']:+6.2f}%  same={r['bit_equal_to_first']}"
                  + (f"  alone {r['alone']['tflops']:.1f} TFLOP/s at {r['alone']['sclk_mhz']} MHz, "
                     f"{r['alone']['power_w']} W" if "alone" in r else ""),
                  flush=True)
    if args.out:
        with open(args.out, "w") as f:
            json.dump({"libs": dict(s.split("=", 1) for s in args.libs), "rounds": args.rounds,
                       "steps": args.steps, "results": results}, f, indent=1)


if __name__ == "__main__":
    main()
