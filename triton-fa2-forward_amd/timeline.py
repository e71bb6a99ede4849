"""Per-workgroup timeline of one forward launch (measurement tool; GPU only).

    python triton-fa2-forward_amd/timeline.py --config C5 [--launches 20] [--csv out.csv]

Runs the product kernel through the measurement library's timeline instance
(fa2_ablate_timeline, include/fa2_ablate.h): the same attention bit for bit, with every
workgroup recording s_memrealtime (100 MHz) at entry, when its prologue is done (Q and the first
K/V tiles in, first barrier passed), when its tile loop is done and when its stores are done, plus
its K/V tile count and the hardware ids of the CU it ran on. The summary of the last launch:

  * span (first entry to last store done) and how full the CU slots were over it;
  * per tile count: how many workgroups, when they started, how long prologue, loop and
    epilogue took, and the loop time per tile;
  * when the second-round workgroups (those that waited for a free slot) started and ended;
  * per XCD: workgroups, tiles of work and when its last workgroup ended.

The timeline instance waits for its stores before the last stamp, which the product kernel does
not; its launch is therefore slightly longer than the product's (reported beside it).
"""

import argparse
import collections
import ctypes
import math
import os
import statistics
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.dirname(HERE))

WORDS = 6          # FA2_ABLATE_TIMELINE_WORDS
MD_HEAD = """# Per-workgroup timeline: fa2::attn_fwd_kernel on {cfg} (one launch, MI355X)

Commands (committed code only; the timeline instance is in libfa2_ablate.so):

    python triton-fa2-forward_amd/timeline.py --config {cfg} --csv {csv}
    python triton-fa2-forward_amd/timeline.py --config {cfg} --from-csv {csv} --md profiles/timeline_{cfg}.md

Every workgroup of the timeline instance (the product kernel, bit for bit, plus s_memrealtime
stamps at 100 MHz) records entry, prologue done (Q and the first K/V tiles in, first barrier),
tile loop done and stores done, its K/V tile count and the hardware id of its CU. It waits for its
stores before the last stamp, which the product kernel does not, so its span is a little longer.
"""
TICK_US = 0.01     # s_memrealtime runs at 100 MHz


def run_timeline(q, k, v, causal, launches):
    """Launch the timeline instance `launches` times; returns (records of the last launch as a
    list of tuples, its output)."""
    import torch

    import ablation
    from fa2 import _lib
    from fa2.kernel import LOG2E

    lib = ablation.ablate_lib()
    fn = lib.fa2_ablate_timeline
    fn.restype = ctypes.c_int
    i32, i64p, vp = ctypes.c_int32, ctypes.POINTER(ctypes.c_int64), ctypes.c_void_p
    fn.argtypes = [vp, vp, vp, vp, i64p, i64p, i64p, i64p] + [i32] * 9 + \
        [ctypes.c_float, vp, ctypes.c_int64, vp]
    B, H_q, N_q, D = q.shape
    H_kv, N_kv = k.shape[1], k.shape[2]
    grid = -(-N_q // 128) * B * H_q
    rec = torch.zeros(grid * WORDS, dtype=torch.int64, device=q.device)
    out = torch.empty_like(q)
    for _ in range(launches):
        rc = fn(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), _lib._strides(q),
                _lib._strides(k), _lib._strides(v), _lib._strides(out), B, H_q, H_kv, N_q, N_kv, D,
                _lib.DTYPE_CODE[q.dtype], int(bool(causal)), 1, LOG2E / math.sqrt(D),
                rec.data_ptr(), rec.numel(), torch.cuda.current_stream().cuda_stream)
        if rc != 0:
            raise RuntimeError(lib.fa2_ablate_last_error().decode(errors="replace"))
    torch.cuda.synchronize()
    r = rec.view(grid, WORDS).cpu().tolist()
    return [tuple(x) for x in r], out


def decode_cu(hw):
    """(xcc, se, sh, cu) from XCC_ID << 32 | HW_ID (gfx9 HW_ID: cu_id bits 8-11, sh_id bit 12,
    se_id bits 13-15; XCC_ID bits 0-3)."""
    hw_id, xcc = hw & 0xFFFFFFFF, (hw >> 32) & 0xF
    return xcc, (hw_id >> 13) & 0x7, (hw_id >> 12) & 1, (hw_id >> 8) & 0xF


def rows_of(recs):
    """Per-workgroup rows (times in us from the first entry) of raw timeline records."""
    t0 = min(r[0] for r in recs)
    rows = []
    for b, (e, p, l, d, tiles, hw) in enumerate(recs):
        rows.append({"block": b, "start": (e - t0) * TICK_US, "prologue": (p - e) * TICK_US,
                     "loop": (l - p) * TICK_US, "epilogue": (d - l) * TICK_US,
                     "end": (d - t0) * TICK_US, "tiles": tiles, "cu": decode_cu(hw)})
    return rows


def rows_from_csv(path):
    """The rows main() --csv wrote (to summarise a saved run again)."""
    rows = []
    with open(path) as f:
        next(f)
        for line in f:
            v = line.strip().split(",")
            rows.append({"block": int(v[0]), "start": float(v[1]), "prologue": float(v[2]),
                         "loop": float(v[3]), "epilogue": float(v[4]), "end": float(v[5]),
                         "tiles": int(v[6]), "cu": tuple(int(x) for x in v[7:11])})
    return rows


def slots_per_cu(rows):
    """The most workgroups resident on one CU at once (two at head_dim 128, three at 64)."""
    best = 0
    by_cu = collections.defaultdict(list)
    for r in rows:
        by_cu[r["cu"]].append(r)
    for g in by_cu.values():
        ev = sorted([(r["start"], 1) for r in g] + [(r["end"], -1) for r in g])
        cur = 0
        for _, d in ev:
            cur += d
            best = max(best, cur)
    return best


def summarize(recs, flops=None):
    return summarize_rows(rows_of(recs), flops)


def summarize_rows(rows, flops=None):
    span = max(r["end"] for r in rows)
    cus = collections.defaultdict(list)
    for r in rows:
        cus[r["cu"]].append(r)
    busy = sum(r["end"] - r["start"] for r in rows)
    slots = slots_per_cu(rows) * len(cus)
    lines = [f"workgroups {len(rows)} on {len(cus)} CUs; span {span:.2f} us"
             + (f" ({flops / (span * 1e-6) / 1e12:.0f} TFLOP/s over the span)" if flops else ""),
             f"resident workgroup-time {busy:.0f} us = {100 * busy / (slots * span):.1f}% of "
             f"{slots} slots ({slots // len(cus)} per CU) x span; summed prologue {sum(r['prologue'] for r in rows):.0f} us, "
             f"loop {sum(r['loop'] for r in rows):.0f} us, epilogue {sum(r['epilogue'] for r in rows):.0f} us",
             "", "| tiles | workgroups | start (us, min-median-max) | prologue us (median) | loop us (median) "
             "| us per tile | epilogue us (median) | end (us, median-max) |", "|---|---|---|---|---|---|---|---|"]
    by_tiles = collections.defaultdict(list)
    for r in rows:
        by_tiles[r["tiles"]].append(r)
    for t in sorted(by_tiles, reverse=True):
        g = by_tiles[t]
        med = lambda key: statistics.median(x[key] for x in g)  # noqa: E731
        lines.append(f"| {t} | {len(g)} | {min(x['start'] for x in g):.1f}-{med('start'):.1f}-"
                     f"{max(x['start'] for x in g):.1f} | {med('prologue'):.2f} | {med('loop'):.2f} | "
                     f"{med('loop') / max(t, 1):.2f} | {med('epilogue'):.2f} | {med('end'):.1f}-"
                     f"{max(x['end'] for x in g):.1f} |")
    late = [r for r in rows if r["start"] > 1.0]
    if late:
        lines += ["", f"second round: {len(late)} workgroups started after 1 us: start "
                  f"{min(r['start'] for r in late):.1f}-{max(r['start'] for r in late):.1f} us, end "
                  f"{min(r['end'] for r in late):.1f}-{max(r['end'] for r in late):.1f} us"]
    xcd = collections.defaultdict(list)
    for r in rows:
        xcd[r["cu"][0]].append(r)
    lines += ["", "| XCD | workgroups | K/V tiles | loop us per tile (median, programs of >= 8 tiles) "
              "| last end (us) |", "|---|---|---|---|---|"]
    for x in sorted(xcd):
        g = xcd[x]
        per_tile = [r["loop"] / r["tiles"] for r in g if r["tiles"] >= 8]
        pt = f"{statistics.median(per_tile):.3f}" if per_tile else "-"
        lines.append(f"| {x} | {len(g)} | {sum(r['tiles'] for r in g)} | {pt} | "
                     f"{max(r['end'] for r in g):.1f} |")
    # the CU that ended last: what it ran
    last_cu = max(cus, key=lambda c: max(r["end"] for r in cus[c]))
    seq = sorted(cus[last_cu], key=lambda r: r["start"])
    lines += ["", "CU that ended last (xcc, se, sh, cu) = %s: " % (last_cu,)
              + "; ".join(f"block {r['block']} {r['tiles']} tiles {r['start']:.1f}-{r['end']:.1f} us"
                          for r in seq)]
    return rows, "\n".join(lines)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="C5")
    ap.add_argument("--launches", type=int, default=20, help="launches before the recorded one")
    ap.add_argument("--csv", default=None, help="also write the per-workgroup rows here")
    ap.add_argument("--from-csv", default=None, help="summarise rows a previous --csv wrote (no GPU)")
    ap.add_argument("--md", default=None,
                    help="with --from-csv: write the summary as a profile (profiles/timeline_<cfg>.md)")
    args = ap.parse_args()
    if args.from_csv:
        import bench

        dt, causal, B, hq, hkv, n, d, scale, outl = bench.WORKLOADS[args.config]
        text = summarize_rows(rows_from_csv(args.from_csv), bench.attn_flops(B, hq, n, n, d, causal))[1]
        if args.md:
            with open(args.from_csv + ".head") if os.path.exists(args.from_csv + ".head") else \
                    open(os.devnull) as f:
                head = f.read().strip()
            with open(args.md, "w") as f:
                f.write(MD_HEAD.format(cfg=args.config, csv=args.from_csv) + "\n" + head + "\n\n"
                        + text + "\n")
        print(text)
        return

    import torch

    import bench
    from ablation import table_free_launch

    q, k, v, causal = bench.make_inputs(args.config, "cuda")
    B, H_q, N, D = q.shape
    flops = bench.attn_flops(B, H_q, N, k.shape[2], D, causal)
    product = table_free_launch(q, k, v, causal)
    bench.settle_clocks(lambda: table_free_launch(q, k, v, causal), min_ms=500.0)
    recs, out = run_timeline(q, k, v, causal, args.launches)
    if not torch.equal(out, product):
        raise SystemExit("the timeline instance's output differs from the product kernel's")
    # the product kernel alone, back to back into one preallocated output (fa2_attn_fwd)
    from fa2 import _lib
    from fa2.kernel import LOG2E

    o = torch.empty_like(q)
    stream = torch.cuda.current_stream().cuda_stream
    scale = LOG2E / math.sqrt(D)
    steps = 200
    prod_ms, _ = bench.time_steps(lambda: _lib.attn_fwd(q, k, v, o, causal, 1, 128, 0, scale, stream),
                                  steps, 5)
    rows, text = summarize(recs, flops)
    head = (f"{bench.describe(args.config)}; output bit-exact with the product kernel; product kernel "
            f"back to back {prod_ms / steps * 1e3:.2f} us per launch")
    print(head)
    print(text)
    if args.csv:
        with open(args.csv + ".head", "w") as f:
            f.write(head + "\n")
        with open(args.csv, "w") as f:
            f.write("block,start_us,prologue_us,loop_us,epilogue_us,end_us,tiles,xcc,se,sh,cu\n")
            for r in rows:
                f.write(f"{r['block']},{r['start']:.2f},{r['prologue']:.2f},{r['loop']:.2f},"
                        f"{r['epilogue']:.2f},{r['end']:.2f},{r['tiles']},{','.join(map(str, r['cu']))}\n")


if __name__ == "__main__":
    main()
