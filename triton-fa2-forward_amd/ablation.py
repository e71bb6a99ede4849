"""Timing variants of the forward kernel: what each kind of its work costs (the counterpart of the
reference's bench/ablation.py). GPU only; a measurement tool, not part of the drop-in.

    python triton-fa2-forward_amd/ablation.py                          # fp16, N 4096 and 16384, causal
    python triton-fa2-forward_amd/ablation.py --seqlens 8192 --dtype bf16 --rounds 5       # C3
    python triton-fa2-forward_amd/ablation.py --seqlens 16384 --batch 2 --hq 16 --hkv 16 \\
        --head-dim 64 --full --input-scale 0.5 --rounds 5                                    # C4
    ... --sustained 2      # also each variant alone for 2 s: its rate, clock and power

Every variant is the product's kernel template instantiated with VARIANT bits
(include/fa2_ablate.h), loaded from the measurement library libfa2_ablate.so, which fa2.kernel
never loads. The reference's variants (bench/ablation.py:1-20, 42-53):

  copy             no switch: the product kernel, bit for bit the launch of fa2_attn_fwd
  scale_first      multiply every score by the scale, then subtract the row max
  mask_every_tile  apply the mask on every K/V tile, not only where needed
  before_fixes     both of the above
  no_exp           exp2 replaced by its argument            (output wrong on purpose)
  no_softmax       no mask, max, exp, sum or rescale        (output wrong on purpose)
  kv_l2            every tile loads K/V tile 0 again: L2 hits instead of HBM reads
  matmul_only      no_softmax + kv_l2: the two products and the loads' issue cost
  no_kv_staging    K/V tiles from the third on are not loaded at all (output wrong on purpose;
                   not in the reference): what staging K/V through LDS costs beyond the first tiles
  split_keys       8 waves per program in two groups over the two halves of its key range,
                   merged through LDS, one workgroup per CU (head_dim 128; still attention; not in
                   the reference): what halving the longest program's path buys
  no_q_load        Q is not read from memory (a lane pattern instead; output wrong on purpose;
                   not in the reference): what a program's Q load costs
  no_store         the output is not written (output wrong on purpose; not in the reference):
                   what a program's store costs
  pack             copy with GQA head packing forced on
  static_order     copy without the dynamic tail of causal grids: workgroup b runs program b
                   (not in the reference; what the run-time dealing of the last programs buys)

Measurement (this repository's bench.py harness): the clocks are settled once (bench.settle_clocks);
then, round after round, every variant runs W warmup launches and K launches back to back between one
pair of HIP events (bench.time_steps), so that each round yields one ms-per-launch figure per variant
and clock drift hits all variants alike. The table gives each variant's median over the rounds, the
spread of its rounds, and the change against `copy`. `attention()` is the shipped call on the same
inputs; on long bf16 problems it adds the key-norm pass and that instance of the kernel (C3), which
the variants do not have, so the deltas are taken against `copy`, not against it.

With --sustained, each variant then also runs alone, back to back, with amdsmi sampling the clock
and the socket power (sustained_run): the chip holds its power near the limit by lowering the
clock, so a switch that saves energy also buys clock, which the interleaved rounds (one clock for
all variants) cannot show; TFLOP/s per GHz separates the two.
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

ABLATE_LIB_PATH = os.path.join(HERE, "libfa2_ablate.so")

# switch -> VARIANT bit (FA2_ABLATE_* in include/fa2_ablate.h)
SWITCH_BITS = {"scale_first": 1, "mask_every_tile": 2, "no_exp": 8, "no_softmax": 16, "kv_l2": 32,
               "static_order": 128, "no_kv_staging": 256, "split_keys": 512, "no_q_load": 1024,
               "no_store": 2048}
KNOBS = tuple(SWITCH_BITS)
VARIANTS = {
    "copy": (),
    "scale_first": ("scale_first",),
    "mask_every_tile": ("mask_every_tile",),
    "before_fixes": ("scale_first", "mask_every_tile"),
    "no_exp": ("no_exp",),
    "no_softmax": ("no_softmax",),
    "kv_l2": ("kv_l2",),
    "matmul_only": ("no_softmax", "kv_l2"),
    "no_kv_staging": ("no_kv_staging",),
    "split_keys": ("split_keys",),
    "no_q_load": ("no_q_load",),
    "no_store": ("no_store",),
    "pack": ("pack",),
    "static_order": ("static_order",),
}
# variants whose output must equal the product's bit for bit (the others change rounding or are
# wrong by design)
EXACT = ("copy", "mask_every_tile", "pack", "static_order")

_LIB = None


def ablate_lib():
    """libfa2_ablate.so, loaded on first use (after torch, which brings the HIP runtime)."""
    global _LIB
    if _LIB is None:
        import torch  # noqa: F401

        if not os.path.exists(ABLATE_LIB_PATH):
            raise RuntimeError(f"{ABLATE_LIB_PATH} is missing; build it with "
                               "python triton-fa2-forward_amd/csrc/build.py")
        lib = ctypes.CDLL(ABLATE_LIB_PATH)
        i32, i64p, vp = ctypes.c_int32, ctypes.POINTER(ctypes.c_int64), ctypes.c_void_p
        lib.fa2_ablate_attn_fwd.restype = ctypes.c_int
        lib.fa2_ablate_attn_fwd.argtypes = [vp, vp, vp, vp, i64p, i64p, i64p, i64p] + [i32] * 9 + \
            [ctypes.c_float, i32, vp]
        lib.fa2_ablate_last_error.restype = ctypes.c_char_p
        lib.fa2_ablate_last_error.argtypes = []
        _LIB = lib
    return _LIB


def variant_bits(switches):
    unknown = set(switches) - set(SWITCH_BITS)
    assert not unknown, f"unknown switches {sorted(unknown)}"
    return sum(SWITCH_BITS[s] for s in switches)


def attention_ablate(q, k, v, causal=True, pack_gqa=False, **knobs):
    """fa2.kernel.attention at the default configuration with the switches in KNOBS turned on
    (the reference's attention_ablate signature, bench/ablation.py:182-200); the argument rules are
    attention()'s."""
    import torch

    from fa2 import _lib
    from fa2.kernel import LOG2E, _default_config, _loadable

    bits = variant_bits([name for name, on in knobs.items() if on])
    assert q.dim() == k.dim() == v.dim() == 4
    B, H_q, N_q, D = q.shape
    H_kv, N_kv = k.shape[1], k.shape[2]
    assert v.shape == k.shape and k.shape[0] == B and k.shape[3] == D
    assert q.dtype == k.dtype == v.dtype and q.dtype in (torch.float16, torch.bfloat16)
    assert H_q % H_kv == 0, "GQA needs H_q divisible by H_kv"
    assert D in (16, 32, 64, 128), "head_dim must be a power of two in [16, 128]"
    if causal:
        assert N_q == N_kv, "causal attention here assumes N_q == N_kv"
    group = H_q // H_kv
    block_m = _default_config(D, True)[0]
    if pack_gqa and block_m % group:
        raise ValueError(f"pack_gqa needs BLOCK_M ({block_m}) to be a multiple of the GQA group ({group})")
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise RuntimeError("attention_ablate runs on the GPU; got CPU tensors")
    out = torch.empty_like(q)
    if out.numel() == 0:
        return out
    q_, k_, v_, o_ = _loadable(q), _loadable(k), _loadable(v), _loadable(out)
    lib = ablate_lib()
    with torch.cuda.device(q.device):
        rc = lib.fa2_ablate_attn_fwd(
            q_.data_ptr(), k_.data_ptr(), v_.data_ptr(), o_.data_ptr(), _lib._strides(q_),
            _lib._strides(k_), _lib._strides(v_), _lib._strides(o_), B, H_q, H_kv, N_q, N_kv, D,
            _lib.DTYPE_CODE[q.dtype], int(bool(causal)), group if pack_gqa else 1,
            LOG2E / math.sqrt(D), bits, torch.cuda.current_stream(q.device).cuda_stream)
    if rc != 0:
        raise RuntimeError(f"fa2_ablate_attn_fwd failed ({rc}): "
                           f"{lib.fa2_ablate_last_error().decode(errors='replace')}")
    if o_ is not out:
        out.copy_(o_)
    return out


def table_free_launch(q, k, v, causal):
    """fa2_attn_fwd at the default configuration: the product kernel without the key-norm table,
    which is what `copy` must equal bit for bit."""
    import torch

    from fa2 import _lib
    from fa2.kernel import LOG2E

    out = torch.empty_like(q)
    _lib.attn_fwd(q, k, v, out, causal, 1, 128, 0, LOG2E / math.sqrt(q.shape[3]),
                  torch.cuda.current_stream().cuda_stream)
    return out


def launcher(name, q, k, v, causal):
    switches = [s for s in VARIANTS[name] if s != "pack"]
    pack = "pack" in VARIANTS[name]
    return lambda: attention_ablate(q, k, v, causal=causal, pack_gqa=pack,
                                    **{s: True for s in switches})


def interleaved_rounds(launchers, rounds, steps, warmup):
    """{name: [ms per launch, one per round]}: bench.time_steps per variant, variants interleaved."""
    import bench

    per_round = {name: [] for name in launchers}
    for _ in range(rounds):
        for name, fn in launchers.items():
            total_ms, _ = bench.time_steps(fn, steps, warmup)
            per_round[name].append(total_ms / steps)
    return per_round


def sustained_run(fn, seconds, flops):
    """One variant alone, back to back for `seconds`, with the clock sampler beside it: the rate,
    graphics clock and socket power it sustains. The chip holds its power near the limit by
    lowering the clock, so work that costs energy (exp, LDS reads) also costs clock; the
    interleaved rounds share one clock between all variants and cannot show that part."""
    import time

    import torch

    import bench

    fn()
    torch.cuda.synchronize()
    # launches per synchronize: ~20 ms of work, so that short kernels (C5: ~30 us) are not timed
    # with a host round trip every few hundred microseconds
    t0 = time.perf_counter()
    for _ in range(10):
        fn()
    torch.cuda.synchronize()
    batch = max(10, int(0.02 / max((time.perf_counter() - t0) / 10, 1e-6)))
    with bench.ClockSampler() as smp:
        t0 = time.perf_counter()
        n = 0
        while time.perf_counter() - t0 < seconds:
            for _ in range(batch):
                fn()
            n += batch
            torch.cuda.synchronize()
        dt = time.perf_counter() - t0
    clk = smp.summary()
    return {"tflops": flops * n / dt / 1e12, "launches": n,
            "sclk_mhz": clk.get("sclk_mhz_median"), "power_w": clk.get("power_w_median")}


def measure_shape(args, N):
    import torch

    import bench
    from fa2.kernel import attention

    dtype = {"fp16": torch.float16, "bf16": torch.bfloat16}[args.dtype]
    causal = not args.full
    g = torch.Generator(device="cpu").manual_seed(0)
    q, k, v = (torch.randn(args.batch, h, N, args.head_dim, generator=g) * args.input_scale
               for h in (args.hq, args.hkv, args.hkv))
    q, k, v = (t.to(dtype).cuda() for t in (q, k, v))
    flops = bench.attn_flops(args.batch, args.hq, N, N, args.head_dim, causal)

    product = table_free_launch(q, k, v, causal)
    shipped = attention(q, k, v, causal=causal)
    launchers = {"attention()": lambda: attention(q, k, v, causal=causal)}
    outputs = {}
    group = args.hq // args.hkv
    for name in args.variants:
        if name == "pack" and (group == 1 or 128 % group):
            print(f"(pack skipped: GQA group {group} does not pack into 128-row programs)")
            continue
        if name == "split_keys" and args.head_dim != 128:
            print(f"(split_keys skipped: built at head_dim 128 only, not {args.head_dim})")
            continue
        launchers[name] = launcher(name, q, k, v, causal)
        outputs[name] = launchers[name]()
    torch.cuda.synchronize()
    checks = {}
    for name, out in outputs.items():
        diff = (out.float() - product.float()).abs().max().item()
        checks[name] = {"bit_exact": bool(torch.equal(out, product)), "max_abs_diff": diff}
        if name in EXACT and not checks[name]["bit_exact"]:
            raise SystemExit(f"variant {name} differs from the product kernel (max diff {diff:.3e})")
    checks["attention()"] = {"bit_exact": bool(torch.equal(shipped, product)),
                             "max_abs_diff": (shipped.float() - product.float()).abs().max().item()}

    bench.settle_clocks(launchers["copy"] if "copy" in launchers else launchers["attention()"])
    per_round = interleaved_rounds(launchers, args.rounds, args.steps, args.warmup)
    base = statistics.median(per_round["copy"]) if "copy" in per_round else None
    sustained = {name: sustained_run(fn, args.sustained, flops) for name, fn in launchers.items()} \
        if args.sustained > 0 else {}
    rows = []
    for name, ms in per_round.items():
        med = statistics.median(ms)
        rows.append({"variant": name, "ms": med, "min_ms": min(ms), "max_ms": max(ms),
                     "vs_copy": (med / base - 1.0) if base else None,
                     "tflops": flops / (med * 1e-3) / 1e12, **checks.get(name, {}),
                     **({"sustained": sustained[name]} if name in sustained else {})})
    del q, k, v, product, shipped, outputs
    torch.cuda.empty_cache()
    return flops, rows


def print_table(args, N, rows):
    shape = (f"B={args.batch} H {args.hq}/{args.hkv} N={N} D={args.head_dim} {args.dtype} "
             f"{'full' if args.full else 'causal'}" + (f" inputs x{args.input_scale}" if args.input_scale != 1 else ""))
    print(f"\n{shape}: {args.rounds} rounds of {args.steps} back-to-back launches per variant")
    sus = all("sustained" in r for r in rows)
    print("| variant | ms per launch (median; min-max over rounds) | vs copy | TFLOP/s | output vs product |"
          + (f" alone for {args.sustained:g} s: TFLOP/s | sclk MHz | power W | TFLOP/s per GHz |" if sus else ""))
    print("|---|---|---|---|---|" + ("---|---|---|---|" if sus else ""))
    for r in rows:
        if r.get("bit_exact"):
            out = "bit-exact"
        elif "max_abs_diff" in r:
            out = f"max diff {r['max_abs_diff']:.2e}"
        else:
            out = ""
        vs = "" if r["vs_copy"] is None or r["variant"] == "copy" else f"{r['vs_copy']:+.1%}"
        extra = ""
        if sus:
            su = r["sustained"]
            ghz = (su["sclk_mhz"] or 0) / 1000.0
            extra = (f" {su['tflops']:.1f} | {su['sclk_mhz'] or '-'} | {su['power_w'] or '-'} | "
                     f"{su['tflops'] / ghz:.1f} |" if ghz else f" {su['tflops']:.1f} | - | - | - |")
        print(f"| {r['variant']} | {r['ms']:.4f} ({r['min_ms']:.4f}-{r['max_ms']:.4f}) | {vs} | "
              f"{r['tflops']:.1f} | {out} |" + extra, flush=True)


def main():
    ap = argparse.ArgumentParser(description="timing variants of the forward kernel")
    ap.add_argument("--seqlens", type=int, nargs="+", default=[4096, 16384])
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--hq", type=int, default=32)
    ap.add_argument("--hkv", type=int, default=8)
    ap.add_argument("--head-dim", type=int, default=128)
    ap.add_argument("--dtype", choices=["fp16", "bf16"], default="fp16")
    ap.add_argument("--full", action="store_true", help="no causal mask")
    ap.add_argument("--input-scale", type=float, default=1.0, help="q, k, v ~ N(0, 1) times this")
    ap.add_argument("--variants", nargs="+", default=list(VARIANTS), choices=list(VARIANTS))
    ap.add_argument("--rounds", type=int, default=3)
    ap.add_argument("--steps", type=int, default=20, help="back-to-back launches per variant per round")
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--sustained", type=float, default=0.0, metavar="SECONDS",
                    help="also run each variant alone for this long with amdsmi clock and power "
                         "sampling (rate, sclk, power, rate per GHz)")
    ap.add_argument("--json", default=None, help="also write the rows here")
    args = ap.parse_args()

    import torch

    if not torch.cuda.is_available():
        raise SystemExit("ablation.py needs the GPU")
    results = []
    for N in args.seqlens:
        flops, rows = measure_shape(args, N)
        print_table(args, N, rows)
        results.append({"seqlen": N, "flops": flops, "rows": rows})
    if args.json:
        with open(args.json, "w") as f:
            json.dump({"args": vars(args), "results": results}, f, indent=1)


if __name__ == "__main__":
    main()
