"""Kernel variants for attributing the kernel's time (counterpart of the reference's
bench/ablation.py). GPU only.

    python triton-fa2-forward_amd/ablation.py                       # N 4096 and 16384, fp16, causal
    python triton-fa2-forward_amd/ablation.py --seqlens 8192 --dtype bf16 --rounds 5

The reference keeps a copy of its kernel with five switches (bench/ablation.py:1-20). Two of them
undo the kernel's two instruction-count choices and still compute attention; here they are
compile-time flags of the one kernel template (attn_fwd_kernel's VARIANT), reached through
fa2_attn_fwd_variant:

  scale_first      multiply every score by the scale, then subtract the row max (two VALU
                   instructions per score) instead of one FMA, s * scale - m
  mask_every_tile  apply the causal / end-of-sequence mask on every K/V tile, not only on the
                   tiles that need it

before_fixes turns both on; copy turns neither on and is the production kernel (bit for bit, as
tests/test_gpu_ablation.py checks); pack forces GQA head packing. The reference's other three
switches (no_exp, no_softmax, kv_l2) skip work and produce wrong outputs by design. They are not
part of this library: their numbers come from a separate, unshipped copy of the kernel.

Timing follows the reference (HIP events around every launch, median and IQR) after bench.py's
1 s clock settle, interleaved over rounds so that clock drift hits every variant alike
(bench/ablation.py:252-255).
"""

import argparse
import json
import math
import os
import statistics
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.dirname(HERE))

KNOBS = ("scale_first", "mask_every_tile")
SKIPPING = ("no_exp", "no_softmax", "kv_l2")     # the reference's, not built here
VARIANTS = {                                       # name -> switches on
    "copy": (),
    "scale_first": ("scale_first",),
    "mask_every_tile": ("mask_every_tile",),
    "before_fixes": ("scale_first", "mask_every_tile"),
    "pack": ("pack",),                             # the copy with GQA head packing forced on
}
VARIANT_BITS = {"scale_first": 1, "mask_every_tile": 2}   # FA2_VARIANT_* in include/fa2_fwd.h


def attention_ablate(q, k, v, causal=True, pack_gqa=False, **knobs):
    """fa2.kernel.attention at the default configuration with the switches in KNOBS
    (bench/ablation.py:182-200). Same argument rules as attention()."""
    import torch

    from fa2 import _lib
    from fa2.kernel import LOG2E, _default_config, _loadable

    skipping = sorted(set(knobs) & set(SKIPPING))
    if skipping:
        raise ValueError(f"switches {skipping} skip work and are not built into this library "
                         "(their timings come from an unshipped copy of the kernel)")
    unknown = set(knobs) - set(KNOBS)
    assert not unknown, f"unknown switches {sorted(unknown)}"
    assert q.dim() == k.dim() == v.dim() == 4
    B, H_q, N_q, D = q.shape
    H_kv, N_kv = k.shape[1], k.shape[2]
    assert v.shape == k.shape and k.shape[0] == B and k.shape[3] == D
    assert q.dtype == k.dtype == v.dtype and q.dtype in (torch.float16, torch.bfloat16)
    assert H_q % H_kv == 0, "GQA needs H_q divisible by H_kv"
    assert D in (16, 32, 64, 128), "head_dim must be a power of two in [16, 128]"
    if causal:
        assert N_q == N_kv, "causal attention here assumes N_q == N_kv"
    bm = _default_config(D, True)[0]
    group = H_q // H_kv
    if pack_gqa and bm % group:
        raise ValueError(f"pack_gqa needs BLOCK_M ({bm}) to be a multiple of the GQA group ({group})")
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise RuntimeError("attention_ablate runs on the GPU; got CPU tensors")
    variant = sum(VARIANT_BITS[kn] for kn, on in knobs.items() if on)
    out = torch.empty_like(q)
    if out.numel() == 0:
        return out
    q_, k_, v_, o_ = _loadable(q), _loadable(k), _loadable(v), _loadable(out)
    with torch.cuda.device(q.device):
        stream = torch.cuda.current_stream(q.device).cuda_stream
        _lib.attn_fwd_variant(q_, k_, v_, o_, causal, group if pack_gqa else 1,
                              1.0 / math.sqrt(D) * LOG2E, variant, stream)
    if o_ is not out:
        out.copy_(o_)
    return out


def _summarize(ms):
    q1, med, q3 = statistics.quantiles(ms, n=4, method="inclusive")
    return {"median_ms": med, "iqr_ms": q3 - q1}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--seqlens", type=int, nargs="+", default=[4096, 16384])
    ap.add_argument("--hq", type=int, default=32)
    ap.add_argument("--hkv", type=int, default=8)
    ap.add_argument("--head-dim", type=int, default=128)
    ap.add_argument("--dtype", choices=["fp16", "bf16"], default="fp16")
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--variants", nargs="+", default=list(VARIANTS), choices=list(VARIANTS))
    ap.add_argument("--rounds", type=int, default=3, help="interleaved rounds; samples are pooled")
    ap.add_argument("--json", default=None)
    args = ap.parse_args()

    import torch

    import bench
    from fa2.kernel import attention

    dtype = {"fp16": torch.float16, "bf16": torch.bfloat16}[args.dtype]
    rows = []
    for N in args.seqlens:
        g = torch.Generator(device="cpu").manual_seed(0)
        q = torch.randn(1, args.hq, N, args.head_dim, generator=g).to("cuda", dtype)
        k = torch.randn(1, args.hkv, N, args.head_dim, generator=g).to("cuda", dtype)
        v = torch.randn(1, args.hkv, N, args.head_dim, generator=g).to("cuda", dtype)
        flops = bench.attn_flops(1, args.hq, N, N, args.head_dim, True)
        ref = attention(q, k, v, causal=True)
        fns = {"production": lambda: attention(q, k, v, causal=True)}
        info = {}
        for name in args.variants:
            knobs = {kn: True for kn in VARIANTS[name] if kn != "pack"}
            fn = (lambda knobs=knobs, pack="pack" in VARIANTS[name]:
                  attention_ablate(q, k, v, causal=True, pack_gqa=pack, **knobs))
            out = fn()
            info[name] = dict(bit_exact=torch.equal(out, ref),
                              max_abs_diff=(out.float() - ref.float()).abs().max().item())
            fns[name] = fn
        bench.settle_clocks(fns["production"])
        samples = {name: [] for name in fns}
        for _ in range(args.rounds):
            for name, fn in fns.items():
                for _ in range(args.warmup):
                    fn()
                samples[name] += bench.time_each(fn, args.iters)
        base = _summarize(samples["production"])
        print(f"\nN={N} {args.dtype} H {args.hq}/{args.hkv} D {args.head_dim} causal  "
              f"(production {base['median_ms']:.3f} ms, {flops / base['median_ms'] / 1e9:.1f} TFLOP/s)")
        print("| variant | ms (IQR) | vs production | TFLOP/s | output |")
        print("|---|---|---|---|---|")
        for name in fns:
            s = _summarize(samples[name])
            delta = s["median_ms"] - base["median_ms"]
            out = ("" if name == "production" else "bit-exact" if info[name]["bit_exact"]
                   else f"max diff {info[name]['max_abs_diff']:.2e}")
            print(f"| {name} | {s['median_ms']:.3f} ({s['iqr_ms']:.3f}) | {delta:+.3f} "
                  f"({delta / base['median_ms']:+.1%}) | {flops / s['median_ms'] / 1e9:.1f} | {out} |",
                  flush=True)
            rows.append(dict(seqlen=N, variant=name, rounds=args.rounds, **s,
                             **info.get(name, {})))
        del q, k, v, ref
        torch.cuda.empty_cache()
    if args.json:
        with open(args.json, "w") as f:
            json.dump({"config": vars(args), "results": rows}, f, indent=1)


if __name__ == "__main__":
    main()
