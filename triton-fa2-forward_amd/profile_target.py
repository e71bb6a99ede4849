"""One workload, a few launches: the process rocprofv3 profiles (counterpart of the reference's
bench/profile_target.py).

    python triton-fa2-forward_amd/profile_target.py --config C3 --launches 3
    python triton-fa2-forward_amd/profile_target.py --config C3 --launches 3 --copy-mib 1024
    python triton-fa2-forward_amd/profile_target.py --pack-short 1 --launches 20

--pack-short N_Q runs the reference's few-queries shape instead (bench.py --pack-short: fp16,
B 16, H 32/8, N_kv 4096, D 128, non-causal, default path: packed, automatic split-KV).

--lib PATH runs another build of the product library (csrc/build.py --variant) through the same
call attention() makes (ab.py's), for the counters of an A/B.

--copy-mib adds one plain device-to-device copy of that many MiB after the attention launches.
Its FETCH_SIZE / WRITE_SIZE reading, against the bytes it is known to move, is the scale factor
that turns the counters' KiB into bytes for the attention kernel.
"""

import argparse
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.dirname(HERE))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="C3")
    ap.add_argument("--launches", type=int, default=3)
    ap.add_argument("--copy-mib", type=int, default=0)
    ap.add_argument("--block-m", type=int, default=None)
    ap.add_argument("--block-n", type=int, default=None)
    ap.add_argument("--pack-short", type=int, default=None, metavar="N_Q")
    ap.add_argument("--lib", default=None, help="another build of libfa2_fwd.so (ab.py's call)")
    args = ap.parse_args()

    import torch

    import bench
    from fa2.kernel import attention

    if args.pack_short is not None:
        c = bench.PACK_SHORT
        g = torch.Generator(device="cpu").manual_seed(0)
        q = torch.randn(c["B"], c["H_q"], args.pack_short, c["D"], generator=g).half().cuda()
        k = torch.randn(c["B"], c["H_kv"], c["N_kv"], c["D"], generator=g).half().cuda()
        v = torch.randn(c["B"], c["H_kv"], c["N_kv"], c["D"], generator=g).half().cuda()
        causal = False
        print(f"profile_target: pack-short N_q={args.pack_short}, {args.launches} launches", flush=True)
    else:
        q, k, v, causal = bench.make_inputs(args.config, "cuda")
        print(f"profile_target: {bench.describe(args.config)}, {args.launches} launches", flush=True)
    if args.lib:
        import ab

        out = torch.empty_like(q)
        call = ab.make_call(ab.load(args.lib), q, k, v, out, causal, True)
        print(f"profile_target: library {args.lib}", flush=True)
    else:
        call = lambda: attention(q, k, v, causal=causal, block_m=args.block_m,  # noqa: E731
                                 block_n=args.block_n)
    for _ in range(args.launches):
        call()
    torch.cuda.synchronize()
    if args.copy_mib:
        n = args.copy_mib << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        print(f"profile_target: copied {args.copy_mib} MiB ({n} bytes read, {n} written)", flush=True)
    print("profile_target: done", flush=True)


if __name__ == "__main__":
    main()
