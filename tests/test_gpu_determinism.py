"""Run-to-run determinism of every shipped kernel instance that spills registers to scratch.

The compiler's resource report (fa2/kernel_resources.json, written by csrc/build.py) shows VGPR
spills to scratch in the head_dim-64 software-pipelined instances held to three waves per SIMD:
bf16 causal and full (2-3 VGPRs, 12-16 bytes per lane), their key-norm instances (4-5, 20-24
bytes), and the fp16 ones (2-5 VGPRs, with and without the key-norm table: the rounded P sum). Scratch loads and stores count in the
same vmcnt counter as the kernel's hand-placed LDS-DMA waits, so a wrong count would show up as a
read of K/V or of a spilled value before it landed: the output would then change from launch to
launch. Each case below runs a full-size grid (C4-sized for full attention, C2-sized for causal)
three times and requires the same bits every time, plus a finite output within the 2x-SDPA rule
of the fp32 oracle on a small shape of the same instance. The reference checks its own invariants
bitwise the same way (tests/test_correctness.py:155-168).
"""

import json
import math
import os

import pytest
import torch

from attn_check import check_against_oracle, make_qkv

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
RESOURCES = os.path.join(ROOT, "triton-fa2-forward_amd", "fa2", "kernel_resources.json")

# (name, dtype, causal, key-norm table, full-size shape B, H, N)
CASES = [
    ("bf16_d64_full", torch.bfloat16, False, False, (2, 16, 16384)),
    ("bf16_d64_causal", torch.bfloat16, True, False, (4, 16, 4096)),
    ("bf16_d64_full_keynorm", torch.bfloat16, False, True, (2, 16, 16384)),
    ("bf16_d64_causal_keynorm", torch.bfloat16, True, True, (4, 16, 4096)),
    ("fp16_d64_full", torch.float16, False, False, (2, 16, 16384)),
    ("fp16_d64_causal", torch.float16, True, False, (4, 16, 4096)),
    ("fp16_d64_full_keynorm", torch.float16, False, True, (2, 16, 16384)),
    ("fp16_d64_causal_keynorm", torch.float16, True, True, (4, 16, 4096)),
]


def _run(q, k, v, causal, table):
    """fa2_attn_fwd_ex at the default configuration; with `table`, a workspace with room for the
    key-norm table, which the library then always uses (the default tiles qualify)."""
    from fa2 import _lib
    from fa2.kernel import LOG2E

    B, H_q, N_q, D = q.shape
    H_kv, N_kv = k.shape[1], k.shape[2]
    out = torch.empty_like(q)
    ws = None
    if table:
        chunks = (N_kv + 63) // 64
        ws = torch.empty((B * H_kv * chunks * 4 + 255) // 256 * 256, dtype=torch.uint8,
                         device=q.device)
    _lib.attn_fwd_ex(q, k, v, out, causal, 1, 128, 0, LOG2E / math.sqrt(D), None, 1, ws,
                     torch.cuda.current_stream().cuda_stream)
    return out


def test_the_spilling_instances_are_the_ones_listed():
    """The cases cover every default-configuration instance that the resource report says spills
    VGPRs (4 waves, 64-key tiles; variant 0 or 4)."""
    if not os.path.exists(RESOURCES):
        pytest.skip("kernel_resources.json not built")
    kernels = json.load(open(RESOURCES))["kernels"].values()
    spilling = {(k["dtype"], k["head_dim"], k["causal"], k["variant"]) for k in kernels
                if k["waves"] == 4 and k["block_n"] == 64 and k.get("vgpr_spills", 0) > 0}
    covered = {("bf16" if dt == torch.bfloat16 else "fp16", 64, causal, 4 if table else 0)
               for _, dt, causal, table, _ in CASES}
    assert spilling <= covered, spilling - covered


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_spilling_instance_is_deterministic_at_full_size(case):
    name, dt, causal, table, (B, H, N) = case
    print(f"determinism: {name} B={B} H={H} N={N} D=64", flush=True)
    q, k, v = make_qkv(B, H, H, N, N, 64, dt, seed=21)
    if dt == torch.float16:
        q, k, v = (t * 0.5 for t in (q, k, v))   # C4's half-scale inputs
    first = _run(q, k, v, causal, table)
    torch.cuda.synchronize()
    assert torch.isfinite(first).all()
    for _ in range(2):
        again = _run(q, k, v, causal, table)
        torch.cuda.synchronize()
        assert torch.equal(again, first)
    # the same instance meets the oracle on a small shape
    qs, ks, vs = make_qkv(2, 4, 4, 333, 333, 64, dt, seed=22)
    check_against_oracle(qs, ks, vs, causal, precision=torch.float32,
                         ours=_run(qs, ks, vs, causal, table))
