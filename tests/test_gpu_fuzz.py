"""Seeded random shapes through fa2.kernel.attention, against the oracle.

The parity suite follows the reference's grid (tests/test_correctness.py:106-218) and adds
chosen edge cases; this file covers the combinations between them: batch, GQA ratio, lengths
(N_q != N_kv when not causal), head_dim, dtype, packing, tile overrides, split-KV and the
log-sum-exp, and strided inputs. The case list is fixed by a seed, printed per case, and each
case is checked with the reference's rule (max-abs <= 2x SDPA's + 1e-4 against naive_attention
in fp32) and, when requested, the log-sum-exp against naive_lse.
"""

import random

import pytest
import torch

from attn_check import check_against_oracle, make_qkv
from oracle import reference as ref

pytestmark = pytest.mark.gpu

LSE_ATOL = 1e-4


def _cases(n=64, seed=20261201, first=0):
    rnd = random.Random(seed)
    cases = []
    for i in range(first, first + n):
        h_kv = rnd.choice([1, 2, 3, 4, 8])
        group = rnd.choice([1, 2, 3, 4, 7, 8])
        causal = rnd.random() < 0.5
        n_q = rnd.choice([1, 5, 17, 64, 100, 128, 255, 333, 600])
        n_kv = n_q if causal else rnd.choice([1, 9, 64, 200, 513, 1024, 1500])
        d = rnd.choice([16, 32, 64, 128])
        dtype = rnd.choice(["fp16", "bf16"])
        block_m = rnd.choice([None, 16, 32, 64, 96, 112, 128, 256])
        block_n = rnd.choice([None, 16, 32, 64, 128])
        pack = rnd.choice([None, False, True])
        if pack and (block_m or 128) % group:
            pack = False
        splits = None if causal else rnd.choice([None, 1, 2, 3, 8])
        lse = rnd.random() < 0.3
        strided = rnd.random() < 0.2
        cases.append((i, rnd.choice([1, 2, 3]), h_kv * group, h_kv, n_q, n_kv, d, dtype, causal,
                      block_m, block_n, pack, splits, lse, strided))
    return cases


@pytest.mark.parametrize("case", _cases() + _cases(seed=20261211, first=1000),
                         ids=lambda c: f"case{c[0]}")
def test_fuzz_against_oracle(case):
    from fa2.kernel import attention

    (i, B, h_q, h_kv, n_q, n_kv, d, dtype, causal, block_m, block_n, pack, splits, lse,
     strided) = case
    print(f"\ncase {case}", flush=True)
    dt = torch.float16 if dtype == "fp16" else torch.bfloat16
    q, k, v = make_qkv(B, h_q, h_kv, n_q, n_kv, d, dt, seed=i)
    if strided:  # [B, N, H, D] storage viewed as [B, H, N, D]
        q, k, v = (t.transpose(1, 2).contiguous().transpose(1, 2) for t in (q, k, v))
    kw = dict(causal=causal, block_m=block_m, block_n=block_n, pack_gqa=pack)
    if splits is not None:
        kw["num_splits"] = splits
    if lse:
        out, got = attention(q, k, v, return_lse=True, **kw)
        want = ref.naive_lse(q.float(), k.float(), None, causal=causal)
        err = (got - want).abs().max().item()
        assert err <= LSE_ATOL, f"log-sum-exp max-abs error {err:.3e}"
    else:
        out = attention(q, k, v, **kw)
    assert out.shape == q.shape and out.stride() == q.stride()
    check_against_oracle(q, k, v, causal, precision=torch.float32, ours=out)
