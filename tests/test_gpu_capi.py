"""The C ABI from a plain C host: tests/capi/fa2_capi_check.c calls fa2_attn_fwd /
fa2_attn_fwd_ex with hipMalloc'd buffers in a process that has no Python or torch (the binding
a non-Python caller of the replaced Triton launch, fa2/kernel.py:247-259, would write).

Each case runs the host as a child process, reads back its seeded inputs and outputs, and checks
them against the oracle with the reference's rule (max-abs <= 2x SDPA's + 1e-4 against
naive_attention in fp64), the log-sum-exp against naive_lse, and the C host's output against
the Python front end's on the same inputs, bit for bit: the two bindings launch the same kernel.
"""

import os
import subprocess

import numpy as np
import pytest
import torch

from attn_check import check_against_oracle
from oracle import reference as ref

pytestmark = pytest.mark.gpu

EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "capi", "fa2_capi_check")
DTYPES = {0: torch.float16, 1: torch.bfloat16}

# (B, H_q, H_kv, N_q, N_kv, D, dtype, causal, pack, block_m, block_n, splits (0 = library's
# pick), lse)
CASES = [
    (2, 8, 2, 300, 300, 128, 1, True, 1, 128, 0, 1, False),      # C3's kind, small
    (2, 8, 2, 77, 1000, 64, 0, False, 4, 128, 0, 0, True),       # packed, split-KV, log-sum-exp
    (1, 4, 4, 129, 129, 32, 0, True, 1, 64, 32, 1, True),        # non-default tiles
    (3, 28, 4, 1000, 1000, 128, 1, True, 7, 112, 0, 1, False),   # C5's shape, packed
    (1, 32, 8, 4096, 4096, 128, 0, True, 1, 128, 0, 1, False),   # a dynamic tail (1024 programs)
]


def _load(path):
    raw = path.read_bytes()
    h = np.frombuffer(raw[:64], dtype=np.int32)
    B, hq, hkv, nq, nkv, d, dtype, causal, pack, bm, bn, splits, has_lse, rc = (int(x) for x in h[:14])
    assert rc == 0
    dt = DTYPES[dtype]
    off = 64

    def take(n, shape):
        nonlocal off
        a = np.frombuffer(raw[off:off + 2 * n], dtype=np.int16).copy()
        off += 2 * n
        return torch.from_numpy(a).view(dt).reshape(shape)

    q = take(B * hq * nq * d, (B, hq, nq, d))
    k = take(B * hkv * nkv * d, (B, hkv, nkv, d))
    v = take(B * hkv * nkv * d, (B, hkv, nkv, d))
    out = take(B * hq * nq * d, (B, hq, nq, d))
    lse = None
    if has_lse:
        lse = torch.from_numpy(np.frombuffer(raw[off:off + 4 * B * hq * nq], dtype=np.float32).copy())
        lse = lse.reshape(B, hq, nq)
    return q, k, v, out, lse, splits


@pytest.mark.skipif(not os.path.exists(EXE), reason="tests/capi/fa2_capi_check is built by csrc/build.py")
@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}_H{}-{}_N{}-{}_D{}_dt{}_c{}_p{}_bm{}_bn{}_s{}_lse{}".format(*c))
def test_c_host_matches_oracle_and_python(case, tmp_path):
    from fa2.kernel import attention

    B, hq, hkv, nq, nkv, d, dtype, causal, pack, bm, bn, splits, lse = case
    path = tmp_path / "case.bin"
    args = [EXE, "run", *(str(int(x)) for x in (B, hq, hkv, nq, nkv, d, dtype, causal, pack, bm, bn,
                                                splits, lse, 7)), str(path)]
    print("\nC host:", " ".join(args[1:-1]), flush=True)
    res = subprocess.run(args, capture_output=True, text=True, timeout=120)
    print(res.stdout.strip(), res.stderr.strip(), flush=True)
    assert res.returncode == 0, res.stderr
    q, k, v, out, lse_c, used_splits = _load(path)
    q, k, v, out = (t.cuda() for t in (q, k, v, out))

    check_against_oracle(q, k, v, causal, ours=out)
    if lse:
        want = ref.naive_lse(q.double(), k.double(), None, causal=causal)
        assert (lse_c.cuda().double() - want).abs().max().item() <= 1e-4

    py = attention(q, k, v, causal=causal, block_m=bm, block_n=bn or None, pack_gqa=pack > 1,
                   num_splits=used_splits, return_lse=bool(lse))
    py_out = py[0] if lse else py
    assert torch.equal(py_out, out)
    if lse:
        assert torch.equal(py[1].cpu(), lse_c)
