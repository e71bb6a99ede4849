"""HIP graph capture of fa2.kernel.attention.

The launch path allocates nothing itself (out, the log-sum-exp and the workspace of split-KV
and of the key-norm table come from torch's caching allocator, which serves graph capture from the graph's private pool) and
records no memset, so a caller can capture attention() in a torch.cuda.CUDAGraph and replay it,
as serving loops do. Each replay here runs on new inputs copied into the captured tensors, with
eager work and synchronisation between replays, and must equal an eager call bit for bit (same
kernels, same tiles, same order).
"""

import pytest
import torch

from attn_check import make_qkv

pytestmark = pytest.mark.gpu


def _attention():
    from fa2.kernel import attention
    return attention


@pytest.mark.parametrize("case", ["causal_gqa", "splitkv_lse", "key_norm_pass"])
def test_graph_replays_match_eager(case):
    attention = _attention()
    if case == "causal_gqa":
        shape, kw = (1, 8, 2, 700, 700, 128, torch.bfloat16), dict(causal=True)
    elif case == "key_norm_pass":
        # long enough for attention() to run the key-norm pass first (2^37 FLOP, 32772 FLOP
        # per byte of K): two kernels and a workspace per call
        from fa2 import _lib
        shape, kw = (1, 8, 2, 8192, 8192, 128, torch.bfloat16), dict(causal=True)
        assert _lib.workspace_bytes_for(1, 8, 2, 8192, 8192, 128, torch.bfloat16, True, 1) > 0
    else:
        shape, kw = (2, 8, 2, 4, 3000, 64, torch.float16), dict(causal=False, num_splits=4,
                                                                  return_lse=True)
    q, k, v = make_qkv(*shape)
    attention(q, k, v, **kw)                    # warm up (library load, allocator) outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            captured = attention(q, k, v, **kw)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    for seed in (1, 2, 3):
        nq, nk, nv = make_qkv(*shape, seed=seed)
        q.copy_(nq), k.copy_(nk), v.copy_(nv)
        graph.replay()
        torch.cuda.synchronize()
        want = attention(nq, nk, nv, **kw)      # eager work between replays
        torch.cuda.synchronize()
        if case == "splitkv_lse":
            assert torch.equal(captured[0], want[0]) and torch.equal(captured[1], want[1])
        else:
            assert torch.equal(captured, want)
