"""fa2_attn_fwd_noalloc, the entry point that allocates nothing (no counterpart in the reference):
through the C ABI, its output must equal fa2_attn_fwd_ex's bit for bit when fa2_attn_fwd_ex gets
a workspace of fa2_workspace_bytes_for(...) bytes. The checks use two calls in a row on the
library's shared scratch, the second with a smaller input, so the first call's leftovers in the
scratch must not reach the second's result. The cases cover split-KV partials (with the
log-sum-exp), the key-norm table (on causal grids that also deal their last programs at run time
from the library's static ticket words, which allocate nothing either), a launch that needs
no scratch, and calls recorded under HIP graph capture (the callers the entry point is for) and
replayed on new inputs.
"""

import math

import pytest
import torch

from attn_check import check_against_oracle, make_qkv

pytestmark = pytest.mark.gpu


def _scale(D):
    from fa2.kernel import LOG2E
    return LOG2E / math.sqrt(D)


def _run_ex(q, k, v, causal, num_splits, want_lse):
    """fa2_attn_fwd_ex with a torch-allocated workspace of fa2_workspace_bytes_for bytes."""
    from fa2 import _lib

    B, H_q, N_q, D = q.shape
    H_kv, N_kv = k.shape[1], k.shape[2]
    out = torch.empty_like(q)
    lse = torch.empty(B, H_q, N_q, dtype=torch.float32, device=q.device) if want_lse else None
    nbytes = _lib.workspace_bytes_for(B, H_q, H_kv, N_q, N_kv, D, q.dtype, causal, num_splits)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=q.device) if nbytes else None
    _lib.attn_fwd_ex(q, k, v, out, causal, 1, 128, 0, _scale(D), lse, num_splits, ws,
                     torch.cuda.current_stream().cuda_stream)
    return out, lse, nbytes


def _run_noalloc(q, k, v, causal, num_splits, want_lse):
    from fa2 import _lib

    B, H_q, N_q, D = q.shape
    out = torch.empty_like(q)
    lse = torch.empty(B, H_q, N_q, dtype=torch.float32, device=q.device) if want_lse else None
    _lib.attn_fwd_noalloc(q, k, v, out, causal, 1, 128, 0, _scale(D), lse, num_splits,
                          torch.cuda.current_stream().cuda_stream)
    return out, lse


def _check_pair(cases):
    """Run the no-allocation entry point on every case in order (one shared scratch), then
    compare each result with fa2_attn_fwd_ex's."""
    results = []
    for (qkv, causal, splits, want_lse) in cases:
        q, k, v = qkv
        print(f"noalloc: B={q.shape[0]} Hq={q.shape[1]} Hkv={k.shape[1]} Nq={q.shape[2]} "
              f"Nkv={k.shape[2]} D={q.shape[3]} {q.dtype} causal={causal} splits={splits}",
              flush=True)
        results.append(_run_noalloc(q, k, v, causal, splits, want_lse))
        torch.cuda.synchronize()
    for (qkv, causal, splits, want_lse), (out, lse) in zip(cases, results):
        q, k, v = qkv
        ref_out, ref_lse, nbytes = _run_ex(q, k, v, causal, splits, want_lse)
        torch.cuda.synchronize()
        assert nbytes > 0 or splits == 1
        assert torch.equal(out, ref_out)
        if want_lse:
            assert torch.equal(lse, ref_lse)
    return results


def test_noalloc_split_kv_equals_workspace_launch():
    """Split-KV partials in the scratch: 16 MiB of them for the few-queries shape (B 16,
    H 32/8, N_q 32, N_kv 4096, 2 splits), then a smaller ragged launch (3 splits, head_dim 64)."""
    big = make_qkv(16, 32, 8, 32, 4096, 128, torch.float16)
    small = make_qkv(2, 8, 2, 7, 777, 64, torch.bfloat16)
    (out_small, lse_small) = _check_pair([(big, False, 2, True), (small, False, 3, True)])[1]
    check_against_oracle(*small, False, ours=out_small)


def test_noalloc_key_table_equals_workspace_launch():
    """The key-norm table in the scratch (bf16, head_dim 128, causal, long enough that it pays):
    C3's shape, then N 4096, which still qualifies; both equal attention()'s output."""
    from fa2 import _lib
    from fa2.kernel import attention

    c3 = make_qkv(1, 32, 8, 8192, 8192, 128, torch.bfloat16)
    smaller = make_qkv(1, 32, 8, 4096, 4096, 128, torch.bfloat16)
    for q, k, v in (c3, smaller):   # the table is in use on both
        assert (_lib.workspace_bytes_for(1, 32, 8, q.shape[2], q.shape[2], 128, q.dtype, True, 1)
                > 0)
    results = _check_pair([(c3, True, 1, False), (smaller, True, 1, False)])
    for (q, k, v), (out, _) in zip((c3, smaller), results):
        assert torch.equal(out, attention(q, k, v, causal=True))


def test_noalloc_without_scratch_needs():
    """A launch that needs no workspace (fp16, short, single pass) never touches the scratch and
    equals fa2_attn_fwd's output; then a split launch on the same scratch."""
    from fa2.kernel import attention

    q, k, v = make_qkv(2, 4, 2, 100, 100, 64, torch.float16)
    out, _ = _run_noalloc(q, k, v, True, 1, False)
    torch.cuda.synchronize()
    assert torch.equal(out, attention(q, k, v, causal=True))
    _check_pair([(make_qkv(1, 8, 8, 1, 1024, 128, torch.bfloat16), False, 4, True)])


@pytest.mark.parametrize("case", ["split_kv", "key_table"])
def test_noalloc_under_graph_capture_replays_exactly(case):
    """fa2_attn_fwd_noalloc recorded in a HIP graph (its device checks and the scratch lookup run
    on the capturing stream; the graph keeps the scratch's address): every replay, on new inputs
    copied into the captured tensors and with eager work and synchronisation in between, equals
    fa2_attn_fwd_ex with a workspace, bit for bit. Split-KV (partials in the scratch, with the
    log-sum-exp) and the key-norm table (C3's shape)."""
    from fa2 import _lib

    if case == "split_kv":
        shape, causal, splits, want_lse = (8, 32, 8, 16, 4096, 128, torch.float16), False, 4, True
    else:
        shape, causal, splits, want_lse = (1, 32, 8, 8192, 8192, 128, torch.bfloat16), True, 1, False
        assert _lib.workspace_bytes_for(1, 32, 8, 8192, 8192, 128, torch.bfloat16, True, 1) > 0
    print(f"noalloc capture: {case} {shape}", flush=True)
    q, k, v = make_qkv(*shape)
    B, H_q, N_q, D = q.shape
    out = torch.empty_like(q)
    lse = torch.empty(B, H_q, N_q, dtype=torch.float32, device=q.device) if want_lse else None
    _run_noalloc(q, k, v, causal, splits, want_lse)   # warm up: library load, scratch lookup
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            _lib.attn_fwd_noalloc(q, k, v, out, causal, 1, 128, 0, _scale(D), lse, splits,
                                  stream.cuda_stream)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    for seed in (1, 2, 3):
        nq, nk, nv = make_qkv(*shape, seed=seed)
        q.copy_(nq), k.copy_(nk), v.copy_(nv)
        graph.replay()
        torch.cuda.synchronize()
        ref_out, ref_lse, _ = _run_ex(nq, nk, nv, causal, splits, want_lse)   # eager, between
        torch.cuda.synchronize()
        assert torch.equal(out, ref_out), seed
        if want_lse:
            assert torch.equal(lse, ref_lse), seed


def test_noalloc_on_new_and_known_streams_equals_workspace_launch():
    """A causal grid with a dynamic tail through fa2_attn_fwd_noalloc on a stream the library has
    not seen (no ticket set: the no-allocation entry point makes none, since a set's event is a
    runtime object, and runs the static order) and on the same stream after a fa2_attn_fwd_ex call
    there gave it a set (the tail): both equal fa2_attn_fwd_ex's output bit for bit. The stream
    is made through the HIP runtime directly (torch pools its own)."""
    import ctypes

    from fa2 import _lib

    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hip.hipStreamDestroy.argtypes = [ctypes.c_void_p]
    hip.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
    q, k, v = make_qkv(1, 32, 8, 4096, 4096, 128, torch.bfloat16, seed=21)
    print("noalloc on a new stream: B=1 Hq=32 Hkv=8 N=4096 D=128 bf16 causal", flush=True)
    want, _, _ = _run_ex(q, k, v, True, 1, False)
    torch.cuda.synchronize()
    h = ctypes.c_void_p()
    assert hip.hipStreamCreate(ctypes.byref(h)) == 0
    try:
        outs = []
        for step in ("new", "ex", "known"):
            out = torch.empty_like(q)
            if step == "ex":
                nbytes = _lib.workspace_bytes_for(1, 32, 8, 4096, 4096, 128, q.dtype, True, 1)
                ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
                _lib.attn_fwd_ex(q, k, v, out, True, 1, 128, 0, _scale(128), None, 1,
                                 ws if nbytes else None, h.value)
            else:
                _lib.attn_fwd_noalloc(q, k, v, out, True, 1, 128, 0, _scale(128), None, 1, h.value)
            assert hip.hipStreamSynchronize(h) == 0
            outs.append((step, out))
        for step, out in outs:
            assert torch.equal(out, want), step
    finally:
        hip.hipStreamSynchronize(h)
        hip.hipStreamDestroy(h)
