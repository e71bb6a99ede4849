"""The dynamic tail of causal grids (attn_fwd_host.hpp: tail_schedule, acquire_tickets;
attn_fwd_schedule.hpp: tail_pick).

Where a causal grid has at least two rounds of programs per XCD, the last programs of every XCD's
static order (program_of's XCD order, or its fallback order where the (batch, kv head) units do
not split evenly over the 8 XCDs) are dealt at run time: each workgroup past the static part
takes a ticket from the launch's shared word, which deals the tail programs to whichever XCD
asks (a build with FA2_TAIL_PRIVATE_PCT > 0 first gives each XCD a queue word of its own for its
heavier tail programs; tests/test_schedule.py checks those rules on the CPU). Every word is
incremented a fixed number of times per launch and wraps, so it is zero again after every launch,
and a few spare workgroups find no program and exit. Which workgroup runs a program changes from
launch to launch; what the program computes does not. So:

* the output equals the static order's (the measurement library's FA2_ABLATE_STATIC_ORDER) bit
  for bit, on shapes with and without GQA packing, ragged, at head_dim 64 and 128;
* calls back to back, with tails of different sizes on one stream, keep that (every launch
  leaves its words at zero for the next);
* two streams running tails at the same time keep it (each stream has its own ticket set);
* a launch recorded under stream capture keeps the static order (one graph can be instantiated
  twice and run twice at once, which would share a set): the measurement library's count of tail
  launches does not move while it is recorded, and its replays equal the eager calls, which use
  the tail, bit for bit;
* a stream destroyed with launches still queued and a new stream created at once (the handle can
  come back while the old launches run): every ticket set's launch waits for the event its previous
  launch signalled when it ended, so the old and new launches never share the words at once;
* streams past the 256 ticket sets a device has run the static order, with the same bits.

The CPU tier (tests/test_schedule.py) checks the same ticket rules over thousands of shapes.
"""

import pytest
import torch

from attn_check import make_qkv

pytestmark = pytest.mark.gpu

# (B, H_q, H_kv, N, D, dtype, pack): all causal, all with a tail at the default 128-row tiles
TAIL_SHAPES = {
    "gqa_d128": (1, 32, 8, 4096, 128, torch.bfloat16, False),   # C3's heads, 1024 programs
    "mha_ragged": (8, 16, 16, 2000, 128, torch.bfloat16, False),  # 128 units, 16 q tiles
    "fp16_d64": (4, 16, 16, 4096, 64, torch.float16, False),     # three workgroups per CU
    "packed": (2, 32, 8, 2048, 128, torch.bfloat16, True),       # GQA head packing
    "fallback": (3, 28, 4, 4096, 128, torch.bfloat16, False),    # 12 units: the fallback order
}


def _static(q, k, v, pack):
    from ablation import attention_ablate
    return attention_ablate(q, k, v, causal=True, pack_gqa=pack, static_order=True)


def _dynamic(q, k, v, pack, stream=None):
    """fa2_attn_fwd at the default configuration (no key-norm table, like the variants)."""
    import math

    from fa2 import _lib
    from fa2.kernel import LOG2E

    out = torch.empty_like(q)
    s = stream if stream is not None else torch.cuda.current_stream()
    _lib.attn_fwd(q, k, v, out, True, q.shape[1] // k.shape[1] if pack else 1, 128, 0,
                  LOG2E / math.sqrt(q.shape[3]), s.cuda_stream)
    return out


def _inputs(name, seed=0):
    B, hq, hkv, n, d, dt, pack = TAIL_SHAPES[name]
    return (*make_qkv(B, hq, hkv, n, n, d, dt, seed=seed), pack)


@pytest.mark.parametrize("name", list(TAIL_SHAPES))
def test_dynamic_tail_is_the_static_order_bit_for_bit(name):
    q, k, v, pack = _inputs(name)
    want = _static(q, k, v, pack)
    for _ in range(3):
        assert torch.equal(_dynamic(q, k, v, pack), want)


def test_tails_of_different_sizes_back_to_back_on_one_stream():
    """Each launch's increments bring the stream's word back to zero; a word left elsewhere would
    shift the next launch's tickets, so that some programs ran twice and others never."""
    cases = {name: _inputs(name, seed=3) for name in ("gqa_d128", "fp16_d64", "mha_ragged")}
    want = {name: _static(*c) for name, c in cases.items()}
    outs = []
    for _ in range(2):
        for name, c in cases.items():
            outs.append((name, _dynamic(*c)))
    torch.cuda.synchronize()
    for name, out in outs:
        assert torch.equal(out, want[name]), name


def test_tails_on_two_streams_at_once():
    a, b = _inputs("gqa_d128", seed=5), _inputs("mha_ragged", seed=6)
    want_a, want_b = _static(*a), _static(*b)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    s1.wait_stream(torch.cuda.current_stream())
    s2.wait_stream(torch.cuda.current_stream())
    outs = []
    for _ in range(3):
        with torch.cuda.stream(s1):
            outs.append(("a", _dynamic(*a, stream=s1)))
        with torch.cuda.stream(s2):
            outs.append(("b", _dynamic(*b, stream=s2)))
    torch.cuda.current_stream().wait_stream(s1)
    torch.cuda.current_stream().wait_stream(s2)
    torch.cuda.synchronize()
    for which, out in outs:
        assert torch.equal(out, want_a if which == "a" else want_b), which


def test_captured_launch_keeps_the_static_order_and_replays_exactly():
    from fa2.kernel import attention

    q, k, v, _ = _inputs("gqa_d128")
    attention(q, k, v, causal=True)             # warm up outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            captured = attention(q, k, v, causal=True)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    for seed in (1, 2, 3):
        nq, nk, nv, _ = _inputs("gqa_d128", seed=seed)
        q.copy_(nq), k.copy_(nk), v.copy_(nv)
        graph.replay()
        torch.cuda.synchronize()
        want = attention(nq, nk, nv, causal=True)   # eager: the tail, on the stream's words
        torch.cuda.synchronize()
        assert torch.equal(captured, want)


def test_capture_records_the_static_order():
    """The launch path's capture check, seen directly: the measurement library (the same host
    code, compiled into it) counts the launches that took a ticket set. An eager launch counts;
    one recorded under capture does not, and its replays equal the static order bit for bit."""
    import ctypes

    from ablation import ablate_lib, attention_ablate

    lib = ablate_lib()
    lib.fa2_ablate_tail_launches.restype = ctypes.c_longlong
    lib.fa2_ablate_tail_launches.argtypes = []
    q, k, v, _ = _inputs("gqa_d128", seed=4)
    want = _static(q, k, v, False)
    before = lib.fa2_ablate_tail_launches()
    eager = attention_ablate(q, k, v, causal=True)
    torch.cuda.synchronize()
    assert lib.fa2_ablate_tail_launches() == before + 1
    assert torch.equal(eager, want)
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            captured = attention_ablate(q, k, v, causal=True)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    assert lib.fa2_ablate_tail_launches() == before + 1   # recorded without a ticket set
    for _ in range(2):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, want)


def test_a_new_stream_on_a_reused_handle_keeps_the_tail_exact():
    """A stream is destroyed with tail launches still queued on it (hipStreamDestroy need not
    wait for them) and a new stream is created at once, which can get the same handle and so the
    same ticket set; its launches wait for the event the old stream's last launch signalled, so
    the two never use the set's words at once. Streams created and destroyed through the HIP
    runtime directly (torch pools its own)."""
    import ctypes
    import math

    from fa2 import _lib
    from fa2.kernel import LOG2E

    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hip.hipStreamDestroy.argtypes = [ctypes.c_void_p]
    hip.hipDeviceSynchronize.argtypes = []
    q, k, v, _ = _inputs("mha_ragged", seed=8)
    want = _static(q, k, v, False)
    torch.cuda.synchronize()
    outs, handles = [], []
    for _ in range(4):
        h = ctypes.c_void_p()
        assert hip.hipStreamCreate(ctypes.byref(h)) == 0
        handles.append(h.value)
        for _ in range(3):   # queued, not waited for, before the destroy
            out = torch.empty_like(q)
            _lib.attn_fwd(q, k, v, out, True, 1, 128, 0, LOG2E / math.sqrt(q.shape[3]), h.value)
            outs.append(out)
        assert hip.hipStreamDestroy(h) == 0
    assert hip.hipDeviceSynchronize() == 0
    print(f"stream handles: {len(set(handles))} distinct of {len(handles)}", flush=True)
    for out in outs:
        assert torch.equal(out, want)


def test_streams_past_the_ticket_sets_run_the_static_order():
    """300 streams that stay alive, one launch of the measurement library on each: the library's
    count of tail launches grows by one for each new stream until its 256 ticket sets are handed
    out (some may have gone to streams of earlier tests in this process) and then stays put; every
    launch, with a tail or without, gives the static order's bits."""
    import ctypes
    import math

    from ablation import ablate_lib
    from fa2 import _lib
    from fa2.kernel import LOG2E

    lib = ablate_lib()
    lib.fa2_ablate_tail_launches.restype = ctypes.c_longlong
    lib.fa2_ablate_tail_launches.argtypes = []
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hip.hipStreamDestroy.argtypes = [ctypes.c_void_p]
    hip.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
    q, k, v, _ = _inputs("gqa_d128", seed=13)
    want = _static(q, k, v, False)
    out = torch.empty_like(q)
    torch.cuda.synchronize()
    B, H_q, N, D = q.shape
    strides = [_lib._strides(t) for t in (q, k, v, out)]
    took, handles = [], []
    try:
        for i in range(300):
            h = ctypes.c_void_p()
            assert hip.hipStreamCreate(ctypes.byref(h)) == 0
            handles.append(h.value)
            before = lib.fa2_ablate_tail_launches()
            out.zero_()
            torch.cuda.synchronize()
            rc = lib.fa2_ablate_attn_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                                         *strides, B, H_q, k.shape[1], N, N, D,
                                         _lib.DTYPE_CODE[q.dtype], 1, 1, LOG2E / math.sqrt(D), 0,
                                         h.value)
            assert rc == 0, lib.fa2_ablate_last_error().decode()
            assert hip.hipStreamSynchronize(h) == 0
            took.append(lib.fa2_ablate_tail_launches() - before)
            assert torch.equal(out, want), f"stream {i} (tail: {took[-1]})"
    finally:
        for h in handles:
            hip.hipStreamSynchronize(h)
            hip.hipStreamDestroy(h)
    first_static = took.index(0) if 0 in took else len(took)
    print(f"streams with a ticket set: {first_static} of {len(took)}", flush=True)
    assert set(took) <= {0, 1}
    assert took == [1] * first_static + [0] * (len(took) - first_static)
    assert 1 <= first_static <= 256


@pytest.mark.parametrize("block_n", [32, 64, 128])
def test_tail_with_lse_and_other_tiles(block_n):
    """The tail with the log-sum-exp output and with 32-, 64- and 128-key tiles (the policy holds
    at every tile width of the 128-row programs): the output within the 2x-SDPA rule of the fp32
    oracle, the same bits as the call without the log-sum-exp, and the log-sum-exp within 1e-4 of
    the oracle's."""
    from attn_check import check_against_oracle
    from fa2.kernel import attention
    from oracle import reference as ref

    q, k, v, _ = _inputs("gqa_d128", seed=11)
    out, lse = attention(q, k, v, causal=True, block_n=block_n, return_lse=True)
    assert torch.equal(out, attention(q, k, v, causal=True, block_n=block_n))
    check_against_oracle(q, k, v, True, precision=torch.float32, ours=out)
    want = ref.naive_lse(q.float(), k.float(), None, causal=True)
    assert (lse - want).abs().max().item() <= 1e-4


def test_tail_with_a_ragged_pack_of_seven():
    """GQA group 7 at block_m 112 (C5's group on a grid long enough for a tail): packed and
    unpacked launches both deal their tails at run time, stay equal bit for bit (packing only
    renumbers rows) and meet the oracle."""
    from attn_check import check_against_oracle
    from fa2.kernel import attention

    q, k, v = make_qkv(2, 56, 8, 2048, 2048, 128, torch.bfloat16, seed=12)
    packed = attention(q, k, v, causal=True, block_m=112, pack_gqa=True)
    unpacked = attention(q, k, v, causal=True, block_m=112, pack_gqa=False)
    assert torch.equal(packed, unpacked)
    check_against_oracle(q, k, v, True, precision=torch.float32, ours=packed)


def test_seeded_random_tail_shapes_are_the_static_order_bit_for_bit():
    """Eight seeded random causal shapes that the policy gives a tail (fa2_ablate_tail_schedule
    says so before the launch): batch 1-6, 1-8 kv heads, GQA groups 1-8, N 1500-6000 (ragged last
    q tiles), head_dim 64 or 128, fp16 or bf16, packed or not where the group divides 128."""
    import ctypes
    import random

    from ablation import ablate_lib

    lib = ablate_lib()
    fn = lib.fa2_ablate_tail_schedule
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_int32] * 7 + [ctypes.POINTER(ctypes.c_int32)] * 3
    rng = random.Random(2026)
    done = 0
    while done < 8:
        B, hkv, group = rng.randint(1, 6), rng.randint(1, 8), rng.choice([1, 2, 4, 7, 8])
        n, d = rng.randint(1500, 6000), rng.choice([64, 128])
        dt = rng.choice([torch.float16, torch.bfloat16])
        pack = group > 1 and 128 % group == 0 and rng.random() < 0.5
        if B * hkv * group * n * d > 6e7:  # keep each case to a few hundred MB at most
            continue
        out = [ctypes.c_int32() for _ in range(3)]
        rc = fn(B, hkv * group, hkv, n, d, 1, group if pack else 1, *(ctypes.byref(o) for o in out))
        if rc != 0 or out[1].value == 0:
            continue
        q, k, v = make_qkv(B, hkv * group, hkv, n, n, d, dt, seed=done)
        want = _static(q, k, v, pack)
        assert torch.equal(_dynamic(q, k, v, pack), want), (B, hkv, group, n, d, dt, pack)
        done += 1
