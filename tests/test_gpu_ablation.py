"""The kernel's timing variants (libfa2_ablate.so via triton-fa2-forward_amd/ablation.py), as the
reference tests its knockout copy (tests/test_ablation.py:16-48):

* with no switch on, the variant is the production kernel, bit for bit (copy): against
  attention() where that launches the table-free kernel, and against fa2_attn_fwd on a shape
  where attention() adds the key-norm pass (there the variants are timed against copy);
* mask_every_tile only adds work: still bit for bit;
* scale_first, and both switches together (the reference's "before_fixes"), still compute
  attention: the 2x-SDPA rule against the fp64 oracle;
* the key split (8 waves in two groups over the halves of each program's key range, merged
  through LDS) is still attention: the 2x-SDPA rule against the fp64 oracle on ragged, GQA,
  causal and full shapes, and C5 at full size against the fp32 oracle;
* the work-skipping knockouts (no_exp, no_softmax, kv_l2, matmul_only, no_kv_staging, no_q_load)
  change the output (tests/test_ablation.py:28-34), on both of the kernel's tile loops
  (software-pipelined at head_dim 64, one tile at a time otherwise), causal or not, and no_store
  writes none.
"""

import math

import pytest
import torch

from attn_check import check_against_oracle, make_qkv

pytestmark = pytest.mark.gpu

BATCH = 2


def _ablate():
    from ablation import attention_ablate
    return attention_ablate


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("pack_gqa", [False, True])
@pytest.mark.parametrize("N", [37, 128])
def test_copy_is_the_production_kernel(causal, pack_gqa, N):
    from fa2.kernel import attention

    q, k, v = make_qkv(BATCH, 8, 2, N, N, 64, torch.float16)
    assert torch.equal(_ablate()(q, k, v, causal=causal, pack_gqa=pack_gqa),
                       attention(q, k, v, causal=causal, pack_gqa=pack_gqa))


def test_copy_is_the_table_free_launch_where_attention_adds_the_key_norm_pass():
    """bf16, head_dim 128, causal, N 4096, H 32/8: attention() asks for the key-norm table here
    (fa2_workspace_bytes_for), the variants never do; copy equals fa2_attn_fwd's launch."""
    from ablation import table_free_launch
    from fa2 import _lib

    q, k, v = make_qkv(1, 32, 8, 4096, 4096, 128, torch.bfloat16)
    assert (_lib.workspace_bytes_for(1, 32, 8, 4096, 4096, 128, q.dtype, True, 1)
            > _lib.workspace_bytes(1, 32, 4096, 128, 1))
    assert torch.equal(_ablate()(q, k, v, causal=True), table_free_launch(q, k, v, True))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [16, 32, 64, 128])
@pytest.mark.parametrize("causal", [True, False])
def test_mask_every_tile_is_bit_exact(dtype, D, causal):
    from fa2.kernel import attention

    # 300 keys: whole tiles (no mask needed) and a ragged last tile
    q, k, v = make_qkv(BATCH, 4, 2, 300, 300, D, dtype)
    assert torch.equal(_ablate()(q, k, v, causal=causal, mask_every_tile=True),
                       attention(q, k, v, causal=causal))


@pytest.mark.parametrize("knobs", [{"scale_first": True}, {"mask_every_tile": True},
                                   {"scale_first": True, "mask_every_tile": True}])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype,D", [(torch.float16, 64), (torch.bfloat16, 128)])
def test_the_kernel_before_its_two_fixes_is_still_attention(knobs, causal, dtype, D):
    q, k, v = make_qkv(BATCH, 4, 2, 128, 128, D, dtype)
    out = _ablate()(q, k, v, causal=causal, **knobs)
    check_against_oracle(q, k, v, causal, ours=out)


def test_scale_first_changes_only_rounding():
    """Scaling before the max moves each exponent by at most an fp32 rounding step: the output
    stays within a few bf16 ulps (2^-7 relative) of the production kernel's."""
    from fa2.kernel import attention

    q, k, v = make_qkv(BATCH, 8, 2, 512, 512, 128, torch.bfloat16)
    a = _ablate()(q, k, v, causal=True, scale_first=True)
    b = attention(q, k, v, causal=True)
    assert (a.float() - b.float()).abs().max().item() <= 2e-2


@pytest.mark.parametrize("knobs", [{"no_exp": True}, {"no_softmax": True}, {"kv_l2": True},
                                   {"no_softmax": True, "kv_l2": True}, {"no_kv_staging": True},
                                   {"no_q_load": True}],
                         ids=["no_exp", "no_softmax", "kv_l2", "matmul_only", "no_kv_staging",
                              "no_q_load"])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype,D", [(torch.float16, 16), (torch.bfloat16, 32),
                                     (torch.float16, 64), (torch.bfloat16, 64),
                                     (torch.bfloat16, 128)])
def test_knockouts_change_the_output(knobs, causal, dtype, D):
    """300 keys span three tiles at every head dim (128-key tiles at 16, 64-key tiles above), so
    kv_l2's repeated first tile differs from the real ones, and no_kv_staging's third tile is a
    stale copy of the first."""
    from fa2.kernel import attention

    q, k, v = make_qkv(BATCH, 4, 2, 300, 300, D, dtype)
    out = _ablate()(q, k, v, causal=causal, **knobs)
    assert not torch.equal(out, attention(q, k, v, causal=causal))


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype,D", [(torch.float16, 64), (torch.bfloat16, 128)])
def test_no_store_writes_nothing(causal, dtype, D):
    """The no_store knockout computes every program and writes no output: a sentinel-filled
    output stays as it was."""
    import ctypes

    from ablation import ablate_lib
    from fa2 import _lib
    from fa2.kernel import LOG2E

    q, k, v = make_qkv(BATCH, 4, 2, 300, 300, D, dtype)
    out = torch.full_like(q, 3.0)
    lib = ablate_lib()
    B, H_q, N, _ = q.shape
    rc = lib.fa2_ablate_attn_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                                 *[_lib._strides(t) for t in (q, k, v, out)], B, H_q, k.shape[1],
                                 N, N, D, _lib.DTYPE_CODE[dtype], int(causal), 1,
                                 LOG2E / math.sqrt(D), 2048,  # FA2_ABLATE_NO_STORE
                                 torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.fa2_ablate_last_error().decode()
    torch.cuda.synchronize()
    assert bool((out == 3.0).all())


@pytest.mark.parametrize("dtype,D,causal", [(torch.bfloat16, 128, True), (torch.float16, 64, False)])
def test_timeline_instance_is_the_product_and_its_records_are_ordered(dtype, D, causal):
    """fa2_ablate_timeline (triton-fa2-forward_amd/timeline.py): the product's output bit for bit,
    and every workgroup's stamps in order (entry <= prologue <= loop <= stores done), its tile
    count that of its program (causal: 2 t + 2 tiles of 64 keys for q tile t, capped at the
    sequence), and hardware ids that name at most 256 CUs."""
    from ablation import table_free_launch
    from timeline import decode_cu, run_timeline

    N = 1000
    q, k, v = make_qkv(2, 8, 2, N, N, D, dtype)
    recs, out = run_timeline(q, k, v, causal, 2)
    assert torch.equal(out, table_free_launch(q, k, v, causal))
    n_tiles_kv = -(-N // 64)
    tiles_seen = sorted(r[4] for r in recs)
    want = sorted(min(2 * t + 2, n_tiles_kv) if causal else n_tiles_kv
                  for t in range(-(-N // 128)) for _ in range(2 * 8))
    assert tiles_seen == want
    for e, p, l, d, tiles, hw in recs:
        assert 0 < e <= p <= l <= d and d - e < 10**6   # under 10 ms
    assert len({decode_cu(r[5]) for r in recs}) <= 256


def test_timeline_records_every_program_once_under_the_dynamic_tail():
    """B1 H32/8 N4096 head_dim 128 causal has a dynamic tail (1024 programs, 128 per XCD): the
    records are indexed by program, so every program's record is written exactly once whichever
    workgroup ran it, and the spare workgroups that found no program leave nothing."""
    from ablation import table_free_launch
    from timeline import run_timeline

    q, k, v = make_qkv(1, 32, 8, 4096, 4096, 128, torch.bfloat16)
    recs, out = run_timeline(q, k, v, True, 2)
    assert torch.equal(out, table_free_launch(q, k, v, True))
    assert sorted(r[4] for r in recs) == sorted(2 * t + 2 for t in range(32) for _ in range(32))
    assert all(0 < r[0] <= r[1] <= r[2] <= r[3] for r in recs)


@pytest.mark.parametrize("causal", [True, False])
def test_static_order_is_copy_bit_for_bit(causal):
    """FA2_ABLATE_STATIC_ORDER changes only which workgroup runs which program."""
    q, k, v = make_qkv(1, 32, 8, 4096, 4096, 128, torch.bfloat16)
    assert torch.equal(_ablate()(q, k, v, causal=causal, static_order=True),
                       _ablate()(q, k, v, causal=causal))


def test_mfma_ceiling_probe_runs_every_mode():
    """fa2_ablate_mfma_ceiling (triton-fa2-forward_amd/ceiling.py): one short launch per mode
    completes and writes a finite value per lane; with constant operands (1.0) every lane's sum
    is exact: 16 accumulator registers x 8 MFMAs per iteration x 16 products of 1.0, per
    accumulator, twice. The VGPR-accumulator mode (inline-asm MFMAs, hazards kept by hand) must
    reproduce the LDS + softmax mode bit for bit: same data, same MFMAs, only the registers the
    accumulators live in differ. The two half-read modes differ only in their LDS allocation
    (the occupancy), so they agree bit for bit too."""
    import ceiling

    lib, fn = ceiling._fn()
    wg, iters = 64, 10
    stream = torch.cuda.current_stream().cuda_stream
    outs = {}
    for name, mode in ceiling.MODES.items():
        out = torch.full((wg * 256,), float("nan"), device="cuda")
        rc = fn(mode, wg, iters, out.data_ptr(), out.numel(), stream)
        assert rc == 0, lib.fa2_ablate_last_error()
        torch.cuda.synchronize()
        assert torch.isfinite(out).all(), mode
        if mode == ceiling.MODES["mfma_const"]:
            assert torch.all(out == 2 * 16 * 8 * iters * 16), out[:4]
        outs[name] = out
    assert torch.equal(outs["mfma_lds_softmax_vacc"], outs["mfma_lds_softmax"])
    # one workgroup per CU instead of two: the same instructions on the same data
    assert torch.equal(outs["half_lds_softmax_vacc_1wave"], outs["half_lds_softmax_vacc"])


def test_hbm_read_probe_reads_every_word():
    """fa2_ablate_hbm_read: every word of the buffer is read once: the XOR of the per-thread
    outputs equals the XOR of the buffer's 32-bit words (grid-stride loop, unrolled by four, and
    its tail), on a size that is not a multiple of the grid's stride."""
    import ctypes

    from ablation import ablate_lib

    lib = ablate_lib()
    rd = lib.fa2_ablate_hbm_read
    rd.restype = ctypes.c_int
    rd.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32,
                   ctypes.c_void_p]
    g = torch.Generator(device="cpu").manual_seed(3)
    words = torch.randint(-2**31, 2**31 - 1, (16 * 12345,), generator=g, dtype=torch.int64).to(torch.int32)
    src = words.cuda()
    for wg in (1, 7, 64):
        out = torch.zeros(wg * 256, dtype=torch.int32, device="cuda")
        rc = rd(src.data_ptr(), src.numel() * 4, out.data_ptr(), out.numel(), wg,
                torch.cuda.current_stream().cuda_stream)
        assert rc == 0, lib.fa2_ablate_last_error()
        torch.cuda.synchronize()
        want = 0
        for w in words.tolist():
            want ^= w & 0xFFFFFFFF
        got = 0
        for w in out.cpu().tolist():
            got ^= w & 0xFFFFFFFF
        assert got == want, wg


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(2, 8, 2, 300), (1, 4, 4, 64), (1, 4, 4, 65), (2, 8, 8, 1000),
                                   (1, 7, 1, 129)])
def test_split_keys_is_attention(shape, dtype, causal):
    """One tile (group 1 idle), 65 keys (group 1 one masked tile), odd tile counts (group 1 one
    tile fewer), rows whose keys all lie in group 0's half (causal), GQA."""
    B, hq, hkv, N = shape
    print(f"split_keys: B={B} Hq={hq} Hkv={hkv} N={N} {dtype} causal={causal}", flush=True)
    q, k, v = make_qkv(B, hq, hkv, N, N, 128, dtype)
    out = _ablate()(q, k, v, causal=causal, split_keys=True)
    check_against_oracle(q, k, v, causal, ours=out)


def test_split_keys_on_c5_meets_the_fp32_oracle():
    import bench

    q, k, v, causal = bench.make_inputs("C5", "cuda")
    print("split_keys: C5 full size", flush=True)
    out = _ablate()(q, k, v, causal=causal, split_keys=True)
    check_against_oracle(q, k, v, causal, precision=torch.float32, ours=out)
    again = _ablate()(q, k, v, causal=causal, split_keys=True)
    assert torch.equal(out, again)


def test_split_keys_needs_head_dim_128():
    q, k, v = make_qkv(1, 4, 4, 64, 64, 64, torch.float16)
    with pytest.raises(RuntimeError):
        _ablate()(q, k, v, causal=True, split_keys=True)
        torch.cuda.synchronize()
