"""GPU parity of the two extensions the reference lacks (its README.md:308-315): the per-row
log-sum-exp output and split-KV.

Ground truth is the oracle: naive_attention for the output (the reference's 2x-SDPA rule,
as in test_gpu_parity.py) and naive_lse for the log-sum-exp, both in fp64 or fp32 on the same
inputs. A split-KV launch must meet the same bar as the single pass; its log-sum-exp, merged
across splits, must match the single pass's to fp32 rounding.
"""

import pytest
import torch

from attn_check import check_against_oracle, make_qkv
from oracle import reference as ref

pytestmark = pytest.mark.gpu

# Log-sum-exp tolerance (absolute, natural-log units). The scores are exact products of the
# 16-bit inputs summed in fp32 in a different order than the oracle's matmul, then exp2 / log2
# in fp32: errors stay near 1e-6 at these sizes. A dropped mask or a base-2 result is off by
# more than 1e-2.
LSE_ATOL = 1e-4


@pytest.fixture(autouse=True)
def _fp32_is_fp32():
    torch.backends.cuda.matmul.allow_tf32 = False
    yield


def _attention():
    from fa2.kernel import attention
    return attention


def lse_truth(q, k, causal, precision=torch.float64):
    return ref.naive_lse(q.to(precision), k.to(precision), None, causal=causal)


def assert_lse(lse, q, k, causal, precision=torch.float64):
    want = lse_truth(q, k, causal, precision)
    assert lse.dtype == torch.float32 and lse.shape == want.shape
    err = (lse.double() - want.double()).abs().max().item()
    assert err <= LSE_ATOL, f"log-sum-exp max-abs error {err:.3e}"


# ------------------------------------------------------------------------------------------
# log-sum-exp from the single-pass kernel
# ------------------------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("D", [16, 32, 64, 128])
@pytest.mark.parametrize("N", [1, 77, 300])
def test_lse_single_pass(dtype, causal, D, N):
    attention = _attention()
    q, k, v = make_qkv(2, 8, 2, N, N, D, dtype)
    out, lse = attention(q, k, v, causal=causal, return_lse=True)
    assert torch.equal(out, attention(q, k, v, causal=causal))  # same kernel, same rounding
    assert_lse(lse, q, k, causal)


@pytest.mark.parametrize("pack_gqa", [False, True])
def test_lse_packed_and_other_tiles(pack_gqa):
    attention = _attention()
    q, k, v = make_qkv(2, 8, 2, 200, 200, 64, torch.bfloat16)
    for bm, bn in ((128, 32), (64, 64), (256, 128), (32, 16)):
        out, lse = attention(q, k, v, causal=True, block_m=bm, block_n=bn, pack_gqa=pack_gqa,
                             return_lse=True)
        check_against_oracle(q, k, v, True, ours=out)
        assert_lse(lse, q, k, True)


# ------------------------------------------------------------------------------------------
# split-KV
# ------------------------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [16, 64, 128])
@pytest.mark.parametrize("splits", [2, 3, 5, 16])
@pytest.mark.parametrize("N_q,N_kv", [(1, 1000), (7, 300), (64, 2048), (130, 777)])
def test_splitkv_matches_oracle(dtype, D, splits, N_q, N_kv):
    attention = _attention()
    q, k, v = make_qkv(2, 8, 2, N_q, N_kv, D, dtype)
    out, lse = attention(q, k, v, causal=False, num_splits=splits, return_lse=True)
    check_against_oracle(q, k, v, False, ours=out)
    assert_lse(lse, q, k, False)
    _, lse1 = attention(q, k, v, causal=False, num_splits=1, return_lse=True)
    assert (lse - lse1).abs().max().item() <= 1e-5


def test_splitkv_packed_equals_unpacked():
    """Same split count, same tiles per row: packed and unpacked agree bit for bit, with an
    explicit count and with the automatic one (which does not look at pack_gqa)."""
    attention = _attention()
    q, k, v = make_qkv(2, 32, 8, 16, 1500, 128, torch.float16)
    for splits in (4, None):
        packed = attention(q, k, v, causal=False, pack_gqa=True, num_splits=splits)
        unpacked = attention(q, k, v, causal=False, pack_gqa=False, num_splits=splits)
        assert torch.equal(packed, unpacked)
        check_against_oracle(q, k, v, False, ours=packed)


def test_splitkv_more_splits_than_tiles():
    """16 splits of a 2-tile key range run as 2 splits; 1 key runs as 1."""
    attention = _attention()
    for n_kv in (100, 1):
        q, k, v = make_qkv(2, 4, 4, 5, n_kv, 64, torch.bfloat16)
        out, lse = attention(q, k, v, causal=False, num_splits=16, return_lse=True)
        check_against_oracle(q, k, v, False, ours=out)
        assert_lse(lse, q, k, False)


def test_splitkv_noncontiguous_output():
    """q (and so out) in [B, N, H, D] storage: the merge honours the output strides."""
    attention = _attention()
    q, k, v = make_qkv(2, 8, 2, 9, 1024, 64, torch.float16)
    q = q.transpose(1, 2).contiguous().transpose(1, 2)
    out = attention(q, k, v, causal=False, num_splits=4)
    assert out.stride() == q.stride()
    check_against_oracle(q, k, v, False, ours=out)


def test_splitkv_deterministic():
    attention = _attention()
    q, k, v = make_qkv(2, 8, 2, 33, 3000, 128, torch.bfloat16)
    a = attention(q, k, v, causal=False, num_splits=8)
    b = attention(q, k, v, causal=False, num_splits=8)
    assert torch.equal(a, b)


@pytest.mark.parametrize("N_q", [1, 16, 32])
def test_pack_short_regime_full_size(N_q):
    """The reference's few-queries table (README.md:282-301): B=16, H_q=32, H_kv=8, N_kv=4096,
    non-causal fp16. The default path packs and picks split-KV; fp32 oracle."""
    from fa2 import _lib
    from fa2.kernel import _cu_count
    attention = _attention()
    q, k, v = make_qkv(16, 32, 8, N_q, 4096, 128, torch.float16)
    splits = _lib.num_splits(16, 32, 8, N_q, 4096, 128, False, 128, 64, _cu_count(q.device))
    assert splits > 1
    out, lse = attention(q, k, v, causal=False, return_lse=True)
    check_against_oracle(q, k, v, False, precision=torch.float32, ours=out)
    assert_lse(lse, q, k, False, precision=torch.float32)


def test_workspace_too_small_is_rejected():
    from fa2 import _lib
    q, k, v = make_qkv(1, 4, 4, 8, 1024, 64, torch.float16)
    out = torch.empty_like(q)
    ws = torch.empty(1024, dtype=torch.uint8, device=q.device)
    with pytest.raises(RuntimeError, match="workspace"):
        _lib.attn_fwd_ex(q, k, v, out, False, 1, 128, 64, 0.18, None, 4, ws,
                         torch.cuda.current_stream().cuda_stream)
