"""The kernel's timing variants (triton-fa2-forward_amd/ablation.py, fa2_attn_fwd_variant), as
the reference tests its knockout copy (tests/test_ablation.py:16-48):

* with no switch on, the variant entry point is the production kernel, bit for bit;
* mask_every_tile only adds work: still bit for bit;
* scale_first, and both switches together (the reference's "before_fixes"), still compute
  attention: the 2x-SDPA rule against the fp64 oracle.

The reference's work-skipping switches (no_exp, no_softmax, kv_l2) are not part of this library;
tests/test_frontend.py checks that asking for them fails.
"""

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
