"""Acceptance helpers shared by the GPU parity tests (restating tests/test_correctness.py:29-44, 90-103).

check_against_oracle runs fa2.kernel.attention, the CPU oracle's naive_attention in a high
precision (fp64 like the reference's tests, or fp32 as BASELINE.json's north star asks) and
torch's own fp16/bf16 SDPA as the yardstick, and applies the reference's rule:
    max|ours - truth| <= 2 * max|sdpa - truth| + 1e-4, and ours is finite.
"""

import torch
import torch.nn.functional as F

from oracle import reference as ref

DEVICE = "cuda"


def make_qkv(B, H_q, H_kv, N_q, N_kv, D, dtype, seed=0, device=DEVICE):
    """q, k, v from one seeded generator on the device, in that order (tests/test_correctness.py:34-39)."""
    g = torch.Generator(device=device).manual_seed(seed)
    q = torch.randn(B, H_q, N_q, D, device=device, dtype=dtype, generator=g)
    k = torch.randn(B, H_kv, N_kv, D, device=device, dtype=dtype, generator=g)
    v = torch.randn(B, H_kv, N_kv, D, device=device, dtype=dtype, generator=g)
    return q, k, v


def sdpa_yardstick(q, k, v, causal):
    """torch's own fp16/bf16 attention on the same inputs, and the backend that produced it.

    K/V are expanded to MHA and made contiguous first, and only the fused GPU backends are
    allowed (torch's math backend runs batched bf16 products on transposed views, which this
    GPU pool forbids); if neither fused backend takes the shape, CPU SDPA is the yardstick.
    """
    from torch.nn.attention import SDPBackend, sdpa_kernel

    group = q.shape[1] // k.shape[1]
    ke = k.repeat_interleave(group, dim=1).contiguous()
    ve = v.repeat_interleave(group, dim=1).contiguous()
    qc = q.contiguous()
    if q.is_cuda:
        for name in ("FLASH_ATTENTION", "EFFICIENT_ATTENTION"):
            try:
                with sdpa_kernel(getattr(SDPBackend, name)):
                    out = F.scaled_dot_product_attention(qc, ke, ve, is_causal=causal)
                torch.cuda.synchronize()
                return out, name.lower()
            except RuntimeError:
                continue
    out = F.scaled_dot_product_attention(qc.cpu(), ke.cpu(), ve.cpu(), is_causal=causal)
    return out.to(q.device), "cpu"


def truth(q, k, v, causal, precision=torch.float64, sm_scale=None):
    return ref.naive_attention(q.to(precision), k.to(precision), v.to(precision),
                               causal=causal, sm_scale=sm_scale)


def check_against_oracle(q, k, v, causal, precision=torch.float64, ours=None, **kw):
    """Run (or take) our output and assert the 2x-SDPA bar. Returns a dict of the numbers."""
    from fa2.kernel import attention

    if ours is None:
        ours = attention(q, k, v, causal=causal, **kw)
    want = truth(q, k, v, causal, precision)
    theirs, backend = sdpa_yardstick(q, k, v, causal)
    ours_abs, ours_rel = ref.errors(ours, want)
    theirs_abs, theirs_rel = ref.errors(theirs, want)
    assert torch.isfinite(ours).all(), "non-finite output"
    assert ref.acceptance(ours_abs, theirs_abs), (
        f"max-abs {ours_abs:.3e} vs torch[{backend}] {theirs_abs:.3e} "
        f"(rel {ours_rel:.3e} vs {theirs_rel:.3e})")
    return {"ours_abs": ours_abs, "sdpa_abs": theirs_abs, "ours_rel": ours_rel,
            "sdpa_rel": theirs_rel, "sdpa_backend": backend}
