"""Pins the CPU oracle (oracle/reference.py) before anything is checked against it.

Every check here is independent of the formula under test: committed brute-force golden
vectors, torch's own SDPA math kernel in fp64, closed forms, and planted mistakes that the
checks must catch. The blocked recurrence is checked against the naive one exactly as the
reference checks its own (tests/test_correctness.py:51-66).
"""

import json
import math
import os

import pytest
import torch
import torch.nn.functional as F

from oracle import reference as ref

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "attention_golden.json")


def make_qkv(B, H_q, H_kv, N_q, N_kv, D, dtype, seed=0):
    """q, k, v from one seeded generator, in that order (tests/test_correctness.py:34-39)."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H_q, N_q, D, dtype=dtype, generator=g)
    k = torch.randn(B, H_kv, N_kv, D, dtype=dtype, generator=g)
    v = torch.randn(B, H_kv, N_kv, D, dtype=dtype, generator=g)
    return q, k, v


# ------------------------------------------------------------------------------------------
# naive_attention
# ------------------------------------------------------------------------------------------

def _golden_cases():
    with open(GOLDEN) as f:
        return json.load(f)["cases"]


@pytest.mark.parametrize("case", _golden_cases(), ids=lambda c: c["name"])
def test_naive_matches_bruteforce_golden(case):
    t = lambda x: torch.tensor(x, dtype=torch.float64)  # noqa: E731
    out = ref.naive_attention(t(case["q"]), t(case["k"]), t(case["v"]),
                              causal=case["causal"], sm_scale=case["sm_scale"])
    torch.testing.assert_close(out, t(case["out"]), atol=1e-12, rtol=1e-12)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("H_q,H_kv", [(4, 4), (4, 2), (6, 1)])
@pytest.mark.parametrize("N_q,N_kv", [(1, 1), (17, 17), (64, 64), (5, 33)])
def test_naive_matches_torch_sdpa_math_fp64(causal, H_q, H_kv, N_q, N_kv):
    if causal and N_q != N_kv:
        pytest.skip("top-left causal is defined here for N_q == N_kv")
    q, k, v = make_qkv(2, H_q, H_kv, N_q, N_kv, 16, torch.float64)
    ke, ve = (t.repeat_interleave(H_q // H_kv, dim=1) for t in (k, v))
    from torch.nn.attention import SDPBackend, sdpa_kernel
    with sdpa_kernel(SDPBackend.MATH):
        lib = F.scaled_dot_product_attention(q, ke, ve, is_causal=causal)
    torch.testing.assert_close(ref.naive_attention(q, k, v, causal=causal), lib, atol=1e-12, rtol=1e-12)


def test_naive_closed_forms():
    q, k, v = make_qkv(2, 4, 2, 7, 7, 16, torch.float64)
    # causal row 0 sees only key 0
    out = ref.naive_attention(q, k, v, causal=True)
    kv_of = torch.arange(4) // 2
    torch.testing.assert_close(out[:, :, 0], v[:, kv_of, 0], atol=1e-14, rtol=0)
    # a single key: every row returns that key's value
    out1 = ref.naive_attention(q, k[:, :, :1], v[:, :, :1], causal=False)
    torch.testing.assert_close(out1, v[:, kv_of, :1].expand_as(out1), atol=1e-14, rtol=0)
    # scale 0 -> uniform weights -> the mean of the visible values (prefix mean when causal)
    out0 = ref.naive_attention(q, k, v, causal=True, sm_scale=0.0)
    prefix_mean = v.cumsum(dim=2) / torch.arange(1, 8, dtype=torch.float64)[:, None]
    torch.testing.assert_close(out0, prefix_mean[:, kv_of], atol=1e-13, rtol=0)
    # identical keys -> equal scores -> mean of v, whatever q is
    k_same = k[:, :, :1].expand_as(k).contiguous()
    out_same = ref.naive_attention(q, k_same, v, causal=False)
    torch.testing.assert_close(out_same, v.mean(dim=2, keepdim=True)[:, kv_of].expand_as(out_same),
                               atol=1e-13, rtol=0)


def test_naive_gqa_equals_mha_on_repeated_heads():
    q, k, v = make_qkv(2, 8, 2, 20, 20, 32, torch.float64)
    ke, ve = (t.repeat_interleave(4, dim=1) for t in (k, v))
    for causal in (True, False):
        torch.testing.assert_close(ref.naive_attention(q, k, v, causal=causal),
                                   ref.naive_attention(q, ke, ve, causal=causal), atol=0, rtol=0)


def test_naive_head_chunking_is_exact():
    q, k, v = make_qkv(2, 6, 3, 30, 30, 16, torch.float64)
    full = ref.naive_attention(q, k, v, causal=True)
    for chunk in (1, 2, 4, 5):
        torch.testing.assert_close(ref.naive_attention(q, k, v, causal=True, heads_per_chunk=chunk),
                                   full, atol=0, rtol=0)


def _planted_naive(kind):
    """naive_attention with one plausible mistake planted (on the CPU, in the checker only)."""
    def run(q, k, v, causal=True, sm_scale=None):
        D = q.shape[-1]
        scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(D)
        group = q.shape[1] // k.shape[1]
        if kind == "wrong_kv_head":
            kv = torch.arange(q.shape[1]) % k.shape[1]
        else:
            kv = torch.arange(q.shape[1]) // group
        kk, vv = k[:, kv], v[:, kv]
        s = q @ kk.transpose(-1, -2) * scale
        n_q, n_kv = s.shape[-2:]
        if causal and kind != "no_mask":
            diag = 1 if kind == "mask_off_by_one" else 0
            s = s.masked_fill(~torch.ones(n_q, n_kv, dtype=torch.bool).tril(diag), float("-inf"))
        return torch.softmax(s, dim=-1) @ vv
    return run


@pytest.mark.parametrize("kind", ["no_mask", "mask_off_by_one", "wrong_kv_head"])
def test_golden_and_sdpa_checks_catch_planted_mistakes(kind):
    """The pins above are strong enough to fail a mistaken oracle."""
    caught = False
    for case in _golden_cases():
        t = lambda x: torch.tensor(x, dtype=torch.float64)  # noqa: E731
        out = _planted_naive(kind)(t(case["q"]), t(case["k"]), t(case["v"]),
                                   causal=case["causal"], sm_scale=case["sm_scale"])
        if not torch.allclose(out, t(case["out"]), atol=1e-9, rtol=0):
            caught = True
    assert caught, f"planted mistake {kind!r} slipped through the golden vectors"


# ------------------------------------------------------------------------------------------
# blocked_attention: the reference's own tier-1 sweep (tests/test_correctness.py:51-66)
# ------------------------------------------------------------------------------------------

@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("H_q,H_kv", [(4, 4), (4, 2), (4, 1)])
@pytest.mark.parametrize("N", [1, 16, 37, 100])
def test_blocked_matches_naive(causal, H_q, H_kv, N):
    q, k, v = make_qkv(2, H_q, H_kv, N, N, 32, torch.float64)
    want = ref.naive_attention(q, k, v, causal=causal)
    got = ref.blocked_attention(q, k, v, causal=causal, block_m=32, block_n=16)
    # fp32 accumulator state inside blocked_attention -> fp32-level agreement
    torch.testing.assert_close(got, want, atol=1e-5, rtol=1e-5)


def test_blocked_noncausal_different_lengths():
    q, k, v = make_qkv(1, 4, 2, 23, 70, 32, torch.float64)
    torch.testing.assert_close(ref.blocked_attention(q, k, v, causal=False),
                               ref.naive_attention(q, k, v, causal=False), atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("block_m,block_n", [(64, 16), (32, 32), (16, 16)])
def test_blocked_other_tiles(block_m, block_n):
    q, k, v = make_qkv(1, 4, 2, 100, 100, 32, torch.float64)
    for causal in (True, False):
        torch.testing.assert_close(
            ref.blocked_attention(q, k, v, causal=causal, block_m=block_m, block_n=block_n),
            ref.naive_attention(q, k, v, causal=causal), atol=1e-5, rtol=1e-5)


def test_blocked_check_catches_planted_mistakes(monkeypatch):
    """Dropping the alpha rescale, or an off-by-one causal mask, must fail the blocked check
    (the reference's own planted-bug exercise, README.md:102-104)."""
    q, k, v = make_qkv(2, 4, 2, 37, 37, 32, torch.float64)
    want = ref.naive_attention(q, k, v, causal=True)

    real_exp2 = torch.exp2

    def no_alpha(x):  # alpha = exp2(m_i - m_new) is the only 1-D exp2 call in the recurrence
        return torch.ones_like(x) if x.dim() == 1 else real_exp2(x)

    monkeypatch.setattr(ref.torch, "exp2", no_alpha)
    bad = ref.blocked_attention(q, k, v, causal=True)
    monkeypatch.setattr(ref.torch, "exp2", real_exp2)
    assert not torch.allclose(bad, want, atol=1e-5, rtol=1e-5)

    good = ref.blocked_attention(q, k, v, causal=True)
    torch.testing.assert_close(good, want, atol=1e-5, rtol=1e-5)

    # off by one: every query also sees the next key
    monkeypatch.setattr(ref, "causal_visible", lambda rows, cols: rows[:, None] + 1 >= cols[None, :])
    bad = ref.blocked_attention(q, k, v, causal=True)
    assert not torch.allclose(bad, want, atol=1e-5, rtol=1e-5)


# ------------------------------------------------------------------------------------------
# helpers and input recipes
# ------------------------------------------------------------------------------------------

def test_attn_flops_counts():
    # one query, one key, D=1: 2 matmuls x 1 MAC x 2 FLOP
    assert ref.attn_flops(1, 1, 1, 1, 1, causal=False) == 4
    assert ref.attn_flops(1, 1, 3, 3, 2, causal=True) == 4 * 6 * 2      # 6 visible pairs
    assert ref.attn_flops(2, 3, 4, 5, 8, causal=False) == 4 * 2 * 3 * 20 * 8
    # C3's FLOP per step: 4 x 32 heads x 8192 x 8193 / 2 visible pairs x 128
    assert abs(ref.attn_flops(1, 32, 8192, 8192, 128, True) - 5.49823e11) / 5.49823e11 < 1e-5


def test_errors_and_acceptance():
    a = torch.zeros(3, dtype=torch.float16)
    b = torch.tensor([0.0, 0.5, -0.25], dtype=torch.float64)
    mx, rel = ref.errors(a, b)
    assert mx == 0.5 and abs(rel - 1.0) < 1e-12
    assert ref.acceptance(2e-3, 1e-3) and not ref.acceptance(2.2e-3, 1e-3)
    assert ref.acceptance(1e-4, 0.0)


def test_baseline_inputs_small():
    q, k, v, causal = ref.baseline_inputs("C1")
    assert causal and q.dtype == torch.float16 and q.shape == (1, 4, 256, 64) and k.shape == v.shape
    # the same seed gives the same bits
    q2, k2, v2, _ = ref.baseline_inputs("C1")
    assert torch.equal(q, q2) and torch.equal(k, k2) and torch.equal(v, v2)
    # q, k, v are the first three fp32 draws of seed 0, in that order
    g = torch.Generator().manual_seed(0)
    torch.testing.assert_close(q, torch.randn(1, 4, 256, 64, generator=g).half(), atol=0, rtol=0)


def test_baseline_inputs_c5_perturbation():
    q, k, v, causal = ref.baseline_inputs("C5")
    assert q.shape == (3, 28, 1000, 128) and k.shape == (3, 4, 1000, 128) and q.dtype == torch.bfloat16
    row_norm = k.float().view(-1, 128).norm(dim=1)
    big = (row_norm > 4 * row_norm.median()).sum().item()
    assert big == 120          # 1% of the 12000 k rows were scaled by 8


def test_c1_blocked_meets_the_2x_bar_on_cpu():
    """C1 end to end on the CPU: the blocked recurrence against fp32 naive, next to CPU SDPA."""
    q, k, v, causal = ref.baseline_inputs("C1")
    truth = ref.naive_attention(q.float(), k.float(), v.float(), causal=causal)
    ours = ref.blocked_attention(q, k, v, causal=causal)
    sdpa = F.scaled_dot_product_attention(q, k, v, is_causal=causal)
    ours_abs, _ = ref.errors(ours, truth)
    sdpa_abs, _ = ref.errors(sdpa, truth)
    assert torch.isfinite(ours).all()
    assert ref.acceptance(ours_abs, sdpa_abs), (ours_abs, sdpa_abs)


# ------------------------------------------------------------------------------------------
# naive_lse: the log-sum-exp output (an extension: the reference has none)
# ------------------------------------------------------------------------------------------

def _bruteforce_lse(q, k, causal, scale):
    """Per-row log-sum-exp in pure-Python float64 (math.exp / math.log), GQA by index."""
    B, H_q, N_q, D = q.shape
    H_kv, N_kv = k.shape[1], k.shape[2]
    group = H_q // H_kv
    Q, K = q.tolist(), k.tolist()
    out = torch.empty(B, H_q, N_q, dtype=torch.float64)
    for b in range(B):
        for h in range(H_q):
            for i in range(N_q):
                scores = [sum(a * c for a, c in zip(Q[b][h][i], K[b][h // group][n])) * scale
                          for n in range(N_kv) if not causal or n <= i]
                m = max(scores)
                out[b, h, i] = m + math.log(sum(math.exp(x - m) for x in scores))
    return out


LSE_CASES = [(True, 2, 1, 6, 6), (True, 4, 2, 9, 9), (False, 2, 2, 3, 11), (False, 4, 1, 7, 5)]


def _lse_inputs(H_q, H_kv, N_q, N_kv, D=8, seed=3):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(2, H_q, N_q, D, generator=g, dtype=torch.float64)
    k = torch.randn(2, H_kv, N_kv, D, generator=g, dtype=torch.float64)
    return q, k


@pytest.mark.parametrize("causal,H_q,H_kv,N_q,N_kv", LSE_CASES)
def test_lse_matches_bruteforce(causal, H_q, H_kv, N_q, N_kv):
    q, k = _lse_inputs(H_q, H_kv, N_q, N_kv)
    got = ref.naive_lse(q, k, k, causal=causal)
    torch.testing.assert_close(got, _bruteforce_lse(q, k, causal, 1 / math.sqrt(8)), atol=1e-12, rtol=0)


def test_lse_closed_forms():
    q, k = _lse_inputs(4, 2, 6, 6)
    # one key: the log-sum-exp is that key's scaled score
    one = ref.naive_lse(q, k[:, :, :1], None, causal=False, sm_scale=0.3)
    want = (q * k[:, [0, 0, 1, 1], :1]).sum(-1) * 0.3
    torch.testing.assert_close(one, want, atol=1e-12, rtol=0)
    # a scale of 0: every visible score is 0, so the result is log(#visible keys)
    causal0 = ref.naive_lse(q, k, None, causal=True, sm_scale=0.0)
    torch.testing.assert_close(causal0, torch.log(torch.arange(1, 7, dtype=torch.float64)).expand(2, 4, 6))
    full0 = ref.naive_lse(q, k, None, causal=False, sm_scale=0.0)
    torch.testing.assert_close(full0, torch.full((2, 4, 6), math.log(6), dtype=torch.float64))
    # identical keys: every score equals s, so the result is s + log N
    same = k[:, :, :1].expand(-1, -1, 6, -1).contiguous()
    lse = ref.naive_lse(q, same, None, causal=False)
    s = (q * same[:, [0, 0, 1, 1], :1]).sum(-1) / math.sqrt(8)
    torch.testing.assert_close(lse, s + math.log(6), atol=1e-12, rtol=0)


@pytest.mark.parametrize("kind", ["no_mask", "base_2"])
def test_lse_check_catches_planted_mistakes(kind):
    """The brute force fails a log-sum-exp with the causal mask dropped or taken in base 2."""
    def planted(q, k, causal):
        wrong = ref.naive_lse(q, k, None, causal=causal and kind != "no_mask")
        return wrong / math.log(2) if kind == "base_2" else wrong
    caught = False
    for causal, H_q, H_kv, N_q, N_kv in LSE_CASES:
        q, k = _lse_inputs(H_q, H_kv, N_q, N_kv)
        if not torch.allclose(planted(q, k, causal), _bruteforce_lse(q, k, causal, 1 / math.sqrt(8)),
                              atol=1e-9, rtol=0):
            caught = True
    assert caught, f"planted mistake {kind!r} slipped through"
