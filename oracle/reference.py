"""CPU oracle of the FlashAttention-2 forward: TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py may import this
module, and only as the checker (or, for blocked_attention, as the timed CPU baseline). The
product path, fa2.kernel.attention, never calls into it and has no CPU fallback.

Each function restates, in this repository's own code, the reference's pure-PyTorch
algorithm or helper it is named after:

  expand_kv           fa2/reference.py:16-19    GQA -> MHA by repeating each KV head
  naive_attention     fa2/reference.py:22-32    textbook softmax(Q K^T * scale [+ tril]) V,
                                                the ground truth (callers pick fp32 or fp64)
  blocked_attention   fa2/reference.py:35-82    the kernel's tiled online-softmax recurrence
                                                with fp32 state; the CPU baseline
  naive_lse           (no counterpart)          log sum exp of the same masked, scaled scores
                                                as naive_attention: the log-sum-exp output,
                                                an extension the reference lacks (its
                                                README.md:308), checked per row
  errors              tests/test_correctness.py:42-44   max-abs and relative-L2 error
  acceptance          tests/test_correctness.py:29-31, 90-103   ours <= 2 x SDPA + 1e-4
  attn_flops          bench/bench.py:83-87      4 B H_q pairs D, causal pairs N(N+1)/2
  baseline_inputs     BASELINE.json "configs"   the five seeded input recipes C1..C5

How each is pinned (tests/test_oracle.py; none of these restates the formula under test):
  naive_attention     golden vectors from an independent pure-Python float64 brute force
                      (tests/golden/make_golden.py), torch's SDPA math kernel in fp64 (a library
                      routine), closed forms (N=1 causal -> v[0]; one key -> v; equal scores ->
                      mean of v; a scale of 0 -> mean of v), GQA == MHA on repeated heads, and
                      planted mistakes (no mask, off-by-one mask, wrong KV head) that must fail.
  naive_lse           an independent pure-Python float64 brute force (math.exp / math.log per
                      row), closed forms (one key -> q.k * scale; a scale of 0 -> log of the
                      visible-key count, i.e. log(i + 1) for causal row i; equal scores ->
                      score + log N), and planted mistakes (mask dropped, base 2 instead of e)
                      that must fail.
  blocked_attention   equal to naive_attention to 1e-5 in fp64 over the reference's own sweep
                      (tests/test_correctness.py:51-66), with planted mistakes (alpha dropped,
                      off-by-one causal mask) that must fail the same check.
  attn_flops          hand counts at small sizes and the published C3 figure (5.49823e11).
  baseline_inputs     shapes, dtypes, seeds and the C5 perturbation count, checked directly.
"""

import math

import torch

LOG2E = 1.4426950408889634

# Absolute slack of the 2x-SDPA rule (tests/test_correctness.py:29-31).
ATOL_FLOOR = 1e-4


def expand_kv(k, v, h_q):
    """GQA -> MHA: query head h reads KV head h // group (fa2/reference.py:16-19)."""
    group = h_q // k.shape[1]
    return k.repeat_interleave(group, dim=1), v.repeat_interleave(group, dim=1)


def naive_attention(q, k, v, causal=True, sm_scale=None, heads_per_chunk=None):
    """softmax(Q K^T * scale [+ top-left tril mask]) V, computed in q's dtype.

    Follows fa2/reference.py:22-32. The score matrix is materialised per chunk of heads so that
    long sequences fit: heads_per_chunk (default: every head at once when the chunk's scores
    stay under 2 GiB) bounds the [B, chunk, N_q, N_kv] temporary.
    """
    B, H_q, N_q, D = q.shape
    H_kv, N_kv = k.shape[1], k.shape[2]
    group = H_q // H_kv
    scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(D)
    if heads_per_chunk is None:
        per_head = B * N_q * N_kv * q.element_size()
        heads_per_chunk = max(1, min(H_q, (2 << 30) // max(1, per_head)))
    mask = None
    if causal:
        mask = torch.ones(N_q, N_kv, dtype=torch.bool, device=q.device).tril()
    out = torch.empty_like(q)
    for h0 in range(0, H_q, heads_per_chunk):
        h1 = min(H_q, h0 + heads_per_chunk)
        kv_idx = torch.arange(h0, h1, device=q.device) // group
        kc = k.index_select(1, kv_idx)
        vc = v.index_select(1, kv_idx)
        s = torch.matmul(q[:, h0:h1], kc.transpose(-1, -2).contiguous()) * scale
        if causal:
            s = s.masked_fill(~mask, float("-inf"))
        out[:, h0:h1] = torch.matmul(torch.softmax(s, dim=-1), vc)
        del s
    return out


def naive_lse(q, k, v, causal=True, sm_scale=None, heads_per_chunk=None):
    """log sum_n exp(q_i . k_n * scale) over the keys row i sees, natural log, in q's dtype:
    [B, H_q, N_q]. The scores and mask are naive_attention's (fa2/reference.py:22-32); the
    reference has no log-sum-exp output. v is accepted for a uniform signature and unused."""
    B, H_q, N_q, D = q.shape
    H_kv, N_kv = k.shape[1], k.shape[2]
    group = H_q // H_kv
    scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(D)
    if heads_per_chunk is None:
        per_head = B * N_q * N_kv * q.element_size()
        heads_per_chunk = max(1, min(H_q, (2 << 30) // max(1, per_head)))
    mask = None
    if causal:
        mask = torch.ones(N_q, N_kv, dtype=torch.bool, device=q.device).tril()
    out = torch.empty(B, H_q, N_q, dtype=q.dtype, device=q.device)
    for h0 in range(0, H_q, heads_per_chunk):
        h1 = min(H_q, h0 + heads_per_chunk)
        kc = k.index_select(1, torch.arange(h0, h1, device=q.device) // group)
        s = torch.matmul(q[:, h0:h1], kc.transpose(-1, -2).contiguous()) * scale
        if causal:
            s = s.masked_fill(~mask, float("-inf"))
        out[:, h0:h1] = torch.logsumexp(s, dim=-1)
        del s
    return out


def causal_visible(rows, cols):
    """Top-left causal rule: key `col` is visible to query `row` iff col <= row."""
    return rows[:, None] >= cols[None, :]


def blocked_attention(q, k, v, causal=True, sm_scale=None, block_m=32, block_n=16):
    """The FA2 tiled recurrence in plain torch, fp32 state (fa2/reference.py:35-82).

    Each (b, h, start_m) iteration is one program of the GPU kernel: Q tile resident, K/V
    tiles streamed, m / l / acc updated online in base 2, normalised once at the end. Causal
    runs the unmasked columns [0, start_m) and then the diagonal block [start_m, end) with the
    elementwise mask, and never touches columns past the block (needs block_m % block_n == 0,
    which the defaults satisfy).
    """
    B, H_q, N_q, D = q.shape
    H_kv, N_kv = k.shape[1], k.shape[2]
    group = H_q // H_kv
    scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(D)
    qk_scale = scale * LOG2E
    out = torch.empty_like(q)
    dev = q.device

    def sweep(acc, l_i, m_i, qt, kh, vh, rows, lo, hi, masked):
        for n0 in range(lo, hi, block_n):
            cols = torch.arange(n0, min(n0 + block_n, N_kv), device=dev)
            kt = kh[cols].float()
            vt = vh[cols].float()
            s = (qt @ kt.T) * qk_scale
            if masked:
                s = s.masked_fill(~causal_visible(rows, cols), float("-inf"))
            m_new = torch.maximum(m_i, s.max(dim=1).values)
            p = torch.exp2(s - m_new[:, None])
            alpha = torch.exp2(m_i - m_new)
            l_i = l_i * alpha + p.sum(dim=1)
            acc = acc * alpha[:, None] + p @ vt
            m_i = m_new
        return acc, l_i, m_i

    for b in range(B):
        for h in range(H_q):
            kh, vh = k[b, h // group], v[b, h // group]
            for m0 in range(0, N_q, block_m):
                rows = torch.arange(m0, min(m0 + block_m, N_q), device=dev)
                qt = q[b, h, rows].float()
                m_i = torch.full((len(rows),), float("-inf"), device=dev)
                l_i = torch.zeros(len(rows), device=dev)
                acc = torch.zeros(len(rows), D, device=dev)
                if causal:
                    acc, l_i, m_i = sweep(acc, l_i, m_i, qt, kh, vh, rows, 0, m0, False)
                    acc, l_i, m_i = sweep(acc, l_i, m_i, qt, kh, vh, rows, m0,
                                          min(m0 + block_m, N_kv), True)
                else:
                    acc, l_i, m_i = sweep(acc, l_i, m_i, qt, kh, vh, rows, 0, N_kv, False)
                out[b, h, rows] = (acc / l_i[:, None]).to(q.dtype)
    return out


def errors(out, ref):
    """(max-abs, relative L2) of out against ref, in fp64 (tests/test_correctness.py:42-44)."""
    diff = out.double() - ref.double()
    return diff.abs().max().item(), (diff.norm() / ref.double().norm()).item()


def acceptance(ours_abs, sdpa_abs):
    """The reference's bar: no worse than twice torch's own SDPA, plus a 1e-4 floor."""
    return ours_abs <= 2.0 * sdpa_abs + ATOL_FLOOR


def attn_flops(B, H_q, N_q, N_kv, D, causal):
    """Two matmuls, 2 FLOPs per multiply-add; causal keeps N(N+1)/2 pairs (bench/bench.py:83-87)."""
    pairs = N_q * (N_q + 1) / 2 if causal else N_q * N_kv
    return 4 * B * H_q * pairs * D


# ------------------------------------------------------------------------------------------
# the same seeded bits on every device
# ------------------------------------------------------------------------------------------

CONFIGS = {
    # name: (dtype, causal, B, H_q, H_kv, N, D, description)
    "C1": (torch.float16, True, 1, 4, 4, 256, 64, "fp16 causal MHA (CPU plumbing)"),
    "C2": (torch.bfloat16, True, 4, 16, 16, 4096, 128, "bf16 causal MHA, EVEN_N"),
    "C3": (torch.bfloat16, True, 1, 32, 8, 8192, 128, "bf16 causal GQA, Llama-3-8B-like heads"),
    "C4": (torch.float16, False, 2, 16, 16, 16384, 64, "fp16 full attention, inputs x0.5"),
    "C5": (torch.bfloat16, True, 3, 28, 4, 1000, 128, "bf16 causal GQA ragged, 1% of k rows x8"),
}


def baseline_inputs(name, device="cpu", seed=0):
    """q, k, v, causal for a BASELINE.json config.

    torch.Generator("cpu") seeded with `seed`; q, k, v drawn with randn in fp32 in that order;
    perturbations applied in fp32; then cast to the config dtype and moved to `device`.
    C4 scales q, k, v by 0.5. C5 draws idx = randperm(B*H_kv*N)[:1%] after v and multiplies
    those rows of k (viewed as [B*H_kv*N, D]) by 8.
    """
    dtype, causal, B, H_q, H_kv, N, D, _ = CONFIGS[name]
    g = torch.Generator("cpu").manual_seed(seed)
    q = torch.randn(B, H_q, N, D, generator=g, dtype=torch.float32)
    k = torch.randn(B, H_kv, N, D, generator=g, dtype=torch.float32)
    v = torch.randn(B, H_kv, N, D, generator=g, dtype=torch.float32)
    if name == "C4":
        q, k, v = q * 0.5, k * 0.5, v * 0.5
    if name == "C5":
        rows = B * H_kv * N
        idx = torch.randperm(rows, generator=g)[: rows // 100]
        k.view(rows, D)[idx] *= 8.0
    return (q.to(dtype).to(device), k.to(dtype).to(device), v.to(dtype).to(device), causal)
