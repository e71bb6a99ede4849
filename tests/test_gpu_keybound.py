"""GPU parity of the key-norm bound: fa2_attn_fwd_ex given room for the key-norm table.

The library then runs the key-norm pass (attn_key_norm.hip: the largest squared key norm of
every 64 keys of every (batch, kv head)) and the kernel instance that uses it: after a row's first
tile, |q| max|k| qk_scale <= m + tau (Cauchy-Schwarz) proves that no later score passes the
row's reference max m by more than tau (15 for fp16, 32 for bf16, in exp2 units), and waves
whose rows all pass skip the per-tile row max. A row whose bound passes m + tau by at most the
lift (4 for fp16 where the bound is at most 19, 8 for bf16) skips as well, with its reference
raised by a whole number to bound - tau or just above. attention() asks for the table only on long
problems (fa2_workspace_bytes_for); these tests force it on small ones by passing the room.

Checked here: the table itself against torch's norms; the output against the oracle with the
reference's rule (2x SDPA's max-abs error + 1e-4) on shapes where every wave skips, where none
does (rows whose bound fails) and mixed; scores that rise far above the first tile's maximum
(P up to ~2^25 in bf16); packed == unpacked bit for bit with the table; split-KV and the
log-sum-exp with the table.
"""

import math

import pytest
import torch

from attn_check import check_against_oracle, make_qkv
from oracle import reference as ref

pytestmark = pytest.mark.gpu

CHUNK = 64  # keys per table entry (kKeyChunk)


@pytest.fixture(autouse=True)
def _fp32_is_fp32():
    torch.backends.cuda.matmul.allow_tf32 = False
    yield


def _table_bytes(B, H_kv, N_kv):
    n = B * H_kv * (-(-N_kv // CHUNK)) * 4
    return (n + 255) // 256 * 256


def run_with_table(q, k, v, causal, pack=1, splits=1, lse=False, table=True):
    """fa2_attn_fwd_ex at the default configuration, with the workspace the split-KV partials
    need plus (table=True) room for the key-norm table. Returns (out, lse, workspace)."""
    from fa2 import _lib
    from fa2.kernel import LOG2E

    B, H_q, N_q, D = q.shape
    H_kv, N_kv = k.shape[1], k.shape[2]
    split_bytes = _lib.workspace_bytes(B, H_q, N_q, D, splits)
    n = split_bytes + (_table_bytes(B, H_kv, N_kv) if table else 0)
    ws = torch.zeros(n, dtype=torch.uint8, device=q.device) if n else None
    out = torch.empty_like(q)
    l = torch.empty((B, H_q, N_q), dtype=torch.float32, device=q.device) if lse else None
    stream = torch.cuda.current_stream(q.device).cuda_stream
    _lib.attn_fwd_ex(q, k, v, out, causal, pack, 128, 0, 1.0 / math.sqrt(D) * LOG2E, l, splits,
                     ws, stream)
    torch.cuda.synchronize()
    return out, l, ws


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [16, 32, 64, 128])
@pytest.mark.parametrize("N_kv", [1, 63, 64, 65, 1000])
def test_key_table_is_the_largest_key_norm_per_chunk(dtype, D, N_kv):
    q, k, v = make_qkv(2, 6, 3, 5, N_kv, D, dtype)
    k = k * torch.linspace(0.5, 2.0, N_kv, device=k.device, dtype=torch.float32).to(dtype)[:, None]
    _, _, ws = run_with_table(q, k, v, False)
    chunks = -(-N_kv // CHUNK)
    got = ws[: 2 * 3 * chunks * 4].view(torch.float32).reshape(2, 3, chunks)
    norms = k.float().pow(2).sum(-1)                                   # [B, H_kv, N_kv]
    padded = torch.zeros(2, 3, chunks * CHUNK, device=k.device)
    padded[..., :N_kv] = norms
    want = padded.reshape(2, 3, chunks, CHUNK).amax(-1)
    torch.testing.assert_close(got, want, rtol=1e-5, atol=0)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("D", [16, 32, 64, 128])
@pytest.mark.parametrize("N", [1, 100, 700])
def test_key_bound_matches_oracle(dtype, causal, D, N):
    q, k, v = make_qkv(2, 8, 2, N, N, D, dtype)
    out, _, _ = run_with_table(q, k, v, causal)
    check_against_oracle(q, k, v, causal, ours=out)
    # the same attention as the launch without the table (the bits may differ)
    plain, _, _ = run_with_table(q, k, v, causal, table=False)
    check_against_oracle(q, k, v, causal, ours=plain)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_key_bound_packed_equals_unpacked(causal, dtype):
    q, k, v = make_qkv(2, 16, 4, 333, 333, 128, dtype)
    packed, _, _ = run_with_table(q, k, v, causal, pack=4)
    unpacked, _, _ = run_with_table(q, k, v, causal, pack=1)
    assert torch.equal(packed, unpacked)
    again, _, _ = run_with_table(q, k, v, causal, pack=4)
    assert torch.equal(packed, again)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [True, False])
def test_key_bound_rows_that_fail_keep_the_row_max(dtype, causal):
    """Some query rows 40x longer (their bound cannot hold: those waves keep the row max and
    its rescaling), a few keys 8x longer (C5's outliers), the rest as usual: mixed waves."""
    q, k, v = make_qkv(2, 8, 2, 600, 600, 128, dtype)
    q[:, 0, ::7] *= 40
    k[:, 1, ::97] *= 8
    out, _, _ = run_with_table(q, k, v, causal)
    check_against_oracle(q, k, v, causal, precision=torch.float32, ours=out)


@pytest.mark.parametrize("D,causal,N,scale", [(64, False, 4096, 1.0), (64, True, 2048, 1.0),
                                               (128, True, 1024, 0.9), (128, False, 1024, 0.9)])
def test_key_bound_lifted_rows_match_oracle(D, causal, N, scale):
    """fp16: rows whose bound lands just past tau (15) above their first tile's maximum still
    skip, with their reference raised by a whole number (at most 4, kBoundLift) so that
    P <= 2^15 holds, where the bound is at most 19 (kBoundLiftMax: no P below 2^-24). The test
    first finds such rows on the host, then checks the output against the fp32 oracle."""
    B, H_q, H_kv = 2, 8, 2
    q, k, v = make_qkv(B, H_q, H_kv, N, N, D, torch.float16, seed=5)
    q = (q.float() * scale).to(torch.float16)
    qk = 1.0 / math.sqrt(D) * 1.4426950408889634
    qf, kf = q.float(), k.float().repeat_interleave(H_q // H_kv, dim=1)
    s0 = (qf @ kf[:, :, :64].transpose(-1, -2)) * qk                    # first tile's scores
    if causal:
        s0 = s0.masked_fill(torch.ones(N, 64, dtype=torch.bool, device=q.device).triu(1), -float("inf"))
    m0 = s0.amax(-1)
    kn2 = kf.pow(2).sum(-1)                                            # [B, H_q, N]
    if causal:   # a row sees keys 0..pos: the running max of the norms, in 64-key chunks
        kmax = kn2.reshape(B, H_q, N // 64, 64).amax(-1).cummax(-1).values.repeat_interleave(64, -1)
    else:
        kmax = kn2.amax(-1, keepdim=True).expand(B, H_q, N)
    bound = (qf.pow(2).sum(-1) * kmax).sqrt() * qk * (1 + 2 ** -10)
    lift = torch.ceil(bound - 15.0 - m0)
    lifted = int(((lift > 0) & (lift <= 4) & (bound <= 19.0)).sum().item())
    print(f"fp16 D={D} causal={causal}: {lifted} of {B * H_q * N} rows lifted", flush=True)
    assert lifted >= 32
    out, _, _ = run_with_table(q, k, v, causal)
    check_against_oracle(q, k, v, causal, precision=torch.float32, ours=out)


@pytest.mark.parametrize("dtype,top", [(torch.bfloat16, 25.0), (torch.float16, 13.0)])
@pytest.mark.parametrize("causal", [True, False])
def test_key_bound_scores_far_above_the_first_tile(dtype, top, causal):
    """The first 64 keys are short, later ones point along the queries: a row's later scores
    reach ~top (exp2 units) above a first-tile maximum near 0, so P grows to ~2^top with no
    rescaling. The bound still holds (|q| |k| qk_scale ~ top < tau)."""
    B, H, N, D = 1, 4, 512, 128
    qk_scale = 1.0 / math.sqrt(D) * 1.4426950408889634
    g = torch.Generator(device="cuda").manual_seed(3)
    dirs = torch.nn.functional.normalize(torch.randn(B, H, 1, D, device="cuda", generator=g), dim=-1)
    qn = math.sqrt(top / qk_scale)  # |q| |k| = top / qk_scale when aligned
    q = dirs.expand(B, H, N, D) * qn + 0.05 * torch.randn(B, H, N, D, device="cuda", generator=g)
    k = 0.02 * torch.randn(B, H, N, D, device="cuda", generator=g)
    k[:, :, 64:] += dirs * qn * torch.linspace(0.2, 1.0, N - 64, device="cuda")[:, None]
    v = torch.randn(B, H, N, D, device="cuda", generator=g)
    q, k, v = (t.to(dtype).contiguous() for t in (q, k, v))
    out, lse, _ = run_with_table(q, k, v, causal, lse=True)
    assert torch.isfinite(out).all()
    check_against_oracle(q, k, v, causal, precision=torch.float32, ours=out)
    want = ref.naive_lse(q.double(), k.double(), None, causal=causal)
    assert (lse.double() - want).abs().max().item() <= 1e-4


@pytest.mark.parametrize("splits", [2, 3])
def test_key_bound_with_split_kv_and_lse(splits):
    q, k, v = make_qkv(2, 8, 2, 40, 2000, 128, torch.bfloat16)
    out, lse, _ = run_with_table(q, k, v, False, splits=splits, lse=True)
    check_against_oracle(q, k, v, False, ours=out)
    want = ref.naive_lse(q.double(), k.double(), None, causal=False)
    assert (lse.double() - want).abs().max().item() <= 1e-4


@pytest.mark.parametrize("causal", [True, False])
def test_key_bound_strided_inputs(causal):
    """[B, N, H, D] storage viewed as [B, H, N, D] (the reference's strided test,
    tests/test_correctness.py:134-140): the key-norm pass steps by the sequence stride H*D."""
    q, k, v = make_qkv(2, 8, 2, 500, 500, 64, torch.bfloat16)
    q, k, v = (t.transpose(1, 2).contiguous().transpose(1, 2) for t in (q, k, v))
    out, _, ws = run_with_table(q, k, v, causal)
    check_against_oracle(q, k, v, causal, ours=out)
    chunks = -(-500 // CHUNK)
    got = ws[: 2 * 2 * chunks * 4].view(torch.float32).reshape(2, 2, chunks)
    norms = torch.zeros(2, 2, chunks * CHUNK, device=k.device)
    norms[..., :500] = k.float().pow(2).sum(-1)
    torch.testing.assert_close(got, norms.reshape(2, 2, chunks, CHUNK).amax(-1), rtol=1e-5, atol=0)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_key_bound_long_key_range(dtype):
    """40000 keys (625 table entries: the kernel folds the entries past the first 256 in its
    prologue) against 128 queries, non-causal, with and without split-KV."""
    q, k, v = make_qkv(1, 4, 1, 128, 40000, 64, dtype)
    out, _, _ = run_with_table(q, k, v, False)
    check_against_oracle(q, k, v, False, precision=torch.float32, ours=out)
    out2, _, _ = run_with_table(q, k, v, False, splits=3)
    check_against_oracle(q, k, v, False, precision=torch.float32, ours=out2)


def _fuzz_cases(n=48, seed=20261202, first=0):
    import random
    rnd = random.Random(seed)
    cases = []
    for i in range(first, first + n):
        h_kv = rnd.choice([1, 2, 3, 4])
        group = rnd.choice([1, 2, 4, 7, 8])
        causal = rnd.random() < 0.5
        n_q = rnd.choice([1, 17, 64, 129, 300, 777])
        n_kv = n_q if causal else rnd.choice([1, 64, 65, 500, 1500])
        d = rnd.choice([16, 32, 64, 128])
        dtype = rnd.choice([torch.float16, torch.bfloat16])
        pack = group if (group > 1 and 128 % group == 0 and rnd.random() < 0.5) else 1
        splits = 1 if causal else rnd.choice([1, 1, 2, 4])
        lse = rnd.random() < 0.4
        strided = rnd.random() < 0.25
        scale = rnd.choice([0.25, 1.0, 3.0])  # small, usual and large scores
        cases.append((i, rnd.choice([1, 2]), h_kv * group, h_kv, n_q, n_kv, d, dtype, causal, pack,
                      splits, lse, strided, scale))
    return cases


@pytest.mark.parametrize("case", _fuzz_cases() + _fuzz_cases(seed=20261212, first=1000),
                         ids=lambda c: f"case{c[0]}")
def test_key_bound_fuzz(case):
    """Seeded random shapes with the key-norm table forced: every combination of GQA group,
    packing, lengths, head_dim, dtype, split-KV, log-sum-exp, strides and score scale."""
    i, B, h_q, h_kv, n_q, n_kv, d, dtype, causal, pack, splits, lse, strided, scale = case
    print(f"\ncase {case}", flush=True)
    q, k, v = make_qkv(B, h_q, h_kv, n_q, n_kv, d, dtype, seed=100 + i)
    q = (q.float() * scale).to(dtype)
    if strided:
        q, k, v = (t.transpose(1, 2).contiguous().transpose(1, 2) for t in (q, k, v))
    out, l, _ = run_with_table(q, k, v, causal, pack=pack, splits=splits, lse=lse)
    check_against_oracle(q, k, v, causal, precision=torch.float32, ours=out)
    if lse:
        want = ref.naive_lse(q.float(), k.float(), None, causal=causal)
        assert (l - want).abs().max().item() <= 1e-4
