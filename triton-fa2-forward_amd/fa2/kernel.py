"""FlashAttention-2 forward on AMD MI355X (gfx950): the drop-in for the reference's fa2.kernel.

Scope, as the reference (fa2/kernel.py:1-51): forward only, FP16/BF16 inputs, optional causal
mask (top-left aligned, N_q == N_kv), GQA. q is [B, H_q, N_q, D], k/v are [B, H_kv, N_kv, D],
H_q % H_kv == 0; every H_q // H_kv consecutive query heads share one KV head.

The arithmetic runs in one hand-written HIP kernel for gfx950 (csrc/attn_fwd_kernel.hpp), reached
through the C ABI of include/fa2_fwd.h. This module keeps the reference's host-side contract:
the same arguments, the same assertions and ValueErrors, the same default-tile and head-packing
policy, and `out = torch.empty_like(q)` as the caller-visible allocation. There is no CPU or
PyTorch fallback: without the built library or without GPU tensors, attention() raises.

Tile semantics on gfx950:
  block_m   rows of (position, head) pairs per program, exactly as in the reference. The
            kernel runs ceil(block_m / 32) wave64s of 32 rows (rounded up to 1, 2, 4 or 8
            waves); rows past block_m are computed on zeros and dropped.
  block_n   keys per K/V tile, rounded up to 32, 64 or 128 (the MFMA tile is 32 keys).
  num_warps, num_stages
            accepted for signature compatibility with the reference's Triton launch. The wave
            count follows block_m and the K/V pipeline depth is fixed (one tile in LDS, the
            next in flight), so these two do not change the launch.
"""

import math

import torch

from . import _lib

LOG2E = 1.4426950408889634


def _default_config(head_dim, on_cuda):
    """(BLOCK_M, BLOCK_N, num_waves, num_stages) for gfx950; counterpart of the reference's
    _default_config (fa2/kernel.py:186-195) and of fa2_default_config in the C ABI.

    on_cuda=False returns the reference's small CPU tile; this module cannot compute on the
    CPU, but the value still drives should_pack_gqa for callers that ask.
    """
    if not on_cuda:
        return 32, 16, 1, 1
    if head_dim not in (16, 32, 64, 128):
        raise ValueError(f"head_dim must be one of 16, 32, 64, 128, got {head_dim}")
    # sweep.py on MI355X: 64-key tiles (C2, C3, C5 at head_dim 128; C4 at 64, where 64-key tiles
    # get the software-pipelined loop), 128-key tiles at head_dim 16
    return 128, (128 if head_dim == 16 else 64), 4, 2


def _tile_efficiency(rows, block_m):
    """Fraction of a program's rows in use (fa2/kernel.py:198-199)."""
    return rows / (-(-rows // block_m) * block_m)


def should_pack_gqa(n_q, group, block_m):
    """FlashAttention-3's rule (fa2/kernel.py:202-207): pack when the unpacked tiles are less
    than 90% as full as the packed ones. Packing needs block_m to be a multiple of the group."""
    if group == 1 or block_m % group:
        return False
    return _tile_efficiency(n_q, block_m) < 0.9 * _tile_efficiency(n_q * group, block_m)


# K/V rows further apart than this (elements) are copied first: the C ABI takes up to 2^22, as
# the kernel builds a K/V tile's buffer resource from 32-bit products of the row stride.
_MAX_KV_ROW_STRIDE = 1 << 22


def _loadable(t, max_row_stride=None):
    """t itself if the kernel's 16-byte loads can address it, else a dense copy. A contiguous
    tensor qualifies when it is 16-byte aligned: its strides are multiples of head_dim, itself a
    multiple of 8 (the fast path, checked first: this runs four times per call). With
    `max_row_stride`, a sequence stride above it also takes the copy (K and V)."""
    if t.is_contiguous() and t.data_ptr() % 16 == 0:
        return t
    ok = (t.stride(-1) == 1 and t.data_ptr() % 16 == 0
          and all(n == 1 or s % 8 == 0 for n, s in zip(t.shape[:3], t.stride()[:3]))
          and (max_row_stride is None or t.shape[2] == 1 or t.stride(2) <= max_row_stride))
    return t if ok else t.clone(memory_format=torch.contiguous_format)


_CU_COUNT = {}


def _cu_count(device):
    if device not in _CU_COUNT:
        _CU_COUNT[device] = torch.cuda.get_device_properties(device).multi_processor_count
    return _CU_COUNT[device]


def attention(q, k, v, causal=True, sm_scale=None, block_m=None, block_n=None,
              num_warps=None, num_stages=None, pack_gqa=None, *, num_splits=None,
              return_lse=False):
    """softmax(Q K^T * sm_scale [+ causal mask]) V, fused (fa2/kernel.py:210-260).

    q: [B, H_q, N_q, D]; k, v: [B, H_kv, N_kv, D]; returns [B, H_q, N_q, D] laid out like q.
    pack_gqa: put each GQA group's query heads into one program; None decides with
    should_pack_gqa.

    Keyword-only extensions (the reference has neither, README.md:308-315):
    num_splits: split-KV, cut every program's key range into this many workgroups and merge
        their partial results in a second kernel (non-causal only); None picks it from the
        grid size and the GPU's CU count (1 when the grid already fills the GPU). The pick
        does not depend on pack_gqa, so packed and unpacked results stay equal bit for bit.
    return_lse: also return the natural-log log-sum-exp of every row's scaled scores, fp32
        [B, H_q, N_q], i.e. (out, lse).
    """
    assert q.dim() == k.dim() == v.dim() == 4
    B, H_q, N_q, D = q.shape
    Bk, H_kv, N_kv, Dk = k.shape
    assert v.shape == k.shape and Bk == B and Dk == D
    assert q.dtype == k.dtype == v.dtype and q.dtype in (torch.float16, torch.bfloat16)
    assert H_q % H_kv == 0, "GQA needs H_q divisible by H_kv"
    assert D in (16, 32, 64, 128), "head_dim must be a power of two in [16, 128]"
    if causal:
        # Top-left aligned causal mask (prefill); bottom-right alignment is out of scope.
        assert N_q == N_kv, "causal attention here assumes N_q == N_kv"

    bm, bn, nw, ns = _default_config(D, q.is_cuda)
    bm, bn = block_m or bm, block_n or bn
    nw, ns = num_warps or nw, num_stages or ns
    group = H_q // H_kv
    if pack_gqa is None:
        pack_gqa = should_pack_gqa(N_q, group, bm)
    elif pack_gqa and bm % group:
        raise ValueError(f"pack_gqa needs BLOCK_M ({bm}) to be a multiple of the GQA group ({group})")
    pack = group if pack_gqa else 1

    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    if not sm_scale > 0:
        raise ValueError(f"sm_scale must be positive (the row max is scaled after it is taken), got {sm_scale}")
    qk_scale = sm_scale * LOG2E  # exp(x) == exp2(x * log2 e)
    if num_splits is not None:
        if not 1 <= num_splits <= 16:
            raise ValueError(f"num_splits must be in [1, 16], got {num_splits}")
        if num_splits > 1 and causal:
            raise ValueError("num_splits > 1 (split-KV) needs causal=False")

    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise RuntimeError("fa2.kernel.attention runs on the GPU (gfx950 HIP kernel); got CPU tensors")
    if not (q.device == k.device == v.device):
        raise RuntimeError(f"q, k, v must be on one device, got {q.device}, {k.device}, {v.device}")

    if num_splits is None:
        num_splits = 1 if causal else _lib.num_splits(B, H_q, H_kv, N_q, N_kv, D, causal, bm, bn,
                                                      _cu_count(q.device))

    out = torch.empty_like(q)
    lse = torch.empty((B, H_q, N_q), dtype=torch.float32, device=q.device) if return_lse else None
    if out.numel() == 0:
        return (out, lse) if return_lse else out
    q_ = _loadable(q)
    k_, v_ = (_loadable(t, _MAX_KV_ROW_STRIDE) for t in (k, v))
    o_ = _loadable(out)

    def launch():
        stream = torch.cuda.current_stream(q.device).cuda_stream
        # split-KV partials and, on long enough problems, the key-norm table
        ws_bytes = _lib.workspace_bytes_for(B, H_q, H_kv, N_q, N_kv, D, q.dtype, causal,
                                            num_splits)
        if ws_bytes == 0 and lse is None:
            _lib.attn_fwd(q_, k_, v_, o_, causal, pack, bm, bn, qk_scale, stream)
        else:
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes else None
            _lib.attn_fwd_ex(q_, k_, v_, o_, causal, pack, bm, bn, qk_scale, lse, num_splits,
                             ws, stream)

    # the launch must run with q's device current; switch only when it is not (the switch costs
    # more than the rest of a small call)
    if q.device.index == torch.cuda.current_device():
        launch()
    else:
        with torch.cuda.device(q.device):
            launch()
    if o_ is not out:
        out.copy_(o_)
    return (out, lse) if return_lse else out
