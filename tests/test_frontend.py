"""CPU tests of the host side: the drop-in's policy and errors, and the C ABI of libfa2_fwd.so.

None of these launch a kernel. The C-ABI calls here all stop at argument checking (or at the
empty-output early return), which touches no GPU.
"""

import ctypes
import os
import re

import pytest
import torch

from fa2 import _lib
from fa2.kernel import _default_config, attention, should_pack_gqa

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fa2_fwd.h")

needs_lib = pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH),
                               reason="libfa2_fwd.so not built (python triton-fa2-forward_amd/csrc/build.py)")


def cpu_qkv(B, H_q, H_kv, N_q, N_kv, D, dtype=torch.float16):
    g = torch.Generator().manual_seed(0)
    return (torch.randn(B, H_q, N_q, D, generator=g).to(dtype),
            torch.randn(B, H_kv, N_kv, D, generator=g).to(dtype),
            torch.randn(B, H_kv, N_kv, D, generator=g).to(dtype))


# ------------------------------------------------------------------------------------------
# policy (fa2/kernel.py:186-207) and the reference's known answers
# ------------------------------------------------------------------------------------------

def test_should_pack_gqa_follows_tile_efficiency():
    """tests/test_correctness.py:189-198, verbatim known answers."""
    assert should_pack_gqa(1, 4, 128)
    assert should_pack_gqa(64, 4, 128)
    assert not should_pack_gqa(4096, 4, 128)
    assert not should_pack_gqa(1000, 4, 128)
    assert not should_pack_gqa(64, 1, 128)
    assert not should_pack_gqa(64, 3, 128)


def test_should_pack_gqa_c5_does_not_pack_by_rule():
    # BASELINE C5 (group 7, N=1000): 128 % 7 != 0, and even at block_m 112 the rule says no
    assert not should_pack_gqa(1000, 7, 128)
    assert not should_pack_gqa(1000, 7, 112)
    assert should_pack_gqa(1, 7, 112)


def test_default_config_table():
    for d in (16, 32, 64, 128):
        bm, bn, nw, ns = _default_config(d, True)
        assert bm % 32 == 0 and bn in (32, 64, 128) and nw == bm // 32 and ns >= 1
    assert _default_config(64, False) == (32, 16, 1, 1)


# ------------------------------------------------------------------------------------------
# the reference's argument errors, raised before anything reaches the GPU
# ------------------------------------------------------------------------------------------

def test_pack_gqa_needs_block_m_divisible_by_group():
    q, k, v = cpu_qkv(1, 6, 2, 16, 16, 64)     # group 3 does not divide BLOCK_M
    with pytest.raises(ValueError, match="BLOCK_M"):
        attention(q, k, v, causal=True, pack_gqa=True)


def test_sm_scale_must_be_positive():
    q, k, v = cpu_qkv(1, 4, 2, 16, 16, 64)
    with pytest.raises(ValueError, match="sm_scale"):
        attention(q, k, v, sm_scale=-0.125)
    with pytest.raises(ValueError, match="sm_scale"):
        attention(q, k, v, sm_scale=0.0)


@pytest.mark.parametrize("bad", ["rank", "dtype", "head_dim", "gqa", "causal_lengths", "kv_shape"])
def test_shape_and_dtype_assertions(bad):
    q, k, v = cpu_qkv(1, 4, 2, 16, 16, 64)
    if bad == "rank":
        q = q[0]
    elif bad == "dtype":
        q, k, v = q.float(), k.float(), v.float()
    elif bad == "head_dim":
        q, k, v = (t[..., :48].contiguous() for t in (q, k, v))
    elif bad == "gqa":
        q = torch.cat([q, q[:, :1]], dim=1)    # 5 query heads over 2 KV heads
    elif bad == "causal_lengths":
        k, v = k[:, :, :8], v[:, :, :8]
    elif bad == "kv_shape":
        v = v[:, :, :8]
    with pytest.raises(AssertionError):
        attention(q, k, v, causal=True)


def test_cpu_tensors_fail_loudly():
    """No silent CPU or PyTorch fallback exists on the product path."""
    q, k, v = cpu_qkv(1, 4, 2, 16, 16, 64)
    with pytest.raises(RuntimeError, match="GPU"):
        attention(q, k, v, causal=True)


# ------------------------------------------------------------------------------------------
# the C ABI: load, exports, policy agreement, argument checks
# ------------------------------------------------------------------------------------------

def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(fa2_[a-z0-9_]+)\s*\(", text))


def test_loadable_copies_only_what_the_kernel_cannot_address():
    """fa2.kernel._loadable (CPU tensors: the check is on strides and alignment only): views the
    16-byte loads can address pass through; a K/V row stride above the C ABI's 2^22 elements is
    copied, one at the limit is not (the reference's attention() takes any stride)."""
    from fa2 import kernel

    base = torch.empty(1, 4, 64, 64, dtype=torch.float16)
    assert kernel._loadable(base) is base
    bnhd = torch.empty(1, 64, 4, 64, dtype=torch.float16).transpose(1, 2)  # [B, N, H, D] view
    assert kernel._loadable(bnhd, kernel._MAX_KV_ROW_STRIDE) is bnhd
    odd = torch.empty(1, 4, 64, 68, dtype=torch.float16)[..., :60]        # stride 68: not x8
    assert kernel._loadable(odd) is not odd and kernel._loadable(odd).is_contiguous()
    store = torch.empty(1 << 23, dtype=torch.float16)
    at = store.as_strided((1, 1, 2, 64), (1 << 23, 1 << 23, 1 << 22, 1))
    below = store.as_strided((1, 1, 2, 64), (1 << 23, 1 << 23, (1 << 22) - 8, 1))
    wide = torch.empty((1 << 22) + 8 + 64, dtype=torch.float16).as_strided(
        (1, 1, 2, 64), ((1 << 22) + 72, (1 << 22) + 72, (1 << 22) + 8, 1))
    assert kernel._loadable(at, kernel._MAX_KV_ROW_STRIDE) is at
    assert kernel._loadable(below, kernel._MAX_KV_ROW_STRIDE) is below
    copied = kernel._loadable(wide, kernel._MAX_KV_ROW_STRIDE)
    assert copied is not wide and copied.is_contiguous() and torch.equal(copied, wide)
    assert kernel._loadable(wide) is wide   # q and out: no row-stride limit in the C ABI


@needs_lib
def test_library_exports_every_declared_symbol():
    declared = _declared_functions()
    assert {"fa2_attn_fwd", "fa2_default_config", "fa2_should_pack_gqa",
            "fa2_last_error", "fa2_version"} <= declared
    lib = _lib.lib()
    for name in declared:
        assert hasattr(lib, name), name
    assert set(_lib.SIGNATURES) == declared
    assert b"gfx950" in lib.fa2_version()


@needs_lib
def test_c_policy_matches_python():
    lib = _lib.lib()
    for n_q in (1, 3, 16, 64, 100, 1000, 4096):
        for group in (1, 2, 3, 4, 7, 8, 32):
            for bm in (16, 32, 64, 112, 128, 256):
                assert bool(lib.fa2_should_pack_gqa(n_q, group, bm)) == should_pack_gqa(n_q, group, bm)
    for d in (16, 32, 64, 128):
        out = [ctypes.c_int32() for _ in range(4)]
        assert lib.fa2_default_config(d, *(ctypes.byref(o) for o in out)) == 0
        assert tuple(o.value for o in out) == _default_config(d, True)
    assert lib.fa2_default_config(48, None, None, None, None) == -1


def _call(**over):
    """fa2_attn_fwd with valid defaults except `over`; pointers are fake (16-byte aligned)."""
    a = dict(q=0x1000, k=0x2000, v=0x3000, out=0x4000, sq=(8192, 2048, 64, 1), sk=(4096, 2048, 64, 1),
             sv=(4096, 2048, 64, 1), so=(8192, 2048, 64, 1), batch=1, h_q=4, h_kv=2, n_q=32, n_kv=32,
             head_dim=64, dtype=0, causal=1, pack=1, block_m=128, block_n=64, qk_scale=0.18, stream=None)
    a.update(over)
    arr = lambda s: (ctypes.c_int64 * 4)(*s)  # noqa: E731
    lib = _lib.lib()
    rc = lib.fa2_attn_fwd(a["q"], a["k"], a["v"], a["out"], arr(a["sq"]), arr(a["sk"]), arr(a["sv"]),
                          arr(a["so"]), a["batch"], a["h_q"], a["h_kv"], a["n_q"], a["n_kv"],
                          a["head_dim"], a["dtype"], a["causal"], a["pack"], a["block_m"], a["block_n"],
                          a["qk_scale"], a["stream"])
    return rc, _lib.last_error()


@needs_lib
@pytest.mark.parametrize("over,code,msg", [
    (dict(head_dim=48), -1, "head_dim"),
    (dict(h_q=5), -1, "divisible"),
    (dict(dtype=2), -1, "dtype"),
    (dict(n_kv=16), -1, "N_q == N_kv"),
    (dict(pack=3), -1, "pack"),
    (dict(pack=2, block_m=127), -1, "BLOCK_M"),
    (dict(block_m=0), -1, "BLOCK_M"),
    (dict(block_m=257), -1, "BLOCK_M"),
    (dict(block_n=129), -1, "BLOCK_N"),
    (dict(qk_scale=0.0), -1, "qk_scale"),
    (dict(qk_scale=-1.0), -1, "qk_scale"),
    (dict(q=0x1008), -2, "aligned"),
    (dict(sq=(8192, 2048, 64, 2)), -2, "stride"),
    (dict(sk=(4096, 2048, 60, 1)), -2, "multiples of 8"),
    (dict(q=0), -1, "null"),
    # grids past 2^31 - 1 workgroups, including sizes whose product overflows int64
    (dict(batch=1 << 20, h_q=1 << 20, h_kv=1 << 20, n_q=4096, n_kv=4096), -1, "too large"),
    (dict(batch=2**31 - 1, h_q=2**31 - 1, h_kv=1, n_q=2**31 - 257, n_kv=2**31 - 257, block_m=1),
     -1, "too large"),
    # 32-bit positions in the kernel: sequences up to 2^31 - 257, causal or not
    (dict(n_q=2**31 - 1, n_kv=2**31 - 1, block_m=100), -1, "at most"),
    (dict(causal=0, n_q=32, n_kv=2**31 - 200), -1, "at most"),
    # a packed launch whose rows (n_q * pack) pass 2^31 although the grid is small: B 1, H 8/1,
    # N 2^28 + 1 (q is 64 GiB at head_dim 16, which fits in HBM); the row index would wrap
    (dict(h_q=8, h_kv=1, pack=8, n_q=2**28 + 1, n_kv=2**28 + 1, head_dim=16,
          sq=(8 * (2**28 + 1) * 16, (2**28 + 1) * 16, 16, 1), sk=((2**28 + 1) * 16, (2**28 + 1) * 16, 16, 1),
          sv=((2**28 + 1) * 16, (2**28 + 1) * 16, 16, 1), so=(8 * (2**28 + 1) * 16, (2**28 + 1) * 16, 16, 1)),
     -1, "32-bit row index"),
    (dict(h_q=8, h_kv=1, pack=8, n_q=2**28 + 1, n_kv=2**28 + 1, block_m=256),
     -1, "32-bit row index"),
    # K/V row strides past 2^22 elements: the kernel builds a tile's buffer resource from 32-bit
    # products of the row stride
    (dict(sk=(1 << 40, 1 << 30, (1 << 22) + 8, 1)), -1, "sequence stride"),
    (dict(sv=(1 << 40, 1 << 30, (1 << 22) + 8, 1)), -1, "sequence stride"),
])
def test_c_abi_rejects_bad_arguments(over, code, msg):
    rc, err = _call(**over)
    assert rc == code and msg in err, (rc, err)


@needs_lib
def test_c_abi_empty_output_is_a_no_op():
    assert _call(batch=0, q=0, k=0, v=0, out=0)[0] == 0
    assert _call(n_q=0, n_kv=0, q=0, k=0, v=0, out=0)[0] == 0


# ------------------------------------------------------------------------------------------
# fa2_attn_fwd_ex: log-sum-exp output and split-KV (extensions; no reference counterpart)
# ------------------------------------------------------------------------------------------

def _call_ex(**over):
    """fa2_attn_fwd_ex, non-causal, with fake pointers: every case below fails before a launch."""
    a = dict(q=0x1000, k=0x2000, v=0x3000, out=0x4000, sq=(8192, 2048, 64, 1), sk=(65536, 16384, 64, 1),
             sv=(65536, 16384, 64, 1), so=(8192, 2048, 64, 1), batch=1, h_q=4, h_kv=2, n_q=32, n_kv=256,
             head_dim=64, dtype=0, causal=0, pack=1, block_m=128, block_n=64, qk_scale=0.18, lse=None,
             num_splits=4, workspace=None, ws_bytes=0, stream=None)
    a.update(over)
    arr = lambda s: (ctypes.c_int64 * 4)(*s)  # noqa: E731
    lib = _lib.lib()
    rc = lib.fa2_attn_fwd_ex(a["q"], a["k"], a["v"], a["out"], arr(a["sq"]), arr(a["sk"]), arr(a["sv"]),
                             arr(a["so"]), a["batch"], a["h_q"], a["h_kv"], a["n_q"], a["n_kv"],
                             a["head_dim"], a["dtype"], a["causal"], a["pack"], a["block_m"],
                             a["block_n"], a["qk_scale"], a["lse"], a["num_splits"], a["workspace"],
                             a["ws_bytes"], a["stream"])
    return rc, _lib.last_error()


@needs_lib
@pytest.mark.parametrize("over,code,msg", [
    (dict(num_splits=0), -1, "num_splits"),
    (dict(num_splits=17), -1, "num_splits"),
    (dict(causal=1, n_kv=32, sk=(8192, 2048, 64, 1), sv=(8192, 2048, 64, 1)), -1, "causal"),
    (dict(workspace=None), -1, "workspace"),
    (dict(workspace=0x100000, ws_bytes=1024), -1, "workspace"),
    (dict(workspace=0x100010, ws_bytes=1 << 30), -2, "256-byte"),
    (dict(lse=0x1002, num_splits=1), -2, "lse"),
    (dict(head_dim=48), -1, "head_dim"),
])
def test_c_abi_ex_rejects_bad_arguments(over, code, msg):
    rc, err = _call_ex(**over)
    assert rc == code and msg in err, (rc, err)


@needs_lib
def test_split_policy():
    lib = _lib.lib()
    # the reference's pack-short regime (README.md:282-301), B=16, H 32/8, N_kv=4096, packed:
    # N_q <= 32 -> 128 programs -> 4 splits fill 256 CUs twice; N_q = 64 -> 256 programs -> 2
    # (the smaller grid is the packed one: 128 programs at N_q <= 32, 256 at N_q = 64)
    for n_q, want in ((1, 2), (16, 2), (32, 2), (64, 1), (128, 1)):
        assert lib.fa2_num_splits(16, 32, 8, n_q, 4096, 128, 0, 128, 64, 256) == want, n_q
    assert lib.fa2_num_splits(16, 32, 8, 1, 4096, 128, 1, 128, 64, 256) == 1      # causal
    assert lib.fa2_num_splits(16, 32, 8, 1, 4096, 128, 0, 127, 64, 256) == 1      # 127 % 4: 512 programs
    assert lib.fa2_num_splits(1, 8, 8, 1, 256, 128, 0, 128, 64, 256) == 1         # 4 tiles only
    assert lib.fa2_num_splits(1, 8, 8, 1, 512, 128, 0, 128, 64, 256) == 2         # 8 tiles: 2 x 4
    assert lib.fa2_num_splits(1, 8, 8, 1, 4096, 128, 0, 128, 64, 256) == 16       # 8 programs, capped
    assert lib.fa2_num_splits(4, 8, 8, 1, 4096, 128, 0, 128, 64, 256) == 8        # 32 x 8 = 256


@needs_lib
def test_workspace_bytes():
    lib = _lib.lib()
    rows = 16 * 32 * 1
    up = lambda x: (x + 255) // 256 * 256  # noqa: E731
    # fp32 partial outputs, then two fp32 partial log-sum-exps (merge weights, exact), each aligned
    assert lib.fa2_workspace_bytes(16, 32, 1, 128, 4) == up(4 * rows * 128 * 4) + 2 * up(4 * rows * 4)
    assert lib.fa2_workspace_bytes(3, 5, 7, 16, 3) == up(3 * 105 * 16 * 4) + 2 * up(3 * 105 * 4)
    assert lib.fa2_workspace_bytes(16, 32, 1, 128, 1) == 0
    assert lib.fa2_workspace_bytes(16, 32, 0, 128, 4) == 0


@needs_lib
def test_workspace_bytes_for_adds_the_key_table_where_it_pays():
    """The key-norm table (one fp32 per batch, kv head and 64 keys, 256-byte rounded) is asked
    for on bf16 at head_dim 128, or (fp16 or bf16) at 64 without the causal mask, when the
    attention does >= 16384 FLOP per byte of K and >= 2^37 FLOP: C3 and C4 qualify; C2 (4097
    FLOP/B), C5 (2.2e10 FLOP), fp16 at head_dim 128 and the few-queries shapes do not."""
    lib = _lib.lib()
    up = lambda x: (x + 255) // 256 * 256  # noqa: E731
    table = lambda B, H_kv, N_kv: up(B * H_kv * -(-N_kv // 64) * 4)  # noqa: E731
    f = lib.fa2_workspace_bytes_for
    F16, BF16 = 0, 1
    assert f(1, 32, 8, 8192, 8192, 128, BF16, 1, 1) == table(1, 8, 8192)          # C3
    assert f(1, 32, 8, 8192, 8192, 128, F16, 1, 1) == 0                           # fp16: no
    assert f(2, 16, 16, 16384, 16384, 64, F16, 0, 1) == table(2, 16, 16384)       # C4 (fp16)
    assert f(2, 16, 16, 16384, 16384, 64, F16, 1, 1) == 0                         # causal D64: no
    assert f(2, 16, 16, 16384, 16384, 64, BF16, 0, 1) == table(2, 16, 16384)      # bf16 full D64
    assert f(1, 32, 8, 8192, 8192, 64, BF16, 1, 1) == 0                           # causal D64: no
    assert f(4, 16, 16, 4096, 4096, 128, BF16, 1, 1) == 0                         # C2
    assert f(3, 28, 4, 1000, 1000, 128, BF16, 1, 1) == 0                          # C5
    assert f(16, 32, 8, 1, 4096, 128, BF16, 0, 2) == lib.fa2_workspace_bytes(16, 32, 1, 128, 2)
    # split-KV partials first, the table after them
    assert f(1, 64, 8, 2048, 16384, 128, BF16, 0, 2) == (lib.fa2_workspace_bytes(1, 64, 2048, 128, 2)
                                                         + table(1, 8, 16384))
    assert f(0, 32, 8, 8192, 8192, 128, BF16, 1, 1) == 0
    assert f(1, 32, 8, 8192, 8192, 48, BF16, 1, 1) == 0


# ------------------------------------------------------------------------------------------
# the measurement library libfa2_ablate.so (include/fa2_ablate.h): the timing variants of the
# reference's bench/ablation.py, kept out of the product library
# ------------------------------------------------------------------------------------------

ABLATE_HEADER = os.path.join(ROOT, "include", "fa2_ablate.h")
ABLATE_LIB = os.path.join(ROOT, "triton-fa2-forward_amd", "libfa2_ablate.so")
needs_ablate = pytest.mark.skipif(not os.path.exists(ABLATE_LIB), reason="libfa2_ablate.so not built")


def _exported(path):
    """Names of the functions a shared library exports (nm -D --defined-only)."""
    import shutil
    import subprocess

    if not shutil.which("nm"):
        pytest.skip("nm (binutils) is not installed")
    res = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True,
                         check=True)
    return {line.split()[-1] for line in res.stdout.splitlines() if line.strip()}


def _c_names(header):
    text = re.sub(r"/\*.*?\*/", "", open(header).read(), flags=re.S)
    return set(re.findall(r"\b(fa2_[a-z0-9_]+)\s*\(", text))


@needs_lib
def test_product_library_exports_its_api_and_no_timing_variant():
    """libfa2_fwd.so exports exactly the C functions of fa2_fwd.h (hidden visibility for the
    rest), and none of the measurement library's: no ablation entry point, and no kernel
    instance with a timing-variant bit (only VARIANT 0, the product, and 4, its key-norm
    instance, are compiled in)."""
    names = _exported(_lib.LIB_PATH)
    c_funcs = {n for n in names if n.startswith("fa2_")}
    assert c_funcs == _declared_functions()
    assert not {n for n in names if "ablate" in n or "variant" in n}
    kernels = [n for n in names if n.startswith("_ZN3fa215attn_fwd_kernel")]
    assert kernels
    for n in kernels:
        variant = int(re.search(r"ELb[01]ELi(\d+)EEEv", n).group(1))
        assert variant in (0, 4), n


@needs_ablate
def test_dynamic_tail_policy_on_the_cpu():
    """fa2_ablate_tail_schedule: which launches deal their last programs at run time, and how many
    (attn_fwd_host.hpp: tail_schedule). Causal grids of at least two rounds of programs per XCD
    (64 slots at head_dim 128, 96 at 64): with whole (batch, kv head) units per XCD the tail is the
    lighter of a quarter of each XCD's programs and half a unit chunk; otherwise (the fallback
    order) a quarter of every XCD's blocks and the remainder; plus 6% spare workgroups (rounded up
    to a multiple of 8). Known answers worked by hand from those rules."""
    from ablation import ablate_lib

    lib = ablate_lib()
    fn = lib.fa2_ablate_tail_schedule
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_int32] * 7 + [ctypes.POINTER(ctypes.c_int32)] * 3

    def tail(B, hq, hkv, n, d, causal, pack=1):
        out = [ctypes.c_int32(-1) for _ in range(3)]
        rc = fn(B, hq, hkv, n, d, int(causal), pack, *(ctypes.byref(o) for o in out))
        return rc, tuple(o.value for o in out)

    # C3: 2048 programs, 256 per XCD, chunk of one unit (256 programs): a quarter, 64 per XCD
    assert tail(1, 32, 8, 8192, 128, True) == (0, (1536, 512, 640))
    # C2: 8 units per XCD in chunks of 4 (2 MiB units): half a chunk = a quarter = 64
    assert tail(4, 16, 16, 4096, 128, True) == (0, (1536, 512, 640))
    # B8 H16 N4096: 512 per XCD; half a chunk (64) is lighter than a quarter (128)
    assert tail(8, 16, 16, 4096, 128, True) == (0, (3584, 512, 760))
    # fp16 head_dim 64 (three workgroups per CU): 256 per XCD >= 2 x 96
    assert tail(4, 16, 16, 4096, 64, True) == (0, (1536, 512, 640))
    # GQA head packing: 1024 programs, 128 per XCD, a quarter = 32
    assert tail(2, 32, 8, 2048, 128, True, pack=4) == (0, (768, 256, 320))
    # the fallback order (12 units): 2688 programs, 336 per XCD, a quarter = 84 per XCD
    assert tail(3, 28, 4, 4096, 128, True) == (0, (2016, 672, 840))
    # ... with a remainder: B1 H20/4 N8192, 1280 programs, 160 per XCD -> 40; 20 units: 5 x 256
    assert tail(1, 20, 4, 8192, 128, True) == (0, (960, 320, 400))
    # static order: non-causal (C4), fewer than two rounds (C5: 672 programs), under two rounds
    assert tail(2, 16, 16, 16384, 64, False) == (0, (0, 0, 0))
    assert tail(3, 28, 4, 1000, 128, True) == (0, (0, 0, 0))
    assert tail(1, 32, 8, 2048, 128, True) == (0, (0, 0, 0))
    assert tail(2, 16, 16, 4096, 64, True) == (0, (0, 0, 0))   # 128 per XCD < 2 x 96
    # sizes attention() rejects
    for bad in ((1, 30, 8, 512, 128, True), (1, 32, 8, 512, 48, True), (1, 32, 8, 512, 128, True, 3)):
        rc, _ = tail(*bad)
        assert rc == -1 and lib.fa2_ablate_last_error(), bad


@needs_ablate
def test_measurement_library_exports_exactly_its_header():
    names = _exported(ABLATE_LIB)
    assert {n for n in names if n.startswith("fa2_")} == _c_names(ABLATE_HEADER) == {
        "fa2_ablate_attn_fwd", "fa2_ablate_timeline", "fa2_ablate_mfma_ceiling",
        "fa2_ablate_hbm_read", "fa2_ablate_tail_schedule", "fa2_ablate_program_map",
        "fa2_ablate_tail_launches", "fa2_ablate_last_error"}
    # the knockouts are compiled into it: kernel instances with the no_exp, no_softmax and
    # kv_l2 bits, matmul_only (no_softmax | kv_l2), no_kv_staging (256), the key split (512,
    # head_dim 128 only), no_q_load (1024) and no_store (2048); and the timeline instance (64)
    variants = {int(m.group(1)) for n in names for m in [re.search(r"ELb[01]ELi(\d+)EEEv", n)] if m}
    assert variants == {0, 1, 2, 3, 8, 16, 32, 48, 64, 256, 512, 1024, 2048}


@needs_ablate
def test_measurement_library_rejects_unbuilt_variants_before_any_launch():
    from ablation import ablate_lib

    arr = lambda s: (ctypes.c_int64 * 4)(*s)  # noqa: E731
    lib = ablate_lib()
    st = arr((8192, 2048, 64, 1))
    # 4: the key-norm instance is the product's, not a variant; 64: the timeline instance runs
    # only through fa2_ablate_timeline, which checks its record buffer
    for bad in (4, 5, 24, 64, 65, -1):
        rc = lib.fa2_ablate_attn_fwd(0x1000, 0x2000, 0x3000, 0x4000, st, st, st, st, 1, 4, 4, 32,
                                     32, 64, 0, 1, 1, 0.18, bad, None)
        assert rc == -1 and b"variant" in lib.fa2_ablate_last_error(), (bad, rc)
    # the product's argument checks apply to every variant
    rc = lib.fa2_ablate_attn_fwd(0x1000, 0x2000, 0x3000, 0x4000, st, st, st, st, 1, 4, 4, 32,
                                 32, 48, 0, 1, 1, 0.18, 8, None)
    assert rc == -1 and b"head_dim" in lib.fa2_ablate_last_error()
    # the key split (512) is built at head_dim 128 only
    rc = lib.fa2_ablate_attn_fwd(0x1000, 0x2000, 0x3000, 0x4000, st, st, st, st, 1, 4, 4, 32,
                                 32, 64, 0, 1, 1, 0.18, 512, None)
    assert rc == -1 and b"key split" in lib.fa2_ablate_last_error()


@needs_ablate
def test_timeline_needs_a_buffer_of_six_words_per_workgroup():
    """fa2_ablate_timeline rejects a missing, misaligned or short record buffer before any
    launch (fake device pointers): B 1, H 4, N 32 -> 4 workgroups -> 24 words."""
    from ablation import ablate_lib

    arr = lambda s: (ctypes.c_int64 * 4)(*s)  # noqa: E731
    lib = ablate_lib()
    fn = lib.fa2_ablate_timeline
    fn.restype = ctypes.c_int
    i32, i64p, vp = ctypes.c_int32, ctypes.POINTER(ctypes.c_int64), ctypes.c_void_p
    fn.argtypes = [vp, vp, vp, vp, i64p, i64p, i64p, i64p] + [i32] * 9 + \
        [ctypes.c_float, vp, ctypes.c_int64, vp]
    st = arr((8192, 2048, 64, 1))
    for rec, words, code, msg in ((None, 24, -1, b"null"), (0x10004, 24, -2, b"aligned"),
                                  (0x10000, 23, -1, b"24 words")):
        rc = fn(0x1000, 0x2000, 0x3000, 0x4000, st, st, st, st, 1, 4, 4, 32, 32, 64, 0, 1, 1,
                0.18, rec, words, None)
        assert rc == code and msg in lib.fa2_ablate_last_error(), (rc, lib.fa2_ablate_last_error())


@needs_ablate
def test_mfma_ceiling_rejects_bad_arguments_before_any_launch():
    """fa2_ablate_mfma_ceiling checks mode, workgroup and iteration counts and its output buffer
    (fake device pointers) without touching the GPU."""
    import ceiling

    lib, fn = ceiling._fn()
    for mode, wg, it, out, words, code, msg in (
            (-1, 8, 1, 0x1000, 2048, -1, b"mode"), (10, 8, 1, 0x1000, 2048, -1, b"mode"),
            (0, 0, 1, 0x1000, 2048, -1, b"workgroups"), (0, 65537, 1, 0x1000, 1 << 30, -1, b"workgroups"),
            (0, 8, 0, 0x1000, 2048, -1, b"iters"), (3, 8, 100001, 0x1000, 2048, -1, b"iters"),
            (0, 8, 1, None, 2048, -1, b"null"), (1, 8, 1, 0x1002, 2048, -2, b"aligned"),
            (2, 8, 1, 0x1000, 2047, -1, b"2048")):
        rc = fn(mode, wg, it, out, words, None)
        assert rc == code and msg in lib.fa2_ablate_last_error(), (mode, wg, it, rc,
                                                                   lib.fa2_ablate_last_error())
    assert ceiling.launch_flops(2048, 6000) == 2048 * 4 * 6000 * 16 * 32768
    rd = lib.fa2_ablate_hbm_read
    rd.restype = ctypes.c_int
    rd.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32,
                   ctypes.c_void_p]
    for src, nb, out, words, wg, code, msg in (
            (None, 1024, 0x1000, 256, 1, -1, b"null"), (0x1008, 1024, 0x1000, 256, 1, -2, b"aligned"),
            (0x1000, 1000, 0x2000, 256, 1, -1, b"multiple of 16"), (0x1000, 1024, 0x2000, 256, 0, -1, b"workgroups"),
            (0x1000, 1024, 0x2000, 511, 2, -1, b"512")):
        rc = rd(src, nb, out, words, wg, None)
        assert rc == code and msg in lib.fa2_ablate_last_error(), (src, nb, rc, lib.fa2_ablate_last_error())
    assert list(ceiling.MODES.values()) == [0, 1, 2, 3, 4, 5, 6, 7, 8, 9]


def test_ablation_front_end_checks_arguments_on_the_cpu():
    from ablation import VARIANTS, attention_ablate, variant_bits

    # the reference's variant names (bench/ablation.py:42-53) and their bits
    assert list(VARIANTS) == ["copy", "scale_first", "mask_every_tile", "before_fixes", "no_exp",
                              "no_softmax", "kv_l2", "matmul_only", "no_kv_staging", "split_keys",
                              "no_q_load", "no_store", "pack", "static_order"]
    assert variant_bits(VARIANTS["matmul_only"]) == 48
    assert variant_bits(VARIANTS["no_kv_staging"]) == 256  # FA2_ABLATE_NO_KV_STAGING
    assert variant_bits(VARIANTS["no_q_load"]) == 1024  # FA2_ABLATE_NO_Q_LOAD
    assert variant_bits(VARIANTS["no_store"]) == 2048  # FA2_ABLATE_NO_STORE
    assert variant_bits(VARIANTS["static_order"]) == 128  # FA2_ABLATE_STATIC_ORDER, host-only
    q = torch.zeros(1, 4, 8, 64, dtype=torch.float16)
    with pytest.raises(AssertionError, match="unknown"):
        attention_ablate(q, q, q, fast=True)
    with pytest.raises(RuntimeError, match="GPU"):
        attention_ablate(q, q, q, no_exp=True)


CAPI_EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "capi", "fa2_capi_check")


@pytest.mark.skipif(not os.path.exists(CAPI_EXE), reason="tests/capi/fa2_capi_check is built by csrc/build.py")
def test_c_host_sees_the_c_abi_errors():
    """The plain-C host (no Python in its process) gets FA2_EINVAL / FA2_EALIGN and the messages
    for rejected arguments, and the policy queries answer; no GPU call is made."""
    import subprocess

    res = subprocess.run([CAPI_EXE, "errors"], capture_output=True, text=True, timeout=60)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "all ok" in res.stdout


def test_split_and_lse_arguments_fail_in_python():
    q = torch.zeros(1, 4, 8, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="num_splits"):
        attention(q, q, q, causal=False, num_splits=0)
    with pytest.raises(ValueError, match="causal"):
        attention(q, q, q, causal=True, num_splits=2)


@needs_lib
def test_c_abi_noalloc_rejects_splits_past_its_scratch():
    """fa2_attn_fwd_noalloc holds FA2_NOALLOC_SCRATCH_BYTES (32 MiB) per GPU: a split-KV launch
    whose partials need more is rejected before any device call (fake pointers here)."""
    arr = lambda s: (ctypes.c_int64 * 4)(*s)  # noqa: E731
    lib = _lib.lib()
    sq = arr((32 * 64 * 128, 64 * 128, 128, 1))
    skv = arr((8 * 4096 * 128, 4096 * 128, 128, 1))
    # B 16, H 32/8, N_q 64, N_kv 4096, 16 splits: 16 x 32768 rows x 128 dims x 4 B = 256 MiB
    assert lib.fa2_workspace_bytes(16, 32, 64, 128, 16) > 32 << 20
    rc = lib.fa2_attn_fwd_noalloc(0x1000, 0x2000, 0x3000, 0x4000, sq, skv, skv, sq, 16, 32, 8, 64,
                                  4096, 128, 0, 0, 1, 128, 0, 0.18, None, 16, None)
    assert rc == -1 and "scratch" in _lib.last_error(), (rc, _lib.last_error())


@needs_lib
def test_build_records_the_resources_of_every_product_instance():
    """csrc/build.py keeps the compiler's resource report of every attn_fwd_kernel instance
    (fa2/kernel_resources.json), and sweep.py finds the instance any tile choice runs."""
    import sweep

    res = sweep.load_resources()
    assert res, "kernel_resources.json missing or empty"
    for dt in (0, 1):
        for d in (16, 32, 64, 128):
            for causal in (False, True):
                for bm in (1, 32, 64, 100, 128, 256):
                    for bn in (16, 32, 64, 128):
                        r = res[sweep.instance_name(dt, d, bm, bn, causal, False)]
                        assert r["vgprs"] > 0 and r["lds_bytes"] > 0 and r["waves_per_simd"] >= 1
                r = res[sweep.instance_name(dt, d, 128, 0 or _default_config(d, True)[1], causal, True)]
                assert r["variant"] == 4


@needs_lib
def test_default_instances_keep_the_occupancy_the_design_counts_on():
    """The compiler's report of the default instances: two waves per SIMD and no VGPR spills at
    head_dim 128 (C2, C3, C5; with and without the key-norm table), three waves per SIMD for the
    fp16 head_dim-64 software-pipelined instances (C4), whose rounded P sum costs a few spilled
    VGPRs (at most 5; tests/test_gpu_determinism.py runs every spilling instance)."""
    import sweep

    res = sweep.load_resources()
    for dt in (0, 1):
        for causal in (False, True):
            for keynorm in (False, True):
                r = res[sweep.instance_name(dt, 128, 128, 64, causal, keynorm)]
                assert r["waves_per_simd"] >= 2 and r["vgpr_spills"] == 0, r
    for keynorm in (False, True):
        r = res[sweep.instance_name(0, 64, 128, 64, False, keynorm)]
        assert r["waves_per_simd"] == 3 and r["vgpr_spills"] <= 5, r


@needs_lib
def test_fa2_installs_as_a_package(tmp_path):
    """`pip install .` puts the drop-in under its reference import name with the built library
    inside, so `from fa2.kernel import
    attention` works without PYTHONPATH edits (setup.cfg maps fa2 to triton-fa2-forward_amd/fa2).
    Installed into a scratch target from a copy of the
    project files (no network: the build backend is the installed setuptools)."""
    import shutil
    import subprocess
    import sys

    src = tmp_path / "src"
    (src / "triton-fa2-forward_amd").mkdir(parents=True)
    shutil.copy(os.path.join(ROOT, "pyproject.toml"), src)
    shutil.copy(os.path.join(ROOT, "setup.cfg"), src)
    shutil.copytree(os.path.join(ROOT, "triton-fa2-forward_amd", "fa2"),
                    src / "triton-fa2-forward_amd" / "fa2",
                    ignore=shutil.ignore_patterns("__pycache__"))
    target = tmp_path / "site"
    res = subprocess.run([sys.executable, "-m", "pip", "install", "--no-build-isolation", "--no-deps",
                          "--no-index", "--quiet", "--target", str(target), str(src)],
                         capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stdout + res.stderr
    assert (target / "fa2" / "libfa2_fwd.so").exists()
    probe = ("import fa2.kernel, fa2._lib as L; print(fa2.kernel.__file__); "
             "print(L.lib().fa2_version().decode())")
    env = {k: v for k, v in os.environ.items() if k != "PYTHONPATH"}
    env["PYTHONPATH"] = str(target)
    res = subprocess.run([sys.executable, "-c", probe], capture_output=True, text=True, timeout=300,
                         cwd=str(tmp_path), env=env)
    assert res.returncode == 0, res.stdout + res.stderr
    kernel_file, version = res.stdout.split("\n")[:2]
    assert kernel_file.startswith(str(target)) and "gfx950" in version


def test_ab_library_suffixes():
    """ab.py's NAME=PATH[@kt|@nt][@bmNNN]: the table mode and the BLOCK_M a build is launched
    with; a path that merely contains '@bm' keeps it."""
    import ab

    assert ab.parse_lib_suffixes("lib.so") == ("lib.so", None, 128)
    assert ab.parse_lib_suffixes("lib.so@kt") == ("lib.so", "kt", 128)
    assert ab.parse_lib_suffixes("lib.so@nt@bm256") == ("lib.so", "nt", 256)
    assert ab.parse_lib_suffixes("v/lib.so@bm64") == ("v/lib.so", None, 64)
    assert ab.parse_lib_suffixes("d@bmx/lib.so") == ("d@bmx/lib.so", None, 128)
