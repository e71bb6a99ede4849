"""triton-fa2-forward_amd/isa_stats.py, the static gfx950 ISA view of the kernel (the counterpart of
the reference's bench/sass_stats.py and its tests, tests/test_sass_stats.py:25-48): the parser on a
hand-written listing, then the product's C3 instance compiled here (hipcc, no GPU)."""

import os
import shutil

import pytest

from isa_stats import (blocks, budget, compile_listing, function_body, histogram, kernel_name, klass,
                       loops, metadata, parse, report)

LISTING = """\t.text
_kern:                                  ; @_kern
; %bb.0:
\ts_load_dwordx4 s[0:3], s[4:5], 0x0
\tv_mov_b32_e32 v1, 0
.LBB0_1:                                ; =>This Inner Loop Header: Depth=1
\tds_read_b128 v[2:5], v1
\ts_waitcnt lgkmcnt(0)
\tv_mfma_f32_32x32x16_bf16 v[8:23], v[2:5], v[6:9], v[8:23]
\tv_fma_f32 v24, v8, s6, -v25
\tv_exp_f32_e32 v24, v24
\tv_dot2c_f32_bf16_e32 v26, v27, v28
\tbuffer_load_dwordx4 v29, s[0:3], 0 offen lds
\ts_barrier
\ts_cbranch_scc1 .LBB0_3
; %bb.2:
\tv_accvgpr_read_b32 v30, a0
\ts_add_i32 s7, s7, 1
.LBB0_3:
\ts_cmp_lt_i32 s7, s8
\ts_cbranch_scc1 .LBB0_1
\ts_endpgm
.Lfunc_end0:
\t.size\t_kern, .Lfunc_end0-_kern
"""


def test_mnemonic_classes():
    assert [klass(op) for op in ("v_mfma_f32_32x32x16_bf16", "v_exp_f32_e32", "v_dot2c_f32_bf16_e32",
                                 "v_accvgpr_read_b32", "v_permlane32_swap_b32_e32", "v_fma_f32",
                                 "ds_read_b64_tr_b16", "buffer_load_dwordx4", "s_load_dwordx4",
                                 "s_waitcnt", "s_cbranch_scc1", "s_add_i32")] == \
        ["mfma", "trans", "dot", "agpr move", "lane move", "valu", "lds", "vmem", "smem",
         "wait/sync", "control", "salu"]


def test_loops_are_backward_branches_and_blocks_split_at_labels_and_branches():
    insts, labels = parse(function_body(LISTING, "_kern"))
    assert len(insts) == 16 and labels == {".LBB0_1": 2, ".LBB0_3": 13}
    assert loops(insts, labels) == [(2, 14)]                  # the forward branch is no loop
    assert [(n, s, e) for n, s, e in blocks(insts, labels, 2, 14)] == \
        [(".LBB0_1", 2, 11), ("+11", 11, 13), (".LBB0_3", 13, 15)]


def test_histogram_and_budget():
    insts, labels = parse(function_body(LISTING, "_kern"))
    by_class, by_op = histogram(insts[2:10])
    assert by_class["mfma"] == 1 and by_class["trans"] == 1 and by_class["dot"] == 1
    assert by_class["lds"] == 1 and by_class["vmem"] == 1 and by_class["wait/sync"] == 2
    assert by_op["v_fma_f32"] == 1
    assert budget(by_class) == {"mfma": 32, "issue": 32, "valu_issue": 12}


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="hipcc not installed")
def test_c3_instance_tile_loop_and_resources():
    """The instance C3 runs (bf16, head_dim 128, 4 waves, 64-key tiles, causal, key-norm): at most
    256 VGPRs and no VGPR spills (two waves per SIMD), 64 KiB of LDS (two K/V buffer pairs) and
    the dynamic tail's ticket (one int, padded to 16 bytes), so that two workgroups fit a CU; its
    tile loop holds the tile's 32 MFMAs (16 for S, 16 for PV), one exp2 per score and lane
    register (32) plus the rescale factor, and the rounded-P row sum's 16 dot2 instructions."""
    asm = compile_listing(1, 128)
    name = kernel_name(1, 128, 4, 64, True, 4)
    meta = metadata(asm, name)
    assert meta["vgpr_count"] <= 256 and meta["vgpr_spill_count"] == 0, meta
    assert meta["group_segment_fixed_size"] == 65536 + 16, meta
    text, (insts, labels, first, last, per_block) = report(asm, name)
    total, _ = histogram(insts[first:last + 1])
    assert total["mfma"] == 32 and total["trans"] == 33 and total["dot"] == 16, total
    with_mfma = [bc for _, bc in per_block if bc["mfma"]]
    assert sorted(bc["mfma"] for bc in with_mfma) == [16, 16]
    assert "tile loop" in text


def test_the_tile_loop_is_the_innermost_loop_with_mfmas():
    """A rare block placed after the loop that branches back to an earlier label makes a backward
    branch spanning the loop and the MFMAs before it; the tile loop is still the inner one."""
    listing = LISTING.replace("\ts_endpgm\n", "\ts_cbranch_execz .LBB0_9\n\ts_endpgm\n.LBB0_9:\n"
                              "\tv_mov_b32_e32 v1, 1\n\ts_branch .LBB0_0\n").replace(
        "; %bb.0:\n", "; %bb.0:\n.LBB0_0:\n\tv_mfma_f32_32x32x16_bf16 v[8:23], v[2:5], v[6:9], v[8:23]\n")
    insts, labels = parse(function_body(listing, "_kern"))
    spans = loops(insts, labels)
    assert len(spans) == 2 and spans[0] == (labels[".LBB0_1"], labels[".LBB0_3"] + 1)
    text, (_, _, first, last, _) = report(listing, "_kern")
    assert (first, last) == spans[0], text


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="hipcc not installed")
def test_c4_instance_pipelined_tile_loop():
    """The instance C4 runs (fp16, head_dim 64, 64-key tiles, full attention, key-norm): the
    pipelined loop holds two tiles per trip, so its tile loop has 2 x 16 MFMAs, 2 x 32 exp2 plus
    the rescale factor and 2 x 16 dot2 (the rounded-P sum), at three waves per SIMD (168 VGPRs)."""
    asm = compile_listing(0, 64)
    name = kernel_name(0, 64, 4, 64, False, 4)
    meta = metadata(asm, name)
    assert meta["vgpr_count"] <= 168, meta
    text, (insts, labels, first, last, per_block) = report(asm, name)
    total, _ = histogram(insts[first:last + 1])
    assert total["mfma"] == 32 and total["trans"] == 65 and total["dot"] == 32, (total, text)
