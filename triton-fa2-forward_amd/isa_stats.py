"""Static gfx950 ISA view of the forward kernel: what one K/V tile costs, instruction by instruction
(the counterpart of the reference's bench/sass_stats.py, for this build's own AMD assembly).

    python triton-fa2-forward_amd/isa_stats.py                                # bf16 D128 causal, key-norm
    python triton-fa2-forward_amd/isa_stats.py --dtype fp16 --head-dim 64 --full --variant 0
    python triton-fa2-forward_amd/isa_stats.py --dump kernel.s                # keep the listing

Compiles csrc/attn_fwd_inst.hip for one (dtype, head_dim) pair to gfx950 assembly (hipcc -S,
device only; no GPU needed) with the library's own flags, takes one instance of
attn_fwd_kernel<DT, D, waves, block_n, causal, VARIANT>, and prints:

  * its resources from the code object's metadata (VGPRs, AGPRs, SGPRs, spills, LDS);
  * every loop (a backward branch and the blocks it spans), and for the tile loop (the innermost
    loop with the most MFMAs) each basic block's instructions by class: a tile runs the blocks on its
    common path, while the mask, rescale and log-sum-exp blocks run only on some tiles;
  * per block, a cycle budget: matrix-core cycles (a 32x32x16 MFMA keeps its SIMD's matrix core
    busy for 8 passes of 4 clocks, 32 cycles, at the peak rate) against issue cycles (a wave
    issues at most one instruction every 4 clocks).
"""

import argparse
import collections
import os
import re
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
sys.path.insert(0, CSRC)

# Instruction classes, matched on the mnemonic; first match wins.
CLASSES = (
    ("mfma", re.compile(r"^v_mfma_")),
    ("trans", re.compile(r"^v_(exp|log|rcp|rsq|sqrt|sin|cos)_")),
    ("dot", re.compile(r"^v_dot\d")),
    ("agpr move", re.compile(r"^v_accvgpr_")),
    ("lane move", re.compile(r"^v_(readlane|readfirstlane|writelane|permlane)")),
    ("valu", re.compile(r"^v_")),
    ("lds", re.compile(r"^ds_")),
    ("vmem", re.compile(r"^(buffer|global|flat|scratch)_")),
    ("smem", re.compile(r"^s_(load|buffer_load|memtime|memrealtime|getreg)")),
    ("wait/sync", re.compile(r"^s_(waitcnt|barrier|setprio|nop|sleep)")),
    ("control", re.compile(r"^s_(branch|cbranch|endpgm|setpc|swappc|getpc)")),
    ("salu", re.compile(r"^s_")),
)
LABEL = re.compile(r"^(\.LBB\d+_\d+):")
BRANCH = re.compile(r"^s_(?:branch|cbranch_\w+)\s+(\.LBB\d+_\d+)")
MFMA_CYCLES = 32     # v_mfma_f32_32x32x16_{bf16,f16}: 8 passes of 4 clocks on its SIMD
ISSUE_CYCLES = 4     # one instruction of a wave per 4 clocks


def klass(op):
    return next((name for name, rx in CLASSES if rx.match(op)), "other")


def function_body(asm, name):
    """The instruction and label lines of function `name` in an assembly listing."""
    m = re.search(r"^" + re.escape(name) + r":.*?\n(.*?)^\.Lfunc_end", asm, re.S | re.M)
    if not m:
        raise KeyError(f"{name} is not in the listing")
    return m.group(1)


def parse(body):
    """-> (instructions, labels): instructions as mnemonic strings in order; labels map a block
    label to the index of its first instruction."""
    insts, labels = [], {}
    for line in body.splitlines():
        t = line.strip()
        if not t or t.startswith(";"):
            continue
        m = LABEL.match(t)
        if m:
            labels[m.group(1)] = len(insts)
            continue
        if t.startswith("."):
            continue
        insts.append(t.split(";")[0].strip())
    return insts, labels


def loops(insts, labels):
    """(first, last) instruction indexes of every backward branch's range, innermost first."""
    out = []
    for i, ins in enumerate(insts):
        m = BRANCH.match(ins)
        if m and m.group(1) in labels and labels[m.group(1)] <= i:
            out.append((labels[m.group(1)], i))
    return sorted(out, key=lambda r: r[1] - r[0])


def blocks(insts, labels, first, last):
    """Basic blocks of insts[first..last] as (label, start, end) with end exclusive: a block starts
    at a label and after a branch."""
    starts = sorted({first} | {i for i in labels.values() if first < i <= last}
                    | {i + 1 for i in range(first, last) if BRANCH.match(insts[i])})
    names = {i: n for n, i in labels.items()}
    ends = starts[1:] + [last + 1]
    return [(names.get(s, f"+{s}"), s, e) for s, e in zip(starts, ends) if s < e]


def histogram(insts):
    by_class, by_op = collections.Counter(), collections.Counter()
    for ins in insts:
        op = ins.split()[0]
        by_class[klass(op)] += 1
        by_op[op] += 1
    return by_class, by_op


def budget(by_class):
    """Cycles per tile and wave: the matrix core's, and issue (every instruction of the wave)."""
    n = sum(by_class.values())
    return {"mfma": by_class["mfma"] * MFMA_CYCLES, "issue": n * ISSUE_CYCLES,
            "valu_issue": (by_class["valu"] + by_class["trans"] + by_class["dot"]
                           + by_class["agpr move"] + by_class["lane move"]) * ISSUE_CYCLES}


def metadata(asm, name):
    """Resource fields of kernel `name` from the amdhsa.kernels metadata of a listing."""
    m = re.search(r"\.name:\s+" + re.escape(name) + r"\s*\n", asm)
    if not m:
        return {}
    # the kernel's metadata entry: from the previous '  - ' item start to the next one
    start = asm.rfind("\n  - ", 0, m.start())
    end = asm.find("\n  - ", m.end())
    entry = asm[start:end if end > 0 else len(asm)]
    fields = {}
    for key in ("vgpr_count", "agpr_count", "sgpr_count", "vgpr_spill_count", "sgpr_spill_count",
                "group_segment_fixed_size", "private_segment_fixed_size"):
        f = re.search(r"\." + key + r":\s+(\d+)", entry)
        if f:
            fields[key] = int(f.group(1))
    return fields


def kernel_name(dt, d, waves, block_n, causal, variant):
    return (f"_ZN3fa215attn_fwd_kernelILi{dt}ELi{d}ELi{waves}ELi{block_n}ELb{int(causal)}"
            f"ELi{variant}EEEvNS_6ParamsE")


def compile_listing(dt, d, out_path=None):
    """gfx950 assembly of csrc/attn_fwd_inst.hip for one (dtype, head_dim) pair, with the
    library's flags (csrc/build.py)."""
    import build

    with tempfile.TemporaryDirectory() as tmp:
        path = out_path or os.path.join(tmp, "kernel.s")
        cmd = [build.hipcc(), *build.common_flags(), "--cuda-device-only", "-S",
               f"-DFA2_DT={dt}", f"-DFA2_D={d}", os.path.join(CSRC, "attn_fwd_inst.hip"),
               "-o", path]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed:\n{res.stderr}")
        return open(path).read()


def report(asm, name):
    lines = []
    meta = metadata(asm, name)
    lines.append(f"{name}")
    lines.append("resources: " + ", ".join(f"{k} {v}" for k, v in meta.items()))
    insts, labels = parse(function_body(asm, name))
    lp = loops(insts, labels)
    lines.append(f"{len(insts)} instructions; loops (first-last instruction, MFMAs): " + ", ".join(
        f"{a}-{b} ({sum(1 for i in insts[a:b + 1] if i.startswith('v_mfma'))})" for a, b in lp))
    if not lp:
        return "\n".join(lines), None
    def n_mfma(r):
        return sum(1 for i in insts[r[0]:r[1] + 1] if i.startswith("v_mfma"))

    # The tile loop: the most MFMAs among the innermost loops that hold any. A backward branch
    # from a block placed after the loop (a rare path jumping back) spans more than the loop,
    # and the range it spans holds the loop and the prologue's MFMAs too.
    with_mfma = [r for r in lp if n_mfma(r)]
    innermost = [r for r in with_mfma
                 if not any(o != r and r[0] <= o[0] and o[1] <= r[1] for o in with_mfma)]
    first, last = max(innermost, key=lambda r: (n_mfma(r), r[0] - r[1]))
    lines += ["", f"tile loop: instructions {first}-{last}", "",
              "| block | instructions | mfma | trans | dot | valu | lane move | agpr move | lds | vmem | "
              "salu | wait/sync | control | mfma cycles | issue cycles |",
              "|---|---|---|---|---|---|---|---|---|---|---|---|---|---|---|"]
    per_block = []
    for bname, s, e in blocks(insts, labels, first, last):
        by_class, _ = histogram(insts[s:e])
        per_block.append((bname, by_class))
        b = budget(by_class)
        lines.append(f"| {bname} | {e - s} | " + " | ".join(
            str(by_class[c]) for c in ("mfma", "trans", "dot", "valu", "lane move", "agpr move", "lds",
                                       "vmem", "salu", "wait/sync", "control"))
            + f" | {b['mfma']} | {b['issue']} |")
    total, _ = histogram(insts[first:last + 1])
    core = collections.Counter()
    for _, bc in per_block:
        if bc["mfma"] or bc["trans"] >= 8:
            core.update(bc)
    lines += ["", "whole loop (every block once): " + ", ".join(f"{c} {n}" for c, n in total.most_common()),
              "blocks every tile runs (those with the MFMAs or the exponentials): "
              + ", ".join(f"{c} {n}" for c, n in core.most_common())]
    return "\n".join(lines), (insts, labels, first, last, per_block)


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--dtype", choices=["fp16", "bf16"], default="bf16")
    ap.add_argument("--head-dim", type=int, default=128, choices=[16, 32, 64, 128])
    ap.add_argument("--full", action="store_true", help="the non-causal instance")
    ap.add_argument("--waves", type=int, default=4)
    ap.add_argument("--block-n", type=int, default=None)
    ap.add_argument("--variant", type=int, default=4, help="0: table-free; 4: key-norm (C3's)")
    ap.add_argument("--dump", default=None, help="also keep the listing here")
    args = ap.parse_args()

    import build

    dt = {"fp16": 0, "bf16": 1}[args.dtype]
    bn = args.block_n or (128 if args.head_dim == 16 else 64)
    name = kernel_name(dt, args.head_dim, args.waves, bn, not args.full, args.variant)
    asm = compile_listing(dt, args.head_dim, args.dump)
    text, _ = report(asm, name)
    print(f"hipcc {' '.join(build.common_flags()[:3])} ... --cuda-device-only -S "
          f"-DFA2_DT={dt} -DFA2_D={args.head_dim} csrc/attn_fwd_inst.hip")
    print(text)


if __name__ == "__main__":
    if shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"):
        raise SystemExit("isa_stats.py needs hipcc")
    main()
