"""Build libfa2_fwd.so, the gfx950 FlashAttention-2 forward library, in-tree, and the
measurement library libfa2_ablate.so beside it.

    python triton-fa2-forward_amd/csrc/build.py [-j 8] [--verbose]

Compiles attn_fwd_inst.hip once per (dtype, head_dim) pair plus the split-KV combine pass
(attn_fwd_combine.hip), the key-norm pass (attn_key_norm.hip) and the C-ABI file fa2_fwd.hip,
in parallel, with hipcc for gfx950 only, and links them into
triton-fa2-forward_amd/fa2/libfa2_fwd.so next to the Python front end that loads it. Then builds
the plain-C host of the C ABI that the tests run (tests/capi/fa2_capi_check).

The measurement library (include/fa2_ablate.h) is the kernel's timing variants: the same kernel
template with work switched off, compiled from attn_fwd_ablate_inst.hip per pair and linked with
its own C-ABI file fa2_ablate.hip into triton-fa2-forward_amd/libfa2_ablate.so, outside the
fa2 package: the product never loads it. It also holds the MFMA ceiling probe (mfma_ceiling.hip):
what the matrix cores sustain under the chip's power limit.

`--variant NAME -D MACRO=VALUE ...` builds only the product library, with those compile-time
definitions, into triton-fa2-forward_amd/variants/NAME/libfa2_fwd.so (objects under build/): a
second build of the same sources for a same-box A/B against the product (ab.py), e.g. another
FA2_TAIL_PRIVATE_PCT. It never replaces the product library.

Both libraries are built with hidden visibility, so each exports exactly the functions its
header declares (FA2_API). The compiler's resource report for every kernel instance (VGPRs,
AGPRs, SGPRs, spills, LDS, occupancy; -Rpass-analysis=kernel-resource-usage) is saved to
triton-fa2-forward_amd/fa2/kernel_resources.json, which sweep.py prints beside its timings.
"""

import argparse
import json
import os
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

CSRC = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(CSRC)
ROOT = os.path.dirname(PKG)
INCLUDE = os.path.join(ROOT, "include")
OBJ_DIR = os.path.join(PKG, "build", "obj")
LIB_PATH = os.path.join(PKG, "fa2", "libfa2_fwd.so")
ABLATE_LIB_PATH = os.path.join(PKG, "libfa2_ablate.so")
RESOURCES_PATH = os.path.join(PKG, "fa2", "kernel_resources.json")
CAPI_DIR = os.path.join(ROOT, "tests", "capi")

ARCH = "gfx950"
DTYPES = (0, 1)            # 0 = fp16, 1 = bf16
HEAD_DIMS = (16, 32, 64, 128)


def hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the gfx950 build needs ROCm's hipcc")
    return path


def common_flags():
    return [
        f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC", "-fvisibility=hidden",
        # no packed fp32 VALU ops (v_pk_*_f32) anywhere in device code
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", CSRC, "-I", INCLUDE,
    ]


def _run(cmd, verbose):
    """Run one build command; returns its stderr (without the host pass's noise)."""
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the device-only target feature; that warning is noise.
    err = "\n".join(line for line in res.stderr.splitlines() if "packed-fp32-ops" not in line)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    return err


_REMARK = re.compile(r"remark:\s+(Function Name|TotalSGPRs|VGPRs|AGPRs|ScratchSize \[bytes/lane\]|"
                     r"Occupancy \[waves/SIMD\]|SGPRs Spill|VGPRs Spill|LDS Size \[bytes/block\]):"
                     r"\s+(\S+)")
_FIELDS = {"TotalSGPRs": "sgprs", "VGPRs": "vgprs", "AGPRs": "agprs",
           "ScratchSize [bytes/lane]": "scratch_bytes_per_lane", "Occupancy [waves/SIMD]": "waves_per_simd",
           "SGPRs Spill": "sgpr_spills", "VGPRs Spill": "vgpr_spills", "LDS Size [bytes/block]": "lds_bytes"}
_KERNEL = re.compile(r"^_ZN3fa215attn_fwd_kernelILi(\d)ELi(\d+)ELi(\d)ELi(\d+)ELb([01])ELi(\d+)EEEvNS_6ParamsE$")


def parse_resources(stderr):
    """kernel-resource-usage remarks -> {mangled name: {field: int}} for the forward kernel."""
    out, cur = {}, None
    for m in _REMARK.finditer(stderr):
        key, val = m.group(1), m.group(2)
        if key == "Function Name":
            cur = out.setdefault(val, {}) if _KERNEL.match(val) else None
        elif cur is not None:
            cur[_FIELDS[key]] = int(val)
    return out


def describe_instance(name):
    """attn_fwd_kernel<DT, D, NW, BN, CAUSAL, VARIANT> template arguments of a mangled name."""
    m = _KERNEL.match(name)
    dt, d, nw, bn, causal, variant = (int(x) for x in m.groups())
    return {"dtype": ("fp16", "bf16")[dt], "head_dim": d, "waves": nw, "block_m": 32 * nw,
            "block_n": bn, "causal": bool(causal), "variant": variant}


VARIANTS_DIR = os.path.join(PKG, "variants")


def build_variant(name, defines, jobs=8, verbose=False):
    """The product library compiled with extra -D definitions, linked to
    variants/NAME/libfa2_fwd.so. Returns its path."""
    if not re.fullmatch(r"[A-Za-z0-9_.-]+", name):
        raise ValueError(f"variant name {name!r}: letters, digits, '_', '.', '-' only")
    obj_dir = os.path.join(PKG, "build", "variants", name)
    out_dir = os.path.join(VARIANTS_DIR, name)
    os.makedirs(obj_dir, exist_ok=True)
    os.makedirs(out_dir, exist_ok=True)
    cc = hipcc()
    flags = [*common_flags(), *(f"-D{d}" for d in defines)]
    cmds = []
    for dt in DTYPES:
        for d in HEAD_DIMS:
            cmds.append([cc, *flags, f"-DFA2_DT={dt}", f"-DFA2_D={d}", "-c",
                         os.path.join(CSRC, "attn_fwd_inst.hip"), "-o",
                         os.path.join(obj_dir, f"attn_fwd_dt{dt}_d{d}.o")])
    for name_ in ("attn_fwd_combine", "attn_key_norm", "fa2_fwd", "fa2_scratch"):
        cmds.append([cc, *flags, "-c", os.path.join(CSRC, name_ + ".hip"), "-o",
                     os.path.join(obj_dir, name_ + ".o")])
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        list(ex.map(lambda cmd: _run(cmd, verbose), cmds))
    path = os.path.join(out_dir, "libfa2_fwd.so")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", path + ".tmp",
          *(c[-1] for c in cmds)], verbose)
    os.replace(path + ".tmp", path)
    with open(os.path.join(out_dir, "defines.txt"), "w") as f:
        f.write("\n".join(defines) + "\n")
    return path


def build(jobs=8, verbose=False):
    """Compile every kernel instance and link both libraries. Returns the product .so path."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    cc = hipcc()
    units, ablate_units = [], []
    for dt in DTYPES:
        for d in HEAD_DIMS:
            obj = os.path.join(OBJ_DIR, f"attn_fwd_dt{dt}_d{d}.o")
            units.append([cc, *common_flags(), "-Rpass-analysis=kernel-resource-usage",
                          f"-DFA2_DT={dt}", f"-DFA2_D={d}", "-c",
                          os.path.join(CSRC, "attn_fwd_inst.hip"), "-o", obj])
            obj = os.path.join(OBJ_DIR, f"attn_fwd_ablate_dt{dt}_d{d}.o")
            ablate_units.append([cc, *common_flags(), f"-DFA2_DT={dt}", f"-DFA2_D={d}", "-c",
                                 os.path.join(CSRC, "attn_fwd_ablate_inst.hip"), "-o", obj])
    shared = []
    for name in ("attn_fwd_combine", "attn_key_norm"):
        shared.append([cc, *common_flags(), "-c", os.path.join(CSRC, name + ".hip"),
                       "-o", os.path.join(OBJ_DIR, name + ".o")])
    api = [cc, *common_flags(), "-c", os.path.join(CSRC, "fa2_fwd.hip"),
           "-o", os.path.join(OBJ_DIR, "fa2_fwd.o")]
    scratch = [cc, *common_flags(), "-c", os.path.join(CSRC, "fa2_scratch.hip"),
               "-o", os.path.join(OBJ_DIR, "fa2_scratch.o")]
    ablate_api = [cc, *common_flags(), "-c", os.path.join(CSRC, "fa2_ablate.hip"),
                  "-o", os.path.join(OBJ_DIR, "fa2_ablate.o")]
    ceiling = [cc, *common_flags(), "-c", os.path.join(CSRC, "mfma_ceiling.hip"),
               "-o", os.path.join(OBJ_DIR, "mfma_ceiling.o")]
    everything = units + shared + [api, scratch] + ablate_units + [ablate_api, ceiling]
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        errs = list(ex.map(lambda cmd: _run(cmd, verbose), everything))

    resources = {}
    for err in errs[:len(units)]:
        for name, fields in parse_resources(err).items():
            resources[name] = {**describe_instance(name), **fields}
    with open(RESOURCES_PATH + ".tmp", "w") as f:
        json.dump({"arch": ARCH, "source": "hipcc -Rpass-analysis=kernel-resource-usage",
                   "kernels": dict(sorted(resources.items()))}, f, indent=1)
    os.replace(RESOURCES_PATH + ".tmp", RESOURCES_PATH)

    def link(objs, path):
        _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", path + ".tmp", *objs], verbose)
        os.replace(path + ".tmp", path)

    shared_objs = [u[-1] for u in shared]
    link([u[-1] for u in units] + shared_objs + [api[-1], scratch[-1]], LIB_PATH)
    link([u[-1] for u in ablate_units] + shared_objs + [ablate_api[-1], ceiling[-1]],
         ABLATE_LIB_PATH)
    build_capi_check(verbose)
    return LIB_PATH


def build_capi_check(verbose=False):
    """The plain-C host of the C ABI that tests/test_gpu_capi.py runs (tests/capi/), linked
    against the library with a relative rpath so that it runs from any checkout."""
    src = os.path.join(CAPI_DIR, "fa2_capi_check.c")
    out = os.path.join(CAPI_DIR, "fa2_capi_check")
    rocm = os.path.dirname(os.path.dirname(os.path.realpath(hipcc())))
    _run(["gcc", "-std=c99", "-O2", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__",
          "-I", os.path.join(rocm, "include"), "-I", INCLUDE, src, "-o", out + ".tmp",
          "-L", os.path.dirname(LIB_PATH), "-lfa2_fwd", "-L", os.path.join(rocm, "lib"),
          "-lamdhip64", "-lm", "-Wl,-rpath,$ORIGIN/../../triton-fa2-forward_amd/fa2",
          "-Wl,-rpath," + os.path.join(rocm, "lib")], verbose)
    os.replace(out + ".tmp", out)
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("-j", "--jobs", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--variant", default=None, help="build only the product library, with -D, "
                    "into variants/VARIANT/libfa2_fwd.so")
    ap.add_argument("-D", dest="defines", action="append", default=[], metavar="MACRO=VALUE")
    args = ap.parse_args()
    if args.variant:
        print(build_variant(args.variant, args.defines, args.jobs, args.verbose))
    elif args.defines:
        ap.error("-D needs --variant (the product library is always built as shipped)")
    else:
        print(build(args.jobs, args.verbose))


if __name__ == "__main__":
    main()
