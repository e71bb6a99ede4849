"""Build libfa2_fwd.so, the gfx950 FlashAttention-2 forward library, in-tree.

    python triton-fa2-forward_amd/csrc/build.py [-j 8] [--verbose]

Compiles attn_fwd_inst.hip once per (dtype, head_dim) pair plus the split-KV combine pass
(attn_fwd_combine.hip), the key-norm pass (attn_key_norm.hip) and the C-ABI file fa2_fwd.hip,
in parallel, with hipcc for gfx950 only, and links them into
triton-fa2-forward_amd/fa2/libfa2_fwd.so next to the Python front end that loads it. Then builds
the plain-C host of the C ABI that the tests run (tests/capi/fa2_capi_check).
"""

import argparse
import os
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
        f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC",
        # no packed fp32 VALU ops (v_pk_*_f32) anywhere in device code
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", CSRC, "-I", INCLUDE,
    ]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the device-only target feature; that warning is noise.
    err = "\n".join(line for line in res.stderr.splitlines() if "packed-fp32-ops" not in line)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(jobs=8, verbose=False):
    """Compile every kernel instance and link the library. Returns the .so path."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    cc = hipcc()
    units = []
    for dt in DTYPES:
        for d in HEAD_DIMS:
            obj = os.path.join(OBJ_DIR, f"attn_fwd_dt{dt}_d{d}.o")
            units.append([cc, *common_flags(), f"-DFA2_DT={dt}", f"-DFA2_D={d}", "-c",
                          os.path.join(CSRC, "attn_fwd_inst.hip"), "-o", obj])
    for name in ("attn_fwd_combine", "attn_key_norm", "fa2_fwd"):
        units.append([cc, *common_flags(), "-c", os.path.join(CSRC, name + ".hip"),
                      "-o", os.path.join(OBJ_DIR, name + ".o")])
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        list(ex.map(lambda cmd: _run(cmd, verbose), units))
    objs = [u[-1] for u in units]
    tmp = LIB_PATH + ".tmp"
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], verbose)
    os.replace(tmp, LIB_PATH)
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
    args = ap.parse_args()
    print(build(args.jobs, args.verbose))


if __name__ == "__main__":
    main()
