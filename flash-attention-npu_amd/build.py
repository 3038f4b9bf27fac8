"""Builds the MI355X FlashAttention libraries in-tree.

  fa_mi355x/lib/libfa_mi355x.so        HIP kernels for gfx950 + the C ABI (include/fa_mi355x.h)
  fa_mi355x/lib/libfa_mi355x_torch.so  torch.ops.fa_mi355x operators over that C ABI
  fa_mi355x/lib/libfa_mi355x_phases.so (only with --phases) the same C ABI with
                                       per-wave real-time stamps in the decode kernel
                                       (FA_DECODE_PHASES), read by bench.py --phases;
                                       never loaded otherwise

Usage: python build.py [--jobs N] [--phases]. hipcc cross-compiles for gfx950,
so this runs on a machine without a GPU.
"""
import argparse
import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "fa_mi355x", "lib")
OBJDIR = os.path.join(HERE, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = os.environ.get("FA_MI355X_ARCH", "gfx950")

HIP_SOURCES = ["fa_fwd.hip", "fa_decode.hip", "fa_kv_prep.hip", "fa_bwd.hip", "fa_api.cpp", "fa_noalloc.hip"]
HIPFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # no packed fp32 ops (v_pk_*_f32) in any generated code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(REPO, "include"),
]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    return out


# Per-source LLVM scheduler choice. The prefill kernels (fa_fwd.hip) are
# scheduled with max-memory-clause: the c4 prefill kernel measured 919-922 us
# against 928-929 us with the default strategy (same box, alternating runs;
# 954 vs 962 us on a second box), max-ilp 977 us, iterative-ilp 1021 us.
# Decode and the backward are faster with the default (max-memory-clause / max-ilp
# were +1-2 % on c2 / c3 decode and +6 % on the backward).
SRC_FLAGS = {
    "fa_fwd.hip": ["-mllvm", "-amdgpu-sched-strategy=max-memory-clause"],
}


def _compile_hip(src, defines=(), tag=""):
    obj = os.path.join(OBJDIR, os.path.basename(src) + tag + ".o")
    cmd = ([HIPCC] + HIPFLAGS + SRC_FLAGS.get(os.path.basename(src), []) + [f"-D{d}" for d in defines]
           + ["-c", os.path.join(CSRC, src), "-o", obj])
    _run(cmd)
    return obj


def _torch_flags():
    import torch
    import torch.utils.cpp_extension as ce
    inc = ce.include_paths()
    libs = ce.library_paths()
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cflags = ["-O2", "-std=c++17", "-fPIC", f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__=1",
              "-DUSE_ROCM=1", "-I", os.path.join(ROCM, "include"), "-I", sysconfig.get_paths()["include"]]
    for i in inc:
        cflags += ["-I", i]
    ldflags = []
    for l in libs:
        ldflags += ["-L", l, f"-Wl,-rpath,{l}"]
    ldflags += ["-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
                "-L", os.path.join(ROCM, "lib"), f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}", "-lamdhip64"]
    return cflags, ldflags


def build(jobs=8, verbose=True, phases=False):
    os.makedirs(LIBDIR, exist_ok=True)
    os.makedirs(OBJDIR, exist_ok=True)
    cflags, ldflags = _torch_flags()
    torch_obj = os.path.join(OBJDIR, "fa_torch_ops.o")
    torch_cmd = ["g++"] + cflags + ["-c", os.path.join(CSRC, "torch_ext", "fa_torch_ops.cpp"), "-o", torch_obj]
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        futs = [ex.submit(_compile_hip, s) for s in HIP_SOURCES]
        pfut = ex.submit(_compile_hip, "fa_decode.hip", ("FA_DECODE_PHASES",), ".phases") if phases else None
        tfut = ex.submit(_run, torch_cmd)
        objs = [f.result() for f in futs]
        pobj = pfut.result() if phases else None
        tfut.result()
    core = os.path.join(LIBDIR, "libfa_mi355x.so")
    tmp = core + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined", "-o", tmp] + objs)
    os.replace(tmp, core)
    if phases:
        plib = os.path.join(LIBDIR, "libfa_mi355x_phases.so")
        pobjs = [pobj if os.path.basename(o) == "fa_decode.hip.o" else o for o in objs]
        # -Bsymbolic: the instrumented library binds its own kernels even beside the product library
        _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined", "-Wl,-Bsymbolic", "-o",
              plib + ".tmp"] + pobjs)
        os.replace(plib + ".tmp", plib)
    tlib = os.path.join(LIBDIR, "libfa_mi355x_torch.so")
    tmp = tlib + ".tmp"
    _run(["g++", "-shared", "-o", tmp, torch_obj, "-L", LIBDIR, "-lfa_mi355x", "-Wl,-rpath,$ORIGIN"] + ldflags)
    os.replace(tmp, tlib)
    if verbose:
        print(f"built {core}\nbuilt {tlib}")
    return core, tlib


def clean():
    shutil.rmtree(OBJDIR, ignore_errors=True)
    shutil.rmtree(LIBDIR, ignore_errors=True)


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=8)
    ap.add_argument("--clean", action="store_true")
    ap.add_argument("--phases", action="store_true",
                    help="also build libfa_mi355x_phases.so (decode kernel with per-wave stamps, bench.py --phases)")
    args = ap.parse_args()
    if args.clean:
        clean()
    build(args.jobs, phases=args.phases)
    sys.exit(0)
