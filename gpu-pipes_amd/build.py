"""Build the gfx950 library (libgpipes.so) and the CPU oracle (liboracle.so).

Both are compiled in-tree so the shared objects travel with the source tree:
  gpu-pipes_amd/gpipes/libgpipes.so   HIP kernels + C ABI (include/gpipes.h)
  gpu-pipes_amd/gpipes/libgpipes_phase.so  the same with the fused MGN kernels'
                                      phase timers compiled in (diagnostics:
                                      bench.py --phase-timers)
  oracle/liboracle.so                 CPU restatement used only by tests/bench
  gpu-pipes_amd/apps/mgn_mlp_cc       C++ driver of the operator (links libgpipes.so)

Usage: python gpu-pipes_amd/build.py [--verbose]
"""
import concurrent.futures as cf
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "gpipes", "libgpipes.so")
PHASE_LIB = os.path.join(PKG, "gpipes", "libgpipes_phase.so")
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_LIB = os.path.join(ORACLE_DIR, "liboracle.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # keep packed-fp32 VALU forms out of the generated code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]
# MFMA accumulators in VGPRs: the AGPR file holds the resident weights of the
# MLP kernels.  The wide GEMM and the fused NeRF kernel keep their 256
# accumulators in AGPRs instead.
VGPR_FORM = ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]

SOURCES = ["mgn_fused.hip", "mgn_pipelined.hip", "stages.hip", "gemm.hip", "nerf_fused.hip", "dlrm_fused.hip", "status.hip",
           "bert_addln_pipelined.hip", "bert_ffn_pipelined.hip", "nerf_a_pipelined.hip", "probe.hip", "synth.hip", "capi.cpp", "ffn.cpp", "mlp.cpp", "arena.cpp"]
SOURCE_FLAGS = {"gemm.hip": [], "nerf_fused.hip": [], "dlrm_fused.hip": []}


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}")
    # hipcc's host pass does not know the packed-fp32 feature flag: drop that noise
    noise = ("packed-fp32-ops", "not a recognized feature", "warning generated")
    out = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if l and not any(n in l for n in noise))
    if verbose and out.strip():
        print(out)


def build_library(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    objs = []
    jobs = []
    for src in SOURCES:
        path = os.path.join(CSRC, src)
        obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
        objs.append(obj)
        lang = ["-x", "hip"] if src.endswith(".hip") else []
        extra = SOURCE_FLAGS.get(src, VGPR_FORM)
        jobs.append([HIPCC] + HIP_FLAGS + extra + lang + ["-c", path, "-o", obj])
    # the diagnostic build's fused MGN object, with the phase timers
    phase_obj = os.path.join(BUILD, "mgn_fused_phase.o")
    jobs.append([HIPCC] + HIP_FLAGS + VGPR_FORM + ["-DGP_PHASE_TIMERS", "-x", "hip", "-c",
                                                   os.path.join(CSRC, "mgn_fused.hip"), "-o", phase_obj])
    with cf.ThreadPoolExecutor(max_workers=min(len(jobs), 8)) as ex:
        list(ex.map(lambda c: _run(c, verbose), jobs))
    for lib, lib_objs in ((LIB, objs), (PHASE_LIB, [phase_obj if o.endswith("mgn_fused.o") else o for o in objs])):
        tmp = lib + ".tmp"
        # --no-undefined: a kernel whose host stub was not emitted fails here, not at load time
        _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined", "-o", tmp] + lib_objs,
             verbose)
        os.replace(tmp, lib)
    return LIB


def build_oracle(verbose=False):
    # x86-64-v3 (AVX2 + FMA) runs on any current server host; OpenMP over rows.
    # synth.c (the input generator) without contraction: each of its steps
    # must round as in the device generator.
    tmp = ORACLE_LIB + ".tmp"
    os.makedirs(BUILD, exist_ok=True)
    objs = []
    for src, extra in (("oracle.c", []), ("synth.c", ["-ffp-contract=off"])):
        obj = os.path.join(BUILD, "oracle_" + os.path.splitext(src)[0] + ".o")
        _run(["gcc", "-O3", "-march=x86-64-v3", "-fopenmp", "-fPIC"] + extra +
             ["-c", os.path.join(ORACLE_DIR, src), "-o", obj], verbose)
        objs.append(obj)
    _run(["gcc", "-fopenmp", "-shared"] + objs + ["-o", tmp, "-lm"], verbose)
    os.replace(tmp, ORACLE_LIB)
    return ORACLE_LIB


APPS = ["mgn_mlp_cc"]


def build_apps(verbose=False):
    outs = []
    for app in APPS:
        exe = os.path.join(PKG, "apps", app)
        _run([HIPCC, "-O2", "-std=c++17", os.path.join(PKG, "apps", app + ".cpp"), "-o", exe + ".tmp",
              "-L" + os.path.dirname(LIB), "-lgpipes", "-Wl,-rpath,$ORIGIN/../gpipes"], verbose)
        os.replace(exe + ".tmp", exe)
        outs.append(exe)
    return outs


def build(verbose=False):
    lib = build_library(verbose)
    return lib, build_oracle(verbose), build_apps(verbose)


if __name__ == "__main__":
    print(build(verbose="--verbose" in sys.argv))
