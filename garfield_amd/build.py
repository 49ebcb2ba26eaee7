"""Build recipe for libgarfield.so (gfx950) and the garfield_search CLI.

Everything is compiled in-tree with hipcc so the built files travel with the
repository snapshot.  Packed-fp32 instructions are disabled for all device
code (-packed-fp32-ops).  MFMA results are kept in ordinary VGPRs
(-amdgpu-mfma-vgpr-form): the brute-force epilogue reads every accumulator
with VALU compares, and AGPR results would cost one v_accvgpr_read each.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libgarfield.so")
CLI = os.path.join(HERE, "garfield_search")
ARCH = os.environ.get("GF_OFFLOAD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wno-deprecated-declarations", "-I", os.path.join(ROOT, "include"),
]
LIB_SOURCES = ["gf_kernels.hip", "gf_host.cpp", "gf_stream.cpp", "gf_io.cpp", "gf_build.cpp",
               "gf_noalloc.cpp"]
OBJ_DIR = os.path.join(HERE, "_build")


def _run(cmd):
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build(verbose=True):
    os.makedirs(OBJ_DIR, exist_ok=True)
    objs, procs = [], []
    for src in LIB_SOURCES:   # compiled concurrently, one hipcc per source
        obj = os.path.join(OBJ_DIR, os.path.splitext(src)[0] + ".o")
        cmd = [HIPCC, *COMMON, "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
        print("+", " ".join(cmd), flush=True)
        procs.append((cmd, subprocess.Popen(cmd)))
        objs.append(obj)
    failed = [cmd for cmd, pr in procs if pr.wait() != 0]
    if failed:
        raise subprocess.CalledProcessError(1, failed[0])
    tmp = LIB + ".tmp"
    _run([HIPCC, *COMMON, "-shared", *objs, "-o", tmp])
    os.replace(tmp, LIB)
    cli_src = os.path.join(CSRC, "gf_cli.cpp")
    if os.path.exists(cli_src):
        _run([HIPCC, *COMMON, "-x", "hip", cli_src, "-o", CLI, "-L", HERE, "-lgarfield",
              "-Wl,-rpath,$ORIGIN"])
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
