"""Build recipe for libg2ptq_hip.so (hipcc, gfx950 only).

``python -m g2ptq_amd.build`` compiles every ``csrc/*.hip`` translation unit
for gfx950 and links them into ``g2ptq_amd/libg2ptq_hip.so`` in-tree, so the
library travels with the source tree, then builds ``csrc/fastcall.c`` (gcc)
into the CPython module ``g2ptq_amd/_fastcall`` beside it.
"""
import concurrent.futures
import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libg2ptq_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Packed-fp32 VALU ops are disabled for every translation unit.
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-fno-gpu-rdc",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable", "-Wno-unused-but-set-variable",
]


# Per-file extra flags.  The quantize / sweep kernels must round every product
# and sum separately (the reference's torch ops never fuse); the flag also
# covers the HIP header's __f*_rn helpers, which a source-level pragma cannot.
EXTRA = {"quant.hip": ["-ffp-contract=off"], "calib.hip": ["-ffp-contract=off"]}


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src):
    obj = os.path.join(BUILD, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *FLAGS, *EXTRA.get(os.path.basename(src), []), "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    return obj, err


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    jobs = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
        results = list(ex.map(_compile, srcs))
    for _, err in results:
        if err.strip() and verbose:
            print(err, file=sys.stderr)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *[o for o, _ in results]]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    build_fastcall()
    return LIB


def build_fastcall():
    """The CPython fast-call module (csrc/fastcall.c) beside the library: gcc,
    linked against libg2ptq_hip.so and resolving it next to itself."""
    ext = os.path.join(HERE, "_fastcall" + sysconfig.get_config_var("EXT_SUFFIX"))
    tmp = ext + ".tmp"
    cmd = ["gcc", "-O2", "-std=c11", "-shared", "-fPIC", "-Wall",
           "-I", sysconfig.get_paths()["include"], os.path.join(CSRC, "fastcall.c"),
           "-L", HERE, "-lg2ptq_hip", "-Wl,-rpath,$ORIGIN", "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"gcc failed for fastcall.c:\n{res.stderr}")
    os.replace(tmp, ext)
    return ext


if __name__ == "__main__":
    print(build(verbose=True))
