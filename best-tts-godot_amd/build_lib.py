"""Build recipe for libkk.so (HIP, gfx950).

Compiles every ``csrc/*.hip`` with hipcc in parallel into ``_build/`` and
links ``libkk.so`` next to this file, so the library travels with the source
tree.  Run ``python build_lib.py`` or call :func:`build`.
"""
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libkk.so")

ARCH = os.environ.get("KK_OFFLOAD_ARCH", "gfx950")

# -ffp-contract=off keeps a*b+c as two roundings, as numpy computes it;
# packed-fp32 instructions are disabled on purpose (hipcc's host pass warns
# that it does not know the feature, which is harmless).
HIPFLAGS = [
    "-std=c++17", "-O3", f"--offload-arch={ARCH}", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument", f"-I{INCLUDE}", f"-I{CSRC}",
]


def _hipcc():
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(exe):
        raise RuntimeError("hipcc not found: libkk needs ROCm's hipcc to build")
    return exe


def _compile(src):
    """Compiles one source; returns (object path, [kernels that spill])."""
    obj = os.path.join(BUILD, os.path.basename(src).replace(".hip", ".o"))
    cmd = [_hipcc(), *HIPFLAGS, "-Rpass-analysis=kernel-resource-usage", "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{res.stderr}")
    spills, name = [], None
    for line in res.stderr.splitlines():
        if "Function Name:" in line:
            name = line.split("Function Name:")[1].split("[")[0].strip()
        elif "ScratchSize [bytes/lane]:" in line:
            size = int(line.split("ScratchSize [bytes/lane]:")[1].split("[")[0])
            if size:
                spills.append(f"{name} ({size} B/lane)")
    return obj, spills


def build(verbose=False):
    """Compile and link libkk.so; returns its path.  Always rebuilds."""
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    workers = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(workers) as ex:
        done = list(ex.map(_compile, srcs))
    objs = [o for o, _ in done]
    # A kernel with private (scratch) memory spills registers to memory:
    # every kernel here is meant to fit, so say which one does not.
    spills = [k for _, ks in done for k in ks]
    if spills:
        print("libkk: kernels using scratch memory: " + ", ".join(spills), file=sys.stderr)
    tmp = LIB + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link of libkk.so failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
