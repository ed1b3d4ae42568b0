"""Build libjasmine_hip.so (gfx950) in-tree with hipcc.

    python jasmine_amd/build.py

Every HIP/C++ source under csrc/ is compiled for gfx950 only, objects go to
jasmine_amd/_build/, the shared library to jasmine_amd/libjasmine_hip.so.
"""
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libjasmine_hip.so")
ARCH = os.environ.get("JAS_OFFLOAD_ARCH", "gfx950")

# Packed-FP32 instructions are disabled for every device compile (the compiler would
# otherwise form v_pk_* from plain float code); hipcc's host pass warns it does not know
# the feature, which is harmless.
HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-parameter", "-Wno-unknown-pragmas",
]


def hipcc():
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found")


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))


def _compile(src):
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    extra = os.environ.get("JAS_EXTRA_CXXFLAGS", "").split()  # e.g. -D tuning switches
    cmd = [hipcc()] + HIPCC_FLAGS + extra + ["-x", "hip", "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (r.stderr or "").splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {os.path.basename(src)}\n{err}")
    return obj, err


def build(verbose=True, jobs=None):
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(8, len(srcs))
    objs = []
    with cf.ThreadPoolExecutor(jobs) as ex:
        for obj, err in ex.map(_compile, srcs):
            objs.append(obj)
            if verbose and err.strip():
                print(err, file=sys.stderr)
    tmp = LIB + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", tmp] + objs + ["-lhiprtc"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stderr)
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources for {ARCH}")
    return LIB


if __name__ == "__main__":
    build()
