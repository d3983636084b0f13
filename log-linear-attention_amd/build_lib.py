"""Build libhattn_hip.so in-tree with hipcc for gfx950.

    python log-linear-attention_amd/build_lib.py

Compiles every ``csrc/*.hip`` / ``csrc/*.cpp`` into
``hattention/_native/libhattn_hip.so``.  No torch extension machinery: the
library is a plain C-ABI shared object loaded with ctypes.
"""
import glob
import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "hattention", "_native")
OUT = os.path.join(OUT_DIR, "libhattn_hip.so")
ARCH = "gfx950"

# Packed-fp32 instructions are disabled for all device code on this pool.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def build(verbose: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))
    objs = []
    tmp = tempfile.mkdtemp(prefix="hattn_build_")
    try:
        for src in srcs:
            obj = os.path.join(tmp, os.path.basename(src) + ".o")
            cmd = [hipcc(), "-c", "-fPIC", "-O3", "-std=c++17", f"--offload-arch={ARCH}",
                   "-I", os.path.join(HERE, "..", "include"), *DEVICE_FLAGS, src, "-o", obj]
            if src.endswith(".cpp"):
                cmd = [hipcc(), "-c", "-fPIC", "-O2", "-std=c++17",
                       "-I", os.path.join(HERE, "..", "include"), src, "-o", obj]
            if verbose:
                print(" ".join(cmd), flush=True)
            r = subprocess.run(cmd, capture_output=True, text=True)
            if r.returncode != 0:
                sys.stderr.write(r.stdout + r.stderr)
                raise RuntimeError(f"compile failed: {src}")
            objs.append(obj)
        tmp_out = OUT + ".tmp"
        cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp_out]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            sys.stderr.write(r.stdout + r.stderr)
            raise RuntimeError("link failed")
        os.replace(tmp_out, OUT)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
