"""Build libhattn_hip.so in-tree with hipcc for gfx950.

    python log-linear-attention_amd/build_lib.py

Compiles every ``csrc/*.hip`` / ``csrc/*.cpp`` into
``hattention/_native/libhattn_hip.so``.  No torch extension machinery: the
library is a plain C-ABI shared object loaded with ctypes.
"""
import concurrent.futures
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


def _compile_cmd(src: str, obj: str) -> list:
    inc = ["-I", os.path.join(HERE, "..", "include")]
    if src.endswith(".cpp"):
        return [hipcc(), "-c", "-fPIC", "-O2", "-std=c++17", *inc, src, "-o", obj]
    return [hipcc(), "-c", "-fPIC", "-O3", "-std=c++17", f"--offload-arch={ARCH}", *inc,
            *DEVICE_FLAGS, src, "-o", obj]


def build(verbose: bool = False, jobs: int = 0) -> str:
    """Compile every source (in parallel, one hipcc process per file) and link."""
    os.makedirs(OUT_DIR, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))
    tmp = tempfile.mkdtemp(prefix="hattn_build_")
    try:
        objs = [os.path.join(tmp, os.path.basename(src) + ".o") for src in srcs]
        cmds = [_compile_cmd(src, obj) for src, obj in zip(srcs, objs)]
        if verbose:
            for cmd in cmds:
                print(" ".join(cmd), flush=True)
        jobs = jobs or min(len(cmds), max(1, (os.cpu_count() or 1) // 2), 8)
        with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
            results = list(ex.map(lambda c: subprocess.run(c, capture_output=True, text=True), cmds))
        for src, r in zip(srcs, results):
            if r.returncode != 0:
                sys.stderr.write(r.stdout + r.stderr)
                raise RuntimeError(f"compile failed: {src}")
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
