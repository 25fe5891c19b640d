"""Build ``libsilogic_hip.so`` in-tree with hipcc for gfx950.

Each ``csrc/*.hip`` file is compiled to an object in parallel, then linked
into ``silogic_amd/lib/libsilogic_hip.so``. Packed-FP32 instruction
selection is disabled (``-packed-fp32-ops``), and no fast-math flag is used,
so fp32 division, ``expf`` and contraction follow IEEE semantics.
"""
import concurrent.futures as cf
import os
import shutil
import subprocess
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIBDIR, "libsilogic_hip.so")
ARCH = os.environ.get("SILOGIC_HIP_ARCH", "gfx950")

FLAGS = ["--offload-arch=" + ARCH, "-O3", "-std=c++17", "-fPIC",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _hipcc():
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def build(verbose=False, jobs=None):
    """Compile every HIP source and link the shared library; return its path."""
    hipcc = _hipcc()
    os.makedirs(LIBDIR, exist_ok=True)
    srcs = sources()
    with tempfile.TemporaryDirectory(prefix="slg_build_") as tmp:
        def compile_one(src):
            obj = os.path.join(tmp, os.path.basename(src)[:-4] + ".o")
            cmd = [hipcc] + FLAGS + ["-c", src, "-o", obj]
            r = subprocess.run(cmd, capture_output=True, text=True)
            if r.returncode != 0:
                raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr[-4000:]}")
            if verbose:
                print("compiled", os.path.basename(src), flush=True)
            return obj

        jobs = jobs or min(len(srcs), os.cpu_count() or 4, 8)
        with cf.ThreadPoolExecutor(jobs) as ex:
            objs = list(ex.map(compile_one, srcs))
        tmp_lib = LIB + ".tmp"
        cmd = [hipcc, "--offload-arch=" + ARCH, "-shared", "-fPIC", "-o", tmp_lib] + objs
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed:\n{r.stderr[-4000:]}")
        os.replace(tmp_lib, LIB)
    if verbose:
        print("built", LIB, flush=True)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
