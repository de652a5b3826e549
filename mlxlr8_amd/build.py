"""Build libmoe_mi355x.so (all HIP kernels + the C ABI) in-tree for gfx950.

    python -m mlxlr8_amd.build            # compile every source, always
"""
import os
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libmoe_mi355x.so"
ARCH = os.environ.get("MOE_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Wall", "-Wno-unused-function",
    # packed fp32 vector ops are kept out of generated code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
# Per-source additions.  The fused decode block claims work with single-lane atomics whose result
# it reads late on purpose; the atomic optimizer would rewrite them into wave-wide atomics that
# read the result at once (and so wait for every memory operation issued before them).
FILE_FLAGS = {
    "k4_layer.hip": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"],
}


def sources():
    return sorted(CSRC.glob("*.hip"))


def build(verbose=False):
    """Compile all sources and link the shared library; raises on any compiler error."""
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    with tempfile.TemporaryDirectory(prefix="moe_build_") as tmp:
        objs = []

        def compile_one(src):
            obj = Path(tmp) / (src.stem + ".o")
            cmd = [hipcc, *FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
            r = subprocess.run(cmd, capture_output=True, text=True)
            if r.returncode != 0:
                raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stderr}")
            if verbose and r.stderr.strip():
                print(r.stderr, file=sys.stderr)
            return obj

        with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
            objs = list(ex.map(compile_one, sources()))
        tmp_lib = LIB.with_suffix(".so.tmp")
        cmd = [hipcc, *FLAGS, "-shared", *map(str, objs), "-o", str(tmp_lib)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed:\n{r.stderr}")
        os.replace(tmp_lib, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
