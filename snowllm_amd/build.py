"""Build the gfx950 kernel library (libsnowverify.so) in-tree with hipcc.

Each csrc/*.hip file is compiled to an object in parallel, then linked into one shared
library next to this file. The library links the HIP runtime by soname, so inside a process
that has imported torch it binds to torch's own libamdhip64.
"""
import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OBJ = HERE / "_build"
LIB = HERE / "libsnowverify.so"
ARCH = os.environ.get("SNOWVERIFY_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable", "-Wno-unused-parameter",
    # no packed FP32 instructions (v_pk_fma_f32 and kin): some of their forms have given
    # wrong results on these boxes
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in VGPRs: the k-quant kernels rescale every sub-block product in VALU, and
    # AGPR results would cost a v_accvgpr_read per element first
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    # the first kernel arguments arrive preloaded in SGPRs (gfx940+ kernarg preload) instead of
    # through a scalar load at the start of every kernel: 3.578 -> 3.533 ms per config-4 step
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-munsafe-fp-atomics",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _compile(src: pathlib.Path) -> pathlib.Path:
    obj = OBJ / (src.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", str(CSRC), "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stderr}")
    if r.stderr.strip():
        sys.stderr.write(r.stderr)
    return obj


def build(verbose: bool = True) -> pathlib.Path:
    OBJ.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources for {ARCH}")
    return LIB


if __name__ == "__main__":
    build()
