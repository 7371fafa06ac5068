"""Build libhymoe.so (the HIP kernels and the C ABI) in-tree for gfx950.

    python -m hyper_amd.build            # compile every source, link hyper_amd/libhymoe.so
    python -m hyper_amd.build --stamps   # the same with -DHY_STAMPS: hyper_amd/libhymoe_stamps.so, whose decode
                                         # kernels record per-block phase times (python bench.py --timeline NAME ...)

Flags every HIP source is compiled with:
  -ffp-contract=off                           every fp32 product/sum is rounded on its own unless the
                                              source calls fmaf (the numeric contract with the CPU oracle)
  -fhip-fp32-correctly-rounded-divide-sqrt    IEEE division (the quantizers' -127/max, 1/iscale, softmax)
  -Xclang -target-feature -Xclang -packed-fp32-ops   no packed-fp32 VALU instructions
  -mllvm -amdgpu-mfma-vgpr-form               MFMA results in VGPRs (the integer scaling reads them next)
"""
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT = PKG / "libhymoe.so"
OUT_STAMPS = PKG / "libhymoe_stamps.so"
BUILD = PKG / "_build"

SOURCES = ["hy_route.hip", "hy_gemv.hip", "hy_gemm.hip", "hy_decode.hip", "hy_capi.cpp", "hy_step.cpp", "hy_gguf.cpp"]
ARCH = os.environ.get("HYMOE_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
FLAGS = [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
         "-fhip-fp32-correctly-rounded-divide-sqrt", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-mllvm", "-amdgpu-mfma-vgpr-form",
         "-Wall", "-Wno-unused-function", "-Wno-unused-variable", "-I", str(PKG.parent / "include")]


def _compile(src: str, stamps: bool = False) -> Path:
    obj = BUILD / (Path(src).stem + ("_stamps.o" if stamps else ".o"))
    cmd = [HIPCC, *FLAGS, *(["-DHY_STAMPS"] if stamps else []), "-c", str(CSRC / src), "-o", str(obj)]
    if src.endswith(".cpp"):
        cmd[1:1] = ["-x", "hip"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "not a recognized feature for this target"
    err = "\n".join(l for l in (r.stderr or "").splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def build(verbose: bool = False, stamps: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    out = OUT_STAMPS if stamps else OUT
    with ThreadPoolExecutor(max_workers=min(4, len(SOURCES))) as ex:
        objs = list(ex.map(lambda src: _compile(src, stamps), SOURCES))
    tmp = out.with_suffix(".so.tmp")
    r = subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    build(verbose=True, stamps="--stamps" in sys.argv[1:])
