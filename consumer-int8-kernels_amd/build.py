"""Build the gfx950 library and the torch op module in-tree.

Outputs (next to the Python package, so they travel with the source tree):
  consumer_int8/libci8_amd.so   -- HIP kernels + the C ABI of include/consumer_int8_amd.h
  consumer_int8/_C.so           -- torch.ops.consumer_int8.* registration (stable ABI)
  consumer_int8/libci8_probe.so -- bench.py's MFMA-loop clock probe (not the drop-in)

Usage: python consumer-int8-kernels_amd/build.py   (or __graft_entry__.build()).
hipcc cross-compiles for gfx950, so this runs on a machine without a GPU.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
CSRC = PKG_ROOT / "csrc"
OUT_DIR = PKG_ROOT / "consumer_int8"
REPO = PKG_ROOT.parent
INCLUDE = REPO / "include"
BUILD_DIR = PKG_ROOT / "_build"

ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")
ARCH = "gfx950"

HIP_SOURCES = ["quantize.hip", "gemm.hip", "gemm_small.hip", "gemm_pp.hip", "gemv.hip", "silu.hip",
               "allspark.hip", "q8block.hip", "gguf_q8.hip", "gemm_grouped.hip", "noalloc.hip", "gemm_bytes.hip"]
HOST_SOURCES = ["abi.cpp"]

# -packed-fp32-ops: keep packed FP32 (v_pk_*_f32) out of the generated code.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _run(cmd: list[str]) -> None:
    result = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    stderr = "\n".join(l for l in result.stderr.splitlines() if noise not in l)
    if result.returncode != 0:
        raise RuntimeError(f"command failed ({result.returncode}): {' '.join(cmd)}\n{stderr}")


# Per-file extra flags. The GEMM's machine scheduler: the default strategy lets the
# register allocator rotate the 224 MFMA accumulators between AGPRs and VGPRs in the
# software-pipelined loop (copies around every MFMA); iterative-minreg keeps every
# accumulator in place.
FILE_FLAGS = {"gemm.hip": ["-mllvm", "-amdgpu-sched-strategy=iterative-minreg"],
              "probe.hip": ["-mllvm", "-amdgpu-sched-strategy=iterative-minreg"]}


def _compile(src: Path, obj: Path) -> Path:
    if src.suffix == ".hip":
        _run([HIPCC, *HIP_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)])
    else:
        _run([HIPCC, "-O2", "-std=c++17", "-fPIC", "-Wall", f"-I{INCLUDE}", f"-I{CSRC}",
              "-D__HIP_PLATFORM_AMD__", f"-I{ROCM / 'include'}", "-x", "c++", "-c", str(src), "-o", str(obj)])
    return obj


def build_library(jobs: int = 8) -> Path:
    BUILD_DIR.mkdir(exist_ok=True)
    sources = [CSRC / s for s in HIP_SOURCES + HOST_SOURCES]
    objects = [BUILD_DIR / (s.stem + ".o") for s in sources]
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        list(pool.map(_compile, sources, objects))
    target = OUT_DIR / "libci8_amd.so"
    tmp = target.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
          *map(str, objects), f"-L{ROCM / 'lib'}", "-lamdhip64",
          f"-Wl,-rpath,{ROCM / 'lib'}", "-Wl,-soname,libci8_amd.so"])
    os.replace(tmp, target)
    return target


def build_probe() -> Path:
    """bench.py's measurement library: the MFMA/HBM probes (probe.hip) and the persistent
    GEMM with clock stamps (probe_pp.hip, built with gemm_pp.hip's flags). It links the
    drop-in library for device_cu_count."""
    BUILD_DIR.mkdir(exist_ok=True)
    objects = [_compile(CSRC / name, BUILD_DIR / (Path(name).stem + ".o"))
               for name in ("probe.hip", "probe_pp.hip")]
    target = OUT_DIR / "libci8_probe.so"
    tmp = target.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects),
          f"-L{OUT_DIR}", "-lci8_amd", "-Wl,-rpath,$ORIGIN",
          f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}",
          "-Wl,-soname,libci8_probe.so"])
    os.replace(tmp, target)
    return target


def build_torch_module() -> Path:
    import torch  # noqa: PLC0415  (only the build needs torch's headers)

    torch_dir = Path(torch.__file__).resolve().parent
    py_include = sysconfig.get_paths()["include"]
    target = OUT_DIR / "_C.so"
    tmp = target.with_suffix(".so.tmp")
    cxx = shutil.which("g++") or "g++"
    _run([cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
          "-DTORCH_STABLE_ONLY", "-DUSE_ROCM", "-DTORCH_TARGET_VERSION=0x020A000000000000",
          f"-I{torch_dir / 'include'}", f"-I{py_include}", f"-I{INCLUDE}",
          str(CSRC / "torch_ops.cpp"), "-o", str(tmp),
          f"-L{OUT_DIR}", "-lci8_amd", "-Wl,-rpath,$ORIGIN",
          f"-L{torch_dir / 'lib'}", "-ltorch_hip", "-ltorch_cpu", "-lc10", f"-Wl,-rpath,{torch_dir / 'lib'}"])
    os.replace(tmp, target)
    return target


def build() -> None:
    build_library()
    build_probe()
    build_torch_module()


if __name__ == "__main__":
    build()
    print("built", OUT_DIR / "libci8_amd.so", OUT_DIR / "_C.so", file=sys.stderr)
