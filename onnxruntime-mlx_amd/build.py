"""Build the gfx950 kernel library and the execution-provider library in-tree.

    python onnxruntime-mlx_amd/build.py            # everything
    python onnxruntime-mlx_amd/build.py kernels    # libortmi_kernels.so only
    python onnxruntime-mlx_amd/build.py stamps     # the decode program with phase stamps

Outputs go to onnxruntime-mlx_amd/lib/. hipcc cross-compiles for gfx950 without a
GPU, so this runs on any host with ROCm installed.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "lib")
OBJ = os.path.join(HERE, "lib", "obj")
INCLUDE = os.path.normpath(os.path.join(HERE, "..", "include"))
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")

KERNEL_SOURCES = ["runtime.hip", "mnb.hip", "attention.hip", "norm.hip", "decode_step.hip",
                  "gqa_ext.hip"]
EP_SOURCES = ["ep/ep.cpp", "ep/graph.cpp", "ep/fuse.cpp", "ep/plan.cpp"]

HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    # Packed-FP32 VALU forms are kept out of generated code on this target.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", INCLUDE,
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")


def _compile(src: str) -> str:
    os.makedirs(OBJ, exist_ok=True)
    obj = os.path.join(OBJ, src.replace("/", "_") + ".o")
    extra = ["-fvisibility=hidden"] if src.startswith("ep/") else []
    _run([HIPCC, *HIP_FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj])
    return obj


def build_kernels(jobs: int = 4) -> str:
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, KERNEL_SOURCES))
    out = os.path.join(LIB, "libortmi_kernels.so")
    tmp = out + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs,
          "-Wl,-soname,libortmi_kernels.so"])
    os.replace(tmp, out)
    return out


def build_ep(jobs: int = 4) -> str | None:
    srcs = [s for s in EP_SOURCES if os.path.exists(os.path.join(CSRC, s))]
    if not srcs:
        return None
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    out = os.path.join(LIB, "libonnxruntime_mi355x_ep.so")
    tmp = out + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs,
          "-L", LIB, "-lortmi_kernels", "-Wl,-rpath,$ORIGIN",
          "-Wl,-soname,libonnxruntime_mi355x_ep.so",
          # Only the two plugin entry points are exported (the ORT plugin contract).
          "-Wl,--version-script=" + os.path.join(CSRC, "ep", "exports.map")])
    os.replace(tmp, out)
    return out


def build_harness() -> str:
    """The in-repo harness host that drives a plugin EP through the ORT plugin ABI."""
    obj = _compile("host/harness.cpp")
    out = os.path.join(LIB, "libortmi_harness.so")
    tmp = out + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, obj, "-ldl",
          "-Wl,-soname,libortmi_harness.so"])
    os.replace(tmp, out)
    return out


def build_stamps() -> str:
    """The decode program with per-phase timestamps compiled in (-DORTMI_DPROG_STAMPS),
    as a library of its own for dprog_stamps.py; the product libraries never have them."""
    os.makedirs(OBJ, exist_ok=True)
    objs = []
    for src in ("runtime.hip", "decode_step.hip"):
        obj = os.path.join(OBJ, "stamps_" + src + ".o")
        _run([HIPCC, *HIP_FLAGS, "-DORTMI_DPROG_STAMPS", "-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    out = os.path.join(LIB, "libortmi_dprog_stamps.so")
    tmp = out + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs,
          "-Wl,-soname,libortmi_dprog_stamps.so"])
    os.replace(tmp, out)
    return out


def build_all(jobs: int = 4) -> list[str]:
    outs = [build_kernels(jobs)]
    ep = build_ep(jobs)
    if ep:
        outs.append(ep)
    outs.append(build_harness())
    outs.append(build_stamps())
    return outs


if __name__ == "__main__":
    what = sys.argv[1] if len(sys.argv) > 1 else "all"
    if what == "kernels":
        print(build_kernels())
    elif what == "stamps":
        print(build_stamps())
    else:
        for p in build_all():
            print(p)
