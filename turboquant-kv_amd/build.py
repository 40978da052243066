"""Build the gfx950 kernel library and the torch.ops registration library in-tree.

    python turboquant-kv_amd/build.py          # rebuild both
    python turboquant-kv_amd/build.py --check  # report what is built

Outputs (git-ignored, shipped with the tree):
    turboquant_kv/_lib/libturboquant_hip.so    HIP kernels + the C ABI (include/turboquant_hip.h)
    turboquant_kv/_lib/libturboquant_torch.so  TORCH_LIBRARY(turboquant) -> C ABI

Every HIP source is compiled with hipcc for gfx950 only, with packed-fp32 code
generation disabled.  The .hip files compile in parallel.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "turboquant_kv", "_lib")
OBJDIR = os.path.join(HERE, "_build")
HIP_LIB = os.path.join(LIBDIR, "libturboquant_hip.so")
TORCH_LIB = os.path.join(LIBDIR, "libturboquant_torch.so")

HIP_SOURCES = ["tq_quantize.hip", "tq_scan.hip", "tq_decode.hip", "tq_paged.hip", "tq_prefill.hip",
               "tq_core_tables.hip", "tq_entropy.hip"]
# host C++ of the torch.ops library: the HIP-device ops and the CPU-tensor kernels of the
# reference schemas
TORCH_SOURCES = ["torch_ops.cpp", "cpu_ops.cpp"]
ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # no packed fp32 (v_pk_*_f32) code generation
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                    if "packed-fp32-ops" not in l and "is not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    return out


def _cxx11_abi() -> int:
    import torch
    return int(torch._C._GLIBCXX_USE_CXX11_ABI)


def _torch_paths():
    import torch.utils.cpp_extension as ce
    inc = ce.include_paths()
    libs = ce.library_paths()
    return inc, libs


def build(verbose: bool = False) -> None:
    os.makedirs(LIBDIR, exist_ok=True)
    os.makedirs(OBJDIR, exist_ok=True)
    objs = []
    jobs = []
    with cf.ThreadPoolExecutor(max_workers=4) as ex:
        for src in HIP_SOURCES:
            obj = os.path.join(OBJDIR, src.replace(".hip", ".o"))
            objs.append(obj)
            cmd = [HIPCC, *DEVICE_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
            jobs.append(ex.submit(_run, cmd))
        inc, libs = _torch_paths()
        torch_objs = []
        for src in TORCH_SOURCES:
            obj = os.path.join(OBJDIR, src.replace(".cpp", ".o"))
            torch_objs.append(obj)
            tcmd = [HIPCC, "-O2", "-std=c++17", "-fPIC", "-x", "c++", "-D__HIP_PLATFORM_AMD__=1",
                    "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={_cxx11_abi()}"]
            for i in inc + ["/opt/rocm/include"]:
                tcmd += ["-isystem", i]
            tcmd += ["-c", os.path.join(CSRC, src), "-o", obj]
            jobs.append(ex.submit(_run, tcmd))
        for j in jobs:
            out = j.result()
            if verbose and out.strip():
                print(out)
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", HIP_LIB])
    link = [HIPCC, "-shared", "-fPIC", *torch_objs, "-o", TORCH_LIB, f"-L{LIBDIR}",
            "-lturboquant_hip", "-Wl,-rpath,$ORIGIN"]
    for l in libs:
        link += [f"-L{l}", f"-Wl,-rpath,{l}"]
    link += ["-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch"]
    _run(link)
    if verbose:
        print(f"built {HIP_LIB}\nbuilt {TORCH_LIB}")


def is_built() -> bool:
    return os.path.exists(HIP_LIB) and os.path.exists(TORCH_LIB)


if __name__ == "__main__":
    if "--check" in sys.argv:
        print("built" if is_built() else "not built")
        sys.exit(0 if is_built() else 1)
    build(verbose=True)
