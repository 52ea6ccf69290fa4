"""In-tree build of the native parts of dvattention_amd.

* ``libdvattn_amd.so`` -- the HIP kernels for gfx950 and the C ABI
  (include/dvattn_amd.h), compiled with hipcc; no torch dependency.
* ``_libdvatt.so``     -- the ``torch.ops.libdvatt`` operator registrations
  (csrc/torch_ops.cpp), a thin host-only C++ layer over the C ABI, compiled with
  g++ against the installed torch and linked to ``libdvattn_amd.so``.

Run ``python dvattention_amd/_build.py`` (or ``__graft_entry__.build()``); both load
this file without importing the package, whose import needs the libraries.
Both libraries land next to this file so they travel with the source tree.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(REPO, "include")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = os.environ.get("DVATTN_ARCH", "gfx950")

CAPI_SO = os.path.join(HERE, "libdvattn_amd.so")
TORCH_SO = os.path.join(HERE, "_libdvatt.so")
# measurement-only library: the paged-read probe behind `bench.py --read-ceiling`
PROBE_SO = os.path.join(HERE, "libdvattn_probe.so")

HIP_SOURCES = ["dv_decode.hip", "dv_chunk.hip", "dv_chunk32.hip", "dv_small.hip", "dv_rope.hip", "dv_cache.hip",
               "dv_capi.hip"]

# gfx950 code only; packed-fp32 instructions are disabled (the host pass of
# hipcc warns that it does not know the feature, which is harmless).
HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "-shared",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fvisibility=hidden",
    "-Wno-unused-result",
]


def _run(cmd: list[str]) -> None:
    print("[dvattention_amd build]", " ".join(cmd), flush=True)
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if out.strip():
        print(out, flush=True)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}")


# Per-source code-generation flags.  dv_chunk.hip: each wave keeps 128 fp32
# accumulators plus 64 query-operand registers live across its stage loop;
# with the MFMAs in VGPR form the loop runs without register-file copies,
# where the compiler's default choice moved accumulators between VGPRs and
# AGPRs around every MFMA.
SOURCE_FLAGS = {"dv_chunk.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=true"]}


def build_capi() -> str:
    hipcc = shutil.which("hipcc") or os.path.join(ROCM, "bin", "hipcc")
    srcs = [s for s in HIP_SOURCES if os.path.exists(os.path.join(CSRC, s))]
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    objs = [os.path.join(objdir, src.replace(".hip", ".o")) for src in srcs]
    cmds = [[hipcc, *flags, *SOURCE_FLAGS.get(src, []), f"-I{INCLUDE}", f"-I{CSRC}", "-c",
             os.path.join(CSRC, src), "-o", obj] for src, obj in zip(srcs, objs)]
    # one compiler per source, a few at a time (each takes about 1 GB)
    workers = max(1, min(len(cmds), 4, os.cpu_count() or 1))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        for fut in [pool.submit(_run, c) for c in cmds]:
            fut.result()
    tmp = CAPI_SO + ".tmp"
    _run([hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp])
    os.replace(tmp, CAPI_SO)
    return CAPI_SO


def build_torch_ops() -> str:
    import torch
    from torch.utils import cpp_extension

    inc = cpp_extension.include_paths()
    libdir = os.path.join(os.path.dirname(torch.__file__), "lib")
    cxx = shutil.which("g++") or "g++"
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    tmp = TORCH_SO + ".tmp"
    cmd = [
        cxx, "-O2", "-std=c++17", "-fPIC", "-shared",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        *[f"-I{p}" for p in inc],
        f"-I{os.path.join(ROCM, 'include')}", f"-I{INCLUDE}",
        os.path.join(CSRC, "torch_ops.cpp"),
        "-o", tmp,
        f"-L{libdir}", f"-L{HERE}",
        "-ldvattn_amd", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
        "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{libdir}",
    ]
    _run(cmd)
    os.replace(tmp, TORCH_SO)
    return TORCH_SO


def build_probe() -> str:
    hipcc = shutil.which("hipcc") or os.path.join(ROCM, "bin", "hipcc")
    tmp = PROBE_SO + ".tmp"
    _run([hipcc, *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", os.path.join(CSRC, "dv_probe.hip"), "-o", tmp])
    os.replace(tmp, PROBE_SO)
    return PROBE_SO


def build_all() -> None:
    build_capi()
    build_torch_ops()
    build_probe()


if __name__ == "__main__":
    build_all()
    sys.exit(0)
