"""Build the three gfx950 libraries in-tree (no cmake, no JIT cache).

    python -m grxcp_amd.build        # or grxcp_amd.build.build()

Outputs, next to this file in ``lib/``:

* ``libgrxrt.so``   runtime subset over HIP (grx_runtime.h)
* ``libgrxblas.so`` grxBLAS host library + GEMM / level-1/2 kernels (grxblas.h)
* ``libgrxdnn.so``  grxDNN host library + norm / attention kernels (grxdnn.h)

Host ``.cpp`` files are compiled with g++ against the HIP runtime API headers;
``.hip`` kernel files with ``hipcc --offload-arch=gfx950``. Every HIP
compile line carries ``-Xclang -target-feature -Xclang -packed-fp32-ops`` so
the compiler emits no packed-fp32 VALU instructions.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "lib")
OBJDIR = os.path.join(HERE, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

INCLUDES = ["-I", os.path.join(ROOT, "include"), "-I", CSRC]
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden", f"--offload-arch={ARCH}",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Wall", "-Wno-unused-result"]
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__",
              "-I", os.path.join(ROCM, "include")]

# Per-file extra flags. Attention keeps its MFMA results (scores and O) in
# VGPRs, where the softmax VALU work reads them without AGPR copies.
EXTRA = {
    "kernels/attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}

LIBS = {
    "libgrxrt.so": (["runtime.cpp"], []),
    "libgrxblas.so": (["grxblas.cpp", "kernels/gemm_mfma.hip", "kernels/sgemm.hip",
                       "kernels/noalloc_scratch.hip"], ["grxrt"]),
    "libgrxdnn.so": (["grxdnn.cpp", "kernels/norms.hip", "kernels/softmax_gelu.hip",
                      "kernels/attention.hip"], ["grxrt"]),
}


def _obj(src: str) -> str:
    return os.path.join(OBJDIR, src.replace("/", "_") + ".o")


def _compile(src: str) -> str:
    path = os.path.join(CSRC, src)
    out = _obj(src)
    if src.endswith(".hip"):
        cmd = [HIPCC, *HIP_FLAGS, *EXTRA.get(src, []), *INCLUDES, "-c", path, "-o", out]
    else:
        cmd = ["g++", *HOST_FLAGS, *INCLUDES, "-c", path, "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature name; that
    # warning is expected and harmless.
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return out


def build(verbose: bool = False) -> dict[str, str]:
    """Compile every source and link the three libraries. Always rebuilds."""
    os.makedirs(OBJDIR, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    sources = sorted({s for srcs, _ in LIBS.values() for s in srcs})
    workers = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(workers) as ex:
        list(ex.map(_compile, sources))
    outputs = {}
    for lib, (srcs, deps) in LIBS.items():  # dict order: libgrxrt first
        out = os.path.join(LIBDIR, lib)
        tmp = out + ".tmp"
        cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", tmp,
               *[_obj(s) for s in srcs], "-L", LIBDIR, *[f"-l{d}" for d in deps],
               "-Wl,-rpath,$ORIGIN", "-Wl,--no-undefined"]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stderr}")
        os.replace(tmp, out)
        outputs[lib] = out
        if verbose:
            print(f"built {out}")
    return outputs


if __name__ == "__main__":
    build(verbose=True)
