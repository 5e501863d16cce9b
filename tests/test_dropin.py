"""The drop-in boundary, as a C/C++ caller sees it, checked on the CPU.

* the reference's own grxBLAS callers -- its three library gates and its cycle
  benchmark (ref tests/libs/test_grxblas.cpp, test_grxblas_ex.cpp,
  test_grxblas_l12.cpp, tests/bench/gemm_cycles.cpp) -- compile unchanged
  against include/ and link against grxcp_amd/lib. They are read in place
  from /root/reference (never copied); without it these cases skip;
* a C99 translation unit that includes every public header compiles with
  -pedantic-errors and links every declared function;
* the CPU host backend (oracle/libgrxblas_ref.so + libgrxrt_ref.so, the
  "host/mock reference backend" BASELINE config 1 runs on) passes the
  reference's three library gates, runs config 1 (fp32 SGEMM 512^3) through
  grxblasSgemm within 1e-4 of numpy float64, and refuses bad arguments with
  the same status as the GPU library.
"""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

import grxcp_amd as g
import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")
REF = O.REF_ROOT
CALLERS = {
    "test_grxblas": "tests/libs/test_grxblas.cpp",
    "test_grxblas_ex": "tests/libs/test_grxblas_ex.cpp",
    "test_grxblas_l12": "tests/libs/test_grxblas_l12.cpp",
    "gemm_cycles": "tests/bench/gemm_cycles.cpp",
}
HOST_GATES = ["test_grxblas", "test_grxblas_ex", "test_grxblas_l12"]
needs_ref = pytest.mark.skipif(not os.path.isdir(REF), reason="/root/reference is not on this machine")


def _link_flags():
    return ["-L", g.LIBDIR, f"-Wl,-rpath,{g.LIBDIR}"]


@needs_ref
@pytest.mark.parametrize("name", sorted(CALLERS))
def test_reference_caller_compiles_and_links_unchanged(tmp_path, name):
    src = os.path.join(REF, CALLERS[name])
    text = open(src).read()
    assert "#include <grx/grx.h>" in text and "#include <grx/grxblas.h>" in text
    out = tmp_path / name
    r = subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", src, "-I", INCLUDE, *_link_flags(),
                        "-lgrxblas", "-lgrxrt", "-o", str(out)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    assert out.exists()


def _declared(header):
    text = open(os.path.join(INCLUDE, "grx", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted({n for n in re.findall(r"\b(grx\w+)\s*\(", text)
                   if not n.startswith("grxCycleSummarize")})


def test_c99_caller_includes_every_header_and_links_every_function(tmp_path):
    names = _declared("grx_runtime.h") + _declared("grxblas.h") + _declared("grxdnn.h")
    assert len(names) > 40
    table = ",\n  ".join(f"(fn)&{n}" for n in names)
    src = tmp_path / "caller.c"
    src.write_text(f"""
#include <grx/grx.h>
#include <grx/grxblas.h>
#include <grx/grxdnn.h>
#include <grx/grx_cycles.h>
#include <stdio.h>
typedef void (*fn)(void);
static const fn every[] = {{
  {table}
}};
int main(void) {{
  grxblasHandle_t h = NULL;
  grxdnnHandle_t d = NULL;
  grxCycleSlot slot = {{0}};
  if (grxblasCreate(&h) != GRXBLAS_STATUS_SUCCESS) return 2;
  if (grxdnnCreate(&d) != GRXDNN_STATUS_SUCCESS) return 3;
  if (slot.start != 0) return 5;
  printf("%u functions, %s\\n", (unsigned)(sizeof every / sizeof every[0]),
         grxblasGetStatusString(GRXBLAS_STATUS_SUCCESS));
  grxdnnDestroy(d);
  return grxblasDestroy(h) == GRXBLAS_STATUS_SUCCESS ? 0 : 4;
}}
""")
    exe = tmp_path / "caller"
    r = subprocess.run(["gcc", "-std=c99", "-pedantic-errors", "-Wall", "-Wextra", "-Werror",
                        str(src), "-I", INCLUDE, *_link_flags(), "-lgrxblas", "-lgrxdnn", "-lgrxrt",
                        "-o", str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert run.returncode == 0, run.stdout + run.stderr
    assert run.stdout.strip() == f"{len(names)} functions, success"


# ---- the CPU host backend ----------------------------------------------------

def _host_gate(name):
    path = os.path.join(O.REF_DIR, "host", name)
    if not os.path.exists(path):
        if not O.build_ref():
            pytest.skip("the reference's gates are not built and /root/reference is absent")
    return path


@pytest.mark.parametrize("name", HOST_GATES)
def test_reference_gate_passes_on_the_host_backend(name):
    exe = _host_gate(name)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout[-3000:]
    assert "PASSED (0 failures)" in r.stdout
    assert "  FAIL" not in r.stdout


@pytest.fixture(scope="module")
def host_blas():
    O.build()
    ctypes.CDLL(O.HOST_RT, mode=ctypes.RTLD_GLOBAL)
    L = ctypes.CDLL(O.HOST_BLAS)
    L.grxblasCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    L.grxblasDestroy.argtypes = [ctypes.c_void_p]
    fp = ctypes.POINTER(ctypes.c_float)
    vp = ctypes.c_void_p
    i = ctypes.c_int
    L.grxblasSgemm.argtypes = [vp, i, i, i, i, i, fp, vp, i, vp, i, fp, vp, i]
    L.grxblasGemmEx.argtypes = [vp, i, i, i, i, i, fp, vp, i, i, vp, i, i, fp, vp, i, i]
    h = ctypes.c_void_p()
    assert L.grxblasCreate(ctypes.byref(h)) == 0
    yield L, h
    L.grxblasDestroy(h)


def _f(v):
    return ctypes.byref(ctypes.c_float(v))


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def test_config1_sgemm_512_cubed_on_the_host_backend(host_blas):
    """BASELINE config 1 in its stated execution mode: fp32 C = A*B, 512^3
    row-major, alpha=1 beta=0, U[-1,1] from seeds 1 and 2, through
    grxblasSgemm on the CPU host backend, mapped to column-major as
    C^T = B^T A^T: Sgemm(N, N, m=512, n=512, k=512, B, 512, A, 512, C, 512)."""
    from grxcp_amd import synth
    L, h = host_blas
    M = N = K = 512
    A = synth.uniform_f32(M * K, 1, -1.0, 1.0)
    B = synth.uniform_f32(K * N, 2, -1.0, 1.0)
    C = np.full(M * N, np.nan, np.float32)       # beta == 0 must not read C
    assert L.grxblasSgemm(h, 0, 0, N, M, K, _f(1.0), _p(B), N, _p(A), K, _f(0.0), _p(C), N) == 0
    want = A.reshape(M, K).astype(np.float64) @ B.reshape(K, N).astype(np.float64)
    got = C.reshape(M, N)
    assert np.isfinite(got).all()
    assert np.max(np.abs(got - want)) / np.max(np.abs(want)) <= 1e-4
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5)


def test_host_backend_gemm_ex_bf16_matches_numpy_exactly(host_blas):
    """bf16 TN GemmEx (config 2's layout) on exact-by-construction values."""
    L, h = host_blas
    m, n, k = 24, 20, 40
    st = O.HalvesStream(7)
    A, B = st.take(k * m), st.take(k * n)          # A stored k x m (op T), B k x n
    C = np.zeros(m * n, np.float32)
    assert L.grxblasGemmEx(h, 1, 0, m, n, k, _f(1.0), _p(O.f32_to_bf16(A)), g.GRX_R_16BF, k,
                           _p(O.f32_to_bf16(B)), g.GRX_R_16BF, k, _f(0.0), _p(C), g.GRX_R_32F, m) == 0
    want = A.reshape(m, k).astype(np.float64) @ B.reshape(n, k).astype(np.float64).T
    assert np.array_equal(C.reshape(n, m).T, want.astype(np.float32))


REFUSALS = [
    # (call name, args builder) -> the status both libraries must return
    ("sgemm negative m", lambda L, h, d: L.grxblasSgemm(h, 0, 0, -1, 4, 4, _f(1), d, 4, d, 4, _f(0), d, 4)),
    ("sgemm null alpha", lambda L, h, d: L.grxblasSgemm(h, 0, 0, 4, 4, 4, None, d, 4, d, 4, _f(0), d, 4)),
    ("sgemm lda < m", lambda L, h, d: L.grxblasSgemm(h, 0, 0, 8, 4, 4, _f(1), d, 7, d, 4, _f(0), d, 8)),
    ("sgemm ldb < n (T)", lambda L, h, d: L.grxblasSgemm(h, 0, 1, 4, 8, 4, _f(1), d, 4, d, 7, _f(0), d, 4)),
    ("sgemm null C", lambda L, h, d: L.grxblasSgemm(h, 0, 0, 4, 4, 4, _f(1), d, 4, d, 4, _f(0), None, 4)),
    ("sgemm empty", lambda L, h, d: L.grxblasSgemm(h, 0, 0, 0, 4, 4, _f(1), None, 4, None, 4, _f(0), None, 4)),
    ("gemmex ldc < m", lambda L, h, d: L.grxblasGemmEx(h, 0, 0, 8, 4, 4, _f(1), d, 2, 8, d, 2, 4, _f(0), d, 0, 7)),
    ("gemmex k>0 null A", lambda L, h, d: L.grxblasGemmEx(h, 0, 0, 4, 4, 4, _f(1), None, 2, 4, d, 2, 4, _f(0), d, 0, 4)),
    ("gemmex empty n", lambda L, h, d: L.grxblasGemmEx(h, 0, 0, 4, 0, 4, _f(1), None, 2, 4, None, 2, 4, _f(0), None, 0, 4)),
]


@pytest.mark.parametrize("case", range(len(REFUSALS)), ids=[c[0] for c in REFUSALS])
def test_host_backend_refuses_like_the_gpu_library(host_blas, case):
    """Validation runs before any device work in both libraries, so the GPU
    library answers these on a machine without a GPU too."""
    L, h = host_blas
    gl = g.load().blas
    gh = ctypes.c_void_p()
    assert gl.grxblasCreate(ctypes.byref(gh)) == 0
    try:
        buf = np.zeros(64, np.float32)
        d = _p(buf)
        name, call = REFUSALS[case]
        want = call(gl, gh, d)
        assert want in (g.SUCCESS, g.INVALID_VALUE), (name, want)
        assert call(L, h, d) == want, name
    finally:
        gl.grxblasDestroy(gh)
