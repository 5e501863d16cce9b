"""The C-ABI boundary, checked without a GPU.

* every function declared in include/grx/*.h is exported by the library that
  implements it, with C linkage;
* argument validation runs before any device work, in the reference's order
  (ref src/libs/grxblas/grxblas.cpp:507-524, 882-897), so the refusal paths
  of the reference's gates (ref tests/libs/test_grxblas.cpp:349-367,
  test_grxblas_ex.cpp:345-371) are checkable on the CPU;
* a configured kernel path that does not hold the kernels fails with
  NOT_INITIALIZED (ref src/libs/grxblas/grxblas.cpp:33-58, 139-146), and a
  machine without a gfx950 reports ARCH_MISMATCH instead of launching.
"""
import ctypes
import os
import re
import subprocess
import sys

import pytest

import grxcp_amd as g

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = {
    "grx_runtime.h": "libgrxrt.so",
    "grxblas.h": "libgrxblas.so",
    "grxdnn.h": "libgrxdnn.so",
}


def declared(header: str) -> list[str]:
    text = open(os.path.join(ROOT, "include", "grx", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    names = re.findall(r"\b(grx\w+)\s*\(", text)
    return sorted({n for n in names if not n.startswith("grxCycleSummarize")})


def exported(lib: str) -> set[str]:
    out = subprocess.run(["nm", "-D", "--defined-only", os.path.join(g.LIBDIR, lib)],
                         capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


@pytest.mark.parametrize("header", sorted(HEADERS))
def test_every_declared_symbol_is_exported(header):
    names = declared(header)
    assert len(names) >= 10
    have = exported(HEADERS[header])
    missing = [n for n in names if n not in have]
    assert not missing, f"{HEADERS[header]} lacks {missing}"


@pytest.mark.parametrize("header", sorted(HEADERS))
def test_nothing_but_the_declared_api_is_exported(header):
    extra = sorted(exported(HEADERS[header]) - set(declared(header)))
    assert not extra, f"{HEADERS[header]} also exports {extra[:10]}"


def test_python_table_matches_headers():
    for header, lib in HEADERS.items():
        assert set(declared(header)) == set(g.EXPORTS[lib]), header


def test_reference_enumerator_values():
    # ref include/grx/grx_types.h:120-134, include/grx/grxblas.h:37-51, 118-125
    assert (g.GRX_R_32F, g.GRX_R_16F, g.GRX_R_8I, g.GRX_R_32I, g.GRX_R_16BF) == (0, 2, 3, 10, 14)
    assert (g.OP_N, g.OP_T) == (0, 1)
    assert (g.TENSOR_FP16, g.TENSOR_INT8, g.TENSOR_BF16) == (0x01, 0x10, 0x40)
    L = g.load().blas
    assert L.grxblasGetStatusString(0) == b"success"
    assert L.grxblasGetStatusString(6) == b"not supported"


def test_handle_lifecycle_without_device():
    L = g.load().blas
    h = ctypes.c_void_p()
    assert L.grxblasCreate(ctypes.byref(h)) == g.SUCCESS
    s = ctypes.c_void_p(1234)
    assert L.grxblasGetStream(h, ctypes.byref(s)) == g.SUCCESS and not s.value
    assert L.grxblasSetStream(h, ctypes.c_void_p(0x10)) == g.SUCCESS
    assert L.grxblasGetStream(h, ctypes.byref(s)) == g.SUCCESS and s.value == 0x10
    assert L.grxblasSetStream(h, None) == g.SUCCESS
    assert L.grxblasCreate(None) == g.INVALID_VALUE
    assert L.grxblasSetStream(None, None) == g.NOT_INITIALIZED
    assert L.grxblasGetStream(None, ctypes.byref(s)) == g.INVALID_VALUE
    assert L.grxblasSetTensorMapSlots(h, 0, 1) == g.SUCCESS
    assert L.grxblasSetTensorMapSlots(h, 1, 1) == g.INVALID_VALUE
    assert L.grxblasSetTensorMapSlots(h, -1, 1) == g.INVALID_VALUE
    assert L.grxblasSetTensorMapSlots(None, 0, 1) == g.NOT_INITIALIZED
    p = ctypes.c_char_p(b"x")
    assert L.grxblasGetLoadedKernelPath(h, ctypes.byref(p)) == g.SUCCESS and p.value is None
    assert L.grxblasSetCycleProbe(h, ctypes.c_void_p(8), 0) == g.INVALID_VALUE
    assert L.grxblasSetCycleProbe(h, None, 0) == g.SUCCESS
    assert L.grxblasCycleSlotsNeeded(h, 64, 64) == 4
    assert L.grxblasCycleSlotsNeeded(h, 65, 64) == 8
    assert L.grxblasCycleSlotsNeeded(h, 0, 64) == 0
    assert L.grxblasDestroy(h) == g.SUCCESS
    assert L.grxblasDestroy(None) == g.NOT_INITIALIZED


FAKE = ctypes.c_void_p(0x1000)  # never dereferenced: every call below stops before device work


def gemm_ex(h, ta, tb, m, n, k, A, at, lda, B, bt, ldb, C, ct, ldc, alpha=1.0, beta=0.0):
    return g.load().blas.grxblasGemmEx(h, ta, tb, m, n, k, g.fptr(alpha), A, at, lda, B, bt, ldb,
                                       g.fptr(beta), C, ct, ldc)


def test_gemm_ex_validation_before_device_work():
    L = g.load().blas
    h = ctypes.c_void_p()
    L.grxblasCreate(ctypes.byref(h))
    F16, F32 = g.GRX_R_16F, g.GRX_R_32F
    # null handle (ref test_grxblas_ex.cpp:366-369)
    assert gemm_ex(None, 0, 0, 8, 4, 8, FAKE, F16, 8, FAKE, F16, 8, FAKE, F32, 8) == g.NOT_INITIALIZED
    # null alpha/beta
    assert L.grxblasGemmEx(h, 0, 0, 8, 4, 8, None, FAKE, F16, 8, FAKE, F16, 8, g.fptr(0), FAKE, F32,
                           8) == g.INVALID_VALUE
    # negative sizes
    assert gemm_ex(h, 0, 0, -1, 4, 8, FAKE, F16, 8, FAKE, F16, 8, FAKE, F32, 8) == g.INVALID_VALUE
    # empty problem succeeds without launching, even with null matrices
    assert gemm_ex(h, 0, 0, 0, 4, 8, None, F16, 8, None, F16, 8, None, F32, 8) == g.SUCCESS
    assert gemm_ex(h, 0, 0, 4, 0, 8, None, F16, 8, None, F16, 8, None, F32, 8) == g.SUCCESS
    # null A/B with k > 0, null C
    assert gemm_ex(h, 0, 0, 8, 4, 8, None, F16, 8, FAKE, F16, 8, FAKE, F32, 8) == g.INVALID_VALUE
    assert gemm_ex(h, 0, 0, 8, 4, 8, FAKE, F16, 8, FAKE, F16, 8, None, F32, 8) == g.INVALID_VALUE
    # lda bounds k when A is transposed (ref test_grxblas_ex.cpp:354-357)
    assert gemm_ex(h, 1, 0, 4, 4, 8, FAKE, F16, 4, FAKE, F16, 8, FAKE, F32, 4) == g.INVALID_VALUE
    # too-small lda (ref test_grxblas_ex.cpp:362-365), ldb, ldc
    assert gemm_ex(h, 0, 0, 8, 4, 8, FAKE, F16, 2, FAKE, F16, 8, FAKE, F32, 8) == g.INVALID_VALUE
    assert gemm_ex(h, 0, 1, 8, 4, 8, FAKE, F16, 8, FAKE, F16, 3, FAKE, F32, 8) == g.INVALID_VALUE
    assert gemm_ex(h, 0, 0, 8, 4, 8, FAKE, F16, 8, FAKE, F16, 8, FAKE, F32, 7) == g.INVALID_VALUE
    # k == 0 with null A/B is legal (C = beta*C); it reaches the device check
    L.grxblasDestroy(h)


def test_sgemm_validation_before_device_work():
    L = g.load().blas
    h = ctypes.c_void_p()
    L.grxblasCreate(ctypes.byref(h))
    one, zero = g.fptr(1.0), g.fptr(0.0)
    # ref test_grxblas.cpp:349-367
    assert L.grxblasSgemm(h, 0, 0, 4, 4, 4, one, FAKE, 2, FAKE, 4, zero, FAKE, 4) == g.INVALID_VALUE
    assert L.grxblasSgemm(h, 0, 0, 4, 4, 4, one, FAKE, 4, FAKE, 4, zero, FAKE, 1) == g.INVALID_VALUE
    assert L.grxblasSgemm(h, 0, 0, 0, 4, 4, one, FAKE, 4, FAKE, 4, zero, FAKE, 4) == g.SUCCESS
    assert L.grxblasSgemm(None, 0, 0, 4, 4, 4, one, FAKE, 4, FAKE, 4, zero, FAKE, 4) == g.NOT_INITIALIZED
    # ref test_grxblas.cpp:338-345
    sb = L.grxblasSgemmStridedBatched
    assert sb(h, 0, 0, 4, 4, 4, one, FAKE, 4, 16, FAKE, 4, 16, zero, FAKE, 4, 16, 0) == g.SUCCESS
    assert sb(h, 0, 0, 4, 4, 4, one, FAKE, 4, 16, FAKE, 4, 16, zero, FAKE, 4, 16, -1) == g.INVALID_VALUE
    L.grxblasDestroy(h)


def test_blas12_validation_before_device_work():
    L = g.load().blas
    h = ctypes.c_void_p()
    L.grxblasCreate(ctypes.byref(h))
    one = g.fptr(1.0)
    assert L.grxblasSaxpy(h, 4, one, FAKE, 0, FAKE, 1) == g.INVALID_VALUE
    assert L.grxblasSaxpy(h, 0, one, None, 1, None, 1) == g.SUCCESS
    assert L.grxblasSaxpy(h, -1, one, FAKE, 1, FAKE, 1) == g.INVALID_VALUE
    assert L.grxblasSscal(h, 4, one, FAKE, -1) == g.INVALID_VALUE
    assert L.grxblasSgemv(h, 0, 4, 4, one, FAKE, 3, FAKE, 1, one, FAKE, 1) == g.INVALID_VALUE
    assert L.grxblasSgemv(None, 0, 4, 4, one, FAKE, 4, FAKE, 1, one, FAKE, 1) == g.NOT_INITIALIZED
    L.grxblasDestroy(h)


def _run_child(code: str, env_extra: dict) -> str:
    env = dict(os.environ, **env_extra)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env,
                       cwd=ROOT, timeout=120)
    assert r.returncode == 0, r.stderr
    return r.stdout.strip()


_PROBE_CALL = """
import ctypes, grxcp_amd as g
L = g.load().blas
h = ctypes.c_void_p(); L.grxblasCreate(ctypes.byref(h))
m = ctypes.c_int(); n = ctypes.c_int(); k = ctypes.c_int()
print(L.grxblasGetTensorTile(h, ctypes.byref(m), ctypes.byref(n), ctypes.byref(k)))
"""


def test_configured_kernel_path_without_kernels_is_not_initialized(tmp_path):
    out = _run_child(_PROBE_CALL, {"GRXBLAS_KERNEL_PATH": str(tmp_path)})
    assert out == str(g.NOT_INITIALIZED)


def test_set_kernel_path_overrides_and_clears():
    code = """
import ctypes, grxcp_amd as g
L = g.load().blas
h = ctypes.c_void_p(); L.grxblasCreate(ctypes.byref(h))
L.grxblasSetKernelPath(b"/nonexistent")
m = ctypes.c_int(); n = ctypes.c_int(); k = ctypes.c_int()
a = L.grxblasGetTensorTile(h, ctypes.byref(m), ctypes.byref(n), ctypes.byref(k))
L.grxblasSetKernelPath(g.LIBDIR.encode())
h2 = ctypes.c_void_p(); L.grxblasCreate(ctypes.byref(h2))
b = L.grxblasGetTensorTile(h2, ctypes.byref(m), ctypes.byref(n), ctypes.byref(k))
p = ctypes.c_char_p()
L.grxblasGetLoadedKernelPath(h2, ctypes.byref(p))
print(a, b if g.device_count() == 0 else 'dev', p.value.decode().endswith('libgrxblas.so'))
"""
    a, b, ok = _run_child(code, {}).split()
    assert int(a) == g.NOT_INITIALIZED
    assert ok == "True"
    if b != "dev":
        assert int(b) == g.ARCH_MISMATCH  # right path, but no gfx950 here


@pytest.mark.skipif(g.device_count() > 0, reason="checks the no-device path")
def test_attention_broadcast_input_passes_validation():
    """An input whose rows share addresses (a broadcast) is accepted, and so
    is an interleaved [B, S, H, D] output: validation passes and the call
    stops at the missing device."""
    D = g.load().dnn
    h = ctypes.c_void_p()
    assert D.grxdnnCreate(ctypes.byref(h)) == g.SUCCESS
    ad = g.AttnDesc(True, 0.125)
    q = g.TensorDesc(g.GRX_R_16BF, [1, 2, 16, 128])
    shared_rows = g.TensorDesc(g.GRX_R_16BF, [1, 2, 16, 128], [4096, 2048, 0, 1])
    bshd = g.TensorDesc(g.GRX_R_16BF, [1, 2, 16, 128], [4096, 128, 256, 1])
    fq, fk, fv, fo = (ctypes.c_void_p(0x100000 * (i + 1)) for i in range(4))
    assert D.grxdnnAttentionForward(h, ad.d, shared_rows.d, fq, q.d, fk, q.d, fv, bshd.d,
                                    fo) == g.ARCH_MISMATCH
    # Q, K and V may overlap one another (here: the same buffer), and O may be
    # Q itself with Q's layout (in place)
    assert D.grxdnnAttentionForward(h, ad.d, q.d, fq, q.d, fq, q.d, fq, q.d, fo) == g.ARCH_MISMATCH
    assert D.grxdnnAttentionForward(h, ad.d, q.d, fq, q.d, fk, q.d, fv, q.d, fq) == g.ARCH_MISMATCH
    assert D.grxdnnDestroy(h) == g.SUCCESS


def test_dnn_cycle_probe_arguments():
    """grxdnnSetCycleProbe follows grxblasSetCycleProbe's argument rules; the
    slot count is workgroups x 8 waves (here the 256-CU default of a host
    without a device: at most one workgroup per CU, a multiple of 8, no more
    than the (batch, head, 256-query) items of the busiest XCD need)."""
    D = g.load().dnn
    h = ctypes.c_void_p()
    assert D.grxdnnCreate(ctypes.byref(h)) == g.SUCCESS
    assert D.grxdnnSetCycleProbe(h, ctypes.c_void_p(8), 0) == g.INVALID_VALUE
    assert D.grxdnnSetCycleProbe(h, ctypes.c_void_p(8), 64) == g.SUCCESS
    assert D.grxdnnSetCycleProbe(h, None, 0) == g.SUCCESS
    assert D.grxdnnSetCycleProbe(None, None, 0) == g.NOT_INITIALIZED
    assert D.grxdnnAttentionCycleSlotsNeeded(h, 1, 1, 1) == 8 * 8
    assert D.grxdnnAttentionCycleSlotsNeeded(h, 2, 8, 512) == 8 * 4 * 8   # 2 heads x 2 tiles per XCD
    assert D.grxdnnAttentionCycleSlotsNeeded(h, 4, 32, 4096) == 256 * 8
    assert D.grxdnnAttentionCycleSlotsNeeded(h, 0, 32, 4096) == 0
    assert D.grxdnnDestroy(h) == g.SUCCESS


def test_attention_output_overlapping_k_or_v_is_refused():
    """A workgroup writes its O rows while workgroups of other query tiles of
    the same head still read K and V: an O that overlaps K or V (or overlaps
    Q other than as Q itself) would race, so validation refuses it."""
    D = g.load().dnn
    h = ctypes.c_void_p()
    assert D.grxdnnCreate(ctypes.byref(h)) == g.SUCCESS
    ad = g.AttnDesc(True, 0.125)
    q = g.TensorDesc(g.GRX_R_16BF, [1, 2, 16, 128])           # 8 KB per tensor
    bshd = g.TensorDesc(g.GRX_R_16BF, [1, 2, 16, 128], [4096, 128, 256, 1])
    att = D.grxdnnAttentionForward
    P = lambda a: ctypes.c_void_p(a)  # noqa: E731
    fq, fk, fv = P(0x100000), P(0x200000), P(0x300000)
    assert att(h, ad.d, q.d, fq, q.d, fk, q.d, fv, q.d, fk) == g.INVALID_VALUE          # O == K
    assert att(h, ad.d, q.d, fq, q.d, fk, q.d, fv, q.d, fv) == g.INVALID_VALUE          # O == V
    assert att(h, ad.d, q.d, fq, q.d, fk, q.d, fv, q.d, P(0x300000 + 4096)) == g.INVALID_VALUE
    assert att(h, ad.d, q.d, fq, q.d, fk, q.d, fv, q.d, P(0x200000 - 4096)) == g.INVALID_VALUE
    assert att(h, ad.d, q.d, fq, q.d, fk, q.d, fv, q.d, P(0x100000 + 256)) == g.INVALID_VALUE
    assert att(h, ad.d, q.d, fq, q.d, fk, q.d, fv, bshd.d, fq) == g.INVALID_VALUE       # Q, other layout
    # touching but not overlapping is fine (stops at the missing device, or runs)
    ok = g.ARCH_MISMATCH if g.device_count() == 0 else None
    if ok is not None:
        assert att(h, ad.d, q.d, fq, q.d, fk, q.d, fv, q.d, P(0x200000 + 8192)) == ok
        assert att(h, ad.d, q.d, fq, q.d, fk, q.d, fv, q.d, P(0x200000 - 8192)) == ok
    # a packed [B, S, 3, H, D] QKV buffer: Q, K and V are views with one set
    # of strides, 2*H*D bytes apart. O written over the Q slot shares no
    # element with K or V (their spans interleave): accepted. O over the K
    # slot, or shifted by one head or by 8 elements, shares elements: refused.
    B_, H_, S_, D_ = 2, 2, 16, 128
    qkv = g.TensorDesc(g.GRX_R_16BF, [B_, H_, S_, D_], [S_ * 3 * H_ * D_, D_, 3 * H_ * D_, 1])
    base = 0x1000000
    pq, pk, pv = P(base), P(base + 2 * H_ * D_), P(base + 4 * H_ * D_)
    assert att(h, ad.d, qkv.d, pk, qkv.d, pk, qkv.d, pv, qkv.d, pk) == g.INVALID_VALUE   # O == K
    assert att(h, ad.d, qkv.d, pq, qkv.d, pk, qkv.d, pv, qkv.d, P(base + 2 * D_)) == g.INVALID_VALUE
    assert att(h, ad.d, qkv.d, pq, qkv.d, pk, qkv.d, pv, qkv.d,
               P(base + 2 * H_ * D_ - 16)) == g.INVALID_VALUE
    assert att(h, ad.d, qkv.d, pq, qkv.d, pk, qkv.d, pv, qkv.d,
               P(base + 4 * H_ * D_ + 2 * D_)) == g.INVALID_VALUE                          # O over V's head 1
    if ok is not None:
        assert att(h, ad.d, qkv.d, pq, qkv.d, pk, qkv.d, pv, qkv.d, pq) == ok              # in place
        # a separate contiguous O: fine
        dense = g.TensorDesc(g.GRX_R_16BF, [B_, H_, S_, D_])
        assert att(h, ad.d, qkv.d, pq, qkv.d, pk, qkv.d, pv, dense.d, P(0x4000000)) == ok
    assert D.grxdnnDestroy(h) == g.SUCCESS


@pytest.mark.skipif(g.device_count() > 0, reason="checks the no-device path")
def test_no_device_is_arch_mismatch_not_a_launch():
    L = g.load().blas
    h = ctypes.c_void_p()
    L.grxblasCreate(ctypes.byref(h))
    assert gemm_ex(h, 1, 0, 64, 64, 64, FAKE, g.GRX_R_16BF, 64, FAKE, g.GRX_R_16BF, 64, FAKE,
                   g.GRX_R_16BF, 64) == g.ARCH_MISMATCH
    types = ctypes.c_uint()
    assert L.grxblasGetTensorTypes(h, ctypes.byref(types)) == g.ARCH_MISMATCH
    L.grxblasDestroy(h)


def test_dnn_descriptors_and_validation():
    D = g.load().dnn
    h = ctypes.c_void_p()
    assert D.grxdnnCreate(ctypes.byref(h)) == g.SUCCESS
    xd = g.TensorDesc(g.GRX_R_16BF, [4, 256])
    wd = g.TensorDesc(g.GRX_R_16BF, [256])
    bad_w = g.TensorDesc(g.GRX_R_16BF, [128])
    i8 = g.TensorDesc(g.GRX_R_8I, [4, 256])
    i8w = g.TensorDesc(g.GRX_R_8I, [256])
    # packed strides are filled in
    t = ctypes.c_int(); nb = ctypes.c_int()
    dims = (ctypes.c_int * 4)(); strides = (ctypes.c_int * 4)()
    assert D.grxdnnGetTensorNdDescriptor(xd.d, 4, ctypes.byref(t), ctypes.byref(nb), dims, strides) == 0
    assert (t.value, nb.value, list(dims)[:2], list(strides)[:2]) == (g.GRX_R_16BF, 2, [4, 256], [256, 1])
    rms = D.grxdnnRMSNormForward
    assert rms(None, xd.d, FAKE, wd.d, FAKE, 1e-6, xd.d, FAKE) == g.NOT_INITIALIZED
    assert rms(h, None, FAKE, wd.d, FAKE, 1e-6, xd.d, FAKE) == g.INVALID_VALUE
    assert rms(h, xd.d, FAKE, bad_w.d, FAKE, 1e-6, xd.d, FAKE) == g.INVALID_VALUE
    assert rms(h, xd.d, FAKE, wd.d, FAKE, -1.0, xd.d, FAKE) == g.INVALID_VALUE
    assert rms(h, xd.d, FAKE, wd.d, FAKE, float("nan"), xd.d, FAKE) == g.INVALID_VALUE
    assert rms(h, i8.d, FAKE, i8w.d, FAKE, 1e-6, i8.d, FAKE) == g.NOT_SUPPORTED
    assert rms(h, xd.d, None, wd.d, FAKE, 1e-6, xd.d, FAKE) == g.INVALID_VALUE
    assert D.grxdnnLayerNormForward(h, xd.d, FAKE, wd.d, FAKE, None, 1e-6, xd.d, FAKE) == g.INVALID_VALUE
    empty = g.TensorDesc(g.GRX_R_16BF, [0, 256])
    assert rms(h, empty.d, None, wd.d, None, 1e-6, empty.d, None) == g.SUCCESS
    strided = g.TensorDesc(g.GRX_R_16BF, [4, 256], [256, 2])
    assert rms(h, strided.d, FAKE, wd.d, FAKE, 1e-6, strided.d, FAKE) == g.NOT_SUPPORTED
    # attention
    ad = g.AttnDesc(True, 0.125)
    q = g.TensorDesc(g.GRX_R_16BF, [1, 2, 16, 128])
    q96 = g.TensorDesc(g.GRX_R_16BF, [1, 2, 16, 96])
    qf32 = g.TensorDesc(g.GRX_R_32F, [1, 2, 16, 128])
    att = D.grxdnnAttentionForward
    assert att(None, ad.d, q.d, FAKE, q.d, FAKE, q.d, FAKE, q.d, FAKE) == g.NOT_INITIALIZED
    assert att(h, None, q.d, FAKE, q.d, FAKE, q.d, FAKE, q.d, FAKE) == g.INVALID_VALUE
    assert att(h, ad.d, q96.d, FAKE, q96.d, FAKE, q96.d, FAKE, q96.d, FAKE) == g.NOT_SUPPORTED
    assert att(h, ad.d, qf32.d, FAKE, qf32.d, FAKE, qf32.d, FAKE, qf32.d, FAKE) == g.NOT_SUPPORTED
    assert att(h, ad.d, q.d, FAKE, q96.d, FAKE, q.d, FAKE, q.d, FAKE) == g.INVALID_VALUE
    assert att(h, ad.d, q.d, None, q.d, FAKE, q.d, FAKE, q.d, FAKE) == g.INVALID_VALUE
    # an output whose rows share addresses is refused
    shared_rows = g.TensorDesc(g.GRX_R_16BF, [1, 2, 16, 128], [4096, 2048, 0, 1])
    assert att(h, ad.d, q.d, FAKE, q.d, FAKE, q.d, FAKE, shared_rows.d, FAKE) == g.INVALID_VALUE
    heads_over_rows = g.TensorDesc(g.GRX_R_16BF, [1, 2, 16, 128], [4096, 64, 128, 1])
    assert att(h, ad.d, q.d, FAKE, q.d, FAKE, q.d, FAKE, heads_over_rows.d, FAKE) == g.INVALID_VALUE
    c = ctypes.c_int(); sc = ctypes.c_float()
    assert D.grxdnnGetAttentionDescriptor(ad.d, ctypes.byref(c), ctypes.byref(sc)) == 0
    assert (c.value, sc.value) == (1, 0.125)
    assert D.grxdnnSetAttentionDescriptor(ad.d, 2, 0.1) == g.INVALID_VALUE
    assert D.grxdnnSetAttentionDescriptor(ad.d, 1, 0.0) == g.INVALID_VALUE
    assert D.grxdnnSetTensorNdDescriptor(xd.d, g.GRX_R_16BF, 0, (ctypes.c_int * 1)(1), None) == g.INVALID_VALUE
    assert D.grxdnnSetTensorNdDescriptor(xd.d, 99, 1, (ctypes.c_int * 1)(1), None) == g.INVALID_VALUE
    assert D.grxdnnDestroy(h) == g.SUCCESS


def test_runtime_without_device():
    rt = g.load().rt
    assert rt.grxGetErrorName(0) == b"grxSuccess"
    assert rt.grxGetErrorName(999) == b"grxErrorUnknown"
    assert rt.grxMalloc(None, 16) == 1  # invalid value
    p = ctypes.c_void_p(5)
    assert rt.grxMalloc(ctypes.byref(p), 0) == 0 and not p.value
    assert rt.grxFree(None) == 0
    assert rt.grxMemcpy(None, None, 0, g.MEMCPY_DEFAULT) == 0
    assert rt.grxMemcpy(FAKE, FAKE, 4, 7) == 6  # invalid direction, checked before HIP
    assert rt.grxStreamDestroy(None) == 7
    assert rt.grxEventRecord(None, None) == 7


@pytest.mark.parametrize("lib", sorted(set(HEADERS.values())))
def test_product_libraries_never_reach_the_oracle(lib):
    """The oracle and the CPU host backend are test infrastructure: no
    product library links them, names their symbols or loads them at run
    time (no dlopen of a path containing them)."""
    path = os.path.join(g.LIBDIR, lib)
    dyn = subprocess.run(["readelf", "-d", path], capture_output=True, text=True, check=True).stdout
    needed = re.findall(r"\(NEEDED\).*\[(.*)\]", dyn)
    assert needed and not any("oracle" in n or "_ref" in n for n in needed), needed
    undefined = subprocess.run(["nm", "-D", "--undefined-only", path], capture_output=True, text=True,
                               check=True).stdout
    assert "oracle_" not in undefined and "dlopen" not in undefined
    strings = subprocess.run(["strings", path], capture_output=True, text=True, check=True).stdout
    assert "libgrx_oracle" not in strings and "libgrxblas_ref" not in strings


def test_product_python_never_imports_the_oracle():
    """grxcp_amd's Python (the ctypes mirror the tests and bench.py use) has
    no route to oracle/: no import of it and no path into it."""
    pkg = os.path.join(ROOT, "grxcp_amd")
    for name in os.listdir(pkg):
        if name.endswith(".py"):
            text = open(os.path.join(pkg, name)).read()
            assert not re.search(r"^\s*(import|from)\s+oracle\b", text, re.M), name
            assert "oracle/" not in text and "libgrx_oracle" not in text, name
