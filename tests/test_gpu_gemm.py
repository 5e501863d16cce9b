"""grxblasGemmEx / grxblasGemmExDequant on gfx950 against the CPU oracle.

Mirrors the reference's GemmEx gate (ref tests/libs/test_grxblas_ex.cpp):
exact-by-construction inputs (multiples of 0.5 in [-4, 4], exact in fp16 and
bf16, products and sums exact in fp32), so the comparison is BIT-EXACT over
the ENTIRE padded C buffer -- inside the window and in the padding -- for
ragged shapes and all four transposes, with the tile shape queried from the
library. int8 is integer and exact. Random-normal cases (the BASELINE config
distributions) use the north-star bound: max relative error <= 1e-2 vs an
fp32/fp64 reference.
"""
import os
import re

import numpy as np
import pytest

import grxcp_amd as g
import oracle as O
from helpers import Guarded, col_major, from_col_major, normwise_rel_err, say, to_dev, window_mask

pytestmark = pytest.mark.gpu

F16, BF16, F32, I8, I32 = g.GRX_R_16F, g.GRX_R_16BF, g.GRX_R_32F, g.GRX_R_8I, g.GRX_R_32I


def logged_plans(capfd, call):
    """Run `call` with GRXBLAS_LOG=1; return the launch plans the library
    printed, as dicts of the key=value fields of each line."""
    capfd.readouterr()
    os.environ["GRXBLAS_LOG"] = "1"
    try:
        call()
    finally:
        del os.environ["GRXBLAS_LOG"]
    lines = [l for l in capfd.readouterr().err.splitlines() if l.startswith("grxblas: gemm ")]
    return [dict(re.findall(r"(\w+)=(\w+)", l)) for l in lines]


def narrow(vals: np.ndarray, t: int) -> np.ndarray:
    return O.f32_to_half(vals) if t == F16 else O.f32_to_bf16(vals)


def widen(bits: np.ndarray, t: int) -> np.ndarray:
    return O.half_to_f32(bits) if t == F16 else O.bf16_to_f32(bits)


def float_case(blas, in_t, out_t, ta, tb, m, n, k, alpha, beta, pad, cpad=None, seed=99,
               guard=False):
    """The reference's run_case (ref test_grxblas_ex.cpp:65-149), for any
    fp16/bf16 input and fp32/fp16/bf16 output. `pad` widens lda/ldb, `cpad`
    (default: pad) widens ldc. With `guard`, C sits between guard bands and a
    changed band counts as one stray write. Returns (#wrong, #stray)."""
    kk = k if k else 1
    a_rows, a_cols = (kk, m) if ta else (m, kk)
    b_rows, b_cols = (n, kk) if tb else (kk, n)
    lda, ldb, ldc = a_rows + pad, b_rows + pad, m + (pad if cpad is None else cpad)
    st = O.HalvesStream(seed)
    A = st.take(lda * a_cols)
    B = st.take(ldb * b_cols)
    C = st.take(ldc * n) * 2.0
    hA, hB = narrow(A, in_t), narrow(B, in_t)
    assert np.array_equal(widen(hA, in_t), A) and np.array_equal(widen(hB, in_t), B)
    if out_t == F32:
        c_host = C
        expected = O.gemm_f32acc(ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc)
    else:
        c_host = narrow(C, out_t)
        c_in = widen(c_host, out_t)
        expected = narrow(O.gemm_f32acc(ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, c_in, ldc), out_t)
        # the padding must come back as uploaded
        inside = window_mask(m, n, ldc)
        expected = np.where(inside, expected, c_host)
    dA, dB = to_dev(hA), to_dev(hB)
    dC = Guarded(c_host) if guard else to_dev(c_host)
    say(f"gemm_ex in={in_t} out={out_t} ta={ta} tb={tb} {m}x{n}x{k} a={alpha} b={beta} pad={pad}")
    s = blas.gemm_ex(ta, tb, m, n, k, alpha, dA.p, in_t, lda, dB.p, in_t, ldb, beta, dC.p, out_t, ldc)
    assert s == g.SUCCESS, g.STATUS[s]
    g.synchronize()
    got = dC.download(c_host.dtype, c_host.size)
    inside = window_mask(m, n, ldc)
    diff = got.view(np.uint32 if got.itemsize == 4 else np.uint16) != \
        expected.astype(c_host.dtype).view(np.uint32 if got.itemsize == 4 else np.uint16)
    stray = int(np.sum(diff & ~inside)) + (0 if not guard or dC.guards_intact() else 1)
    return int(np.sum(diff & inside)), stray


def gate_cases(tm, tn, tk):
    """The reference's case list (ref test_grxblas_ex.cpp:207-242)."""
    cases = [
        (0, 0, tm, tn, tk, 1.0, 0.0, 0), (0, 0, tm * 2, tn * 2, tk * 2, 1.0, 0.0, 0),
        (0, 0, 16, 16, 16, 1.0, 0.0, 0), (0, 0, 5, 3, 7, 1.0, 0.0, 0),
        (0, 0, 17, 9, 13, 1.0, 0.0, 0), (0, 0, 1, 1, 1, 1.0, 0.0, 0),
        (0, 0, 12, 6, 10, 2.5, -1.5, 0), (0, 0, 12, 6, 10, 1.0, 0.0, 3),
        (0, 0, 6, 5, 0, 1.0, 2.0, 0),
    ]
    for which in range(3):
        ta, tb = int(which != 1), int(which != 0)
        cases += [(ta, tb, tm, tn, tk, 1.0, 0.0, 0), (ta, tb, tm * 2, tn * 2, tk * 2, 1.0, 0.0, 0),
                  (ta, tb, 5, 3, 7, 1.0, 0.0, 0), (ta, tb, 17, 9, 13, 1.0, 0.0, 0),
                  (ta, tb, 12, 6, 10, 2.5, -1.5, 3)]
    return cases


def test_tensor_tile_and_types(blas):
    import ctypes
    m, n, k, t = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_uint()
    assert blas.L.grxblasGetTensorTile(blas.h, ctypes.byref(m), ctypes.byref(n), ctypes.byref(k)) == 0
    assert (m.value, n.value, k.value) == (32, 32, 16)
    assert blas.L.grxblasGetTensorTypes(blas.h, ctypes.byref(t)) == 0
    assert t.value & g.TENSOR_FP16 and t.value & g.TENSOR_BF16 and t.value & g.TENSOR_INT8
    p = ctypes.c_char_p()
    assert blas.L.grxblasGetLoadedKernelPath(blas.h, ctypes.byref(p)) == 0
    assert p.value and p.value.decode().endswith("libgrxblas.so")


@pytest.mark.parametrize("in_t,out_t", [(F16, F32), (BF16, F32), (BF16, BF16), (F16, F16)])
def test_reference_gemm_ex_gate(blas, in_t, out_t):
    bad = []
    for case in gate_cases(32, 32, 16):
        ta, tb, m, n, k, a, b, pad = case
        wrong, stray = float_case(blas, in_t, out_t, ta, tb, m, n, k, a, b, pad)
        if wrong or stray:
            bad.append((case, wrong, stray))
    assert not bad, bad


# Fast (TN, K-contiguous) path: still exact-by-construction, at sizes and
# alignments that route to the 256x256 MFMA kernel, with ragged m/n and a k
# that does not fill the last 128-byte stage.
# (m, n, k, pad, cpad): lda = k + pad and ldc = m + cpad are multiples of 8
# wherever the fast path is meant to run.
FAST_SHAPES = [
    (256, 256, 64, 0, 0), (512, 256, 128, 0, 0), (300, 200, 200, 8, 4), (1, 1, 8, 0, 0),
    (257, 513, 1024, 8, 7), (1024, 768, 2048, 0, 0),
]


@pytest.mark.parametrize("in_t,out_t", [(BF16, F32), (BF16, BF16), (F16, F32)])
@pytest.mark.parametrize("m,n,k,pad,cpad", FAST_SHAPES)
def test_fast_path_exact(blas, in_t, out_t, m, n, k, pad, cpad):
    wrong, stray = float_case(blas, in_t, out_t, 1, 0, m, n, k, 1.0, 0.0, pad, cpad)
    assert (wrong, stray) == (0, 0)


def test_fast_path_alpha_beta(blas):
    assert float_case(blas, BF16, F32, 1, 0, 384, 320, 256, 2.5, -1.5, 8) == (0, 0)
    assert float_case(blas, BF16, BF16, 1, 0, 384, 320, 256, 2.5, -1.5, 8) == (0, 0)
    assert float_case(blas, F16, F16, 1, 0, 384, 320, 256, 2.5, -1.5, 8) == (0, 0)


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 1)])
@pytest.mark.parametrize("in_t,out_t", [(BF16, BF16), (BF16, F32), (F16, F16), (F16, F32)])
def test_transposed_copy_paths_exact(blas, in_t, out_t, ta, tb):
    """Layouts other than T,N above the size threshold run the TN kernel behind
    K-contiguous copies of op(A) / op(B) in the handle's workspace: ragged
    shapes, padded leading dimensions, alpha/beta, still bit-exact."""
    assert float_case(blas, in_t, out_t, ta, tb, 320, 264, 512, 1.0, 0.0, 0) == (0, 0)
    assert float_case(blas, in_t, out_t, ta, tb, 264, 300, 520, 2.5, -1.5, 8) == (0, 0)


def test_workspace_grows_and_follows_stream_changes():
    """The transposed-copy workspace: a larger problem after a smaller one
    (the workspace grows), and back-to-back calls alternating between two
    streams with no host synchronisation in between (each stream has its own
    workspace). Every result bit-exact."""
    blas = g.Blas()
    streams = [g.Stream(), g.Stream()]
    try:
        cases = []
        for i, (m, n, k) in enumerate([(256, 256, 512), (512, 384, 1024), (320, 512, 768),
                                       (512, 512, 1024)]):
            st = O.HalvesStream(100 + i)
            A, B = st.take(m * k), st.take(k * n)     # N,N: A m x k (lda m), B k x n (ldb k)
            hA, hB = narrow(A, BF16), narrow(B, BF16)
            want = O.gemm_f32acc(0, 0, m, n, k, 1.0, A, m, B, k, 0.0, np.zeros(m * n, np.float32), m)
            cases.append((m, n, k, to_dev(hA), to_dev(hB), g.DeviceBuffer(m * n * 4), want))
        for i, (m, n, k, dA, dB, dC, _) in enumerate(cases):
            blas.set_stream(streams[i % 2].s)
            say(f"workspace case {i}: {m}x{n}x{k} on stream {i % 2}")
            assert blas.gemm_ex(0, 0, m, n, k, 1.0, dA.p, BF16, m, dB.p, BF16, k, 0.0, dC.p, F32,
                                m) == g.SUCCESS
        g.synchronize()
        for m, n, k, dA, dB, dC, want in cases:
            got = dC.download(np.float32, m * n)
            assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))
    finally:
        blas.close()
        for st in streams:
            st.close()


@pytest.mark.parametrize("in_t,out_t", [(BF16, BF16), (BF16, F32), (F16, F16), (F16, F32)])
@pytest.mark.parametrize("m,n,k,alpha,beta,pad,cpad,kernel", [
    (1024, 1024, 8192, 1.0, 0.0, 0, 0, "tn128"),     # 64 tiles of 128x128, 128 stages
    (300, 520, 4160, 2.5, -1.5, 8, 4, "tn128"),      # ragged m/n, last slice shorter
    (512, 2048, 4096, 1.0, 0.0, 0, 8, "tn128"),      # 64 tiles, 64 stages
    (2048, 1152, 6144, 1.0, 0.0, 0, 0, "tn256"),     # 144 tiles of 128x128: 256x256 slices
])
def test_split_k_exact(blas, capfd, in_t, out_t, m, n, k, alpha, beta, pad, cpad, kernel):
    """Problems with few tiles and a long K are split along K, on 128x128
    tiles where at most 128 of them cover C, else on 256x256 tiles; the
    partial sums of exact inputs are exact, so the result stays bit-exact."""
    res = []
    plans = logged_plans(capfd, lambda: res.append(
        float_case(blas, in_t, out_t, 1, 0, m, n, k, alpha, beta, pad, cpad)))
    assert res == [(0, 0)]
    assert len(plans) == 1 and plans[0]["kernel"] == kernel and int(plans[0]["split"]) >= 2, plans


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 1)])
def test_split_k_after_transposed_copies(blas, capfd, ta, tb):
    res = []
    plans = logged_plans(capfd, lambda: res.append(
        float_case(blas, BF16, BF16, ta, tb, 512, 256, 4096, 1.0, 0.0, 0)))
    assert res == [(0, 0)]
    p = plans[0]
    # the 16-bit operand stored M- (N-) contiguous is read in place by the slices
    assert (p["direct_a"], p["direct_b"]) == (str(1 - ta), str(tb)) and int(p["split"]) >= 2, plans
    assert (p["copy_a"], p["copy_b"]) == ("0", "0"), plans


def test_split_k_plan_limits(blas, capfd):
    """Where the split does not pay: many tiles, short K, a batch."""
    buf = g.DeviceBuffer(4096 * 4096 * 2)
    out = g.DeviceBuffer(4096 * 4096 * 4)
    calls = [
        lambda: blas.gemm_ex(1, 0, 4096, 4096, 4096, 1.0, buf.p, BF16, 4096, buf.p, BF16, 4096,
                             0.0, out.p, F32, 4096),                  # 256 tiles fill the CUs
        lambda: blas.gemm_ex(1, 0, 1024, 1024, 512, 1.0, buf.p, BF16, 512, buf.p, BF16, 512,
                             0.0, out.p, F32, 1024),                  # 8 stages
        lambda: blas.gemm_strided_batched_ex(1, 0, 256, 256, 8192, 1.0, buf.p, BF16, 8192, 0,
                                             buf.p, BF16, 8192, 0, 0.0, out.p, F32, 256,
                                             256 * 256, 2),           # batch of 2
        lambda: blas.gemm_ex(1, 0, 256, 256, 8192, 1.0, buf.p, BF16, 8192, buf.p, BF16, 8192,
                             0.0, out.p, F32, 256),                   # the same, unbatched
    ]
    for want, call in zip(["1", "1", "1", "8"], calls):
        plans = logged_plans(capfd, lambda: (call() == g.SUCCESS) or pytest.fail("call failed"))
        g.synchronize()
        assert [p["split"] for p in plans] == [want], plans


def test_tn128_path_exact(blas, capfd):
    """16-bit and int8 problems of at least 1024 x 1024 with few 256x256 tiles
    and at most 32 stages of K run on 128x128 tiles: every input/output
    type, (T, N) directly and (N, N) with A read where it lies (16-bit) or
    behind the operand copy (int8), ragged n and K, alpha/beta, bit-exact
    against the oracle over the whole padded C, with guard bands; the
    GRXBLAS_LOG line shows the path taken."""
    cases = []
    for ta, tb in ((1, 0), (0, 0)):
        for it, ot in ((BF16, F32), (BF16, BF16), (F16, F16), (F16, F32)):
            cases.append(("f", ta, tb, it, ot))
        cases += [("i8", ta, tb, None, None), ("dq", ta, tb, None, None)]
    bad = []
    for kind, ta, tb, it, ot in cases:
        # C columns and K rows on 16-byte boundaries; m, n and K ragged against the tiles
        m, n, k = 1032, 1100, 200 if kind == "f" else 400
        res = []
        if kind == "f":
            call = lambda: res.append(float_case(blas, it, ot, ta, tb, m, n, k, 1.5, -0.5, 0, 8,
                                                 seed=7 + ta, guard=True))
            ok = (0, 0)
        elif kind == "i8":
            call = lambda: res.append(int8_case(blas, ta, tb, m, n, k, 2.0, 1.0, 0, fill="rand", seed=9,
                                                cpad=0, guard=True))
            ok = 0
        else:
            call = lambda: res.append(dequant_case(blas, ta, tb, m, n, k, 0, 8, seed=11, guard=True))
            ok = (0, 0)
        plans = logged_plans(capfd, call)
        direct = "1" if kind == "f" and ta == 0 else "0"
        if res != [ok] or len(plans) != 1 or plans[0]["kernel"] != "tn128" or \
                plans[0]["direct_a"] != direct or plans[0]["copy_a"] != str(1 - ta - int(direct)):
            bad.append((kind, ta, tb, it, ot, res, plans))
    assert not bad, bad


@pytest.mark.parametrize("it,ot,ta,tb,m,n,k,pad,alpha,beta,ring,direct", [
    (BF16, BF16, 0, 0, 1032, 1100, 200, 8, 1.5, -0.5, "4", "10"),  # lda > m, K ends inside a stage
    (F16, F32, 0, 0, 2176, 2176, 128, 0, 1.0, 0.0, "2", "10"),     # 289 tiles: the two-stage ring
    (BF16, F32, 0, 0, 1024, 2048, 16, 0, 2.5, 1.0, "4", "10"),     # 16 k-rows: one stage, mostly zero fill
    (F16, F16, 0, 0, 1096, 1024, 1000, 0, 1.0, 0.0, "4", "10"),    # 16 stages, the last one partial
    (BF16, BF16, 0, 0, 1030, 1100, 200, 0, 1.0, 0.0, "4", "00"),   # lda = m = 1030: behind the copy
    (BF16, BF16, 1, 1, 1100, 1032, 200, 8, 1.5, -0.5, "4", "01"),  # op(B) = B^T read in place
    (F16, F32, 0, 1, 1032, 1096, 1000, 0, 2.0, 1.0, "4", "11"),    # both in place
    (BF16, F32, 0, 1, 2176, 2176, 128, 0, 1.0, 0.0, "2", "11"),    # both, the two-stage ring
    (F16, F16, 0, 1, 1024, 1030, 200, 0, 1.0, 0.0, "4", "10"),     # ldb = n = 1030: B behind the copy
    # 576 tiles of 128x128: the 256x256 kernel (ring 0) keeps the copies
    (BF16, BF16, 0, 0, 3072, 3080, 64, 8, 1.5, -0.5, "0", "00"),
    (F16, F32, 0, 1, 3080, 3072, 200, 0, 1.0, 0.0, "0", "00"),
])
def test_direct_operands_exact(blas, capfd, it, ot, ta, tb, m, n, k, pad, alpha, beta, ring, direct):
    """16-bit problems on one pass of the 128x128 kernel read an M-contiguous
    A (transa N) and an N-contiguous B (transb T) where they lie (k-rows of
    the tile's 128 m or n staged in LDS and read through transposing reads),
    with no copy (the 256x256 kernel keeps the copies): bit-exact over the padded C with guard bands, both rings, K
    ending inside a stage, leading dimensions above m and n, alpha/beta, fp32
    and 16-bit C; an operand whose columns are off 16-byte boundaries keeps
    its copy. `direct` is the plan's (direct_a, direct_b)."""
    res = []
    plans = logged_plans(capfd, lambda: res.append(
        float_case(blas, it, ot, ta, tb, m, n, k, alpha, beta, pad, (-m) % 8, seed=k + m, guard=True)))
    assert res == [(0, 0)]
    kernel = "tn256" if ring == "0" else "tn128"
    assert len(plans) == 1 and plans[0]["kernel"] == kernel and plans[0]["ring"] == ring, plans
    p = plans[0]
    assert p["direct_a"] + p["direct_b"] == direct and p["split"] == "1", plans
    assert p["copy_a"] == str(1 - ta - int(direct[0])) and p["copy_b"] == str(tb - int(direct[1])), plans


@pytest.mark.parametrize("kind,ta,tb,m,n,k,direct,split", [
    ("i8", 0, 0, 1024, 1040, 400, "10", False),
    ("i8", 1, 1, 1040, 1024, 400, "01", False),
    ("dq", 0, 1, 1024, 1024, 384, "11", False),
    ("i8", 0, 1, 2176, 2176, 256, "11", False),    # 289 tiles: the two-stage ring
    ("i8", 0, 0, 512, 256, 16384, "10", True),     # K slices
    ("i8", 0, 0, 1032, 1040, 400, "00", False),    # m % 16 != 0: behind the copy
])
def test_direct_operands_int8_exact(blas, capfd, kind, ta, tb, m, n, k, direct, split):
    """int8 problems on the 128x128 kernel read an M-contiguous A and an
    N-contiguous B in place (128 k-rows of 128 bytes per stage, fragments
    through ds_read_b64_tr_b8) where m (n) is a multiple of 16: int32 C and
    the dequantised bf16 C bit-exact with guard bands."""
    res = []
    if kind == "i8":
        call = lambda: res.append(int8_case(blas, ta, tb, m, n, k, 2.0, 1.0, 0, fill="rand",  # noqa: E731
                                            seed=k + m, cpad=0, guard=True))
        ok = 0
    else:
        call = lambda: res.append(dequant_case(blas, ta, tb, m, n, k, 0, 0, seed=k, guard=True))  # noqa: E731
        ok = (0, 0)
    plans = logged_plans(capfd, call)
    assert res == [ok]
    p = plans[0]
    assert len(plans) == 1 and p["kernel"] == "tn128" and (int(p["split"]) > 1) == split, plans
    assert p["direct_a"] + p["direct_b"] == direct, plans
    assert p["copy_a"] == str(1 - ta - int(direct[0])) and p["copy_b"] == str(tb - int(direct[1])), plans


@pytest.mark.parametrize("it,ot,ta,tb,m,n,k,cpad,split,staged,direct", [
    (BF16, F32, 0, 0, 512, 256, 4096, 0, True, "0", "10"),     # K slices
    (F16, F16, 1, 1, 512, 264, 4096, 0, True, "0", "01"),
    (BF16, BF16, 0, 1, 1024, 1024, 1000, 1, False, "1", "11"),  # ldc = 1025: C staged, one slice
    (F16, F32, 0, 0, 1024, 512, 8192, 1, True, "1", "10"),      # C staged behind K slices
])
def test_direct_operands_with_slices_and_staged_c(blas, capfd, it, ot, ta, tb, m, n, k, cpad, split,
                                                   staged, direct):
    """The 128x128 kernel's K slices (each slice reading its k-rows of an
    operand in place, kslice rows down) and its staged C (raw partials, then
    the epilogue into an unaligned C) with in-place operands: bit-exact over
    the padded C with guard bands, no copy in the plan."""
    res = []
    plans = logged_plans(capfd, lambda: res.append(
        float_case(blas, it, ot, ta, tb, m, n, k, 1.5, -0.5, 0, cpad, seed=k + m, guard=True)))
    assert res == [(0, 0)]
    p = plans[0]
    assert len(plans) == 1 and p["kernel"] == "tn128" and (int(p["split"]) > 1) == split, plans
    assert p["staged"] == staged and p["direct_a"] + p["direct_b"] == direct, plans
    assert (p["copy_a"], p["copy_b"]) == ("0", "0"), plans


@pytest.mark.parametrize("kind,it,ot,m,n,k", [
    ("f", BF16, F32, 1030, 1100, 64),     # one K stage: the loop's first wait is its last
    ("f", BF16, BF16, 1030, 1100, 64),
    ("f", BF16, F32, 1024, 1056, 2048),   # exactly 32 stages, the plan's upper limit
    ("f", F16, F16, 1030, 1024, 2048),
    ("f", BF16, BF16, 1031, 1100, 200),   # m % 4 != 0: a partial run of rows per lane
    ("f", F16, F32, 1029, 1060, 200),
    ("i8", None, None, 1030, 1100, 128),  # int8: one 128-byte stage, and 32 of them
    ("i8", None, None, 1030, 1100, 4096),
])
def test_tn128_stage_limits_and_ragged_rows(blas, capfd, kind, it, ot, m, n, k):
    """gemm_tn128 at the ends of its K range (1 and 32 stages) and with m not
    a multiple of 4, for fp32 and 16-bit C, bit-exact over the padded C with
    guard bands; the plan must be the 128x128 kernel."""
    res = []
    if kind == "f":
        # ldc = m + cpad keeps C columns on 16-byte boundaries
        cpad = (-m) % 8 if ot != F32 else (-m) % 4
        call = lambda: res.append(float_case(blas, it, ot, 1, 0, m, n, k, 1.0, 0.0, 0, cpad,  # noqa: E731
                                             seed=k + m, guard=True))
        ok = (0, 0)
    else:
        call = lambda: res.append(int8_case(blas, 1, 0, m, n, k, 1.0, 0.0, 0, fill="rand",  # noqa: E731
                                            seed=k, cpad=(-m) % 4, guard=True))
        ok = 0
    plans = logged_plans(capfd, call)
    assert res == [ok], res
    assert len(plans) == 1 and plans[0]["kernel"] == "tn128", plans


def test_tn128_two_stage_ring_exact(blas, capfd):
    """Between 256 and 512 tiles of 128x128 the kernel runs its two-stage LDS
    ring, two workgroups per CU: 16-bit and fp32 C, int8 and dequant, (T, N)
    and (N, N) behind the operand copy, ragged m, n and K, bit-exact over
    the padded C with guard bands; the log must show that ring."""
    m, n = 2312, 2184                     # 19 x 18 = 342 tiles
    cases = [("f", 1, 0, BF16, BF16), ("f", 1, 0, F16, F32), ("f", 0, 0, BF16, F32),
             ("i8", 1, 0, None, None), ("dq", 1, 0, None, None)]
    bad = []
    for kind, ta, tb, it, ot in cases:
        res = []
        if kind == "f":
            call = lambda: res.append(float_case(blas, it, ot, ta, tb, m, n, 136, 1.5, -0.5, 0, 8,  # noqa: E731,B023
                                                 seed=31 + ta, guard=True))
            ok = (0, 0)
        elif kind == "i8":
            call = lambda: res.append(int8_case(blas, ta, tb, m, n, 272, 2.0, 1.0, 0, fill="rand",  # noqa: E731,B023
                                                seed=33, cpad=0, guard=True))
            ok = 0
        else:
            call = lambda: res.append(dequant_case(blas, ta, tb, m, n, 272, 0, 8, seed=35, guard=True))  # noqa: E731,B023
            ok = (0, 0)
        plans = logged_plans(capfd, call)
        if res != [ok] or len(plans) != 1 or plans[0]["kernel"] != "tn128" or plans[0]["ring"] != "2":
            bad.append((kind, ta, tb, it, ot, res, plans))
    assert not bad, bad


@pytest.mark.parametrize("kind,ta,tb,it,ot,k,pad", [
    ("f", 1, 0, BF16, BF16, 1001, 0),   # T,N, K not a multiple of 8
    ("f", 0, 0, F16, F32, 1003, 0),     # N,N
    ("f", 1, 1, BF16, F32, 997, 0),     # T,T
    ("f", 0, 1, F16, F16, 999, 0),      # N,T
    ("f", 1, 0, BF16, BF16, 1024, 1),   # K aligned, lda / ldb odd
    ("i8", 1, 0, None, None, 1001, 0),  # int8: K not a multiple of 16
    ("dq", 0, 0, None, None, 1007, 0),
])
def test_padded_copies_for_unaligned_k(blas, capfd, kind, ta, tb, it, ot, k, pad):
    """K not a multiple of 16 bytes, or operands the TN kernels cannot read as
    they lie, above the copy threshold: both operands are copied K-contiguous
    into rows of K padded with zeros, then the TN kernels run on the padded
    K. Bit-exact over the padded C with guard bands, and the plan shows both
    copies on a TN kernel (no general path)."""
    m, n = 1032, 1100
    res = []
    if kind == "f":
        call = lambda: res.append(float_case(blas, it, ot, ta, tb, m, n, k, 1.5, -0.5, pad, 0,  # noqa: E731
                                             seed=k + pad, guard=True))
        ok = (0, 0)
    elif kind == "i8":
        call = lambda: res.append(int8_case(blas, ta, tb, m, n, k, 2.0, 1.0, pad, fill="rand",  # noqa: E731
                                            seed=k, cpad=0, guard=True))
        ok = 0
    else:
        call = lambda: res.append(dequant_case(blas, ta, tb, m, n, k, pad, 0, seed=k, guard=True))  # noqa: E731
        ok = (0, 0)
    plans = logged_plans(capfd, call)
    assert res == [ok], res
    assert len(plans) == 1 and plans[0]["kernel"] in ("tn128", "tn256"), plans
    assert plans[0]["copy_a"] == "1" and plans[0]["copy_b"] == "1", plans


@pytest.mark.parametrize("kind,ta,tb,it,ot,m,k", [
    ("f", 1, 0, BF16, BF16, 1031, 1024),   # bf16 C, ldc = 1031
    ("f", 1, 0, F16, F32, 1030, 1000),     # fp32 C, ldc * 4 = 4120
    ("f", 0, 0, BF16, BF16, 1027, 1001),   # (N, N), K and C unaligned: padded copies, staged C
    ("f", 1, 0, BF16, F32, 1030, 8192),    # long K: slices, then the staged C
    ("i8", 1, 0, None, None, 1030, 1024),  # int32 C
    ("dq", 1, 0, None, None, 1027, 1024),  # dequantised bf16 C
])
def test_staged_c_for_unaligned_ldc(blas, capfd, kind, ta, tb, it, ot, m, k):
    """C whose columns are not on 16-byte boundaries (ldc = m, m not a
    multiple of 8 for 16-bit C, of 4 for 32-bit C) above the copy threshold:
    the TN kernels write raw partials to the workspace and reduce_splits
    applies alpha, beta and the conversion into C. Bit-exact over the padded
    C with guard bands; the plan shows a TN kernel with C staged."""
    n = 1100
    res = []
    if kind == "f":
        call = lambda: res.append(float_case(blas, it, ot, ta, tb, m, n, k, 1.5, -0.5, 0, 0,  # noqa: E731
                                             seed=m + k, guard=True))
        ok = (0, 0)
    elif kind == "i8":
        call = lambda: res.append(int8_case(blas, ta, tb, m, n, k, 2.0, 1.0, 0, fill="rand",  # noqa: E731
                                            seed=m, cpad=0, guard=True))
        ok = 0
    else:
        call = lambda: res.append(dequant_case(blas, ta, tb, m, n, k, 0, 0, seed=m, guard=True))  # noqa: E731
        ok = (0, 0)
    plans = logged_plans(capfd, call)
    assert res == [ok], res
    assert len(plans) == 1 and plans[0]["kernel"] in ("tn128", "tn256"), plans
    assert plans[0]["staged"] == "1", plans


def test_split_k_workspaces_on_many_streams():
    """Split-K calls rotating over six streams (more than the handle keeps
    workspaces for per device, so workspaces are handed over) with no host
    synchronisation between calls. Every result bit-exact."""
    blas = g.Blas()
    streams = [g.Stream() for _ in range(6)]
    try:
        cases = []
        for i in range(12):
            m, n, k = 256 + 64 * (i % 3), 256, 4096 + 256 * (i % 2)
            st = O.HalvesStream(200 + i)
            A, B = st.take(m * k), st.take(k * n)     # T,N: A^T rows of k, B columns of k
            hA, hB = narrow(A, BF16), narrow(B, BF16)
            want = O.gemm_f32acc(1, 0, m, n, k, 1.0, A, k, B, k, 0.0, np.zeros(m * n, np.float32), m)
            cases.append((m, n, k, to_dev(hA), to_dev(hB), g.DeviceBuffer(m * n * 4), want))
        for i, (m, n, k, dA, dB, dC, _) in enumerate(cases):
            blas.set_stream(streams[i % 6].s)
            say(f"split-k stream case {i}: {m}x{n}x{k} on stream {i % 6}")
            assert blas.gemm_ex(1, 0, m, n, k, 1.0, dA.p, BF16, k, dB.p, BF16, k, 0.0, dC.p, F32,
                                m) == g.SUCCESS
        g.synchronize()
        for m, n, k, dA, dB, dC, want in cases:
            got = dC.download(np.float32, m * n)
            assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))
    finally:
        blas.close()
        for st in streams:
            st.close()


def test_split_k_random_normal_tolerance(blas):
    """1024 x 1024 x 8192 bf16 from N(0,1): split-K result within the
    north-star bound of an fp64 reference."""
    from grxcp_amd import synth
    m = n = 1024
    k = 8192
    a = synth.normal_bf16(m * k, 5)            # A^T rows: k contiguous
    b = synth.normal_bf16(n * k, 6)
    dA, dB, dC = to_dev(a), to_dev(b), g.DeviceBuffer(m * n * 4)
    say("split-k random normal 1024x1024x8192")
    assert blas.gemm_ex(1, 0, m, n, k, 1.0, dA.p, BF16, k, dB.p, BF16, k, 0.0, dC.p, F32, m) == 0
    g.synchronize()
    got = dC.download(np.float32, m * n).reshape(n, m)
    A = O.bf16_to_f32(a).reshape(m, k).astype(np.float64)
    B = O.bf16_to_f32(b).reshape(n, k).astype(np.float64)
    ref = B @ A.T                               # [n][m] = C column-major
    assert normwise_rel_err(got.reshape(-1), ref.reshape(-1)) <= 1e-5


def test_split_k_int8_and_dequant_exact(blas, capfd):
    res = []
    plans = logged_plans(capfd, lambda: res.extend([
        int8_case(blas, 1, 0, 1024, 512, 8192, 3, -2, 0, fill="rand", seed=21),
        int8_case(blas, 1, 0, 300, 260, 8320, 1, 1, 16, fill="rand", seed=22, cpad=4),
        dequant_case(blas, 1, 0, 512, 512, 8192, 0, 0, seed=23)]))
    assert res == [0, 0, (0, 0)]
    assert all(int(p["split"]) >= 2 for p in plans) and len(plans) == 3, plans


def slots_written(blas, call, capacity):
    """Run `call` with a zeroed cycle probe attached; count the slots written."""
    import ctypes
    slot_t = np.dtype([("start", np.uint64), ("end", np.uint64), ("core", np.uint32),
                       ("warp", np.uint32)])
    assert slot_t.itemsize == ctypes.sizeof(g.CycleSlot)
    slots = to_dev(np.zeros(capacity, slot_t))
    assert blas.set_cycle_probe(slots.p, capacity) == g.SUCCESS
    try:
        assert call() == g.SUCCESS
        g.synchronize()
    finally:
        assert blas.set_cycle_probe(None, 0) == g.SUCCESS
    got = slots.download(np.uint8, capacity * slot_t.itemsize).view(slot_t)
    return int(np.count_nonzero(got["end"]))


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 1), (1, 0)])
def test_large_layouts_run_the_tn_kernel(blas, ta, tb):
    """Every layout of a large GemmEx lands on the 256x256-tile kernel (one
    probe slot per wave of its 2x2 tiles), not on the 64x64 general kernel
    (100 slots for this shape)."""
    m, n, k = 320, 264, 512
    a_rows, a_cols = (k, m) if ta else (m, k)
    b_rows, b_cols = (n, k) if tb else (k, n)
    dA, dB = g.DeviceBuffer(a_rows * a_cols * 2), g.DeviceBuffer(b_rows * b_cols * 2)
    dC = g.DeviceBuffer(m * n * 4)
    call = lambda: blas.gemm_ex(ta, tb, m, n, k, 1.0, dA.p, BF16, a_rows, dB.p, BF16, b_rows,  # noqa: E731
                                0.0, dC.p, F32, m)
    assert slots_written(blas, call, blas.cycle_slots_needed(m, n)) == 4 * 2 * 2
    # a probe attached keeps a split-K candidate (few tiles, long K) unsplit
    big = g.DeviceBuffer(256 * 8192 * 2)
    call = lambda: blas.gemm_ex(1, 0, 256, 256, 8192, 1.0, big.p, BF16, 8192, big.p, BF16, 8192,  # noqa: E731
                                0.0, dC.p, F32, 256)
    assert slots_written(blas, call, blas.cycle_slots_needed(256, 256)) == 4
    # below the size threshold the general kernel runs
    call = lambda: blas.gemm_ex(0, 0, 64, 64, 64, 1.0, dA.p, BF16, 64, dB.p, BF16, 64,  # noqa: E731
                                0.0, dC.p, F32, 64)
    assert slots_written(blas, call, blas.cycle_slots_needed(64, 64)) == 4


def int8_case(blas, ta, tb, m, n, k, alpha, beta, pad, fill="ref", seed=0, cpad=None, guard=False):
    """The reference's int8_case (ref test_grxblas_ex.cpp:254-322). With
    `guard`, C sits between guard bands and a changed band counts as one
    wrong element."""
    kk = k if k else 1
    a_rows, a_cols = (kk, m) if ta else (m, kk)
    b_rows, b_cols = (n, kk) if tb else (kk, n)
    lda, ldb, ldc = a_rows + pad, b_rows + pad, m + (pad if cpad is None else cpad)
    if fill == "ref":
        ia = np.arange(lda * a_cols, dtype=np.int64)
        A = ((ia * 7 % 15) - 7).astype(np.int8)
        B = ((np.arange(ldb * b_cols, dtype=np.int64) * 5 % 13) - 6).astype(np.int8)
        C = ((np.arange(ldc * n, dtype=np.int64) * 3 % 41) - 20).astype(np.int32)
    else:
        r = np.random.default_rng(seed)
        A = r.integers(-127, 128, lda * a_cols).astype(np.int8)
        B = r.integers(-127, 128, ldb * b_cols).astype(np.int8)
        C = r.integers(-1000, 1000, ldc * n).astype(np.int32)
    want = O.igemm(ta, tb, m, n, k, int(alpha), A, lda, B, ldb, int(beta), C, ldc)
    dA, dB = to_dev(A), to_dev(B)
    dC = Guarded(C) if guard else to_dev(C)
    say(f"igemm ta={ta} tb={tb} {m}x{n}x{k} a={alpha} b={beta} pad={pad}")
    s = blas.gemm_ex(ta, tb, m, n, k, alpha, dA.p, I8, lda, dB.p, I8, ldb, beta, dC.p, I32, ldc)
    assert s == g.SUCCESS, g.STATUS[s]
    g.synchronize()
    got = dC.download(np.int32, C.size)
    return int(np.sum(got != want)) + (0 if not guard or dC.guards_intact() else 1)


def test_reference_int8_gate(blas):
    # ref test_grxblas_ex.cpp:324-331
    cases = [(0, 0, 32, 32, 16, 1, 0, 0), (0, 0, 16, 16, 32, 1, 0, 0), (0, 0, 5, 3, 7, 1, 0, 0),
             (0, 0, 17, 9, 29, 2, -1, 3), (1, 0, 13, 7, 19, 1, 0, 0), (0, 1, 13, 7, 19, 1, 0, 0),
             (1, 1, 13, 7, 19, 1, 1, 0)]
    bad = [(c, int8_case(blas, *c)) for c in cases]
    assert all(n == 0 for _, n in bad), bad


@pytest.mark.parametrize("m,n,k,pad,cpad", [(256, 256, 128, 0, 0), (300, 200, 272, 16, 4),
                                            (512, 768, 4096, 0, 0), (1, 2, 16, 0, 0),
                                            (1000, 1000, 1040, 0, 0)])
def test_int8_fast_path_exact(blas, m, n, k, pad, cpad):
    assert int8_case(blas, 1, 0, m, n, k, 1, 0, pad, fill="rand", seed=m + n + k, cpad=cpad) == 0
    assert int8_case(blas, 1, 0, m, n, k, 3, -2, pad, fill="rand", seed=m + n + k + 1, cpad=cpad) == 0


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 1)])
def test_int8_transposed_copy_paths_exact(blas, ta, tb):
    assert int8_case(blas, ta, tb, 300, 280, 512, 1, 0, 0, fill="rand", seed=7) == 0
    assert int8_case(blas, ta, tb, 264, 256, 528, 3, -2, 16, fill="rand", seed=8, cpad=0) == 0


def test_int8_refusals(blas):
    d = g.DeviceBuffer(4096)
    # ref test_grxblas_ex.cpp:334-340
    assert blas.gemm_ex(0, 0, 8, 4, 16, 2.5, d.p, I8, 8, d.p, I8, 16, 0.0, d.p, I32, 8) == g.INVALID_VALUE
    assert blas.gemm_ex(0, 0, 8, 4, 16, 1.0, d.p, I8, 8, d.p, I8, 16, 0.5, d.p, I32, 8) == g.INVALID_VALUE
    # ref test_grxblas_ex.cpp:345-371
    assert blas.gemm_ex(1, 0, 4, 4, 8, 1.0, d.p, F16, 4, d.p, F16, 8, 0.0, d.p, F32, 4) == g.INVALID_VALUE
    assert blas.gemm_ex(0, 0, 8, 4, 8, 1.0, d.p, F32, 8, d.p, F16, 8, 0.0, d.p, F32, 8) == g.NOT_SUPPORTED
    assert blas.gemm_ex(0, 0, 8, 4, 8, 1.0, d.p, F16, 2, d.p, F16, 8, 0.0, d.p, F32, 8) == g.INVALID_VALUE
    assert blas.gemm_ex(0, 0, 8, 4, 8, 1.0, d.p, F16, 8, d.p, BF16, 8, 0.0, d.p, F32, 8) == g.NOT_SUPPORTED
    assert blas.gemm_ex(0, 0, 8, 4, 8, 1.0, d.p, I8, 8, d.p, I8, 8, 0.0, d.p, F32, 8) == g.NOT_SUPPORTED
    assert blas.gemm_ex_dequant(0, 0, 8, 4, 8, d.p, I8, 8, d.p, I8, 8, None, d.p, BF16, 8) == g.INVALID_VALUE
    assert blas.gemm_ex_dequant(0, 0, 8, 4, 8, d.p, I8, 8, d.p, I8, 8, d.p, d.p, F32, 8) == g.NOT_SUPPORTED


def dequant_case(blas, ta, tb, m, n, k, pad, cpad, seed, guard=False):
    kk = k if k else 1
    a_rows, a_cols = (kk, m) if ta else (m, kk)
    b_rows, b_cols = (n, kk) if tb else (kk, n)
    lda, ldb, ldc = a_rows + pad, b_rows + pad, m + cpad
    r = np.random.default_rng(seed)
    A = r.integers(-127, 128, lda * a_cols).astype(np.int8)
    B = r.integers(-127, 128, ldb * b_cols).astype(np.int8)
    scale = r.uniform(0.001, 0.01, n).astype(np.float32)
    acc = O.igemm(ta, tb, m, n, k, 1, A, lda, B, ldb, 0, np.zeros(m * n, np.int32), m)
    want = O.dequant(m, n, acc, m, scale, ldc)
    poison = np.full(ldc * n, 0x7FC1, np.uint16)
    dA, dB, dS = to_dev(A), to_dev(B), to_dev(scale)
    dC = Guarded(poison) if guard else to_dev(poison)
    say(f"dequant ta={ta} tb={tb} {m}x{n}x{k} pad={pad}")
    s = blas.gemm_ex_dequant(ta, tb, m, n, k, dA.p, I8, lda, dB.p, I8, ldb, dS.p, dC.p, BF16, ldc)
    assert s == g.SUCCESS, g.STATUS[s]
    g.synchronize()
    got = dC.download(np.uint16, ldc * n)
    inside = window_mask(m, n, ldc)
    stray = int(np.sum((got != poison) & ~inside)) + (0 if not guard or dC.guards_intact() else 1)
    return int(np.sum((got != want) & inside)), stray


@pytest.mark.parametrize("ta,tb,m,n,k,pad,cpad", [
    (1, 0, 256, 256, 256, 0, 0), (1, 0, 300, 260, 528, 16, 4), (0, 0, 37, 29, 45, 3, 3),
    (1, 1, 33, 65, 77, 0, 0), (0, 1, 64, 64, 64, 0, 0), (1, 0, 5, 3, 0, 0, 0),
    # above the size threshold: N,N / N,T / T,T through the transposed copies
    (0, 0, 320, 264, 512, 0, 0), (0, 1, 256, 300, 528, 16, 8), (1, 1, 264, 256, 512, 0, 8),
])
def test_dequant_bit_exact(blas, ta, tb, m, n, k, pad, cpad):
    assert dequant_case(blas, ta, tb, m, n, k, pad, cpad, seed=m * 7 + n + k) == (0, 0)


def test_bf16_random_normal_tolerance(blas):
    """Config-2 distribution (N(0,1) bf16, TN, bf16 out) at 1024^3 and a
    ragged shape: max relative error vs a float64 reference <= 1e-2."""
    for (m, n, k) in [(1024, 1024, 1024), (777, 555, 1000)]:
        r = np.random.default_rng(m)
        A = O.f32_to_bf16(r.standard_normal(m * k).astype(np.float32))   # op(A) row-major m x k
        B = O.f32_to_bf16(r.standard_normal(n * k).astype(np.float32))   # col-major k x n
        dA, dB, dC = to_dev(A), to_dev(B), g.DeviceBuffer(m * n * 2)
        say(f"bf16 normal {m}x{n}x{k}")
        assert blas.gemm_ex(1, 0, m, n, k, 1.0, dA.p, BF16, k, dB.p, BF16, k, 0.0, dC.p, BF16, m) == 0
        g.synchronize()
        got = O.bf16_to_f32(dC.download(np.uint16, m * n))
        ref = O.sgemm(1, 0, m, n, k, 1.0, O.bf16_to_f32(A), k, O.bf16_to_f32(B), k, 0.0,
                      np.zeros(m * n, np.float32), m)
        assert normwise_rel_err(got, ref) <= 1e-2


@pytest.mark.parametrize("size", [8192, 4096])
def test_config2_bf16_full(blas, size):
    """BASELINE config 2 at both of its sizes: bf16 8192^3 and 4096^3, TN
    (row-major A x column-major B), bf16 C. Sampled rows x columns against the
    fp64 oracle on the same bf16 inputs, max relative error <= 1e-2; every
    output finite. At both sizes the whole matrix is also checked against
    numpy's float64 product (an independent BLAS), normwise <= 1e-2 and per
    element within bf16 rounding of the exact value plus the fp32 accumulation
    error."""
    from grxcp_amd import synth
    M = N = K = size
    A = synth.normal_bf16(M * K, 21)   # op(A): row-major M x K  (grxBLAS: transa=T, lda=K)
    B = synth.normal_bf16(N * K, 22)   # column-major K x N      (transb=N, ldb=K)
    dA, dB, dC = to_dev(A), to_dev(B), g.DeviceBuffer(M * N * 2)
    say(f"config2 bf16 {size}^3")
    assert blas.gemm_ex(1, 0, M, N, K, 1.0, dA.p, BF16, K, dB.p, BF16, K, 0.0, dC.p, BF16, M) == 0
    g.synchronize()
    C = O.bf16_to_f32(dC.download(np.uint16, M * N)).reshape(N, M)   # C[j, i] (column-major)
    assert np.isfinite(C).all()
    af = O.bf16_to_f32(A).reshape(M, K).astype(np.float64)
    bf = O.bf16_to_f32(B).reshape(N, K).astype(np.float64)
    full = bf @ af.T                                   # [j, i] like C
    assert normwise_rel_err(C, full) <= 1e-2
    # bf16 output: half an ulp (2^-9 relative) of rounding, plus fp32
    # accumulation over K terms of magnitude |a||b| (~K * 2^-24 * sum|ab|)
    bound = 2.0 ** -8 * np.abs(full) + K * 2.0 ** -23 * (np.abs(bf) @ np.abs(af).T)
    assert np.all(np.abs(C - full) <= bound)
    del af, bf, full, bound
    r = np.random.default_rng(0)
    rows = np.sort(np.concatenate([[0, 255, 256, M - 1], r.choice(M, 12, replace=False)]))
    cols = np.sort(np.concatenate([[0, 255, 256, N - 1], r.choice(N, 124, replace=False)]))
    a = O.bf16_to_f32(A.reshape(M, K)[rows])          # len(rows) x K
    b = O.bf16_to_f32(B.reshape(N, K)[cols])          # len(cols) x K
    m, n = len(rows), len(cols)
    ref = O.sgemm(1, 0, m, n, K, 1.0, a.reshape(-1), K, b.reshape(-1), K, 0.0,
                  np.zeros(m * n, np.float32), m).reshape(n, m)
    got = C[np.ix_(cols, rows)]
    assert normwise_rel_err(got, ref) <= 1e-2


def test_config3_int8_full_size(blas):
    """BASELINE config 3 at full size: M=4096 tokens, K=8192, N=28672; int8
    U[-127,127]. int32 C bit-exact on sampled rows x columns against the
    oracle, plus the whole-matrix checksum identity
    sum_ij C = sum_l (sum_i A[i,l]) (sum_j B[l,j]) and its every row and
    column, and all outputs against float64 BLAS (exact here); then the
    per-channel dequant to bf16 bit-exact on the same samples and over all
    outputs (the oracle's dequant of that int32 C)."""
    from grxcp_amd import synth
    M, K, N = 4096, 8192, 28672
    A = synth.uniform_int8(M * K, 31)   # row-major M x K  (transa=T, lda=K)
    B = synth.uniform_int8(N * K, 32)   # column-major K x N (transb=N, ldb=K)
    scale = synth.uniform_f32(N, 33, 0.001, 0.01)
    dA, dB, dC = to_dev(A), to_dev(B), g.DeviceBuffer(M * N * 4)
    say("config3 int8 int32 full size")
    assert blas.gemm_ex(1, 0, M, N, K, 1.0, dA.p, I8, K, dB.p, I8, K, 0.0, dC.p, I32, M) == 0
    g.synchronize()
    C = dC.download(np.int32, M * N).reshape(N, M)
    colsum_a = A.reshape(M, K).sum(0, dtype=np.int64)
    rowsum_b = B.reshape(N, K).sum(0, dtype=np.int64)
    assert int(C.sum(dtype=np.int64)) == int(np.dot(colsum_a, rowsum_b))
    # every column and every row, exactly: sum_i C[i, j] = (sum_i A[i, :]) . B[:, j]
    # and sum_j C[i, j] = A[i, :] . (sum_j B[:, j]), so each 256 x 256 tile
    # is pinned by the sums of the rows and columns through it
    assert np.array_equal(C.sum(1, dtype=np.int64), B.reshape(N, K).astype(np.int64) @ colsum_a)
    assert np.array_equal(C.sum(0, dtype=np.int64), A.reshape(M, K).astype(np.int64) @ rowsum_b)
    # and all 117 M outputs bit for bit against float64 BLAS: every product
    # (|p| <= 127^2) and every partial sum (|s| < 2^27) is an integer that
    # float64 holds exactly, so the float64 product is the exact int32 result
    full = B.reshape(N, K).astype(np.float64) @ A.reshape(M, K).astype(np.float64).T   # [j, i] like C
    assert np.array_equal(C, full.astype(np.int32))
    del full
    r = np.random.default_rng(1)
    rows = np.sort(np.concatenate([[0, 255, 256, M - 1], r.choice(M, 12, replace=False)]))
    cols = np.sort(np.concatenate([[0, 255, 256, N - 1], r.choice(N, 252, replace=False)]))
    m, n = len(rows), len(cols)
    a = np.ascontiguousarray(A.reshape(M, K)[rows])
    b = np.ascontiguousarray(B.reshape(N, K)[cols])
    want = O.igemm(1, 0, m, n, K, 1, a.reshape(-1), K, b.reshape(-1), K, 0, np.zeros(m * n, np.int32),
                   m).reshape(n, m)
    assert np.array_equal(C[np.ix_(cols, rows)], want)
    dC.close()
    dS, dY = to_dev(scale), g.DeviceBuffer(M * N * 2)
    say("config3 int8 dequant full size")
    assert blas.gemm_ex_dequant(1, 0, M, N, K, dA.p, I8, K, dB.p, I8, K, dS.p, dY.p, BF16, M) == 0
    g.synchronize()
    Y = dY.download(np.uint16, M * N).reshape(N, M)
    yw = O.dequant(m, n, want.reshape(-1), m, scale[cols], m).reshape(n, m)
    assert np.array_equal(Y[np.ix_(cols, rows)], yw)
    # all 117 M bf16 outputs, bit for bit: the oracle's dequant of the int32
    # result checked above (its sampled values exact, its row and column sums
    # exact)
    assert np.array_equal(Y, O.dequant(M, N, C.reshape(-1), M, scale, M).reshape(N, M))
    del C
