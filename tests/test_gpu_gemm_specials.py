"""IEEE special values and subnormals through the GEMM paths.

The oracle follows IEEE arithmetic (ref tests/libs/test_grxblas.cpp:63-80 and
test_grxblas_ex.cpp:45-63 accumulate in plain C float/double): a NaN operand
poisons its row or column of C, Inf * 0 is NaN, Inf plus finite stays Inf,
and subnormal inputs and products are kept, not flushed. The matrix cores
must agree on every path: results are compared bit for bit on the
exact-by-construction GemmEx inputs (NaN positions compared as positions),
with the fp16 subnormals written as bit patterns (the reference's own
float -> half helper, ref tests/common/fp16.h:21-62, flushes them; fp16 C is
compared with IEEE rounding, subnormals kept, for the same reason), and
Sgemm's finite cells at the reference gate's bound, its special and
subnormal cells exactly.
"""
import numpy as np
import pytest

import grxcp_amd as g
import oracle as O
from helpers import say, to_dev
from test_gpu_gemm import logged_plans, narrow, widen

pytestmark = pytest.mark.gpu

F16, BF16, F32 = g.GRX_R_16F, g.GRX_R_16BF, g.GRX_R_32F


def plant_specials(A: np.ndarray, B: np.ndarray, in_t: int) -> tuple[np.ndarray, np.ndarray]:
    """A (m rows of k) and B (n rows of k) as narrow bit patterns, with NaN,
    +-Inf, Inf * 0 and subnormal rows planted. C[i, j] = sum_l A[i, l] B[j, l]."""
    A, B = A.copy(), B.copy()
    A[0, 0] = np.nan                      # row 0 of C: NaN
    A[1, 1] = np.inf                      # row 1: +-Inf, NaN where B[j, 1] == 0
    B[2, 1] = 0.0
    B[3, 5] = -np.inf                     # column 3: -+Inf, NaN where A[i, 5] == 0
    A[4, 5] = 0.0
    hA, hB = narrow(A.ravel(), in_t).reshape(A.shape), narrow(B.ravel(), in_t).reshape(B.shape)
    if in_t == F16:
        hA[10, :] = 0x0010                # 2^-20, subnormal in fp16
        hA[12, :] = 0x0001                # 2^-24, the smallest subnormal
    else:
        hA[10, :] = 0x0004                # 2^-131, subnormal in bf16
        hA[12, :] = 0x0d00                # 2^-101: normal, but its products with 2^-30 are not
    one = 0x3c00 if in_t == F16 else 0x3f80
    hB[11, :] = one
    hB[13, :] = one if in_t == F16 else 0x3080   # bf16 2^-30
    return hA, hB


@pytest.mark.parametrize("in_t,out_t", [(BF16, F32), (BF16, BF16), (F16, F32), (F16, F16)])
@pytest.mark.parametrize("name,ta,tb,m,n,k,kernel,split", [
    ("tn256", 1, 0, 2944, 2944, 64, "tn256", False),     # over 512 tiles of 128x128
    ("general64", 1, 0, 37, 29, 45, "general64", False),
    ("split K", 1, 0, 512, 2048, 4096, "tn128", True),
    ("split K, 256x256 tiles", 1, 0, 2048, 1152, 6144, "tn256", True),
    ("tn128", 1, 0, 1032, 1100, 200, "tn128", False),
    ("operand copy (N,N)", 0, 0, 320, 264, 512, "tn128", False),
])
def test_gemm_ex_specials_and_subnormals(blas, capfd, in_t, out_t, name, ta, tb, m, n, k, kernel, split):
    st = O.HalvesStream(m + n + k)
    A0 = st.take(m * k).reshape(m, k)
    B0 = st.take(n * k).reshape(n, k)
    hA, hB = plant_specials(A0, B0, in_t)
    # the library's layout: op(A) = A (m x k); ta=1 stores it as m rows of k
    # (lda = k), ta=0 as k rows of m (lda = m)
    a_store = hA if ta else np.ascontiguousarray(hA.T)
    lda = k if ta else m
    b_store = hB                          # tb=0: B stored as n columns of k (ldb = k)
    Aw, Bw = widen(hA.ravel(), in_t), widen(hB.ravel(), in_t)
    want = O.gemm_f32acc(1, 0, m, n, k, 1.0, Aw, k, Bw, k, 0.0, np.zeros(m * n, np.float32), m)
    dA, dB = to_dev(a_store.ravel()), to_dev(b_store.ravel())
    c0 = np.zeros(m * n, np.float32 if out_t == F32 else np.uint16)
    dC = to_dev(c0)
    res = []

    def call():
        say(f"specials {name} in={in_t} out={out_t} {m}x{n}x{k}")
        res.append(blas.gemm_ex(ta, tb, m, n, k, 1.0, dA.p, in_t, lda, dB.p, in_t, k, 0.0, dC.p, out_t, m))
        g.synchronize()
    plans = logged_plans(capfd, call)
    assert res == [g.SUCCESS], res
    assert len(plans) == 1 and plans[0]["kernel"] == kernel, plans
    assert (int(plans[0]["split"]) >= 2) == split, plans
    if out_t == F32:
        got = dC.download(np.float32, m * n)
        ref = want
    elif out_t == BF16:
        got = widen(dC.download(np.uint16, m * n), BF16)
        ref = widen(narrow(want, BF16), BF16)
    else:
        # IEEE round to nearest even with subnormals kept (numpy's float16);
        # the reference's float -> half test helper flushes them
        got = dC.download(np.uint16, m * n).view(np.float16).astype(np.float32)
        ref = want.astype(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan), (name, int(np.isnan(got).sum()), int(nan.sum()))
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32)), name
    assert np.isinf(ref).sum() > 0 and nan.sum() > 0       # the planted specials reach C
    sub = ref[11 * m + 10], ref[13 * m + 12]
    assert all(v != 0.0 for v in sub)                       # the subnormal rows are not flushed


@pytest.mark.parametrize("name,m,n,k,kernel", [
    ("sgemm_mfma", 300, 200, 100, None),
    ("tn256 fp32", 4096, 4096, 64, "tn256"),
])
def test_sgemm_specials_and_subnormals(blas, capfd, name, m, n, k, kernel):
    A = O.fill_quarters(k * m, 3).reshape(m, k)
    B = O.fill_quarters(k * n, 5).reshape(n, k)
    A[0, 0] = np.nan
    A[1, 1] = np.inf
    B[2, 1] = 0.0
    A[10, :] = 2.0 ** -130                # subnormal fp32 input
    B[11, :] = 1.0
    A[12, :] = 2.0 ** -100                # normal inputs, subnormal products
    B[13, :] = 2.0 ** -30
    want = O.sgemm(1, 0, m, n, k, 1.0, A.ravel(), k, B.ravel(), k, 0.0, np.zeros(m * n, np.float32), m)
    dA, dB, dC = to_dev(A.ravel()), to_dev(B.ravel()), to_dev(np.zeros(m * n, np.float32))
    res = []

    def call():
        say(f"specials {name} {m}x{n}x{k}")
        res.append(blas.sgemm(1, 0, m, n, k, 1.0, dA.p, k, dB.p, k, 0.0, dC.p, m))
        g.synchronize()
    plans = logged_plans(capfd, call)
    assert res == [g.SUCCESS], res
    assert (plans == []) if kernel is None else (len(plans) == 1 and plans[0]["kernel"] == kernel), plans
    got = dC.download(np.float32, m * n)
    special = ~np.isfinite(want)
    assert np.array_equal(np.isnan(got), np.isnan(want)) and np.array_equal(np.isinf(got), np.isinf(want))
    assert np.array_equal(got[special & ~np.isnan(want)], want[special & ~np.isnan(want)])
    assert np.max(np.abs(got[~special] - want[~special])) <= 1e-5 * (k + 1)
    for i, j in ((10, 11), (12, 13)):     # subnormal sums, kept exactly
        assert got[j * m + i] == want[j * m + i] != 0.0, (i, j, got[j * m + i], want[j * m + i])


I8, I32 = g.GRX_R_8I, g.GRX_R_32I


@pytest.mark.parametrize("alpha,beta", [(1, 0), (3, -2)])
def test_int8_full_range_and_int32_wraparound(blas, capfd, alpha, beta):
    """int8 operands over the whole range, -128 included, and a K long enough
    that one accumulator passes 2^31: row 0 of A and column 0 of B all -128,
    so C[0, 0] = 131328 * 16384 = 2151677952, which wraps to -2143289344
    as in the oracle's (and C's) int32 arithmetic; alpha and beta also apply
    in wrapping int32. Few tiles and a long K: the problem is split along K,
    so the wrap passes through the partial sums and their reduction."""
    m, n, k = 64, 96, 131328
    r = np.random.default_rng(alpha + 7)
    A = r.integers(-128, 128, (m, k)).astype(np.int8)     # ta=1: m rows of k
    B = r.integers(-128, 128, (n, k)).astype(np.int8)     # tb=0: n columns of k
    A[0, :] = -128
    B[0, :] = -128
    C = r.integers(-1000, 1000, m * n).astype(np.int32)
    want = O.igemm(1, 0, m, n, k, alpha, A.ravel(), k, B.ravel(), k, beta, C, m)
    exact = alpha * k * 16384 + beta * int(C[0])
    assert exact > 2 ** 31 - 1 and int(want[0]) == (exact + 2 ** 31) % 2 ** 32 - 2 ** 31
    dA, dB, dC = to_dev(A.ravel()), to_dev(B.ravel()), to_dev(C)
    res = []

    def call():
        say(f"int8 wrap {m}x{n}x{k} alpha={alpha} beta={beta}")
        res.append(blas.gemm_ex(1, 0, m, n, k, float(alpha), dA.p, I8, k, dB.p, I8, k, float(beta),
                                dC.p, I32, m))
        g.synchronize()
    plans = logged_plans(capfd, call)
    assert res == [g.SUCCESS], res
    assert len(plans) == 1 and int(plans[0]["split"]) >= 2, plans
    got = dC.download(np.int32, m * n)
    assert np.array_equal(got, want), int(np.sum(got != want))


def test_int8_dequant_of_a_wrapped_accumulator(blas):
    """GemmExDequant takes the same wrapped int32 accumulator through
    float(acc) * scale to bf16, bit-exact against the oracle."""
    m, n, k = 64, 96, 131328
    r = np.random.default_rng(11)
    A = r.integers(-128, 128, (m, k)).astype(np.int8)
    B = r.integers(-128, 128, (n, k)).astype(np.int8)
    A[0, :] = -128
    B[0, :] = -128
    scale = r.uniform(0.001, 0.01, n).astype(np.float32)
    acc = O.igemm(1, 0, m, n, k, 1, A.ravel(), k, B.ravel(), k, 0, np.zeros(m * n, np.int32), m)
    want = O.dequant(m, n, acc, m, scale, m)
    dA, dB, dS = to_dev(A.ravel()), to_dev(B.ravel()), to_dev(scale)
    dC = to_dev(np.zeros(m * n, np.uint16))
    say(f"dequant wrap {m}x{n}x{k}")
    s = blas.gemm_ex_dequant(1, 0, m, n, k, dA.p, I8, k, dB.p, I8, k, dS.p, dC.p, BF16, m)
    assert s == g.SUCCESS, g.STATUS[s]
    g.synchronize()
    got = dC.download(np.uint16, m * n)
    assert np.array_equal(got, want), int(np.sum(got != want))
    assert acc[0] < 0                                      # the wrapped value went through
