"""beta == 0 never reads C, on every GEMM path.

The reference's contract (ref src/libs/grxblas/kernels/sgemm.cpp:80-85, and
the cuBLAS convention its header follows): with beta == 0, C is written and
never read, so a NaN already in C must not reach the result (0 * NaN would).
Every path the planner can pick -- the one-pass 256x256 TN kernel, split K
with its reduction, the 128x128 kernel, the general 64x64 kernel, the
transposed operand copies, the strided batch, the allocation-free entry
point, and Sgemm's small-tile, 256x256 and split-K forms -- runs here with C
filled with NaN. Inside the m x n window the result must equal the oracle's
(computed with C = 0), bit for bit on GemmEx's exact-by-construction inputs;
outside it (ldc padding, gaps between batch members) the NaNs must come back
untouched. The GRXBLAS_LOG line of each call shows the path taken.
"""
import numpy as np
import pytest

import grxcp_amd as g
import oracle as O
from helpers import Guarded, say, to_dev, window_mask
from test_gpu_gemm import logged_plans, narrow, widen

pytestmark = pytest.mark.gpu

F16, BF16, F32 = g.GRX_R_16F, g.GRX_R_16BF, g.GRX_R_32F
NAN16 = np.uint16(0x7FC1)


def nan_fill(n: int, out_t: int) -> np.ndarray:
    if out_t == F32:
        return np.full(n, np.nan, np.float32)
    return np.full(n, NAN16, np.uint16)


def gemm_ex_case(blas, out_t, ta, tb, m, n, k, ldc_pad, seed, noalloc=False):
    """GemmEx bf16 in, `out_t` out, alpha 1.5, beta 0, C all NaN. Returns
    (#wrong in the window, #changed outside it)."""
    a_rows, a_cols = (k, m) if ta else (m, k)
    b_rows, b_cols = (n, k) if tb else (k, n)
    lda, ldb, ldc = a_rows, b_rows, m + ldc_pad
    st = O.HalvesStream(seed)
    A, B = st.take(lda * a_cols), st.take(ldb * b_cols)
    hA, hB = narrow(A, BF16), narrow(B, BF16)
    want = O.gemm_f32acc(ta, tb, m, n, k, 1.5, widen(hA, BF16), lda, widen(hB, BF16), ldb, 0.0,
                         np.zeros(ldc * n, np.float32), ldc)
    c0 = nan_fill(ldc * n, out_t)
    dA, dB, dC = to_dev(hA), to_dev(hB), Guarded(c0)
    say(f"beta0 gemm_ex out={out_t} ta={ta} tb={tb} {m}x{n}x{k} ldc={ldc} noalloc={noalloc}")
    call = blas.gemm_ex_noalloc if noalloc else blas.gemm_ex
    s = call(ta, tb, m, n, k, 1.5, dA.p, BF16, lda, dB.p, BF16, ldb, 0.0, dC.p, out_t, ldc)
    assert s == g.SUCCESS, g.STATUS[s]
    g.synchronize()
    got = dC.download(c0.dtype, c0.size)
    inside = window_mask(m, n, ldc)
    if out_t == F32:
        wrong = got.view(np.uint32) != want.astype(np.float32).view(np.uint32)
    else:
        wrong = got != narrow(want, out_t)
    bits = np.uint32 if got.itemsize == 4 else np.uint16
    stray = int(np.sum((got.view(bits) != c0.view(bits)) & ~inside))
    return int(np.sum(wrong & inside)), stray + (0 if dC.guards_intact() else 1)


@pytest.mark.parametrize("name,out_t,ta,tb,m,n,k,ldc_pad,kernel,split", [
    # more than 512 tiles of 128x128: the 256x256 kernel, one pass
    ("tn256 one pass", BF16, 1, 0, 2944, 2944, 64, 8, "tn256", 0),
    ("tn256 one pass f32 C", F32, 1, 0, 2952, 2944, 80, 4, "tn256", 0),
    ("tn128, two-stage ring", BF16, 1, 0, 2312, 2184, 136, 8, "tn128", 0),
    ("tn128 split K", BF16, 1, 0, 512, 2048, 4096, 8, "tn128", 2),
    ("tn256 split K", BF16, 1, 0, 2048, 1152, 6144, 8, "tn256", 2),
    ("tn128", BF16, 1, 0, 1032, 1100, 200, 8, "tn128", 0),
    ("general64", BF16, 0, 1, 37, 29, 45, 3, "general64", 0),
    ("operand copies (N,N)", BF16, 0, 0, 320, 264, 512, 8, "tn128", 0),
])
def test_gemm_ex_beta_zero_ignores_nan_c(blas, capfd, name, out_t, ta, tb, m, n, k, ldc_pad, kernel, split):
    res = []
    plans = logged_plans(capfd, lambda: res.append(
        gemm_ex_case(blas, out_t, ta, tb, m, n, k, ldc_pad, seed=m + k)))
    assert res == [(0, 0)], (name, res)
    assert len(plans) == 1 and plans[0]["kernel"] == kernel, (name, plans)
    assert (int(plans[0]["split"]) >= 2) == (split >= 2), (name, plans)


def test_gemm_ex_noalloc_beta_zero_ignores_nan_c(blas):
    """The allocation-free entry point on a split-K plan (its partials in the
    static scratch array)."""
    assert gemm_ex_case(blas, BF16, 1, 0, 512, 2048, 2048, 8, seed=5, noalloc=True) == (0, 0)


def test_gemm_strided_batched_ex_beta_zero_ignores_nan_c(blas):
    """Three batch members with NaN gaps between their C blocks; the gaps and
    the ldc padding must come back unchanged."""
    m, n, k, batch = 264, 300, 128, 3
    lda, ldb, ldc = k, k, m + 8
    sa, sb, sc = lda * m + 64, ldb * n + 32, ldc * n + 40
    st = O.HalvesStream(17)
    A, B = st.take(sa * batch), st.take(sb * batch)
    hA, hB = narrow(A, BF16), narrow(B, BF16)
    c0 = nan_fill(sc * batch, BF16)
    dA, dB, dC = to_dev(hA), to_dev(hB), Guarded(c0)
    say(f"beta0 batched {m}x{n}x{k} batch={batch}")
    s = blas.gemm_strided_batched_ex(1, 0, m, n, k, 1.0, dA.p, BF16, lda, sa, dB.p, BF16, ldb, sb, 0.0,
                                     dC.p, BF16, ldc, sc, batch)
    assert s == g.SUCCESS, g.STATUS[s]
    g.synchronize()
    got = dC.download(np.uint16, c0.size)
    inside = np.zeros(c0.size, bool)
    for bi in range(batch):
        want = O.gemm_f32acc(1, 0, m, n, k, 1.0, widen(hA[bi * sa:bi * sa + lda * m], BF16), lda,
                             widen(hB[bi * sb:bi * sb + ldb * n], BF16), ldb, 0.0,
                             np.zeros(ldc * n, np.float32), ldc)
        w = window_mask(m, n, ldc)
        blk = got[bi * sc:bi * sc + ldc * n]
        assert np.array_equal(blk[w], narrow(want, BF16)[w]), bi
        inside[bi * sc:bi * sc + ldc * n] = w
    assert np.array_equal(got[~inside], c0[~inside]) and dC.guards_intact()


@pytest.mark.parametrize("name,ta,tb,m,n,k,kernel,split", [
    ("sgemm_mfma small tiles", 0, 0, 300, 200, 100, None, 0),
    ("tn256 fp32", 1, 0, 4096, 4096, 64, "tn256", 0),
    ("tn256 fp32 split K", 1, 0, 2048, 2048, 1024, "tn256", 4),
])
def test_sgemm_beta_zero_ignores_nan_c(blas, capfd, name, ta, tb, m, n, k, kernel, split):
    lda, ldb, ldc = (k if ta else m), (n if tb else k), m + 4
    A = O.fill_quarters(lda * (m if ta else k), 3)
    B = O.fill_quarters(ldb * (k if tb else n), 5)
    want = O.sgemm(ta, tb, m, n, k, 1.0, A, lda, B, ldb, 0.0, np.zeros(ldc * n, np.float32), ldc)
    c0 = nan_fill(ldc * n, F32)
    dA, dB, dC = to_dev(A), to_dev(B), Guarded(c0)
    res = []

    def call():
        say(f"beta0 sgemm ta={ta} tb={tb} {m}x{n}x{k}")
        res.append(blas.sgemm(ta, tb, m, n, k, 1.0, dA.p, lda, dB.p, ldb, 0.0, dC.p, ldc))
        g.synchronize()
    plans = logged_plans(capfd, call)
    assert res == [g.SUCCESS], g.STATUS[res[0]]
    got = dC.download(np.float32, c0.size)
    inside = window_mask(m, n, ldc)
    assert not np.isnan(got[inside]).any(), name
    assert np.max(np.abs(got[inside] - want[inside])) <= 1e-5 * (k + 1), name    # the reference gate's bound
    assert np.isnan(got[~inside]).all() and dC.guards_intact(), name
    if kernel is None:
        assert plans == [], (name, plans)             # sgemm_mfma logs no GemmEx plan
    else:
        assert len(plans) == 1 and plans[0]["kernel"] == kernel, (name, plans)
        assert int(plans[0]["split"]) == split or (split == 0 and int(plans[0]["split"]) <= 1), (name, plans)
