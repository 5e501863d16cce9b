"""grxblasSgemm / SgemmStridedBatched and level 1/2 on gfx950.

Mirrors the reference's sgemm gate (ref tests/libs/test_grxblas.cpp:265-367):
LCG quarter-integer inputs, tolerance 1e-5*(k+1) inside the m x n window and
BIT-EXACT outside it (stray writes into the padding fail), the batched
tolerance 1e-4*(|exp|+1)*(k+1) over the whole buffer including slack between
batch members, and the BASELINE config-1 problem (512^3, U[-1,1]) at 1e-4
relative against the fp64 oracle. Level 1/2 follow
ref tests/libs/test_grxblas_l12.cpp: small integers, so comparisons are exact.
"""
import numpy as np
import pytest

import grxcp_amd as g
import oracle as O
from helpers import normwise_rel_err, say, to_dev, window_mask

pytestmark = pytest.mark.gpu


def run_case(blas, ta, tb, m, n, k, alpha, beta, pad=0):
    lda = max(1, (k if ta else m) + pad)
    ldb = max(1, (n if tb else k) + pad)
    ldc = max(1, m + pad)
    A = O.fill_quarters(lda * (m if ta else k), 1)
    B = O.fill_quarters(ldb * (k if tb else n), 7)
    C = O.fill_quarters(ldc * n, 13)
    expected = O.sgemm(ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc)
    dA = to_dev(A if A.size else np.zeros(1, np.float32))
    dB = to_dev(B if B.size else np.zeros(1, np.float32))
    dC = to_dev(C)
    say(f"sgemm ta={ta} tb={tb} {m}x{n}x{k} a={alpha} b={beta} pad={pad}")
    s = blas.sgemm(ta, tb, m, n, k, alpha, dA.p, lda, dB.p, ldb, beta, dC.p, ldc)
    assert s == g.SUCCESS, g.STATUS[s]
    g.synchronize()
    got = dC.download(np.float32, C.size)
    inside = window_mask(m, n, ldc)
    tol = 1e-5 * (k + 1)
    bad = np.abs(got - expected) > tol
    stray = got.view(np.uint32) != expected.view(np.uint32)
    return int(np.sum(bad & inside)), int(np.sum(stray & ~inside))


def test_reference_sgemm_gate(blas):
    # ref test_grxblas.cpp:305-317
    cases = [(0, 0, 4, 4, 4, 1.0, 0.0, 0), (0, 0, 8, 5, 3, 1.0, 0.0, 0), (0, 0, 7, 6, 5, 2.5, -1.5, 0),
             (1, 0, 6, 4, 5, 1.0, 0.0, 0), (0, 1, 5, 7, 4, 1.0, 0.0, 0), (1, 1, 4, 5, 6, 1.0, 0.5, 0),
             (0, 0, 16, 16, 16, 1.0, 0.0, 0), (1, 1, 16, 16, 16, 1.0, 0.0, 0), (0, 0, 1, 1, 9, 1.0, 0.0, 0),
             (0, 0, 5, 4, 6, 1.0, 0.0, 3), (1, 1, 6, 5, 4, 2.0, -1.0, 2), (0, 0, 4, 3, 0, 1.0, 2.0, 0)]
    bad = [(c, run_case(blas, *c)) for c in cases]
    assert all(r == (0, 0) for _, r in bad), bad


def test_sgemm_larger_ragged_all_transposes(blas):
    for ta in (0, 1):
        for tb in (0, 1):
            assert run_case(blas, ta, tb, 133, 97, 150, 1.0, 0.5, 5) == (0, 0)


def run_batched(blas, ta, tb, m, n, k, alpha, beta, batch, gap, broadcast_b):
    """ref test_grxblas.cpp:88-172"""
    lda, ldb, ldc = max(1, k if ta else m), max(1, n if tb else k), max(1, m)
    a_el, b_el, c_el = lda * (m if ta else k), ldb * (k if tb else n), ldc * n
    sa, sb, sc = a_el + gap, (0 if broadcast_b else b_el + gap), c_el + gap
    A = O.fill_quarters(sa * (batch - 1) + a_el + gap, 3)
    B = O.fill_quarters((b_el + gap) if broadcast_b else sb * (batch - 1) + b_el + gap, 11)
    C = O.fill_quarters(sc * (batch - 1) + c_el + gap, 17)
    expected = C.copy()
    for bi in range(batch):
        cb = O.sgemm(ta, tb, m, n, k, alpha, A[sa * bi:], lda, B[sb * bi:], ldb, beta,
                     expected[sc * bi:], ldc)
        expected[sc * bi: sc * bi + c_el] = cb[:c_el]
    dA, dB, dC = to_dev(A), to_dev(B), to_dev(C)
    say(f"sgemm batched ta={ta} tb={tb} {m}x{n}x{k} batch={batch} gap={gap} bcast={broadcast_b}")
    s = blas.sgemm_strided_batched(ta, tb, m, n, k, alpha, dA.p, lda, sa, dB.p, ldb, sb, beta, dC.p,
                                   ldc, sc, batch)
    assert s == g.SUCCESS, g.STATUS[s]
    g.synchronize()
    got = dC.download(np.float32, C.size)
    return int(np.sum(np.abs(got - expected) > 1e-4 * (np.abs(expected) + 1) * (k + 1)))


def test_reference_batched_gate(blas):
    # ref test_grxblas.cpp:320-333
    assert run_batched(blas, 0, 0, 6, 5, 4, 1.0, 0.0, 3, 0, False) == 0
    assert run_batched(blas, 0, 0, 6, 5, 4, 2.0, -1.0, 4, 7, False) == 0
    assert run_batched(blas, 0, 0, 6, 5, 4, 1.0, 0.0, 3, 5, True) == 0
    assert run_batched(blas, 1, 1, 5, 4, 6, 1.0, 0.5, 3, 3, False) == 0
    assert run_batched(blas, 0, 0, 7, 3, 5, 1.0, 0.0, 1, 4, False) == 0


def test_large_sgemm_runs_the_256_tile_kernel(blas, capfd):
    """Problems that fill the GPU with 256x256 tiles run the GemmEx TN kernel
    on fp32 (the other layouts behind K-contiguous copies): a batch of 64
    512x512 products in every layout, gaps between batch members and a
    broadcast B, and a ragged batched shape; the batched gate's tolerance over
    the whole buffer, gaps included. The library's GRXBLAS_LOG line names the
    kernel each call ran."""
    from test_gpu_gemm import logged_plans
    cases = [(ta, tb, 512, 512, 132, 1.5, -0.5, 64, 4, tb == 1) for ta in (0, 1) for tb in (0, 1)]
    cases += [(0, 0, 300, 500, 240, 1.0, 0.0, 64, 0, False), (1, 0, 300, 500, 240, 1.0, 1.0, 64, 8, True)]
    for c in cases:
        res = []
        plans = logged_plans(capfd, lambda: res.append(run_batched(blas, *c)))
        assert res == [0], (c, res)
        assert len(plans) == 1 and plans[0]["kernel"] == "tn256", (c, plans)
        assert plans[0]["copy_a"] == str(int(not c[0])) and plans[0]["copy_b"] == str(int(c[1])), (c, plans)


def test_sgemm_split_k_on_the_256_tile_kernel(blas, capfd):
    """Too few 256x256 tiles for the GPU but long enough in K: the fp32 problem
    is split along K (64 tiles x 4 slices) on the same kernel, after the
    operand copy for (N, N); the reference gate's tolerance in the m x n
    window and bit-exact padding, against the oracle."""
    from test_gpu_gemm import logged_plans
    for ta in (1, 0):
        res = []
        plans = logged_plans(capfd, lambda: res.append(run_case(blas, ta, 0, 2048, 2048, 1024, 1.0, 0.5)))
        assert res == [(0, 0)], (ta, res)
        assert len(plans) == 1 and plans[0]["kernel"] == "tn256" and int(plans[0]["split"]) == 4, plans


def test_large_sgemm_workspaces_on_many_streams(capfd):
    """(N, N) Sgemm on the 256x256 kernel copies A into the workspace of the
    calling stream: twelve calls rotating over six streams (more than the
    handle keeps workspaces for, so workspaces are handed over) with no host
    synchronisation between them, each bit-equal to the same call made alone
    and synchronised, and the first of those within the gate's tolerance of
    the oracle."""
    m = n = 512
    k, batch = 128, 64
    blas = g.Blas()
    streams = [g.Stream() for _ in range(6)]
    try:
        sets = []
        for j in range(3):
            A = O.fill_quarters(m * k * batch, 40 + j)
            B = O.fill_quarters(k * n * batch, 50 + j)
            sets.append((A, to_dev(A), B, to_dev(B)))
        def call(j, dC):
            _, dA, _, dB = sets[j]
            return blas.sgemm_strided_batched(0, 0, m, n, k, 1.0, dA.p, m, m * k, dB.p, k, k * n, 0.0,
                                              dC.p, m, m * n, batch)
        from test_gpu_gemm import logged_plans
        alone = []
        for j in range(3):
            dC = g.DeviceBuffer(m * n * batch * 4)
            st = []
            plans = logged_plans(capfd, lambda: st.append(call(j, dC)))
            assert st == [g.SUCCESS]
            assert len(plans) == 1 and plans[0]["kernel"] == "tn256" and plans[0]["copy_a"] == "1", plans
            g.synchronize()
            alone.append(dC.download(np.float32, m * n * batch))
        A0, _, B0, _ = sets[0]
        want = O.sgemm(0, 0, m, n, k, 1.0, A0, m, B0, k, 0.0, np.zeros(m * n, np.float32), m)
        assert np.max(np.abs(alone[0][:m * n] - want)) <= 1e-5 * (k + 1)
        outs = []
        for i in range(12):
            blas.set_stream(streams[i % 6].s)
            dC = g.DeviceBuffer(m * n * batch * 4)
            say(f"sgemm stream case {i}: set {i % 3} on stream {i % 6}")
            assert call(i % 3, dC) == g.SUCCESS
            outs.append(dC)
        g.synchronize()
        for i, dC in enumerate(outs):
            got = dC.download(np.float32, m * n * batch)
            assert np.array_equal(got.view(np.uint32), alone[i % 3].view(np.uint32)), i
    finally:
        blas.close()
        for st in streams:
            st.close()


def test_config1_sgemm_512_cubed(blas):
    """fp32 C = A*B, 512^3 row-major, alpha=1 beta=0, U[-1,1]
    from seeds 1 and 2, mapped to column-major as C^T = B^T A^T:
    Sgemm(N, N, m=512, n=512, k=512, B, 512, A, 512, C, 512)."""
    from grxcp_amd import synth
    M = N = K = 512
    A = synth.uniform_f32(M * K, 1, -1.0, 1.0)   # row-major M x K
    B = synth.uniform_f32(K * N, 2, -1.0, 1.0)   # row-major K x N
    dA, dB, dC = to_dev(A), to_dev(B), g.DeviceBuffer(M * N * 4)
    say("config1 sgemm 512^3")
    assert blas.sgemm(0, 0, N, M, K, 1.0, dB.p, N, dA.p, K, 0.0, dC.p, N) == 0
    g.synchronize()
    got = dC.download(np.float32, M * N)           # = row-major C
    ref = O.sgemm(0, 0, N, M, K, 1.0, B, N, A, K, 0.0, np.zeros(M * N, np.float32), N)
    assert normwise_rel_err(got, ref) <= 1e-4
    # and against numpy as an independent row-major statement
    np.testing.assert_allclose(got.reshape(M, N), A.reshape(M, K).astype(np.float64)
                               @ B.reshape(K, N).astype(np.float64), rtol=0, atol=1e-4)


# ---- level 1 / 2 (ref tests/libs/test_grxblas_l12.cpp) ----------------------

def blas_index(i, n, inc):
    return i * inc if inc > 0 else (n - 1 - i) * (-inc)


def span(n, inc):
    return 0 if n <= 0 else (n - 1) * abs(inc) + 1


@pytest.mark.parametrize("n,incx,incy", [(1, 1, 1), (37, 1, 1), (1000, 2, 3), (64, -1, 1), (65, 2, -3)])
def test_saxpy(blas, n, incx, incy):
    x = (np.arange(span(n, incx)) % 7 - 3).astype(np.float32)
    y = (np.arange(span(n, incy)) % 5 - 2).astype(np.float32)
    want = y.copy()
    for i in range(n):
        want[blas_index(i, n, incy)] += 3.0 * x[blas_index(i, n, incx)]
    dx, dy = to_dev(x), to_dev(y)
    say(f"saxpy n={n} incx={incx} incy={incy}")
    assert blas.L.grxblasSaxpy(blas.h, n, g.fptr(3.0), dx.p, incx, dy.p, incy) == 0
    g.synchronize()
    assert np.array_equal(dy.download(np.float32, y.size), want)


@pytest.mark.parametrize("n,incx", [(1, 1), (100, 1), (33, 3)])
def test_sscal(blas, n, incx):
    x = (np.arange(span(n, incx)) % 9 - 4).astype(np.float32)
    want = x.copy()
    want[: span(n, incx): incx] *= -2.0
    dx = to_dev(x)
    say(f"sscal n={n} incx={incx}")
    assert blas.L.grxblasSscal(blas.h, n, g.fptr(-2.0), dx.p, incx) == 0
    g.synchronize()
    assert np.array_equal(dx.download(np.float32, x.size), want)


@pytest.mark.parametrize("trans", [0, 1])
@pytest.mark.parametrize("m,n,lda,incx,incy,beta", [(7, 5, 7, 1, 1, 0.0), (33, 17, 40, 2, -1, 2.0),
                                                    (300, 260, 301, -1, 3, 0.0)])
def test_sgemv(blas, trans, m, n, lda, incx, incy, beta):
    A = (np.arange(lda * n) % 11 - 5).astype(np.float32)
    xl, yl = (m, n) if trans else (n, m)
    x = (np.arange(span(xl, incx)) % 3 - 1).astype(np.float32)
    y = (np.arange(span(yl, incy)) % 4).astype(np.float32)
    if beta == 0.0:
        y[:] = np.nan  # beta == 0 must not read y
    Am = A.reshape(n, lda)[:, :m].T.astype(np.float64)   # m x n
    op = Am.T if trans else Am
    xv = np.array([x[blas_index(i, xl, incx)] for i in range(xl)], np.float64)
    res = 2.0 * (op @ xv)
    want = y.copy()
    for i in range(yl):
        yi = blas_index(i, yl, incy)
        want[yi] = res[i] + (beta * y[yi] if beta != 0.0 else 0.0)
    dA, dx, dy = to_dev(A), to_dev(x), to_dev(y)
    say(f"sgemv trans={trans} {m}x{n}")
    assert blas.L.grxblasSgemv(blas.h, trans, m, n, g.fptr(2.0), dA.p, lda, dx.p, incx, g.fptr(beta),
                               dy.p, incy) == 0
    g.synchronize()
    got = dy.download(np.float32, y.size)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(got[~np.isnan(want)], want[~np.isnan(want)].astype(np.float32))
