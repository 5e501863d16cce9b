"""grxblasGemmExNoAlloc against grxblasGemmEx, through the C ABI, on the GPU.

The allocation-free entry point runs grxblasGemmEx's plans with the
library's static per-device scratch in place of the handle's workspace, so
its output must be bit-identical to grxblasGemmEx's on the same inputs. Two
calls in a row, the second smaller than the first, each on a plan that uses
the scratch (split-K partials, then a transposed operand copy); a problem
that needs more scratch than the library holds is refused before anything is
launched, and its output buffer is left as it was.
"""
import numpy as np
import pytest

import grxcp_amd as g
from grxcp_amd import synth
from helpers import say, to_dev
from test_gpu_gemm import logged_plans

pytestmark = pytest.mark.gpu

BF16, F32, I8, I32 = g.GRX_R_16BF, g.GRX_R_32F, g.GRX_R_8I, g.GRX_R_32I


def _pair(blas, capfd, ta, tb, m, n, k, it, ot, seed):
    """Run GemmEx and GemmExNoAlloc on the same inputs; return both outputs
    and the two logged plans."""
    r = np.random.default_rng(seed)
    a_rows, a_cols = (k, m) if ta else (m, k)
    b_rows, b_cols = (n, k) if tb else (k, n)
    if it == I8:
        A = r.integers(-127, 128, a_rows * a_cols).astype(np.int8)
        B = r.integers(-127, 128, b_rows * b_cols).astype(np.int8)
        ctype, esize = np.int32, 4
    else:
        A = synth.f32_to_bf16_bits(r.standard_normal(a_rows * a_cols).astype(np.float32))
        B = synth.f32_to_bf16_bits(r.standard_normal(b_rows * b_cols).astype(np.float32))
        ctype, esize = (np.float32, 4) if ot == F32 else (np.uint16, 2)
    dA, dB = to_dev(A), to_dev(B)
    poison = np.full(m * n, 0x7FC1 if esize == 2 else 0x7FC00001, np.uint16 if esize == 2 else np.uint32)
    dC1, dC2 = to_dev(poison), to_dev(poison)
    say(f"noalloc pair ta={ta} tb={tb} {m}x{n}x{k} in={it} out={ot}")
    plans = []
    for fn, dC in ((blas.gemm_ex, dC1), (blas.gemm_ex_noalloc, dC2)):
        got = logged_plans(capfd, lambda: plans.append(  # noqa: B023
            fn(ta, tb, m, n, k, 1.0, dA.p, it, a_rows, dB.p, it, b_rows, 0.0, dC.p, ot, m)))
        plans.append(got)
    g.synchronize()
    assert plans[0] == g.SUCCESS and plans[2] == g.SUCCESS, (plans[0], plans[2])
    c1 = dC1.download(ctype, m * n)
    c2 = dC2.download(ctype, m * n)
    return c1, c2, plans[1], plans[3]


def test_noalloc_matches_gemm_ex_on_two_calls_in_a_row(blas, capfd):
    # 1: few tiles, long K -> split-K partials in the scratch (13 slices of
    #    1024 x 1024 fp32 = 52 MiB)
    c1, c2, p1, p2 = _pair(blas, capfd, 1, 0, 1024, 1024, 8192, BF16, BF16, seed=1)
    assert p1 == p2 and len(p2) == 1 and int(p2[0]["split"]) > 1, (p1, p2)
    assert np.array_equal(c1.view(np.uint16), c2.view(np.uint16))
    # 2: smaller, (N, N) -> the transposed copy of A in the scratch, fp32 C
    c1, c2, p1, p2 = _pair(blas, capfd, 0, 0, 768, 512, 2048, BF16, F32, seed=2)
    assert p1 == p2 and len(p2) == 1 and p2[0]["copy_a"] == "1", (p1, p2)
    assert np.array_equal(c1.view(np.uint32), c2.view(np.uint32))


def test_noalloc_int8_and_no_scratch_plans(blas, capfd):
    # int8 split-K (int32 partials) and a plain TN problem that needs no scratch
    c1, c2, p1, p2 = _pair(blas, capfd, 1, 0, 512, 512, 16384, I8, I32, seed=3)
    assert p1 == p2 and int(p2[0]["split"]) > 1, (p1, p2)
    assert np.array_equal(c1, c2)
    c1, c2, p1, p2 = _pair(blas, capfd, 1, 0, 640, 384, 256, BF16, F32, seed=4)
    assert p1 == p2 and p2[0]["split"] == "1" and p2[0]["copy_a"] == "0", (p1, p2)
    assert np.array_equal(c1.view(np.uint32), c2.view(np.uint32))


def test_noalloc_refuses_more_scratch_than_it_holds(blas, capfd):
    """(N, N) 4096 x 4096 x 8200 bf16 would copy A (4096 x 8200 bf16, 67 MB)
    into more than the 64 MiB scratch: NOT_SUPPORTED with a message, nothing
    launched, C untouched. The buffers are full size, so nothing could
    fault even if a launch happened."""
    m, n, k = 4096, 4096, 8200
    dA, dB = g.DeviceBuffer(m * k * 2), g.DeviceBuffer(k * n * 2)
    poison = np.full(m * n, 0x7FC00001, np.uint32)
    dC = to_dev(poison)
    capfd.readouterr()
    s = blas.gemm_ex_noalloc(0, 0, m, n, k, 1.0, dA.p, BF16, m, dB.p, BF16, k, 0.0, dC.p, F32, m)
    err = capfd.readouterr().err
    g.synchronize()
    assert s == g.NOT_SUPPORTED, g.STATUS[s]
    assert "grxblasGemmExNoAlloc" in err and "scratch" in err
    assert np.array_equal(dC.download(np.uint32, m * n), poison)
