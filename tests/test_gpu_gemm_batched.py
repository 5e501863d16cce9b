"""grxblasGemmStridedBatchedEx on gfx950 against the CPU oracle, batch by batch.

The batched entry point has no counterpart in the reference; it combines
GemmEx's type triples and alpha/beta rules (ref tests/libs/test_grxblas_ex.cpp)
with SgemmStridedBatched's stride convention (ref tests/libs/test_grxblas.cpp:
320-348: signed strides in elements, zero stride broadcasts). Inputs are the
GemmEx gate's exact-by-construction halves (or int8), so every batch must match
the oracle's GemmEx BIT-EXACTLY, and the C elements between batches (a stride
larger than one C) must come back as uploaded.
"""
import ctypes

import numpy as np
import pytest

import grxcp_amd as g
import oracle as O
from helpers import say, to_dev

pytestmark = pytest.mark.gpu

F16, BF16, F32, I8, I32 = g.GRX_R_16F, g.GRX_R_16BF, g.GRX_R_32F, g.GRX_R_8I, g.GRX_R_32I


def narrow(vals, t):
    return O.f32_to_half(vals) if t == F16 else O.f32_to_bf16(vals)


def widen(bits, t):
    return O.half_to_f32(bits) if t == F16 else O.bf16_to_f32(bits)


def slabs(size, batch, mode, align=16):
    """(stride, total elements, offset of the pointer passed, offset of batch b)."""
    packed = -(-size // align) * align + (align if mode == "gap" else 0)
    if mode == "zero":
        return 0, size, 0, lambda b: 0
    if mode == "neg":
        return -packed, packed * (batch - 1) + size, packed * (batch - 1), \
            lambda b: packed * (batch - 1 - b)
    return packed, packed * (batch - 1) + size, 0, lambda b: packed * b


def batched_case(blas, in_t, out_t, ta, tb, m, n, k, alpha, beta, batch, amode, bmode, cmode,
                 seed=7):
    """Returns the number of C elements (window, padding and gaps) that differ."""
    kk = k if k else 1
    a_rows, a_cols = (kk, m) if ta else (m, kk)
    b_rows, b_cols = (n, kk) if tb else (kk, n)
    lda, ldb, ldc = a_rows, b_rows, m
    sa, na, pa, oa = slabs(lda * a_cols, batch, amode)
    sb, nb, pb, ob = slabs(ldb * b_cols, batch, bmode)
    sc, nc, pc, oc = slabs(ldc * n, batch, cmode)
    st = O.HalvesStream(seed)
    eb = 1 if in_t == I8 else 2
    if in_t == I8:
        r = np.random.default_rng(seed)
        A = r.integers(-127, 128, na).astype(np.int8)
        B = r.integers(-127, 128, nb).astype(np.int8)
        C = r.integers(-1000, 1000, nc).astype(np.int32)
        hA, hB, c_host = A, B, C
    else:
        A, B, C = st.take(na), st.take(nb), st.take(nc) * 2.0
        hA, hB = narrow(A, in_t), narrow(B, in_t)
        c_host = C if out_t == F32 else narrow(C, out_t)
    expected = c_host.copy()
    for b in range(batch):
        a0, b0, c0 = oa(b), ob(b), oc(b)
        Ab, Bb = A[a0:a0 + lda * a_cols], B[b0:b0 + ldb * b_cols]
        Cb = c_host[c0:c0 + ldc * n]
        if in_t == I8:
            res = O.igemm(ta, tb, m, n, k, int(alpha), Ab, lda, Bb, ldb, int(beta), Cb, ldc)
        elif out_t == F32:
            res = O.gemm_f32acc(ta, tb, m, n, k, alpha, Ab, lda, Bb, ldb, beta, Cb, ldc)
        else:
            res = narrow(O.gemm_f32acc(ta, tb, m, n, k, alpha, Ab, lda, Bb, ldb, beta,
                                       widen(Cb, out_t), ldc), out_t)
        expected[c0:c0 + ldc * n] = res
    dA, dB, dC = to_dev(hA), to_dev(hB), to_dev(c_host)
    osz = c_host.itemsize
    say(f"gemm_strided_batched_ex in={in_t} out={out_t} ta={ta} tb={tb} {m}x{n}x{k} "
        f"batch={batch} a={amode} b={bmode} c={cmode}")
    s = blas.gemm_strided_batched_ex(
        ta, tb, m, n, k, alpha, ctypes.c_void_p(dA.ptr.value + pa * eb), in_t, lda, sa,
        ctypes.c_void_p(dB.ptr.value + pb * eb), in_t, ldb, sb, beta,
        ctypes.c_void_p(dC.ptr.value + pc * osz), out_t, ldc, sc, batch)
    assert s == g.SUCCESS, g.STATUS[s]
    g.synchronize()
    got = dC.download(c_host.dtype, c_host.size)
    view = np.uint32 if osz == 4 else np.uint16
    return int(np.sum(got.view(view) != expected.view(view)))


@pytest.mark.parametrize("in_t,out_t", [(BF16, BF16), (BF16, F32), (F16, F16), (F16, F32)])
@pytest.mark.parametrize("ta,tb,m,n,k", [(1, 0, 256, 256, 128),   # TN fast path
                                         (1, 0, 72, 40, 48),       # TN fast path, ragged
                                         (0, 0, 17, 9, 13),        # general path
                                         (0, 1, 33, 20, 24)])
def test_batched_float_exact(blas, in_t, out_t, ta, tb, m, n, k):
    assert batched_case(blas, in_t, out_t, ta, tb, m, n, k, 1.0, 0.0, 3, "packed", "packed",
                        "gap") == 0
    assert batched_case(blas, in_t, out_t, ta, tb, m, n, k, 2.5, -1.5, 4, "neg", "zero",
                        "packed", seed=11) == 0


@pytest.mark.parametrize("ta,tb,m,n,k", [(1, 0, 256, 256, 256), (1, 0, 100, 60, 80),
                                         (0, 0, 13, 7, 19), (1, 1, 13, 7, 19)])
def test_batched_int8_exact(blas, ta, tb, m, n, k):
    assert batched_case(blas, I8, I32, ta, tb, m, n, k, 1, 0, 3, "packed", "zero", "gap") == 0
    assert batched_case(blas, I8, I32, ta, tb, m, n, k, 3, -2, 2, "zero", "neg", "packed",
                        seed=5) == 0


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 1)])
def test_batched_transposed_copy_paths(blas, ta, tb):
    """Large non-TN batches: per-batch operand copies (one copy when the
    stride broadcasts), then the TN kernel."""
    assert batched_case(blas, BF16, BF16, ta, tb, 256, 256, 512, 1.0, 0.0, 3, "packed", "neg",
                        "gap") == 0
    assert batched_case(blas, F16, F32, ta, tb, 256, 264, 512, 2.5, -1.5, 2, "zero", "zero",
                        "packed", seed=4) == 0
    assert batched_case(blas, I8, I32, ta, tb, 256, 256, 512, 2, 1, 2, "neg", "packed", "gap",
                        seed=6) == 0


def test_batched_attention_shape(blas):
    """Many small TN products in one launch (per-head score blocks): 32 batches
    of 256 x 256 x 128 bf16, each identical to its own GemmEx."""
    assert batched_case(blas, BF16, BF16, 1, 0, 256, 256, 128, 1.0, 0.0, 32, "packed", "packed",
                        "packed", seed=3) == 0


def test_batched_refusals(blas):
    one = 1.0
    d = g.DeviceBuffer(4096)
    c0 = np.arange(64, dtype=np.float32)
    dc = to_dev(c0)
    args = lambda batch, at=BF16, ct=F32, alpha=one: blas.gemm_strided_batched_ex(
        1, 0, 4, 4, 8, alpha, d.p, at, 8, 32, d.p, at, 8, 32, 0.0, dc.p, ct, 4, 16, batch)
    assert args(-1) == g.INVALID_VALUE
    assert args(0) == g.SUCCESS
    g.synchronize()
    assert np.array_equal(dc.download(np.float32, 64), c0)      # batch 0 writes nothing
    assert args(65536) == g.NOT_SUPPORTED
    assert args(2, at=F32) == g.NOT_SUPPORTED                   # not a GemmEx triple
    assert blas.gemm_strided_batched_ex(1, 0, 4, 4, 8, 1.5, d.p, I8, 8, 32, d.p, I8, 8, 32, 0.0,
                                        dc.p, I32, 4, 16, 2) == g.INVALID_VALUE  # int8 alpha
    assert blas.gemm_strided_batched_ex(1, 0, 4, 4, 8, one, d.p, BF16, 7, 32, d.p, BF16, 8, 32,
                                        0.0, dc.p, F32, 4, 16, 2) == g.INVALID_VALUE  # lda < k


def test_batched_runs_the_128_tile_kernel(blas, capfd):
    """Batches whose 128x128 workgroups number at most 512 (batch x tiles)
    run on the 128x128-tile kernel, its four-stage ring up to 256 of them and
    its two-stage ring up to 512: every batch bit-exact, strides packed,
    broadcast (0) and negative, C gaps untouched; the plan log shows the
    kernel and the ring."""
    from test_gpu_gemm import logged_plans
    cases = [(BF16, BF16, 256, 256, 128, 3, "packed", "zero", "gap", "4"),      # 12 workgroups
             (F16, F32, 512, 512, 128, 32, "packed", "packed", "packed", "2"),  # 512
             (I8, I32, 256, 256, 256, 12, "neg", "packed", "gap", "4")]        # 48
    bad = []
    for it, ot, m, n, k, batch, am, bm, cm, ring in cases:
        res = []
        plans = logged_plans(capfd, lambda: res.append(batched_case(  # noqa: B023
            blas, it, ot, 1, 0, m, n, k, 1.0, 0.0, batch, am, bm, cm, seed=batch)))
        if res != [0] or len(plans) != 1 or plans[0]["kernel"] != "tn128" or plans[0]["ring"] != ring:
            bad.append((it, ot, m, n, k, batch, res, plans))
    assert not bad, bad


def test_batched_direct_operands(blas, capfd):
    """16-bit and int8 batches on one pass of the 128x128 kernel read each
    batch's M-contiguous A and N-contiguous B where they lie: strides packed,
    broadcast (0) and negative, both rings, every batch bit-exact, C gaps
    untouched, no copy."""
    from test_gpu_gemm import logged_plans
    cases = [(BF16, BF16, 0, 0, 256, 256, 512, 3, "neg", "packed", "gap", "4"),
             (F16, F32, 0, 0, 512, 512, 128, 32, "zero", "packed", "packed", "2"),
             (F16, F16, 0, 0, 256, 264, 512, 5, "packed", "zero", "gap", "4"),
             (BF16, F32, 0, 1, 256, 256, 512, 4, "packed", "neg", "gap", "4"),
             (F16, F16, 1, 1, 264, 256, 512, 3, "zero", "zero", "packed", "4"),
             (I8, I32, 0, 1, 256, 256, 512, 3, "neg", "packed", "gap", "4"),
             (I8, I32, 0, 0, 512, 512, 128, 32, "packed", "zero", "packed", "2")]
    bad = []
    for it, ot, ta, tb, m, n, k, batch, am, bm, cm, ring in cases:
        res = []
        alpha, beta = (2.0, -1.0) if it == I8 else (1.5, -0.5)   # int32 C: integral alpha, beta
        plans = logged_plans(capfd, lambda: res.append(batched_case(  # noqa: B023
            blas, it, ot, ta, tb, m, n, k, alpha, beta, batch, am, bm, cm, seed=batch)))
        if res != [0] or len(plans) != 1 or plans[0]["kernel"] != "tn128" or plans[0]["ring"] != ring \
                or plans[0]["direct_a"] != str(1 - ta) or plans[0]["direct_b"] != str(tb) \
                or plans[0]["copy_a"] != "0" or plans[0]["copy_b"] != "0":
            bad.append((it, ot, ta, tb, m, n, k, batch, res, plans))
    assert not bad, bad


def test_batched_padded_copies_for_unaligned_k(blas, capfd):
    """K not a multiple of 16 bytes above the copy threshold, in a batch:
    both operands are copied per batch (once where a stride of 0 broadcasts)
    into rows of K padded with zeros, then the TN kernel; every batch
    bit-exact, C gaps untouched, both copies in the plan."""
    from test_gpu_gemm import logged_plans
    cases = [(BF16, BF16, 256, 264, 1001, 2, "packed", "zero", "gap"),
             (I8, I32, 256, 256, 1001, 3, "neg", "packed", "packed")]
    bad = []
    for it, ot, m, n, k, batch, am, bm, cm in cases:
        res = []
        plans = logged_plans(capfd, lambda: res.append(batched_case(  # noqa: B023
            blas, it, ot, 1, 0, m, n, k, 1.0, 0.0, batch, am, bm, cm, seed=k)))
        if res != [0] or len(plans) != 1 or plans[0]["copy_a"] != "1" or plans[0]["copy_b"] != "1":
            bad.append((it, ot, m, n, k, batch, res, plans))
    assert not bad, bad


def test_batched_probe_capacity(blas):
    """A cycle probe must hold batchCount times one GemmEx's slots."""
    m = n = 256
    per = blas.cycle_slots_needed(m, n)
    batch = 3
    slot_t = np.dtype([("start", np.uint64), ("end", np.uint64), ("core", np.uint32),
                       ("warp", np.uint32)])
    assert slot_t.itemsize == ctypes.sizeof(g.CycleSlot)
    slots = to_dev(np.zeros(per * batch, slot_t))
    dA = g.DeviceBuffer(m * 64 * 2 * batch)
    dC = g.DeviceBuffer(m * n * 4 * batch)
    assert blas.set_cycle_probe(slots.p, per * batch - 1) == g.SUCCESS
    st = blas.gemm_strided_batched_ex(1, 0, m, n, 64, 1.0, dA.p, BF16, 64, m * 64, dA.p, BF16, 64,
                                      m * 64, 0.0, dC.p, F32, m, m * n, batch)
    assert st == g.INVALID_VALUE
    assert blas.set_cycle_probe(slots.p, per * batch) == g.SUCCESS
    st = blas.gemm_strided_batched_ex(1, 0, m, n, 64, 1.0, dA.p, BF16, 64, m * 64, dA.p, BF16, 64,
                                      m * 64, 0.0, dC.p, F32, m, m * n, batch)
    assert st == g.SUCCESS
    g.synchronize()
    assert blas.set_cycle_probe(None, 0) == g.SUCCESS
    got = slots.download(np.uint8, per * batch * slot_t.itemsize).view(slot_t)
    # one 256x256 tile per batch on the TN fast path: 4 waves each, in launch order
    written = np.nonzero(got["end"])[0]
    assert written.tolist() == list(range(4 * batch))
    assert np.all(got["end"][written] >= got["start"][written])
