"""grxdnnSoftmaxForward / grxdnnGeluForward on gfx950 against the CPU oracle.

Neither exists in the reference (planned: ref
docs/designs/grxcp_roadmap.md:864-877); the oracle follows the definitions
(pinned in tests/test_oracle.py). The kernels compute in fp32 from the
rounded inputs and round the output once, so each result is checked against
the fp64 oracle on the same rounded inputs within a bound set by the output
type: half an output ulp plus the fp32 arithmetic (bf16 2^-8, fp16 2^-10,
fp32 4e-6 relative). Exact cases: constant rows give 1/n, -inf entries give 0
and an all -inf row NaN, GELU(0) = 0, the row padding is never written.
"""
import numpy as np
import pytest

import grxcp_amd as g
import oracle as O
from helpers import say, to_dev
from test_gpu_dnn import BF16, F16, F32, dec, enc, nptype

pytestmark = pytest.mark.gpu

REL = {BF16: 2.0 ** -8, F16: 2.0 ** -10, F32: 4e-6}


def run_rows(dnn, op, t, x, pitch=None, mode=0, inplace=False):
    rows, hidden = x.shape
    pitch = pitch or hidden
    xe = enc(x, t)
    xq = dec(xe, t)
    xbuf = np.zeros((rows, pitch), nptype(t))
    xbuf[:, :hidden] = xe
    poison = np.full((rows, pitch), 0x7FC1 if t != F32 else np.float32(np.nan), nptype(t))
    dx = to_dev(xbuf)
    dy = dx if inplace else to_dev(poison)
    xd = g.TensorDesc(t, [rows, hidden], [pitch, 1])
    say(f"{op} t={t} rows={rows} hidden={hidden} pitch={pitch} mode={mode} inplace={inplace}")
    s = dnn.softmax(xd, dx.p, xd, dy.p) if op == "softmax" else dnn.gelu(mode, xd, dx.p, xd, dy.p)
    assert s == g.SUCCESS, g.STATUS[s]
    g.synchronize()
    got = dy.download(nptype(t), rows * pitch).reshape(rows, pitch)
    if pitch > hidden and not inplace:
        assert np.array_equal(got[:, hidden:].view(np.uint8), poison[:, hidden:].view(np.uint8))
    y = dec(np.ascontiguousarray(got[:, :hidden]), t)
    ref = O.softmax(xq) if op == "softmax" else O.gelu(xq, mode).reshape(rows, hidden)
    return y, ref


def check(y, ref, t, atol=0.0):
    err = np.abs(y.astype(np.float64) - ref.astype(np.float64))
    bound = REL[t] * np.abs(ref.astype(np.float64)) + atol
    bad = err > bound
    assert not bad.any(), (int(bad.sum()), float(err.max()))


SOFTMAX_SHAPES = [(1, 1), (3, 7), (5, 64), (17, 1000), (64, 512), (5, 2056), (8, 4096), (4, 8192),
                  (3, 8200), (3, 12000), (2, 32768), (2, 100003)]


@pytest.mark.parametrize("t", [BF16, F16, F32])
@pytest.mark.parametrize("rows,hidden", SOFTMAX_SHAPES)
def test_softmax_vs_oracle(dnn, t, rows, hidden):
    x = (2.0 * np.random.default_rng(rows * 7 + hidden).standard_normal((rows, hidden))).astype(np.float32)
    y, ref = run_rows(dnn, "softmax", t, x)
    # tiny probabilities: the fp32 exp of the kernel is relative, the output
    # type's subnormal range is not
    check(y, ref, t, atol={BF16: 0.0, F16: 6e-8, F32: 1e-30}[t])


def test_softmax_padded_rows_and_exact_cases(dnn):
    x = np.random.default_rng(3).standard_normal((6, 300)).astype(np.float32)
    y, ref = run_rows(dnn, "softmax", BF16, x, pitch=312)
    check(y, ref, BF16)
    for n in (1, 8, 1024, 4096):
        y, _ = run_rows(dnn, "softmax", BF16, np.full((4, n), 3.25, np.float32))
        assert np.array_equal(y, np.full((4, n), 1.0 / n, np.float32))
    x = np.zeros((3, 64), np.float32)
    x[0, 5:] = -np.inf           # row 0: five equal finite entries
    x[1, :] = -np.inf            # row 1: nothing finite -> NaN, as the formula gives
    x[2, ::2] = -np.inf
    y, _ = run_rows(dnn, "softmax", F32, x)
    assert np.array_equal(y[0, :5], np.full(5, 0.2, np.float32)) and not y[0, 5:].any()
    assert np.isnan(y[1]).all()
    assert not y[2, ::2].any() and np.allclose(y[2, 1::2], 1.0 / 32, rtol=1e-6)
    # the same special rows through the workgroup-per-row kernel
    x = np.zeros((3, 4096), np.float32)
    x[0, 5:] = -np.inf
    x[1, :] = -np.inf
    x[2, ::2] = -np.inf
    y, _ = run_rows(dnn, "softmax", F32, x)
    assert np.array_equal(y[0, :5], np.full(5, 0.2, np.float32)) and not y[0, 5:].any()
    assert np.isnan(y[1]).all()
    assert not y[2, ::2].any() and np.allclose(y[2, 1::2], 1.0 / 2048, rtol=1e-6)


@pytest.mark.parametrize("mode", [g.GELU_ERF, g.GELU_TANH])
@pytest.mark.parametrize("t", [BF16, F16, F32])
@pytest.mark.parametrize("rows,hidden,pitch", [(1, 1, 1), (3, 7, 7), (5, 333, 340), (64, 4096, 4096),
                                               (7, 1000, 1000), (6, 1024, 1040), (1, 1 << 20, 1 << 20)])
def test_gelu_vs_oracle(dnn, mode, t, rows, hidden, pitch):
    x = (3.0 * np.random.default_rng(hidden + rows).standard_normal((rows, hidden))).astype(np.float32)
    y, ref = run_rows(dnn, "gelu", t, x, pitch=pitch, mode=mode)
    # near gelu's zero at x = 0 the fp32 erf/tanh relative error is absolute
    check(y, ref, t, atol={BF16: 1e-6, F16: 1e-6, F32: 1e-7}[t])


def test_gelu_in_place_and_zero(dnn):
    x = np.random.default_rng(5).standard_normal((9, 256)).astype(np.float32)
    x[0, :] = 0.0
    y, ref = run_rows(dnn, "gelu", BF16, x, mode=g.GELU_ERF, inplace=True)
    check(y, ref, BF16, atol=1e-6)
    assert not y[0].any()


def test_refusals(dnn):
    d = g.TensorDesc(BF16, [2, 8])
    d32 = g.TensorDesc(F32, [2, 8])
    buf = to_dev(np.zeros(16, np.float32))
    assert dnn.gelu(7, d, buf.p, d, buf.p) == g.INVALID_VALUE
    assert dnn.softmax(d, buf.p, d32, buf.p) == g.NOT_SUPPORTED
    assert dnn.softmax(d, None, d, buf.p) == g.INVALID_VALUE
    assert dnn.softmax(d, buf.p, g.TensorDesc(BF16, [2, 9]), buf.p) == g.INVALID_VALUE
    empty = g.TensorDesc(BF16, [0, 8])
    assert dnn.softmax(empty, None, empty, None) == g.SUCCESS
