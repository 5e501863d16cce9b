"""IEEE special values through the grxDNN kernels, against the CPU oracle.

The reference has no grxDNN (ref docs/designs/grxcp_roadmap.md:864-877); the
oracle evaluates each definition as written, in float64 (pinned in
tests/test_oracle.py), and the kernels must give the same non-finite results
in the same places:
- norms: a NaN anywhere in a row makes the whole row NaN; an infinity makes
  RMSNorm's scale 0 (the row's finite elements become 0, the infinity
  0 * inf = NaN) and LayerNorm's whole row NaN (inf - inf in the variance);
  no row leaks into the other rows of its workgroup;
- softmax: a NaN or +inf in a row makes the row NaN, a very large finite
  entry takes all the weight;
- GELU: gelu(+inf) = +inf, gelu(-inf) = NaN (-inf * 0, as the formula
  gives), NaN stays NaN, and the negative tail keeps its relative precision
  down to outputs of 2^-120 (1 + erf and 1 + tanh are not formed);
- attention: a NaN in Q row i makes O row i NaN; a NaN in K row j makes the
  rows that attend to key j NaN and leaves the others (masked keys are
  replaced by -inf, not added to); a +inf key score makes its row NaN, a
  -inf score drops the key. A NaN in V row j, column d is NaN in column d of
  every row that attends to key j; under the causal mask it also reaches
  the rows before j inside j's 64-key tile, whose P * V product multiplies
  the masked key's weight 0 by it (0 * NaN = NaN), and no other row.
"""
import numpy as np
import pytest

import grxcp_amd as g
import oracle as O
from helpers import normwise_rel_err, say, to_dev
from test_gpu_dnn import BF16, F16, F32, check_norm, dec, enc, nptype, run_attention

pytestmark = pytest.mark.gpu

TINY = {BF16: 2.0 ** -126, F16: 2.0 ** -25, F32: 2.0 ** -126}   # output underflow
# GELU's tail results below this may come from fp32-subnormal intermediates
# (erfc of x / sqrt 2, or the reciprocal of exp(-2z)), which the hardware's
# exp and reciprocal do not keep: 13.5 * 2^-126 < 2^-120.
GELU_TINY = {BF16: 2.0 ** -120, F16: 2.0 ** -25, F32: 2.0 ** -120}
REL = {BF16: 2.0 ** -8, F16: 2.0 ** -10, F32: 4e-6}


def same_specials(y, ref):
    """Identical NaN positions and identical infinities."""
    assert np.array_equal(np.isnan(y), np.isnan(ref)), (int(np.isnan(y).sum()), int(np.isnan(ref).sum()))
    inf = np.isinf(ref)
    assert np.array_equal(np.isinf(y), inf) and np.array_equal(y[inf], ref[inf])


def norm_rows(rows, hidden, t, seed):
    """N(0,1) rows with specials planted in rows 1-5 and 10 (row 11, its
    partner in a two-row workgroup, stays clean)."""
    r = np.random.default_rng(seed)
    x = r.standard_normal((rows, hidden)).astype(np.float32)
    x[1, 3 % hidden] = np.nan
    x[2, 5 % hidden] = np.inf
    x[3, 7 % hidden] = -np.inf
    x[4, :] = 0.0
    x[5, 0] = np.inf
    x[5, hidden - 1] = -np.inf if hidden > 1 else np.inf
    if rows > 11:
        x[10, hidden // 2] = np.nan
    return x


@pytest.mark.parametrize("layer", [False, True])
@pytest.mark.parametrize("t,rows,hidden", [(BF16, 8, 1000), (BF16, 8, 8192), (BF16, 8, 333),
                                           (F16, 8, 4096), (F32, 8, 1000), (BF16, 2048, 4096)])
def test_norm_specials(dnn, layer, t, rows, hidden):
    x = norm_rows(rows, hidden, t, seed=rows + hidden)
    r = np.random.default_rng(hidden)
    gamma = (1 + 0.02 * r.standard_normal(hidden)).astype(np.float32)
    beta = (0.02 * r.standard_normal(hidden)).astype(np.float32)
    xe, ge, be = enc(x, t), enc(gamma, t), enc(beta, t)
    xq, gq, bq = dec(xe, t), dec(ge, t), dec(be, t)
    dx, dg, db = to_dev(xe), to_dev(ge), to_dev(be)
    dy = to_dev(np.zeros_like(xe))
    xd, wd = g.TensorDesc(t, [rows, hidden]), g.TensorDesc(t, [hidden])
    say(f"norm specials layer={layer} t={t} rows={rows} hidden={hidden}")
    if layer:
        s = dnn.layernorm(xd, dx.p, wd, dg.p, db.p, 1e-6, xd, dy.p)
    else:
        s = dnn.rmsnorm(xd, dx.p, wd, dg.p, 1e-6, xd, dy.p)
    assert s == g.SUCCESS, g.STATUS[s]
    g.synchronize()
    y = dec(dy.download(nptype(t), rows * hidden), t).reshape(rows, hidden)
    ref = O.layernorm(xq, gq, bq, 1e-6) if layer else O.rmsnorm(xq, gq, 1e-6)
    same_specials(y, ref)
    special = np.zeros(rows, bool)
    special[[1, 2, 3, 5] + ([10] if rows > 11 else [])] = True
    assert np.isnan(y[1]).all()
    if rows > 11:
        assert np.isnan(y[10]).all() and np.isfinite(y[11]).all()
    for i in (2, 3, 5):              # infinities in the row
        if layer:
            assert np.isnan(y[i]).all()
        else:
            fin = np.isfinite(xq[i])
            assert np.isnan(y[i][~fin]).all() and not y[i][fin].any()
    check_norm(y[~special], ref[~special], bq if layer else None, t)


def softmax_rows(rows, hidden, seed):
    r = np.random.default_rng(seed)
    x = r.standard_normal((rows, hidden)).astype(np.float32)
    x[1, 3 % hidden] = np.nan
    x[2, 5 % hidden] = np.inf
    x[3, 0] = np.inf
    x[3, hidden - 1] = np.inf
    x[6, 9 % hidden] = 60000.0       # finite in every type; exp(-60000) is 0
    return x


@pytest.mark.parametrize("t", [BF16, F16, F32])
@pytest.mark.parametrize("rows,hidden", [(8, 1000), (8, 8192), (8, 12000), (8, 333)])
def test_softmax_specials(dnn, t, rows, hidden):
    x = softmax_rows(rows, hidden, seed=hidden)
    xe = enc(x, t)
    xq = dec(xe, t)
    dx, dy = to_dev(xe), to_dev(np.zeros_like(xe))
    xd = g.TensorDesc(t, [rows, hidden])
    say(f"softmax specials t={t} rows={rows} hidden={hidden}")
    s = dnn.softmax(xd, dx.p, xd, dy.p)
    assert s == g.SUCCESS, g.STATUS[s]
    g.synchronize()
    y = dec(dy.download(nptype(t), rows * hidden), t).reshape(rows, hidden)
    ref = O.softmax(xq)
    same_specials(y, ref)
    for i in (1, 2, 3):
        assert np.isnan(y[i]).all(), i
    one_hot = np.zeros(hidden, np.float32)
    one_hot[9 % hidden] = 1.0
    assert np.array_equal(y[6], one_hot)
    clean = [0, 4, 5, 7]
    err = np.abs(y[clean].astype(np.float64) - ref[clean])
    assert np.all(err <= REL[t] * np.abs(ref[clean]) + TINY[t]), float(err.max())


def gelu_inputs(t):
    """Specials, the largest finite values, and both tails densely."""
    big = {BF16: 3.3895314e38, F16: 65504.0, F32: 3.4028235e38}[t]
    far = [1e30, -1e30] if t != F16 else [60000.0, -60000.0]
    tails = np.concatenate([-np.geomspace(2.0, 15.0, 4000), np.geomspace(2.0, 15.0, 500),
                            np.linspace(-2.0, 2.0, 501)])
    x = np.concatenate([[np.inf, -np.inf, np.nan, 0.0, -0.0, big, -big], far, tails]).astype(np.float32)
    return np.concatenate([x, np.zeros(-x.size % 8, np.float32)])   # whole 16-byte chunks


def cond(x, mode):
    """Relative condition number of the fp32 evaluation's argument: how much
    a relative error of the argument (x / sqrt 2, or z) grows in the result."""
    x = np.abs(x.astype(np.float64))
    if mode == g.GELU_ERF:
        return 1.0 + x * x
    return 1.0 + 1.6 * x + 0.22 * x ** 3


@pytest.mark.parametrize("mode", [g.GELU_ERF, g.GELU_TANH])
@pytest.mark.parametrize("t", [BF16, F16, F32])
@pytest.mark.parametrize("layout", ["flat", "rows", "scalar"])
def test_gelu_specials_and_tails(dnn, mode, t, layout):
    x0 = gelu_inputs(t)
    n = x0.size
    # flat: one contiguous array; rows: 16-byte-aligned rows with a pitch
    # (row by row); scalar: rows of a length that is not a multiple of 8
    hidden = {"flat": n, "rows": 512, "scalar": 509}[layout]
    rows = -(-n // hidden)
    pitch = hidden + (8 if layout == "rows" else 0)
    x = np.zeros(rows * hidden, np.float32)
    x[:n] = x0
    x = x.reshape(rows, hidden)
    xe = enc(x, t)
    xq = dec(xe, t)
    xbuf = np.zeros((rows, pitch), nptype(t))
    xbuf[:, :hidden] = xe
    dx, dy = to_dev(xbuf), to_dev(np.zeros_like(xbuf))
    xd = g.TensorDesc(t, [rows, hidden], [pitch, 1])
    say(f"gelu specials mode={mode} t={t} layout={layout} rows={rows} hidden={hidden}")
    s = dnn.gelu(mode, xd, dx.p, xd, dy.p)
    assert s == g.SUCCESS, g.STATUS[s]
    g.synchronize()
    y = dec(np.ascontiguousarray(dy.download(nptype(t), rows * pitch).reshape(rows, pitch)[:, :hidden]), t)
    ref = O.gelu(xq, mode).reshape(rows, hidden)
    same_specials(y, ref)
    yv, rv, xv = y.ravel()[:n], ref.ravel()[:n], xq.ravel()[:n]
    assert yv[0] == np.inf and np.isnan(yv[1]) and np.isnan(yv[2])
    assert yv[3] == 0.0 and yv[4] == 0.0
    fin = np.isfinite(rv)
    rel = REL[t] + (cond(xv[fin], mode) * 2.0 ** -21 if t == F32 else 0.0)
    err = np.abs(yv[fin].astype(np.float64) - rv[fin])
    bad = err > rel * np.abs(rv[fin]) + GELU_TINY[t]
    assert not bad.any(), (int(bad.sum()), xv[fin][bad][:5], yv[fin][bad][:5], rv[fin][bad][:5])
    # the tail is resolved: results that are normal numbers of the output type are not 0
    small = fin & (np.abs(rv) >= GELU_TINY[t]) & (np.abs(rv) < 1e-6)
    if t != F16:
        assert small.sum() > 500 and (yv[small] != 0).all()


@pytest.mark.parametrize("t", [BF16, F16])
@pytest.mark.parametrize("D,causal", [(128, True), (64, True), (128, False)])
def test_attention_specials(dnn, t, D, causal):
    B, H, S = 1, 3, 200
    r = np.random.default_rng(D + causal)
    q = r.standard_normal((B, H, S, D)).astype(np.float32)
    k = r.standard_normal((B, H, S, D)).astype(np.float32)
    v = r.standard_normal((B, H, S, D)).astype(np.float32)
    q[0, 0, 5, 3] = np.nan           # head 0: Q row 5
    k[0, 0, 70, 9] = np.nan          # head 0: K row 70 (key tile 64-127)
    k[0, 1, 130, 0] = np.inf         # head 1: key 130's score is +-inf by the sign of q[i, 0]
    v[0, 2, 150, 4] = np.nan         # head 2: V row 150, column 4 (key tile 128-191)
    o, qq, kq, vq = run_attention(dnn, t, B, H, S, D, causal, seed=0, q=q, k=k, v=v)
    scale = D ** -0.5
    for h in range(H):
        ref = O.attention_head(qq[0, h], kq[0, h], vq[0, h], causal, scale)
        got = o[0, h]
        if h == 2 and causal:
            # the documented reach of a non-finite V: rows 128..149 of column 4
            assert np.isnan(got[128:150, 4]).all() and not np.isnan(ref[128:150, 4]).any()
            ref = ref.copy()
            ref[128:150, 4] = np.nan
        same_specials(got, ref)
        fin = np.isfinite(ref).all(axis=1)
        assert fin.any() or (not causal and h in (0, 2)), h     # full: NaN reaches every row
        if fin.any():
            assert normwise_rel_err(got[fin], ref[fin]) <= 1e-2, h
        if h == 2:
            cols = np.arange(D) != 4
            assert np.isfinite(got[:, cols]).all()
            assert normwise_rel_err(got[:, cols], ref[:, cols]) <= 1e-2
    # head 0: row 5 and (causal) rows >= 70, or (full) every row, are NaN
    nan_rows = np.isnan(o[0, 0]).any(axis=1)
    want = np.zeros(S, bool)
    want[5] = True
    want[70 if causal else 0:] = True
    assert np.array_equal(nan_rows, want)
    # head 1: a row is NaN exactly where its score with key 130 is +inf or NaN
    s130 = qq[0, 1, :, 0] * np.inf
    hit = (np.arange(S) >= 130) if causal else np.ones(S, bool)
    assert np.array_equal(np.isnan(o[0, 1]).any(axis=1), hit & ~(s130 < 0))
