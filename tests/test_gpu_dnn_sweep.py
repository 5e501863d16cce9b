"""Seeded randomized sweep of the grxDNN entry points, with guard bands.

Draws shapes, element types, row pitches, LayerNorm/RMSNorm, causal/full
attention and both GELU forms from fixed seeds, and checks every call
against the CPU oracle (the bounds of the targeted tests: norms element-wise
at half an output ulp plus fp32 arithmetic, with eps drawn too; attention
1e-2 normwise per head; softmax and GELU
element-wise at the output type's rounding, with the targeted tests'
absolute floors). Every output buffer sits between two 4 KB guard bands
filled with a byte pattern; a call that writes one byte outside its output
fails the test, and so does a change to the row padding inside it.
"""
import numpy as np
import pytest

import grxcp_amd as g
import oracle as O
from helpers import Guarded, normwise_rel_err, say, to_dev
from test_gpu_dnn import dec, enc, norm_violations, nptype
from test_gpu_softmax_gelu import check

pytestmark = pytest.mark.gpu

BF16, F16, F32 = g.GRX_R_16BF, g.GRX_R_16F, g.GRX_R_32F
def _pick(r, seq):
    return seq[int(r.integers(len(seq)))]


def _hidden(r):
    """Row lengths on both sides of the kernels' thresholds, some not a multiple of 8."""
    if r.integers(4) == 0:
        return int(r.integers(1, 3000))
    return 8 * int(_pick(r, [r.integers(1, 64), r.integers(64, 256), r.integers(256, 1024),
                             r.integers(1024, 2100)]))


def _rows_input(r, t, rows, hidden, pitch):
    x = r.standard_normal((rows, hidden)).astype(np.float32)
    xe = enc(x, t)
    buf = np.zeros((rows, pitch), nptype(t))
    buf[:, :hidden] = xe
    return buf, dec(xe, t)


def test_norm_sweep(dnn):
    r = np.random.default_rng(30301)
    bad = []
    for i in range(24):
        t = _pick(r, [BF16, BF16, F16, F32])
        layer = bool(r.integers(2))
        rows, hidden = int(r.integers(1, 160)), _hidden(r)
        pitch = hidden + (_pick(r, [0, 8, 24]) if hidden % 8 == 0 else int(r.integers(0, 5)))
        xbuf, xq = _rows_input(r, t, rows, hidden, pitch)
        gamma = (1 + 0.02 * r.standard_normal(hidden)).astype(np.float32)
        beta = (0.02 * r.standard_normal(hidden)).astype(np.float32)
        ge, be = enc(gamma, t), enc(beta, t)
        poison = np.full((rows, pitch), 0x7FC1 if t != F32 else np.float32(np.nan), nptype(t))
        dx, dg, db, dy = to_dev(xbuf), to_dev(ge), to_dev(be), Guarded(poison)
        xd = g.TensorDesc(t, [rows, hidden], [pitch, 1])
        wd = g.TensorDesc(t, [hidden])
        eps = float(_pick(r, [1e-6, 1e-6, 1e-5, 1e-3, 0.1, 1.0]))
        say(f"norm sweep {i}: layer={layer} t={t} rows={rows} hidden={hidden} pitch={pitch} eps={eps}")
        s = (dnn.layernorm(xd, dx.p, wd, dg.p, db.p, eps, xd, dy.p) if layer
             else dnn.rmsnorm(xd, dx.p, wd, dg.p, eps, xd, dy.p))
        assert s == g.SUCCESS, g.STATUS[s]
        g.synchronize()
        got = dy.download(nptype(t)).reshape(rows, pitch)
        y = dec(np.ascontiguousarray(got[:, :hidden]), t)
        gq, bq = dec(ge, t), dec(be, t)
        ref = O.layernorm(xq, gq, bq, eps) if layer else O.rmsnorm(xq, gq, eps)
        ok = (norm_violations(y, ref, bq if layer else None, t) == 0 and dy.guards_intact()
              and np.array_equal(got[:, hidden:].view(np.uint8), poison[:, hidden:].view(np.uint8)))
        if not ok:
            bad.append((i, t, layer, rows, hidden, pitch))
    assert not bad, bad


def test_softmax_gelu_sweep(dnn):
    r = np.random.default_rng(30302)
    bad = []
    for i in range(24):
        op = _pick(r, ["softmax", "gelu"])
        t = _pick(r, [BF16, F16, F32])
        mode = int(r.integers(2))
        rows, hidden = int(r.integers(1, 120)), _hidden(r)
        pitch = hidden + (_pick(r, [0, 8, 40]) if hidden % 8 == 0 else int(r.integers(0, 5)))
        xbuf, xq = _rows_input(r, t, rows, hidden, pitch)
        poison = np.full((rows, pitch), 0x7FC1 if t != F32 else np.float32(np.nan), nptype(t))
        dx, dy = to_dev(xbuf), Guarded(poison)
        xd = g.TensorDesc(t, [rows, hidden], [pitch, 1])
        say(f"row-op sweep {i}: {op} t={t} mode={mode} rows={rows} hidden={hidden} pitch={pitch}")
        s = dnn.softmax(xd, dx.p, xd, dy.p) if op == "softmax" else dnn.gelu(mode, xd, dx.p, xd, dy.p)
        assert s == g.SUCCESS, g.STATUS[s]
        g.synchronize()
        got = dy.download(nptype(t)).reshape(rows, pitch)
        y = dec(np.ascontiguousarray(got[:, :hidden]), t)
        ref = O.softmax(xq) if op == "softmax" else O.gelu(xq, mode).reshape(rows, hidden)
        try:
            atol = ({BF16: 0.0, F16: 6e-8, F32: 1e-30} if op == "softmax"
                    else {BF16: 1e-6, F16: 1e-6, F32: 1e-7})[t]
            check(y, ref, t, atol=atol)
            ok = True
        except AssertionError:
            ok = False
        ok = ok and dy.guards_intact() and np.array_equal(got[:, hidden:].view(np.uint8),
                                                           poison[:, hidden:].view(np.uint8))
        if not ok:
            bad.append((i, op, t, mode, rows, hidden, pitch))
    assert not bad, bad


def test_attention_sweep(dnn):
    r = np.random.default_rng(30303)
    bad = []
    for i in range(12):
        t = _pick(r, [BF16, F16])
        B, H = int(r.integers(1, 3)), int(r.integers(1, 4))
        S, D = int(r.integers(1, 600)), _pick(r, [64, 128])
        causal = bool(r.integers(2))
        shp = (B, H, S, D)
        q, k, v = (enc(r.standard_normal(shp).astype(np.float32), t) for _ in range(3))
        dq, dk, dv = to_dev(q), to_dev(k), to_dev(v)
        do = Guarded(np.full(q.size, 0x7FC1, np.uint16))
        desc = g.TensorDesc(t, list(shp))
        ad = g.AttnDesc(causal, D ** -0.5)
        say(f"attention sweep {i}: t={t} B={B} H={H} S={S} D={D} causal={causal}")
        s = dnn.attention(ad, desc, dq.p, desc, dk.p, desc, dv.p, desc, do.p)
        assert s == g.SUCCESS, g.STATUS[s]
        g.synchronize()
        o = dec(do.download(np.uint16), t).reshape(shp)
        qf, kf, vf = (dec(a, t).reshape(shp) for a in (q, k, v))
        ok = do.guards_intact()
        for b in range(B):
            for h in range(H):
                ref = O.attention_head(qf[b, h], kf[b, h], vf[b, h], causal, D ** -0.5)
                ok = ok and normwise_rel_err(o[b, h], ref) <= 1e-2
        if not ok:
            bad.append((i, t, B, H, S, D, causal))
    assert not bad, bad
