"""grxDNN RMSNorm / LayerNorm / attention on gfx950 against the CPU oracle.

The reference has no grxDNN code to compare with (ref
docs/designs/grxcp_roadmap.md:864-877), so the oracle follows the
definitions (pinned in tests/test_oracle.py). Norms: the kernels compute
in fp32 from the rounded inputs and round each output once, so every element
is held to half an output ulp plus the fp32 arithmetic (`norm_bound`), far
inside the north star's 1e-2; eps is pinned by rows where it dominates.
Attention: max relative error 1e-2 of the fp64 reference. Closed forms are
checked exactly where the arithmetic is exact (LayerNorm of a constant row is
beta; attention row 0 is V[0]).
"""
import ctypes

import numpy as np
import pytest

import grxcp_amd as g
import oracle as O
from helpers import normwise_rel_err, say, to_dev

pytestmark = pytest.mark.gpu

BF16, F16, F32 = g.GRX_R_16BF, g.GRX_R_16F, g.GRX_R_32F


def enc(x: np.ndarray, t: int) -> np.ndarray:
    if t == BF16:
        return O.f32_to_bf16(x)
    if t == F16:
        return O.f32_to_half(x)
    return np.ascontiguousarray(x, np.float32)


def dec(b: np.ndarray, t: int) -> np.ndarray:
    if t == BF16:
        return O.bf16_to_f32(b)
    if t == F16:
        return O.half_to_f32(b)
    return b


def nptype(t):
    return np.float32 if t == F32 else np.uint16


# Per-element bound for the norms: |y - ref| <= OUT_REL * |ref| (half an output
# ulp: 8 significant bits in bf16, 11 in fp16 -- 2^-10 keeps a margin -- and
# 24 in fp32) + ARITH * (|ref - beta| + |beta| + rms_row(ref - beta)) (fp32
# arithmetic: the mean, variance and scale are fp32 reductions over the row,
# so their rounding is an error on the row's scale, which reaches even the
# elements near the mean; then one rsqrt, a multiply by gamma and an add of
# beta on the element's own terms) + FLOOR (fp16's subnormal spacing). ref is
# the fp64 oracle on the same rounded inputs.
OUT_REL = {BF16: 2.0 ** -8, F16: 2.0 ** -10, F32: 2.0 ** -24}
ARITH = {BF16: 2.0 ** -16, F16: 2.0 ** -16, F32: 2.0 ** -18}
FLOOR = {BF16: 0.0, F16: 2.0 ** -25, F32: 0.0}


def norm_bound(ref, beta, t):
    ref = np.asarray(ref, np.float64)
    b = np.zeros_like(ref) if beta is None else np.broadcast_to(np.asarray(beta, np.float64), ref.shape)
    d = ref - b
    row_rms = np.sqrt(np.mean(d * d, axis=-1, keepdims=True))
    return OUT_REL[t] * np.abs(ref) + ARITH[t] * (np.abs(d) + np.abs(b) + row_rms) + FLOOR[t]


def norm_violations(y, ref, beta, t):
    """Number of elements outside norm_bound (0 = pass)."""
    err = np.abs(np.asarray(y, np.float64) - np.asarray(ref, np.float64))
    return int(np.sum(~(err <= norm_bound(ref, beta, t))))


def check_norm(y, ref, beta, t):
    bad = norm_violations(y, ref, beta, t)
    err = np.abs(np.asarray(y, np.float64) - np.asarray(ref, np.float64))
    assert bad == 0, (bad, float(err.max()))


def run_norm(dnn, layer, t, rows, hidden, seed, pitch=None, x=None, eps=1e-6):
    r = np.random.default_rng(seed)
    pitch = pitch or hidden
    if x is None:
        x = r.standard_normal((rows, hidden)).astype(np.float32)
    gamma = (1 + 0.02 * r.standard_normal(hidden)).astype(np.float32)
    beta = (0.02 * r.standard_normal(hidden)).astype(np.float32)
    xe, ge, be = enc(x, t), enc(gamma, t), enc(beta, t)
    xq, gq, bq = dec(xe, t), dec(ge, t), dec(be, t)       # what the kernel sees
    xbuf = np.zeros((rows, pitch), nptype(t))
    xbuf[:, :hidden] = xe
    poison = np.full((rows, pitch), 0x7FC1 if t != F32 else np.float32(np.nan), nptype(t))
    dx, dg, db, dy = to_dev(xbuf), to_dev(ge), to_dev(be), to_dev(poison)
    xd = g.TensorDesc(t, [rows, hidden], [pitch, 1])
    wd = g.TensorDesc(t, [hidden])
    say(f"{'layernorm' if layer else 'rmsnorm'} t={t} rows={rows} hidden={hidden} pitch={pitch}")
    if layer:
        s = dnn.layernorm(xd, dx.p, wd, dg.p, db.p, eps, xd, dy.p)
    else:
        s = dnn.rmsnorm(xd, dx.p, wd, dg.p, eps, xd, dy.p)
    assert s == g.SUCCESS, g.STATUS[s]
    g.synchronize()
    got = dy.download(nptype(t), rows * pitch).reshape(rows, pitch)
    if pitch > hidden:  # the row padding is never written
        pad = got[:, hidden:]
        assert np.array_equal(pad.view(np.uint8), poison[:, hidden:].view(np.uint8))
    yg = dec(np.ascontiguousarray(got[:, :hidden]), t)
    ref = O.layernorm(xq, gq, bq, eps) if layer else O.rmsnorm(xq, gq, eps)
    return yg, ref, (bq if layer else None)


SHAPES = [(1, 1), (3, 7), (5, 100), (64, 512), (33, 2048), (16, 4096), (8, 8192), (4, 16384),
          (2, 16392), (2, 65536)]


@pytest.mark.parametrize("layer", [False, True])
@pytest.mark.parametrize("rows,hidden", SHAPES)
def test_norm_bf16_vs_oracle(dnn, layer, rows, hidden):
    y, ref, beta = run_norm(dnn, layer, BF16, rows, hidden, seed=rows + hidden)
    if hidden == 1 and layer:
        # a one-element row normalises to beta exactly
        assert np.array_equal(y, O.bf16_to_f32(O.f32_to_bf16(ref)))
    check_norm(y, ref, beta, BF16)


@pytest.mark.parametrize("t", [F16, F32])
@pytest.mark.parametrize("layer", [False, True])
def test_norm_other_types(dnn, t, layer):
    y, ref, beta = run_norm(dnn, layer, t, 24, 1024, seed=5)
    check_norm(y, ref, beta, t)


def eps_rows(hidden):
    """Rows on which eps decides the result (RMSNorm: mean(x^2) comparable to
    eps or below it; LayerNorm: variance comparable to eps): constant 1e-3
    rows (mean square 1e-6), N(0, 1e-6) rows, an all-zero row (must give 0,
    not NaN) and N(0,1) rows (with a large eps)."""
    r = np.random.default_rng(hidden)
    return np.stack([np.full(hidden, 1e-3, np.float32),
                     np.full(hidden, -1e-3, np.float32),
                     (1e-3 * r.standard_normal(hidden)).astype(np.float32),
                     np.zeros(hidden, np.float32),
                     r.standard_normal(hidden).astype(np.float32),
                     (0.5 * r.standard_normal(hidden)).astype(np.float32)])


# (eps, hidden): the BASELINE eps on rows of its own scale, then eps values
# that dominate unit-scale rows; hidden lengths reach the wave, block and
# element-wise kernels.
EPS_CASES = [(1e-6, 8192), (1e-6, 1024), (1e-1, 8192), (0.5, 4096), (1.0, 1000), (1e-6, 8200)]


@pytest.mark.parametrize("layer", [False, True])
@pytest.mark.parametrize("eps,hidden", EPS_CASES)
def test_norm_eps_pinned(dnn, layer, eps, hidden):
    x = eps_rows(hidden)
    y, ref, beta = run_norm(dnn, layer, BF16, x.shape[0], hidden, seed=3, x=x, eps=eps)
    assert np.isfinite(y).all()
    check_norm(y, ref, beta, BF16)
    if not layer:
        assert not np.any(y[3]), "an all-zero row gives 0"


@pytest.mark.parametrize("layer", [False, True])
@pytest.mark.parametrize("t,rows,hidden", [
    (BF16, 5, 2056), (BF16, 7, 4104), (BF16, 3, 8200), (BF16, 3, 32768),   # ragged / full blocks
    (F32, 6, 8192), (F32, 3, 3000), (F16, 4, 12000)])
def test_norm_block_paths(dnn, t, layer, rows, hidden):
    """Every workgroup-per-row configuration (256, 512, 1024 threads; two or
    four chunks each), with row lengths that leave most of the last chunks
    idle as well as ones that fill the block exactly."""
    y, ref, beta = run_norm(dnn, layer, t, rows, hidden, seed=rows * hidden)
    check_norm(y, ref, beta, t)


@pytest.mark.parametrize("layer", [False, True])
@pytest.mark.parametrize("t,rows,hidden,pitch", [
    (BF16, 4099, 8192, 8192), (BF16, 2048, 4104, 4112), (F32, 2051, 3000, 3000)])
def test_norm_block_two_rows_per_workgroup(dnn, t, layer, rows, hidden, pitch):
    """From 2048 rows on, norm_block runs two adjacent rows per workgroup
    with gamma and beta held in registers and the partial sums alternating
    between two LDS slots: every row checked, odd row counts (the last
    workgroup has one row), a padded pitch, bf16 and fp32."""
    y, ref, beta = run_norm(dnn, layer, t, rows, hidden, seed=rows + 7 * hidden, pitch=pitch)
    check_norm(y, ref, beta, t)


@pytest.mark.parametrize("layer", [False, True])
def test_norm_padded_rows(dnn, layer):
    y, ref, beta = run_norm(dnn, layer, BF16, 40, 1000, seed=9, pitch=1008)
    check_norm(y, ref, beta, BF16)


def test_layernorm_constant_rows_give_beta_exactly(dnn):
    rows, hidden = 6, 8192
    x = np.repeat(np.array([1.5, -2.25, 0.0, 3.0, 1e-3, -7.0], np.float32)[:, None], hidden, 1)
    y, _, bq = run_norm(dnn, True, BF16, rows, hidden, seed=2, x=x)
    assert np.array_equal(y, np.tile(O.bf16_to_f32(O.f32_to_bf16(bq)), (rows, 1)))


def test_config4_full_size(dnn):
    """BASELINE config 4 at full size (16384 x 8192 bf16): every row against
    the oracle element by element (half a bf16 ulp plus fp32 arithmetic)."""
    from grxcp_amd import synth
    rows, hidden = 16384, 8192
    xb = synth.normal_bf16(rows * hidden, 41).reshape(rows, hidden)
    gb = synth.normal_bf16(hidden, 42, 1.0, 0.02)
    bb = synth.normal_bf16(hidden, 43, 0.0, 0.02)
    dx, dg, db, dy = to_dev(xb), to_dev(gb), to_dev(bb), g.DeviceBuffer(rows * hidden * 2)
    xd, wd = g.TensorDesc(BF16, [rows, hidden]), g.TensorDesc(BF16, [hidden])
    for layer in (False, True):
        say(f"config4 {'layernorm' if layer else 'rmsnorm'} full size")
        s = (dnn.layernorm(xd, dx.p, wd, dg.p, db.p, 1e-6, xd, dy.p) if layer
             else dnn.rmsnorm(xd, dx.p, wd, dg.p, 1e-6, xd, dy.p))
        assert s == 0
        g.synchronize()
        y = dy.download(np.uint16, rows * hidden).reshape(rows, hidden)
        xs = O.bf16_to_f32(xb)
        gf, bf = O.bf16_to_f32(gb), O.bf16_to_f32(bb)
        ref = O.layernorm(xs, gf, bf, 1e-6) if layer else O.rmsnorm(xs, gf, 1e-6)
        yf = O.bf16_to_f32(y)
        for r0 in range(0, rows, 2048):      # in slices, to bound host memory
            check_norm(yf[r0:r0 + 2048], ref[r0:r0 + 2048], bf if layer else None, BF16)
        del xs, ref
        assert np.isfinite(yf).all()
        # every row, size-independent: (y - beta) / gamma has mean square
        # ms / (ms + eps) = 1 - O(1e-6) on these rows, and mean 0 for LayerNorm,
        # up to bf16 rounding of y (2^-9 per element, far less on row means)
        u = (yf.astype(np.float64) - (bf if layer else 0.0)) / gf
        rms = np.sqrt(np.mean(u * u, axis=1))
        assert np.max(np.abs(rms - 1.0)) < 2e-3, float(np.max(np.abs(rms - 1.0)))
        if layer:
            assert np.max(np.abs(np.mean(u, axis=1))) < 2e-3


# ---- attention -----------------------------------------------------------------

def run_attention(dnn, t, B, H, S, D, causal, seed, q=None, k=None, v=None, scale=None):
    r = np.random.default_rng(seed)
    scale = D ** -0.5 if scale is None else scale
    shp = (B, H, S, D)
    q = r.standard_normal(shp).astype(np.float32) if q is None else q
    k = r.standard_normal(shp).astype(np.float32) if k is None else k
    v = r.standard_normal(shp).astype(np.float32) if v is None else v
    qe, ke, ve = enc(q, t), enc(k, t), enc(v, t)
    dq, dk, dv = to_dev(qe), to_dev(ke), to_dev(ve)
    do = g.DeviceBuffer(qe.nbytes)
    desc = g.TensorDesc(t, list(shp))
    ad = g.AttnDesc(causal, scale)
    say(f"attention t={t} B={B} H={H} S={S} D={D} causal={causal} scale={scale:g}")
    s = dnn.attention(ad, desc, dq.p, desc, dk.p, desc, dv.p, desc, do.p)
    assert s == g.SUCCESS, g.STATUS[s]
    g.synchronize()
    o = dec(do.download(np.uint16, qe.size), t).reshape(shp)
    return o, dec(qe, t).reshape(shp), dec(ke, t).reshape(shp), dec(ve, t).reshape(shp)


@pytest.mark.parametrize("t", [BF16, F16])
@pytest.mark.parametrize("S,D,causal", [(128, 128, True), (256, 128, True), (256, 128, False),
                                        (200, 128, True), (1, 128, True), (130, 64, True),
                                        (333, 64, False), (64, 128, False)])
def test_attention_vs_oracle(dnn, t, S, D, causal):
    B, H = 2, 3
    o, q, k, v = run_attention(dnn, t, B, H, S, D, causal, seed=S + D)
    for b in range(B):
        for h in range(H):
            ref = O.attention_head(q[b, h], k[b, h], v[b, h], causal, D ** -0.5)
            assert normwise_rel_err(o[b, h], ref) <= 1e-2, (b, h)


def test_attention_closed_forms(dnn):
    B, H, S, D = 1, 2, 256, 128
    r = np.random.default_rng(1)
    v = r.standard_normal((B, H, S, D)).astype(np.float32)
    o, _, _, vq = run_attention(dnn, BF16, B, H, S, D, True, seed=3, v=v)
    # row 0 attends to key 0 only: O[0] == V[0] exactly
    assert np.array_equal(o[:, :, 0], vq[:, :, 0])
    # Q = 0: uniform weights over the causal prefix -> running mean of V
    o0, _, _, vq0 = run_attention(dnn, BF16, B, H, S, D, True, seed=4, q=np.zeros((B, H, S, D), np.float32),
                                  v=v)
    want = np.cumsum(vq0.astype(np.float64), 2) / np.arange(1, S + 1)[None, None, :, None]
    assert normwise_rel_err(o0, want) <= 1e-2
    # V constant along keys -> O = V
    vc = np.broadcast_to(r.standard_normal((B, H, 1, D)).astype(np.float32), (B, H, S, D)).copy()
    oc, _, _, vqc = run_attention(dnn, BF16, B, H, S, D, True, seed=5, v=vc)
    assert normwise_rel_err(oc, vqc) <= 1e-2


@pytest.mark.parametrize("t", [BF16, F16])
@pytest.mark.parametrize("case", ["growing", "huge_scale", "all_negative"])
@pytest.mark.parametrize("D,causal", [(128, True), (64, False)])
def test_attention_extreme_logits(dnn, t, case, D, causal):
    """Logits the online softmax must rescale for: key magnitudes growing
    along the sequence (each tile's maximum keeps overtaking the running one,
    so the rescale of O and l runs again and again), a softmax scale of 20
    (logits of a few hundred: exp overflows without the running-maximum
    shift) and logits of about -4000 everywhere (exp underflows without it).
    Every head against the float64 oracle, which shifts by the exact row
    maximum."""
    B, H, S = 1, 2, 300
    r = np.random.default_rng({"growing": 61, "huge_scale": 62, "all_negative": 63}[case] + D)
    shp = (B, H, S, D)
    q, k, v = (r.standard_normal(shp).astype(np.float32) for _ in range(3))
    scale = D ** -0.5
    if case == "growing":
        q *= 3.0
        k *= (1.0 + 3.0 * np.arange(S, dtype=np.float32) / S)[None, None, :, None]
    elif case == "huge_scale":
        scale = 20.0
    else:
        q, k = np.abs(q), -np.abs(k)
        scale = 50.0
    o, qd, kd, vd = run_attention(dnn, t, B, H, S, D, causal, seed=0, q=q, k=k, v=v, scale=scale)
    assert np.isfinite(o).all()
    for b in range(B):
        for h in range(H):
            ref = O.attention_head(qd[b, h], kd[b, h], vd[b, h], causal, scale)
            assert normwise_rel_err(o[b, h], ref) <= 1e-2, (case, b, h)


@pytest.mark.parametrize("B,H,S,D,causal", [(4, 256, 64, 128, True), (4, 256, 64, 64, False),
                                             (2, 128, 300, 128, True), (1, 512, 100, 64, True)])
def test_attention_many_items_per_workgroup(dnn, B, H, S, D, causal):
    """Enough heads that every persistent workgroup runs several items, with
    items of one or two tiles: the K/V loads issued two tiles ahead cross
    into the next items, and each item's Q and O move at item boundaries.
    Every head checked."""
    o, q, k, v = run_attention(dnn, BF16, B, H, S, D, causal, seed=B * H + S + D)
    for b in range(B):
        for h in range(H):
            ref = O.attention_head(q[b, h], k[b, h], v[b, h], causal, D ** -0.5)
            assert normwise_rel_err(o[b, h], ref) <= 1e-2, (b, h)


@pytest.mark.parametrize("B,H,S,D,causal", [(2, 3, 256, 128, True), (2, 3, 333, 64, False),
                                             (4, 256, 64, 128, True), (4, 256, 64, 64, False),
                                             (2, 128, 300, 128, True), (1, 64, 520, 128, False)])
def test_attention_in_place(dnn, B, H, S, D, causal):
    """O written over Q (the same buffer and descriptor): a workgroup loads
    each item's Q before it stores that item's O, and the next item's Q rows
    are other rows, so the result equals the out-of-place one. Shapes where
    every persistent workgroup runs several items, causal and not, both head
    dimensions, S beyond one query tile. Every head against the oracle
    computed from the original Q."""
    r = np.random.default_rng(B * H + S + D + 7)
    shp = (B, H, S, D)
    q, k, v = (O.f32_to_bf16(r.standard_normal(shp).astype(np.float32)) for _ in range(3))
    dq, dk, dv = to_dev(q), to_dev(k), to_dev(v)
    desc = g.TensorDesc(BF16, list(shp))
    ad = g.AttnDesc(causal, D ** -0.5)
    say(f"attention in place B={B} H={H} S={S} D={D} causal={causal}")
    assert dnn.attention(ad, desc, dq.p, desc, dk.p, desc, dv.p, desc, dq.p) == g.SUCCESS
    g.synchronize()
    o = O.bf16_to_f32(dq.download(np.uint16, q.size)).reshape(shp)
    qf, kf, vf = (O.bf16_to_f32(a).reshape(shp) for a in (q, k, v))
    assert np.array_equal(dk.download(np.uint16, k.size), k.ravel())
    assert np.array_equal(dv.download(np.uint16, v.size), v.ravel())
    for b in range(B):
        for h in range(H):
            ref = O.attention_head(qf[b, h], kf[b, h], vf[b, h], causal, D ** -0.5)
            assert normwise_rel_err(o[b, h], ref) <= 1e-2, (b, h)


@pytest.mark.parametrize("causal", [True, False])
def test_attention_packed_qkv_output_over_q(dnn, causal):
    """A packed [B, S, 3, H, D] QKV buffer with O written over its Q slot
    (O == Q, same strides): K and V, whose rows interleave with Q's, are left
    as they were, and every head matches the oracle on the original Q."""
    B, H, S, D = 2, 8, 384, 128
    r = np.random.default_rng(17 + causal)
    qkv = O.f32_to_bf16(r.standard_normal((B, S, 3, H, D)).astype(np.float32))
    dbuf = to_dev(qkv)
    strides = [S * 3 * H * D, D, 3 * H * D, 1]
    desc = g.TensorDesc(BF16, [B, H, S, D], strides)
    pq = dbuf.p.value
    pk, pv = pq + 2 * H * D, pq + 4 * H * D
    ad = g.AttnDesc(causal, D ** -0.5)
    say(f"attention packed QKV, O over Q, causal={causal}")
    st = dnn.attention(ad, desc, ctypes.c_void_p(pq), desc, ctypes.c_void_p(pk), desc,
                       ctypes.c_void_p(pv), desc, ctypes.c_void_p(pq))
    assert st == g.SUCCESS, g.STATUS[st]
    g.synchronize()
    got = dbuf.download(np.uint16, qkv.size).reshape(B, S, 3, H, D)
    assert np.array_equal(got[:, :, 1:], qkv[:, :, 1:])
    o = O.bf16_to_f32(got[:, :, 0])
    x = O.bf16_to_f32(qkv)
    for b in range(B):
        for h in range(H):
            ref = O.attention_head(x[b, :, 0, h], x[b, :, 1, h], x[b, :, 2, h], causal, D ** -0.5)
            assert normwise_rel_err(o[b, :, h], ref) <= 1e-2, (b, h)


def test_attention_key_permutation_invariant(dnn):
    """Keys and their values permuted together leave every row of full
    attention unchanged, and the last row of causal attention (which sees
    every key); only the summation order differs. The kernel's tiling puts
    the permuted keys in different tiles, so this also checks that the
    online softmax across tiles is order-independent."""
    B, H, S, D = 1, 2, 320, 128
    r = np.random.default_rng(21)
    q, k, v = (r.standard_normal((B, H, S, D)).astype(np.float32) for _ in range(3))
    perm = r.permutation(S)
    for causal in (False, True):
        o1, _, _, _ = run_attention(dnn, BF16, B, H, S, D, causal, seed=0, q=q, k=k, v=v)
        o2, _, _, _ = run_attention(dnn, BF16, B, H, S, D, causal, seed=0, q=q,
                                    k=np.ascontiguousarray(k[:, :, perm]),
                                    v=np.ascontiguousarray(v[:, :, perm]))
        rows = slice(None) if not causal else slice(S - 1, S)
        assert normwise_rel_err(o2[:, :, rows], o1[:, :, rows].astype(np.float64)) <= 5e-3, causal


def test_rmsnorm_scale_invariant_and_one_hot(dnn):
    """RMSNorm(x * 2^k) == RMSNorm(x) up to eps (a power-of-two scale is exact
    in bf16 and leaves every fp32 step's relative rounding unchanged), and a
    one-hot row a*e_j gives gamma_j * a / sqrt(a^2/H + eps) at j and 0
    elsewhere."""
    rows, hidden = 6, 8192
    r = np.random.default_rng(5)
    x = r.standard_normal((rows, hidden)).astype(np.float32)
    y1, _, _ = run_norm(dnn, False, BF16, rows, hidden, seed=8, x=x, eps=0.0)
    y2, _, _ = run_norm(dnn, False, BF16, rows, hidden, seed=8, x=x * 16.0, eps=0.0)
    assert np.array_equal(y1, y2)
    oh = np.zeros((rows, hidden), np.float32)
    js = [0, 1, 4095, 4096, 8190, 8191]
    amps = [1.0, -3.0, 0.5, 7.25, -0.125, 100.0]
    for i, (j, a) in enumerate(zip(js, amps)):
        oh[i, j] = a
    y, ref, _ = run_norm(dnn, False, BF16, rows, hidden, seed=9, x=oh, eps=1e-6)
    check_norm(y, ref, None, BF16)
    for i, j in enumerate(js):
        assert np.count_nonzero(y[i]) == 1 and y[i, j] != 0
        want = ref[i, j]
        assert abs(y[i, j] - want) <= 2.0 ** -8 * abs(want)


def test_attention_strided_layout(dnn):
    """[B, S, H, D] storage described by strides (heads interleaved)."""
    B, H, S, D = 2, 4, 192, 128
    r = np.random.default_rng(11)
    x = [r.standard_normal((B, S, H, D)).astype(np.float32) for _ in range(3)]
    enc3 = [O.f32_to_bf16(a) for a in x]
    dev = [to_dev(a) for a in enc3]
    do = g.DeviceBuffer(enc3[0].nbytes)
    strides = [S * H * D, D, H * D, 1]
    desc = g.TensorDesc(BF16, [B, H, S, D], strides)
    ad = g.AttnDesc(True, D ** -0.5)
    say("attention strided [B,S,H,D]")
    assert dnn.attention(ad, desc, dev[0].p, desc, dev[1].p, desc, dev[2].p, desc, do.p) == 0
    g.synchronize()
    o = O.bf16_to_f32(do.download(np.uint16, enc3[0].size)).reshape(B, S, H, D)
    qf, kf, vf = (O.bf16_to_f32(a).reshape(B, S, H, D) for a in enc3)
    for b in range(B):
        for h in range(H):
            ref = O.attention_head(qf[b, :, h], kf[b, :, h], vf[b, :, h], True, D ** -0.5)
            assert normwise_rel_err(o[b, :, h], ref) <= 1e-2


def test_attention_output_row_stride_and_span_limit(dnn):
    """O rows far apart (128 KB sequence stride, heads back to back): every
    row is right, and nothing else in the buffer is written -- not the gaps
    between rows, not the rows past S of a query tile (S = 100: the last
    tile's rows 100..127 would land on the next head's first rows), not the
    guard rows after the last head. A stride whose 32-bit span check fails
    is refused before any launch."""
    B, H, S, D = 1, 2, 100, 128
    o_ss = 1 << 16
    r = np.random.default_rng(31)
    shp = (B, H, S, D)
    q, k, v = (O.f32_to_bf16(r.standard_normal(shp).astype(np.float32)) for _ in range(3))
    dq, dk, dv = to_dev(q), to_dev(k), to_dev(v)
    total = (H * S + 32) * o_ss                       # 32 guard rows after the last head
    sentinel = np.full(total, 0xFFFF, np.uint16)       # a bf16 NaN pattern
    do = to_dev(sentinel)
    din = g.TensorDesc(BF16, list(shp))
    dout = g.TensorDesc(BF16, list(shp), [H * S * o_ss, S * o_ss, o_ss, 1])
    ad = g.AttnDesc(True, D ** -0.5)
    say("attention O sequence stride 2^16")
    assert dnn.attention(ad, din, dq.p, din, dk.p, din, dv.p, dout, do.p) == g.SUCCESS
    g.synchronize()
    got = do.download(np.uint16, total)
    rows = got[:H * S * o_ss].reshape(H, S, o_ss)
    qf, kf, vf = (O.bf16_to_f32(a).reshape(shp) for a in (q, k, v))
    for h in range(H):
        ref = O.attention_head(qf[0, h], kf[0, h], vf[0, h], True, D ** -0.5)
        assert normwise_rel_err(O.bf16_to_f32(rows[h, :, :D]), ref) <= 1e-2, h
    assert (rows[:, :, D:] == 0xFFFF).all()
    assert (got[H * S * o_ss:] == 0xFFFF).all()
    # (S + 256) rows of 2 * o_ss bytes reach 2^31: NOT_SUPPORTED, O untouched
    o_big = 3_100_000
    big = g.DeviceBuffer(((S - 1) * o_big + D) * 2)
    dbig = g.TensorDesc(BF16, [1, 1, S, D], [S * o_big, S * o_big, o_big, 1])
    one = g.TensorDesc(BF16, [1, 1, S, D])
    assert dnn.attention(ad, one, dq.p, one, dk.p, one, dv.p, dbig, big.p) == g.NOT_SUPPORTED


def test_config5_full_size(dnn):
    """BASELINE config 5 at full size (B4 H32 S4096 D128 bf16, causal): every
    query row of every head against the oracle (relative error of the row
    <= 1e-2), plus size-independent properties."""
    from grxcp_amd import synth
    B, H, S, D = 4, 32, 4096, 128
    n = B * H * S * D
    qb, kb, vb = (synth.normal_bf16(n, s) for s in (51, 52, 53))
    dq, dk, dv, do = to_dev(qb), to_dev(kb), to_dev(vb), g.DeviceBuffer(n * 2)
    desc = g.TensorDesc(BF16, [B, H, S, D])
    ad = g.AttnDesc(True, D ** -0.5)
    say("config5 attention full size")
    assert dnn.attention(ad, desc, dq.p, desc, dk.p, desc, dv.p, desc, do.p) == 0
    g.synchronize()
    o = do.download(np.uint16, n).reshape(B, H, S, D)
    worst = 0.0
    for b in range(B):
        for h in range(H):
            q = O.bf16_to_f32(qb.reshape(B, H, S, D)[b, h])
            k = O.bf16_to_f32(kb.reshape(B, H, S, D)[b, h])
            v = O.bf16_to_f32(vb.reshape(B, H, S, D)[b, h])
            ref = O.attention_head(q, k, v, True, D ** -0.5).astype(np.float64)
            got = O.bf16_to_f32(o[b, h]).astype(np.float64)
            rel = np.linalg.norm(got - ref, axis=1) / np.linalg.norm(ref, axis=1)
            worst = max(worst, float(rel.max()))
            assert rel.max() <= 1e-2, (b, h, int(rel.argmax()), float(rel.max()))
    say(f"config5 worst row relative error {worst:.2e}")
    of = O.bf16_to_f32(o)
    assert np.isfinite(of).all()
    # every head, size-independent: row 0 attends to key 0 alone (O = V[0],
    # exactly), and every output is a convex combination of the V rows of its
    # causal prefix, so it lies between their running minimum and maximum
    # (up to O's bf16 rounding and the fp32 accumulation)
    vf = O.bf16_to_f32(vb).reshape(B, H, S, D)
    assert np.array_equal(of[:, :, 0], vf[:, :, 0])
    lo = np.minimum.accumulate(vf, axis=2)
    hi = np.maximum.accumulate(vf, axis=2)
    tol = 2.0 ** -8 * np.maximum(np.abs(lo), np.abs(hi)) + 1e-3
    assert np.all(of >= lo - tol) and np.all(of <= hi + tol)
