"""Pinning the CPU oracle before trusting it.

The reference ships no fixture files; its numerical gates generate inputs with
an LCG and compare against CPU reference functions (ref
tests/libs/test_grxblas.cpp:45-80, test_grxblas_ex.cpp:45-63, 254-281). The
oracle restates those functions; here each one is checked against something
it does not share code with -- known-answer tests from the reference, numpy /
torch library routines in float64, closed forms and invariants -- and each
check is shown to FAIL when a plausible mistake is planted in the oracle
(oracle_set_mutation), so a passing check means something.
"""
import numpy as np
import pytest
import torch

import oracle as O


@pytest.fixture(autouse=True)
def _no_mutation():
    O.set_mutation(0)
    yield
    O.set_mutation(0)


def col_major(mat: np.ndarray, ld: int) -> np.ndarray:
    """Store a (rows x cols) matrix column-major with leading dimension ld."""
    rows, cols = mat.shape
    buf = np.zeros(ld * cols, mat.dtype)
    for j in range(cols):
        buf[j * ld: j * ld + rows] = mat[:, j]
    return buf


def from_col_major(buf: np.ndarray, rows: int, cols: int, ld: int) -> np.ndarray:
    return np.stack([buf[j * ld: j * ld + rows] for j in range(cols)], axis=1)


# ---- generators and narrow formats ----------------------------------------

def test_lcg_matches_reference_recurrence():
    # seed*1664525 + 1013904223 mod 2^32; value ((s >> 16) % 17 - 8) * 0.25
    s, vals = 1, []
    for _ in range(5):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        vals.append(((s >> 16) % 17 - 8) * 0.25)
    assert O.fill_quarters(5, 1).tolist() == vals
    st = O.HalvesStream(99)
    a = st.take(3)
    b = st.take(2)  # the stream continues across calls, as in the gate
    assert np.array_equal(np.concatenate([a, b]), O.HalvesStream(99).take(5))
    assert set(np.unique(O.fill_quarters(4000, 7))) <= {i * 0.25 for i in range(-8, 9)}


def test_half_to_float_all_patterns_vs_numpy():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.half_to_f32(bits)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_float_to_half_rne_vs_numpy():
    g = np.random.default_rng(0)
    x = np.concatenate([
        g.standard_normal(200000).astype(np.float32) * 100,
        (g.integers(-8, 9, 1000) * 0.5).astype(np.float32),
        np.array([65504, 65520, 65519.996, 1e9, -1e9, 6.104e-5, np.inf, -np.inf], np.float32),
    ])
    got = O.f32_to_half(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16)
    # numpy keeps subnormal halves; the reference conversion flushes them to
    # signed zero (ref tests/common/fp16.h:32), so compare where numpy's result
    # is normal, infinite or zero.
    rb = ref.view(np.uint16)
    normal = ((rb & 0x7C00) != 0) | ((rb & 0x7FFF) == 0)
    assert np.array_equal(got[normal], rb[normal])
    sub = ~normal
    assert np.all((got[sub] & 0x7FFF) == 0)


def test_bf16_rne_vs_torch():
    g = np.random.default_rng(1)
    x = np.concatenate([
        g.standard_normal(300000).astype(np.float32),
        g.standard_normal(1000).astype(np.float32) * 1e30,
        np.array([0.0, -0.0, np.inf, -np.inf, 3.0e38, 1e-40, -1e-40], np.float32),
        # exact ties: low 16 bits 0x8000, both parities of bit 16
        (np.array([0x3F808000, 0x3F818000, 0xBF808000], np.uint32)).view(np.float32),
    ])
    got = O.f32_to_bf16(x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
    assert np.array_equal(O.bf16_to_f32(got), torch.from_numpy(want.view(np.int16)).view(
        torch.bfloat16).float().numpy())
    nan = O.f32_to_bf16(np.array([np.nan], np.float32))
    assert (nan[0] & 0x7F80) == 0x7F80 and (nan[0] & 0x7F) != 0


# ---- GEMMs ------------------------------------------------------------------

def test_sgemm_known_answer():
    # A = [[1,2],[3,4]], B = [[5,6],[7,8]] -> [[19,22],[43,50]]; C col-major.
    A = col_major(np.array([[1, 2], [3, 4]], np.float32), 2)
    B = col_major(np.array([[5, 6], [7, 8]], np.float32), 2)
    C = np.zeros(4, np.float32)
    assert O.sgemm(0, 0, 2, 2, 2, 1.0, A, 2, B, 2, 0.0, C, 2).tolist() == [19, 43, 22, 50]
    # op(A) = A^T reads the same storage transposed: A^T B = [[26,30],[38,44]]
    assert O.sgemm(1, 0, 2, 2, 2, 1.0, A, 2, B, 2, 0.0, C, 2).tolist() == [26, 38, 30, 44]
    # alpha, beta: 2*AB - 1*[[1,1],[1,1]]
    C1 = np.ones(4, np.float32)
    assert O.sgemm(0, 0, 2, 2, 2, 2.0, A, 2, B, 2, -1.0, C1, 2).tolist() == [37, 85, 43, 99]


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
@pytest.mark.parametrize("pad", [0, 3])
def test_sgemm_vs_numpy(ta, tb, pad):
    g = np.random.default_rng(ta * 2 + tb + 10 * pad)
    m, n, k = 13, 7, 29
    opA = g.standard_normal((m, k)).astype(np.float32)
    opB = g.standard_normal((k, n)).astype(np.float32)
    Cm = g.standard_normal((m, n)).astype(np.float32)
    lda = (k if ta else m) + pad
    ldb = (n if tb else k) + pad
    ldc = m + pad
    A = col_major(opA.T.copy() if ta else opA, lda)
    B = col_major(opB.T.copy() if tb else opB, ldb)
    C = col_major(Cm, ldc)
    got = O.sgemm(ta, tb, m, n, k, 1.5, A, lda, B, ldb, -0.5, C, ldc)
    want = 1.5 * (opA.astype(np.float64) @ opB.astype(np.float64)) - 0.5 * Cm.astype(np.float64)
    np.testing.assert_allclose(from_col_major(got, m, n, ldc), want, rtol=1e-6, atol=1e-6)
    # padding rows untouched
    for j in range(n):
        assert np.array_equal(got[j * ldc + m:(j + 1) * ldc], C[j * ldc + m:(j + 1) * ldc])


def test_sgemm_beta_zero_does_not_read_c():
    A = np.ones(4, np.float32)
    C = np.full(4, np.nan, np.float32)
    got = O.sgemm(0, 0, 2, 2, 2, 1.0, A, 2, A, 2, 0.0, C, 2)
    assert got.tolist() == [2, 2, 2, 2]


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_gemm_f32acc_exact_inputs_vs_numpy(ta, tb):
    # Multiples of 0.5 in [-4, 4]: products and sums are exact in fp32, so the
    # fp32-accumulating oracle must equal a float64 matmul bit for bit.
    st = O.HalvesStream(99)
    m, n, k, pad = 17, 9, 13, 2
    lda = (k if ta else m) + pad
    ldb = (n if tb else k) + pad
    ldc = m + pad
    A = st.take(lda * (m if ta else k))
    B = st.take(ldb * (k if tb else n))
    C = st.take(ldc * n) * 2
    got = O.gemm_f32acc(ta, tb, m, n, k, 2.5, A, lda, B, ldb, -1.5, C, ldc)
    opA = from_col_major(A, k, m, lda).T if ta else from_col_major(A, m, k, lda)
    opB = from_col_major(B, n, k, ldb).T if tb else from_col_major(B, k, n, ldb)
    want = 2.5 * (opA.astype(np.float64) @ opB.astype(np.float64)) - 1.5 * from_col_major(C, m, n, ldc)
    assert np.array_equal(from_col_major(got, m, n, ldc), want.astype(np.float32))


def test_igemm_reference_known_answers():
    # ref src/backends/npu_c930/test_npu_c930.cc:183-238 (row-major 2x2 cases)
    for a, b, want in [([1, 2, 3, 4], [5, 6, 7, 8], [19, 22, 43, 50]),
                       ([-1, 2, 3, -4], [5, -6, 7, 8], [9, 22, -13, -50])]:
        A = col_major(np.array(a, np.int8).reshape(2, 2), 2)
        B = col_major(np.array(b, np.int8).reshape(2, 2), 2)
        C = np.zeros(4, np.int32)
        got = O.igemm(0, 0, 2, 2, 2, 1, A, 2, B, 2, 0, C, 2)
        assert from_col_major(got, 2, 2, 2).reshape(-1).tolist() == want


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_igemm_vs_numpy_full_range(ta, tb):
    g = np.random.default_rng(5 + ta + 2 * tb)
    m, n, k = 19, 11, 300
    opA = g.integers(-128, 128, (m, k)).astype(np.int8)
    opB = g.integers(-128, 128, (k, n)).astype(np.int8)
    Cm = g.integers(-1000, 1000, (m, n)).astype(np.int32)
    lda, ldb, ldc = (k if ta else m) + 1, (n if tb else k) + 2, m + 3
    A = col_major(opA.T.copy() if ta else opA, lda)
    B = col_major(opB.T.copy() if tb else opB, ldb)
    C = col_major(Cm, ldc)
    got = O.igemm(ta, tb, m, n, k, 3, A, lda, B, ldb, -2, C, ldc)
    want = 3 * (opA.astype(np.int64) @ opB.astype(np.int64)) - 2 * Cm.astype(np.int64)
    assert np.array_equal(from_col_major(got, m, n, ldc), want.astype(np.int32))


def test_igemm_wraps_like_int32():
    A = col_major(np.full((1, 4), 127, np.int8), 1)
    B = col_major(np.full((4, 1), 127, np.int8), 4)
    got = O.igemm(0, 0, 1, 1, 4, 70000, A, 1, B, 4, 0, np.zeros(1, np.int32), 1)
    want = (np.int64(4 * 127 * 127) * 70000 + 2**31) % 2**32 - 2**31
    assert int(got[0]) == int(want)


def test_dequant_vs_numpy_and_torch():
    g = np.random.default_rng(3)
    m, n, ld = 33, 21, 40
    acc = g.integers(-(127 * 127 * 8192), 127 * 127 * 8192, ld * n).astype(np.int32)
    scale = g.uniform(0.001, 0.01, n).astype(np.float32)
    got = O.dequant(m, n, acc, ld, scale, m)
    a = from_col_major(acc, m, n, ld).astype(np.float32)     # RNE int -> float
    prod = a * scale[None, :]                                  # one RNE multiply
    want = torch.from_numpy(prod).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(from_col_major(got, m, n, m), want)
    # scale == 1 reduces to bf16(float(acc))
    ones = O.dequant(m, n, acc, ld, np.ones(n, np.float32), m)
    assert np.array_equal(from_col_major(ones, m, n, m),
                          torch.from_numpy(a).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))


# ---- norms ------------------------------------------------------------------

def test_rmsnorm_closed_forms_and_torch():
    g = np.random.default_rng(4)
    H = 512
    gamma = (1 + 0.02 * g.standard_normal(H)).astype(np.float32)
    for c in (np.float32(1.75), np.float32(1e-3)):  # at 1e-3, c^2 == eps: eps matters
        x = np.full((1, H), c, np.float32)
        y = O.rmsnorm(x, gamma, 1e-6)
        np.testing.assert_allclose(y[0], gamma * np.float64(c) / np.sqrt(np.float64(c) ** 2 + 1e-6),
                                   rtol=1e-6)
    xr = g.standard_normal((8, H)).astype(np.float32)
    # scale invariance with eps = 0
    np.testing.assert_allclose(O.rmsnorm(xr * 3.0, gamma, 0.0), O.rmsnorm(xr, gamma, 0.0), rtol=1e-5)
    want = torch.nn.functional.rms_norm(torch.from_numpy(xr).double(), (H,),
                                        torch.from_numpy(gamma).double(), eps=1e-6)
    np.testing.assert_allclose(O.rmsnorm(xr, gamma, 1e-6), want.numpy(), rtol=1e-6, atol=1e-6)


def test_layernorm_closed_forms_and_torch():
    g = np.random.default_rng(6)
    H = 384
    gamma = (1 + 0.02 * g.standard_normal(H)).astype(np.float32)
    beta = (0.02 * g.standard_normal(H)).astype(np.float32)
    x = np.full((2, H), -3.25, np.float32)
    assert np.array_equal(O.layernorm(x, gamma, beta, 1e-6), np.stack([beta, beta]))
    # a row of +-d: mean 0, variance d^2 -> y = gamma * (+-d) / sqrt(d^2 + eps) + beta
    d = 1e-3
    xs = np.tile(np.array([d, -d], np.float32), H // 2)[None]
    want_s = gamma * xs[0].astype(np.float64) / np.sqrt(d * d + 1e-6) + beta
    np.testing.assert_allclose(O.layernorm(xs, gamma, beta, 1e-6)[0], want_s, rtol=1e-5, atol=1e-7)
    xr = g.standard_normal((8, H)).astype(np.float32)
    np.testing.assert_allclose(O.layernorm(xr + 5.0, gamma, beta, 1e-6), O.layernorm(xr, gamma, beta, 1e-6),
                               rtol=1e-4, atol=1e-5)
    want = torch.nn.functional.layer_norm(torch.from_numpy(xr).double(), (H,), torch.from_numpy(gamma).double(),
                                          torch.from_numpy(beta).double(), eps=1e-6)
    np.testing.assert_allclose(O.layernorm(xr, gamma, beta, 1e-6), want.numpy(), rtol=1e-6, atol=1e-6)


# ---- attention --------------------------------------------------------------

def _torch_attention(q, k, v, causal, scale):
    t = lambda a: torch.from_numpy(a).double()[None, None]
    return torch.nn.functional.scaled_dot_product_attention(t(q), t(k), t(v), is_causal=causal,
                                                            scale=scale)[0, 0].numpy()


@pytest.mark.parametrize("causal", [True, False])
def test_attention_vs_torch_sdpa(causal):
    g = np.random.default_rng(7)
    S, D = 70, 64
    q, k, v = (g.standard_normal((S, D)).astype(np.float32) for _ in range(3))
    got = O.attention_head(q, k, v, causal, D ** -0.5)
    np.testing.assert_allclose(got, _torch_attention(q, k, v, causal, D ** -0.5), rtol=1e-5, atol=1e-6)


def test_attention_closed_forms():
    g = np.random.default_rng(8)
    S, D = 40, 32
    q, k, v = (g.standard_normal((S, D)).astype(np.float32) for _ in range(3))
    o = O.attention_head(q, k, v, True, 0.3)
    assert np.array_equal(o[0], v[0])                            # row 0 sees only key 0
    o0 = O.attention_head(np.zeros_like(q), k, v, True, 0.3)     # uniform weights
    np.testing.assert_allclose(o0, np.cumsum(v, 0) / np.arange(1, S + 1)[:, None], rtol=1e-5, atol=1e-6)
    vu = np.tile(v[:1], (S, 1))
    np.testing.assert_allclose(O.attention_head(q, k, vu, True, 0.3), vu, rtol=1e-6)
    # permuting keys (with their values) inside the causal prefix of the last row
    perm = g.permutation(S)
    last = O.attention_head(q, k[perm], v[perm], False, 0.3)
    np.testing.assert_allclose(last, O.attention_head(q, k, v, False, 0.3), rtol=1e-5, atol=1e-6)


def test_softmax_closed_forms_and_torch():
    g = np.random.default_rng(11)
    # constant rows -> 1/n (exact for n a power of two)
    for n in (1, 8, 1024):
        y = O.softmax(np.full((3, n), 2.5, np.float32))
        assert np.array_equal(y, np.full((3, n), 1.0 / n, np.float32))
    # two elements: the logistic function
    a, b = 0.75, -1.25
    y = O.softmax(np.array([[a, b]], np.float32))
    np.testing.assert_allclose(y[0, 0], 1.0 / (1.0 + np.exp(b - a)), rtol=1e-7)
    x = (3.0 * g.standard_normal((37, 301))).astype(np.float32)
    y = O.softmax(x)
    np.testing.assert_allclose(y.sum(axis=1), 1.0, rtol=1e-6)
    np.testing.assert_allclose(O.softmax(x + np.float32(7.0)), y, rtol=1e-5, atol=1e-9)
    ref = torch.softmax(torch.from_numpy(x).double(), dim=1).float().numpy()
    np.testing.assert_allclose(y, ref, rtol=1e-6, atol=1e-12)


def test_gelu_published_values_identity_and_torch():
    # Phi(1) = 0.841344746068543, Phi(2) = 0.977249868051821 (standard normal table)
    x = np.array([0.0, 1.0, -1.0, 2.0], np.float32)
    y = O.gelu(x, 0)
    np.testing.assert_allclose(y, [0.0, 0.841344746068543, -0.158655253931457, 2 * 0.977249868051821],
                               rtol=1e-6, atol=1e-12)
    g = np.random.default_rng(12)
    x = (2.5 * g.standard_normal(4001)).astype(np.float32)
    for mode, approx in ((0, "none"), (1, "tanh")):
        y, ym = O.gelu(x, mode), O.gelu(-x, mode)
        np.testing.assert_allclose(y - ym, x, rtol=1e-5, atol=1e-6)   # gelu(x) - gelu(-x) = x
        ref = torch.nn.functional.gelu(torch.from_numpy(x).double(), approximate=approx).float().numpy()
        np.testing.assert_allclose(y, ref, rtol=1e-6, atol=1e-7)


def test_gelu_far_tails_and_specials():
    """The negative tail to relative precision, where 1 + erf and 1 + tanh
    cancel in double (x < -8.3 and x < -6): against scipy's normal CDF
    (x Phi(x), computed through erfc) and logistic (x expit(2z), the tanh
    form's sigmoid), neither of which shares code with the oracle; and the
    specials: gelu(+inf) = +inf, gelu(-inf) = NaN (-inf times 0, as the
    formula gives), NaN stays NaN, far tails to +x and -0."""
    import scipy.special as sp
    x = np.concatenate([-np.geomspace(3.0, 40.0, 2000), np.geomspace(3.0, 40.0, 200)]).astype(np.float32)
    xd = x.astype(np.float64)
    z = np.sqrt(2.0 / np.pi) * (xd + 0.044715 * xd ** 3)
    for mode, want in ((0, xd * sp.ndtr(xd)), (1, xd * sp.expit(2.0 * z))):
        y = O.gelu(x, mode).astype(np.float64)
        w = want.astype(np.float32).astype(np.float64)       # the oracle rounds once to fp32
        normal = np.abs(w) >= np.finfo(np.float32).tiny
        assert normal.sum() > 1000                          # down to x = -13 (erf), -10 (tanh)
        np.testing.assert_allclose(y[normal], w[normal], rtol=2e-7, atol=0)
        assert np.all(np.abs(y[~normal] - w[~normal]) <= 2.0 ** -149)
    s = np.array([np.inf, -np.inf, np.nan, 1e30, -1e30], np.float32)
    for mode in (0, 1):
        y = O.gelu(s, mode)
        assert y[0] == np.inf and np.isnan(y[1]) and np.isnan(y[2])
        assert y[3] == np.float32(1e30) and y[4] == 0.0 and np.signbit(y[4])


# ---- the checks above fail when a mistake is planted --------------------------

@pytest.mark.parametrize("mutation,check", [
    (1, lambda: test_sgemm_vs_numpy(1, 0, 0)),
    (2, lambda: test_sgemm_vs_numpy(0, 0, 0)),
    (3, lambda: test_sgemm_known_answer()),
    (1, lambda: test_gemm_f32acc_exact_inputs_vs_numpy(1, 1)),
    (2, lambda: test_igemm_reference_known_answers()),
    (3, lambda: test_igemm_vs_numpy_full_range(0, 0)),
    (4, lambda: test_rmsnorm_closed_forms_and_torch()),
    (4, lambda: test_layernorm_closed_forms_and_torch()),
    (4, lambda: test_attention_vs_torch_sdpa(True)),
    (5, lambda: test_attention_closed_forms()),
    (6, lambda: test_dequant_vs_numpy_and_torch()),
    (7, lambda: test_softmax_closed_forms_and_torch()),
    (8, lambda: test_gelu_published_values_identity_and_torch()),
])
def test_planted_mistake_is_caught(mutation, check):
    O.set_mutation(mutation)
    with pytest.raises(AssertionError):
        check()
