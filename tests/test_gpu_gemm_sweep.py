"""Seeded randomized sweep of grxblasGemmEx / grxblasGemmExDequant.

The targeted GemmEx tests check one mechanism at a time; this sweep draws
combinations of them from a fixed seed: fp16/bf16 inputs with fp32 or
16-bit C, int8 with int32 C, int8 dequant to bf16, all four transposes,
ragged and padded shapes, alpha/beta, K from 1 up to 4160, sized so that
some cases take the 256x256-tile kernel directly, some through transposed
operand copies, some split along K and some the general kernel. Inputs are
exact by construction (the reference's method, ref
tests/libs/test_grxblas_ex.cpp:1-14), so every case is compared BIT-EXACT
over the whole padded C buffer against the CPU oracle, with 4 KB guard
bands on both sides of C that must come back unchanged. The path each call
took is read from the library's GRXBLAS_LOG line, and each test asserts that
its cases covered every path.
"""
import numpy as np
import pytest

import grxcp_amd as g
from test_gpu_gemm import dequant_case, float_case, int8_case, logged_plans

pytestmark = pytest.mark.gpu

F16, BF16, F32, I8, I32 = g.GRX_R_16F, g.GRX_R_16BF, g.GRX_R_32F, g.GRX_R_8I, g.GRX_R_32I


def _pick(r, seq):
    return seq[int(r.integers(len(seq)))]


def _shape(r, kind, elem_bytes):
    """(ta, tb, m, n, k, pad, cpad) for one kind of case."""
    ta, tb = int(r.integers(2)), int(r.integers(2))
    unit = 16 // elem_bytes                     # K elements per 16 bytes
    if kind == "small":                         # the general kernel
        m, n, k = (int(v) for v in r.integers(1, 80, 3))
        return ta, tb, m, n, k, _pick(r, [0, 1, 3]), _pick(r, [0, 2, 5])
    if kind == "medium":                        # either kernel, odd K included
        m, n = (int(v) for v in r.integers(60, 700, 2))
        return ta, tb, m, n, int(r.integers(1, 700)), _pick(r, [0, 1, 8]), _pick(r, [0, 3, 8])
    # "split" and "copy": aligned so that the 256x256-tile kernel can run,
    # and m*n*k >= 2^25 so that other layouts take the transposed copies
    m = 8 * int(r.integers(40, 96))
    n = int(r.integers(300, 768))
    if kind == "split":                         # few tiles, K of 32 to 65 stages
        k = unit * int(r.integers(4096 // 16, 8320 // 16))
    else:                                       # a layout other than (T, N), one pass
        ta, tb = _pick(r, [(0, 0), (0, 1), (1, 1)])
        k = unit * int(r.integers(512 // unit, 1008 // unit))
    return ta, tb, m, n, k, _pick(r, [0, unit]), _pick(r, [0, 8])


def _covered(plans):
    return {"split": any(int(p["split"]) > 1 for p in plans),
            "copy_a": any(p["copy_a"] == "1" for p in plans),
            "copy_b": any(p["copy_b"] == "1" for p in plans),
            "tn128": any(p["kernel"] == "tn128" for p in plans),
            "general64": any(p["kernel"] == "general64" for p in plans)}


def test_float_sweep(blas, capfd):
    r = np.random.default_rng(20261)
    kinds = ["small", "medium", "split", "copy"]
    bad, plans = [], []
    for i in range(48):
        in_t = _pick(r, [F16, BF16])
        out_t = _pick(r, [F32, in_t])
        ta, tb, m, n, k, pad, cpad = _shape(r, kinds[i % 4], 2)
        alpha = _pick(r, [1.0, 2.5, -0.5])
        beta = _pick(r, [0.0, 1.0, -1.5])
        res = []
        got = logged_plans(capfd, lambda: res.append(
            float_case(blas, in_t, out_t, ta, tb, m, n, k, alpha, beta, pad, cpad, seed=1000 + i,
                       guard=True)))
        plans += got
        if res != [(0, 0)]:
            bad.append((i, in_t, out_t, ta, tb, m, n, k, alpha, beta, pad, cpad, res, got))
    assert not bad, bad
    cov = _covered(plans)
    assert all(cov.values()), cov


def test_int8_sweep(blas, capfd):
    r = np.random.default_rng(20262)
    kinds = ["small", "medium", "split", "copy"]
    bad, plans = [], []
    for i in range(24):
        ta, tb, m, n, k, pad, cpad = _shape(r, kinds[i % 4], 1)
        alpha = _pick(r, [1.0, 3.0, -2.0])
        beta = _pick(r, [0.0, 1.0, -1.0])
        res = []
        got = logged_plans(capfd, lambda: res.append(
            int8_case(blas, ta, tb, m, n, k, alpha, beta, pad, fill="rand", seed=2000 + i, cpad=cpad,
                      guard=True)))
        plans += got
        if res != [0]:
            bad.append((i, ta, tb, m, n, k, alpha, beta, pad, cpad, res, got))
    assert not bad, bad
    cov = _covered(plans)
    assert all(cov.values()), cov


def test_dequant_sweep(blas, capfd):
    r = np.random.default_rng(20263)
    kinds = ["small", "medium", "split", "copy"]
    bad, plans = [], []
    for i in range(16):
        ta, tb, m, n, k, pad, cpad = _shape(r, kinds[i % 4], 1)
        res = []
        got = logged_plans(capfd, lambda: res.append(
            dequant_case(blas, ta, tb, m, n, k, pad, cpad, seed=3000 + i, guard=True)))
        plans += got
        if res != [(0, 0)]:
            bad.append((i, ta, tb, m, n, k, pad, cpad, res, got))
    assert not bad, bad
    cov = _covered(plans)
    assert all(cov.values()), cov


def test_in_place_operand_sweep(blas, capfd):
    """16-bit problems of the layouts other than (T, N) on the 128x128
    kernel, drawn from a fixed seed: one pass, K slices and staged C (an
    odd ldc), m a multiple of 8, n and the padding random, so that A and B
    are read in place where their columns sit on 16 bytes and copied where
    not. Bit-exact over the padded C with guard bands; the plan's direct_a /
    direct_b must be what the alignment rule says, and the sweep must cover
    both operands in place, a copy, K slices and a staged C."""
    r = np.random.default_rng(20264)
    bad, plans = [], []
    for i in range(15):
        in_t = _pick(r, [F16, BF16])
        out_t = _pick(r, [F32, in_t])
        ta, tb = _pick(r, [(0, 0), (0, 1), (1, 1)])
        long_k = i % 3 == 2                     # few tiles, long K: K slices
        m = 8 * int(r.integers(40, 80)) if long_k else 8 * int(r.integers(66, 140))
        n = int(r.integers(300, 700)) if long_k else int(r.integers(520, 1100))
        k = 8 * int(r.integers(300, 700)) if long_k else 8 * int(r.integers(8, 200))
        pad = _pick(r, [0, 0, 8, 2])
        cpad = _pick(r, [0, 8, 1]) if out_t != F32 else _pick(r, [0, 4, 1])
        alpha, beta = _pick(r, [1.0, 2.5, -0.5]), _pick(r, [0.0, 1.0, -1.5])
        res = []
        got = logged_plans(capfd, lambda: res.append(
            float_case(blas, in_t, out_t, ta, tb, m, n, k, alpha, beta, pad, cpad, seed=4000 + i,
                       guard=True)))
        plans += got
        lda, ldb = (k if ta else m) + pad, (n if tb else k) + pad
        ok = len(got) == 1 and res == [(0, 0)]
        if ok and got[0]["kernel"] == "tn128" and pad != 2:
            want_a = str(int(ta == 0 and lda % 8 == 0))
            want_b = str(int(tb == 1 and n % 8 == 0 and ldb % 8 == 0))
            ok = (got[0]["direct_a"], got[0]["direct_b"]) == (want_a, want_b)
        if not ok:
            bad.append((i, in_t, out_t, ta, tb, m, n, k, pad, cpad, res, got))
    assert not bad, bad
    cov = {"direct_a": any(p["direct_a"] == "1" for p in plans),
           "direct_b": any(p["direct_b"] == "1" for p in plans),
           "copy": any(p["copy_a"] == "1" or p["copy_b"] == "1" for p in plans),
           "split": any(int(p["split"]) > 1 and p["direct_a"] + p["direct_b"] != "00" for p in plans),
           "staged": any(p["staged"] == "1" and p["direct_a"] + p["direct_b"] != "00" for p in plans)}
    assert all(cov.values()), (cov, plans)
