"""grxblasSetCycleProbe on gfx950: one grxCycleSlot per wave.

Mirrors the reference's own use of the probe (ref tests/bench/gemm_cycles.cpp):
slots sized by grxblasCycleSlotsNeeded(h, m, n), zeroed, attached, one call,
detached, read back, on the same small shapes with all-ones inputs. On gfx950
every wave of the GEMM kernels writes slot blockIdx*4 + wave: s_memtime at
entry and at exit, core = XCD << 16 | CU id, warp = wave in its workgroup. A
capacity below what the launch needs is refused before any launch (ref
src/libs/grxblas/grxblas.cpp:690-692, 929-932).
"""
import ctypes

import numpy as np
import pytest

import grxcp_amd as g
from helpers import say, to_dev

pytestmark = pytest.mark.gpu

SLOT = ctypes.sizeof(g.CycleSlot)
SLOT_DTYPE = np.dtype([("start", "<u8"), ("end", "<u8"), ("core", "<u4"), ("warp", "<u4")])
F16_ONE, BF16_ONE = 0x3C00, 0x3F80
GEMM_CYCLES_SHAPES = [(16, 16, 16), (16, 16, 32), (16, 16, 64), (32, 32, 32), (32, 32, 64)]


def probe_call(blas, nslots, call):
    buf = g.DeviceBuffer(nslots * SLOT)
    buf.memset(0)
    assert blas.set_cycle_probe(buf.p, nslots) == g.SUCCESS
    status = call()
    g.synchronize()
    assert blas.set_cycle_probe(None, 0) == g.SUCCESS
    raw = buf.download(np.uint8, nslots * SLOT)
    return status, np.frombuffer(raw.tobytes(), dtype=SLOT_DTYPE)


def check_written(slots, expected):
    written = np.nonzero((slots["start"] != 0) | (slots["end"] != 0))[0]
    assert written.tolist() == list(expected)
    w = slots[written]
    assert np.all(w["end"] > w["start"])
    assert np.all(w["end"] - w["start"] < 10**9)
    assert np.all((w["core"] >> 16) < 8), "XCD id"
    assert np.all(w["warp"] == written % 4)
    return w


@pytest.mark.parametrize("m,n,k", GEMM_CYCLES_SHAPES)
def test_probe_gemm_ex_f16(blas, m, n, k):
    nslots = blas.cycle_slots_needed(m, n)
    assert nslots == 4
    dA = to_dev(np.full(m * k, F16_ONE, np.uint16))
    dB = to_dev(np.full(k * n, F16_ONE, np.uint16))
    dC = to_dev(np.zeros(m * n, np.float32))
    say(f"probe GemmEx f16 NN {m}x{n}x{k}")
    s, slots = probe_call(blas, nslots, lambda: blas.gemm_ex(
        0, 0, m, n, k, 1.0, dA.p, g.GRX_R_16F, m, dB.p, g.GRX_R_16F, k, 0.0, dC.p, g.GRX_R_32F, m))
    assert s == g.SUCCESS, g.STATUS[s]
    assert np.all(dC.download(np.float32, m * n) == k)
    w = check_written(slots, range(4))
    assert len(set(w["core"].tolist())) == 1, "one workgroup runs on one CU"


@pytest.mark.parametrize("m,n,k", GEMM_CYCLES_SHAPES)
def test_probe_sgemm(blas, m, n, k):
    nslots = blas.cycle_slots_needed(m, n)
    dA = to_dev(np.ones(m * k, np.float32))
    dB = to_dev(np.ones(k * n, np.float32))
    dC = to_dev(np.zeros(m * n, np.float32))
    say(f"probe Sgemm NN {m}x{n}x{k}")
    s, slots = probe_call(blas, nslots, lambda: blas.sgemm(
        0, 0, m, n, k, 1.0, dA.p, m, dB.p, k, 0.0, dC.p, m))
    assert s == g.SUCCESS, g.STATUS[s]
    assert np.all(dC.download(np.float32, m * n) == k)
    w = check_written(slots, range(4))
    assert len(set(w["core"].tolist())) == 1


def test_probe_fast_path_bf16(blas):
    m = n = k = 512  # TN, 16-byte rows: the 256x256-tile kernel, 4 workgroups
    nslots = blas.cycle_slots_needed(m, n)
    assert nslots == 4 * 8 * 8
    dA = to_dev(np.full(m * k, BF16_ONE, np.uint16))
    dB = to_dev(np.full(k * n, BF16_ONE, np.uint16))
    dC = to_dev(np.zeros(m * n, np.uint16))
    say("probe GemmEx bf16 TN 512^3 (fast path)")
    s, slots = probe_call(blas, nslots, lambda: blas.gemm_ex(
        1, 0, m, n, k, 1.0, dA.p, g.GRX_R_16BF, k, dB.p, g.GRX_R_16BF, k, 0.0, dC.p, g.GRX_R_16BF, m))
    assert s == g.SUCCESS, g.STATUS[s]
    assert np.all(dC.download(np.uint16, m * n) == 0x4400)  # bf16(512)
    check_written(slots, range(16))


def test_probe_batched_sgemm_needs_slots_per_member(blas):
    m = n = k = 16
    batch = 3
    need = blas.cycle_slots_needed(m, n) * batch
    dA = to_dev(np.ones(m * k * batch, np.float32))
    dB = to_dev(np.ones(k * n * batch, np.float32))
    dC = to_dev(np.zeros(m * n * batch, np.float32))
    call = lambda: blas.sgemm_strided_batched(0, 0, m, n, k, 1.0, dA.p, m, m * k, dB.p, k, k * n,
                                              0.0, dC.p, m, m * n, batch)
    say("probe SgemmStridedBatched 16^3 x3, one slot short")
    s, slots = probe_call(blas, need - 1, call)
    assert s == g.INVALID_VALUE
    assert not np.any(slots["end"])
    assert np.all(dC.download(np.float32, m * n * batch) == 0), "refused before any launch"
    say("probe SgemmStridedBatched 16^3 x3")
    s, slots = probe_call(blas, need, call)
    assert s == g.SUCCESS, g.STATUS[s]
    assert np.all(dC.download(np.float32, m * n * batch) == k)
    check_written(slots, range(need))


def test_probe_capacity_refused_for_gemm_ex(blas):
    m = n = k = 32
    dA = to_dev(np.full(m * k, F16_ONE, np.uint16))
    dB = to_dev(np.full(k * n, F16_ONE, np.uint16))
    dC = to_dev(np.full(m * n, 7.0, np.float32))
    say("probe GemmEx with too few slots")
    s, slots = probe_call(blas, blas.cycle_slots_needed(m, n) - 1, lambda: blas.gemm_ex(
        0, 0, m, n, k, 1.0, dA.p, g.GRX_R_16F, m, dB.p, g.GRX_R_16F, k, 0.0, dC.p, g.GRX_R_32F, m))
    assert s == g.INVALID_VALUE
    assert np.all(dC.download(np.float32, m * n) == 7.0)
    assert not np.any(slots["end"])


def test_probe_level12(blas):
    """Level 1/2 calls write one slot per wave of their 256-thread workgroups
    (the reference writes one per block there, ref grxblas.cpp:764-766)."""
    n = 1000  # saxpy / sscal: 4 workgroups
    dx = to_dev(np.arange(n, dtype=np.float32))
    dy = to_dev(np.ones(n, np.float32))
    say("probe saxpy n=1000, one slot short")
    s, slots = probe_call(blas, 15, lambda: blas.L.grxblasSaxpy(blas.h, n, g.fptr(2.0), dx.p, 1, dy.p, 1))
    assert s == g.INVALID_VALUE and not np.any(slots["end"])
    assert np.all(dy.download(np.float32, n) == 1.0)
    say("probe saxpy n=1000")
    s, slots = probe_call(blas, 16, lambda: blas.L.grxblasSaxpy(blas.h, n, g.fptr(2.0), dx.p, 1, dy.p, 1))
    assert s == g.SUCCESS
    assert np.array_equal(dy.download(np.float32, n), 2.0 * np.arange(n, dtype=np.float32) + 1.0)
    check_written(slots, range(16))
    say("probe sscal n=1000")
    s, slots = probe_call(blas, 16, lambda: blas.L.grxblasSscal(blas.h, n, g.fptr(0.5), dx.p, 1))
    assert s == g.SUCCESS
    check_written(slots, range(16))
    m, nn = 300, 5
    dA = to_dev(np.ones(m * nn, np.float32))
    dv = to_dev(np.ones(max(m, nn), np.float32))
    dw = to_dev(np.zeros(max(m, nn), np.float32))
    for trans, blocks in ((0, 2), (1, nn)):
        say(f"probe sgemv trans={trans} {m}x{nn}")
        s, slots = probe_call(blas, 4 * blocks, lambda: blas.L.grxblasSgemv(
            blas.h, trans, m, nn, g.fptr(1.0), dA.p, m, dv.p, 1, g.fptr(0.0), dw.p, 1))
        assert s == g.SUCCESS
        out = dw.download(np.float32, nn if trans else m)
        assert np.all(out == (m if trans else nn))
        check_written(slots, range(4 * blocks))


def test_probe_attention(dnn):
    """grxdnnSetCycleProbe: one slot per attention wave that has work, at
    workgroup * 8 + wave. One (batch, head) of 512 queries is two 256-query
    items, both on the head's XCD share (workgroups 0 and 8 of 16: XCD
    share = workgroup % 8); the other shares have no work and write nothing.
    Workgroups 0 and 8 run on one hardware XCD, which the kernel's head split
    assumes. With one slot too few the call is refused before any launch."""
    import oracle as O
    B, H, S, D = 1, 1, 512, 128
    nslots = dnn.attention_cycle_slots_needed(B, H, S)
    assert nslots == 16 * 8
    r = np.random.default_rng(7)
    q, k, v = (O.f32_to_bf16(r.standard_normal((S, D)).astype(np.float32)) for _ in range(3))
    dq, dk, dv = to_dev(q), to_dev(k), to_dev(v)
    do = to_dev(np.full(S * D, 0x7FC0, np.uint16))
    desc = g.TensorDesc(g.GRX_R_16BF, [B, H, S, D])
    ad = g.AttnDesc(True, D ** -0.5)
    call = lambda: dnn.attention(ad, desc, dq.p, desc, dk.p, desc, dv.p, desc, do.p)  # noqa: E731
    say("probe attention, one slot short")
    s, slots = probe_call(dnn, nslots - 1, call)
    assert s == g.INVALID_VALUE and not np.any(slots["end"])
    assert np.all(do.download(np.uint16, S * D) == 0x7FC0)
    say("probe attention B=1 H=1 S=512 D=128 causal")
    s, slots = probe_call(dnn, nslots, call)
    assert s == g.SUCCESS, g.STATUS[s]
    written = np.nonzero((slots["start"] != 0) | (slots["end"] != 0))[0]
    assert written.tolist() == list(range(0, 8)) + list(range(64, 72))
    w = slots[written]
    assert np.all(w["end"] > w["start"]) and np.all(w["end"] - w["start"] < 10**9)
    assert np.all(w["warp"] == written % 8)
    assert len(set((w["core"] >> 16).tolist())) == 1, "workgroups 0 and 8 on one XCD"
    assert len(set(w[:8]["core"].tolist())) == 1 and len(set(w[8:]["core"].tolist())) == 1
    o = O.bf16_to_f32(do.download(np.uint16, S * D)).reshape(S, D)
    ref = O.attention_head(O.bf16_to_f32(q).reshape(S, D), O.bf16_to_f32(k).reshape(S, D),
                           O.bf16_to_f32(v).reshape(S, D), True, D ** -0.5)
    assert np.max(np.abs(o - ref)) / np.max(np.abs(ref)) <= 1e-2
