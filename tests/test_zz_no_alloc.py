"""grxblasGemmExNoAlloc against grxblasGemmEx, through the C ABI, on the GPU.

The allocation-free entry point runs grxblasGemmEx's plans with the
library's static per-device scratch in place of the handle's workspace, so
its output must be bit-identical to grxblasGemmEx's on the same inputs. Two
calls in a row, the second smaller than the first, each on a plan that uses
the scratch (split-K partials, then a transposed operand copy); a problem
that needs more scratch than the library holds is refused before anything is
launched, and its output buffer is left as it was. Calls on two streams that
would overlap take turns on the scratch; calls on a fresh handle leave the
device's free memory unchanged; the scratch is only loaded by a process that
calls the entry point; a call captured in a HIP graph gives the same bits on
every replay.
"""
import ctypes
import json
import os
import subprocess
import sys

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
    # 2: smaller, (T, T) with n = 508 (B's columns off 16 bytes, so not read
    #    in place) -> the transposed copy of B in the scratch, fp32 C
    c1, c2, p1, p2 = _pair(blas, capfd, 1, 1, 768, 508, 2048, BF16, F32, seed=2)
    assert p1 == p2 and len(p2) == 1 and p2[0]["copy_b"] == "1", (p1, p2)
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
    """(T, T) 4096 x 4092 x 8208 bf16 (B's columns, ldb = n = 4092, off 16
    bytes, so B is not read in place) would copy B (4092 x 8208 bf16, 67.2
    MB) into more than the 64 MiB scratch: NOT_SUPPORTED with a message,
    nothing launched, C untouched. The buffers are full size, so nothing
    could fault even if a launch happened."""
    m, n, k = 4096, 4092, 8208
    dA, dB = g.DeviceBuffer(m * k * 2), g.DeviceBuffer(k * n * 2)
    poison = np.full(m * n, 0x7FC00001, np.uint32)
    dC = to_dev(poison)
    capfd.readouterr()
    s = blas.gemm_ex_noalloc(1, 1, m, n, k, 1.0, dA.p, BF16, k, dB.p, BF16, n, 0.0, dC.p, F32, m)
    err = capfd.readouterr().err
    g.synchronize()
    assert s == g.NOT_SUPPORTED, g.STATUS[s]
    assert "grxblasGemmExNoAlloc" in err and "scratch" in err
    assert np.array_equal(dC.download(np.uint32, m * n), poison)


def test_noalloc_without_room_for_padded_copies_takes_the_general_path(blas, capfd):
    """K not a multiple of 16 bytes: grxblasGemmEx pads it in copies of both
    operands. Where those copies exceed the 64 MiB scratch (2048 x 2048 x
    8199 bf16: 67 MB) the allocation-free entry point runs the plan without
    them, the general kernel, rather than refusing a problem it ran before
    such copies existed. Exact inputs (halves), so both give the same bits."""
    import oracle as O
    m, n, k = 2048, 2048, 8199
    st = O.HalvesStream(77)
    dA, dB = to_dev(O.f32_to_bf16(st.take(m * k))), to_dev(O.f32_to_bf16(st.take(k * n)))
    got, plans = [], []
    for fn in (blas.gemm_ex, blas.gemm_ex_noalloc):
        dC = g.DeviceBuffer(m * n * 4)
        say(f"padded-copy plan {m}x{n}x{k} through {fn.__name__}")
        status = []
        plans += logged_plans(capfd, lambda: status.append(  # noqa: B023
            fn(1, 0, m, n, k, 1.0, dA.p, BF16, k, dB.p, BF16, k, 0.0, dC.p, F32, m)))
        g.synchronize()
        assert status == [g.SUCCESS], status
        got.append(dC.download(np.float32, m * n))
    assert [(p["kernel"], p["copy_a"], p["copy_b"]) for p in plans] == \
        [("tn128", "1", "1"), ("general64", "0", "0")], plans
    assert np.array_equal(got[0].view(np.uint32), got[1].view(np.uint32))


def _bf16_operands(r, m, n, k):
    A = synth.f32_to_bf16_bits(r.standard_normal(m * k).astype(np.float32))
    B = synth.f32_to_bf16_bits(r.standard_normal(n * k).astype(np.float32))
    return to_dev(A), to_dev(B)


def _free_bytes() -> int:
    free, total = ctypes.c_size_t(0), ctypes.c_size_t(0)
    g.check_rt(g.load().rt.grxMemGetInfo(ctypes.byref(free), ctypes.byref(total)), "grxMemGetInfo")
    return free.value


def test_noalloc_calls_on_two_streams_take_turns(gpu):
    """Two handles on two streams issue split-K NoAlloc calls (52 MiB of
    partials each) back to back with no synchronisation between them: the
    second stream waits for the first's launch, so both results are
    bit-identical to GemmEx's. Four rounds, the streams alternating."""
    m, n, k = 1024, 1024, 8192
    r = np.random.default_rng(11)
    streams = [g.Stream(), g.Stream()]
    handles = [g.Blas(), g.Blas()]
    for h, st in zip(handles, streams):
        h.set_stream(st.s)
    ops = [_bf16_operands(r, m, n, k) for _ in range(2)]
    ref_blas = g.Blas()
    refs = []
    for dA, dB in ops:
        dC = g.DeviceBuffer(m * n * 2)
        g.check(ref_blas.gemm_ex(1, 0, m, n, k, 1.0, dA.p, BF16, k, dB.p, BF16, k, 0.0, dC.p, BF16, m),
                "GemmEx")
        g.synchronize()
        refs.append(dC.download(np.uint16, m * n))
        dC.close()
    outs = [g.DeviceBuffer(m * n * 2) for _ in range(2)]
    for rnd in range(4):
        order = (0, 1) if rnd % 2 == 0 else (1, 0)
        for o in outs:
            o.memset(0xFF)
        say(f"noalloc two streams round {rnd} order {order}")
        for i in order:
            dA, dB = ops[i]
            g.check(handles[i].gemm_ex_noalloc(1, 0, m, n, k, 1.0, dA.p, BF16, k, dB.p, BF16, k, 0.0,
                                               outs[i].p, BF16, m), "GemmExNoAlloc")
        g.synchronize()
        for i in range(2):
            assert np.array_equal(outs[i].download(np.uint16, m * n), refs[i]), (rnd, i)
    for h in handles + [ref_blas]:
        h.close()
    for st in streams:
        st.close()


def test_noalloc_allocates_nothing_on_a_fresh_handle(blas):
    """After the device's first NoAlloc call (which resolves the scratch),
    NoAlloc calls on a new handle -- split-K first, then a transposed copy
    -- leave the device's free memory exactly as it was: no workspace is
    allocated for the handle (GemmEx would allocate 52 MiB here)."""
    r = np.random.default_rng(12)
    m, n, k = 1024, 1024, 8192
    dA, dB = _bf16_operands(r, m, n, k)
    dC = g.DeviceBuffer(m * n * 2)
    g.check(blas.gemm_ex_noalloc(1, 0, m, n, k, 1.0, dA.p, BF16, k, dB.p, BF16, k, 0.0, dC.p, BF16, m),
            "GemmExNoAlloc warm-up")
    g.synchronize()
    fresh = g.Blas()
    say("noalloc fresh handle, free memory before and after")
    before = _free_bytes()
    for _ in range(3):
        g.check(fresh.gemm_ex_noalloc(1, 0, m, n, k, 1.0, dA.p, BF16, k, dB.p, BF16, k, 0.0, dC.p,
                                      BF16, m), "GemmExNoAlloc split-K")
        g.check(fresh.gemm_ex_noalloc(0, 0, 768, 512, 2048, 1.0, dA.p, BF16, 768, dB.p, BF16, 2048,
                                      0.0, dC.p, BF16, 768), "GemmExNoAlloc copy")
    g.synchronize()
    after = _free_bytes()
    fresh.close()
    assert after == before, (before, after)


_PROBE = r"""
import ctypes, json, sys
import numpy as np
sys.path.insert(0, sys.argv[1])
import grxcp_amd as g
L = g.load()
g.check_rt(L.rt.grxSetDevice(0), "grxSetDevice")
def free():
    f, t = ctypes.c_size_t(0), ctypes.c_size_t(0)
    g.check_rt(L.rt.grxMemGetInfo(ctypes.byref(f), ctypes.byref(t)), "grxMemGetInfo")
    return f.value
m, n, k = 1024, 1024, 8192
dA, dB, dC = g.DeviceBuffer(m * k * 2), g.DeviceBuffer(n * k * 2), g.DeviceBuffer(m * n * 4)
for d in (dA, dB, dC):
    d.memset(0)
b = g.Blas()
g.synchronize()
f0 = free()
# a TN GemmEx that needs no scratch (one launch of the GEMM kernels)
g.check(b.gemm_ex(1, 0, 256, 256, 256, 1.0, dA.p, g.GRX_R_16BF, 256, dB.p, g.GRX_R_16BF, 256, 0.0,
                  dC.p, g.GRX_R_32F, 256), "GemmEx")
g.synchronize()
f1 = free()
g.check(b.gemm_ex_noalloc(1, 0, m, n, k, 1.0, dA.p, g.GRX_R_16BF, k, dB.p, g.GRX_R_16BF, k, 0.0,
                          dC.p, g.GRX_R_16BF, m), "GemmExNoAlloc")
g.synchronize()
f2 = free()
print(json.dumps({"before": f0, "after_gemm_ex": f1, "after_noalloc": f2}))
"""


def test_scratch_is_held_only_by_processes_that_call_noalloc(gpu):
    """In a fresh process: loading the library and running GemmEx does not
    take the 64 MiB scratch; the first NoAlloc call does."""
    say("noalloc scratch residency, fresh process")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _PROBE, root], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    v = json.loads(r.stdout.strip().splitlines()[-1])
    mib = 1 << 20
    assert v["before"] - v["after_gemm_ex"] < 32 * mib, v
    assert v["after_gemm_ex"] - v["after_noalloc"] >= 64 * mib, v


def test_noalloc_under_hip_graph_capture(blas):
    """A split-K NoAlloc call captured in a HIP graph (torch.cuda.graph on
    the library's handle) gives GemmEx's bits on every one of five replays,
    with eager GemmEx work, other NoAlloc calls and synchronisations between
    the replays. The device's first NoAlloc call is made before capture."""
    torch = pytest.importorskip("torch")
    m, n, k = 1024, 1024, 8192
    r = np.random.default_rng(13)
    dA, dB = _bf16_operands(r, m, n, k)
    want = g.DeviceBuffer(m * n * 2)
    g.check(blas.gemm_ex(1, 0, m, n, k, 1.0, dA.p, BF16, k, dB.p, BF16, k, 0.0, want.p, BF16, m),
            "GemmEx")
    g.synchronize()
    ref = want.download(np.uint16, m * n)
    dC = g.DeviceBuffer(m * n * 2)
    g.check(blas.gemm_ex_noalloc(1, 0, m, n, k, 1.0, dA.p, BF16, k, dB.p, BF16, k, 0.0, dC.p, BF16, m),
            "GemmExNoAlloc before capture")
    g.synchronize()
    cap = g.Blas()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    torch.cuda.synchronize()
    say("noalloc graph capture")
    with torch.cuda.graph(graph, stream=side):
        cap.set_stream(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        st = cap.gemm_ex_noalloc(1, 0, m, n, k, 1.0, dA.p, BF16, k, dB.p, BF16, k, 0.0, dC.p, BF16, m)
    assert st == g.SUCCESS, g.STATUS[st]
    other = g.DeviceBuffer(m * n * 2)
    for rep in range(5):
        dC.memset(0xFF)
        g.synchronize()
        say(f"noalloc graph replay {rep}")
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(dC.download(np.uint16, m * n), ref), rep
        # eager work on the same scratch between replays
        g.check(blas.gemm_ex_noalloc(1, 0, m, n, k, 1.0, dB.p, BF16, k, dA.p, BF16, k, 0.0, other.p,
                                     BF16, m), "GemmExNoAlloc eager")
        g.check(blas.gemm_ex(1, 0, m, n, k, 1.0, dA.p, BF16, k, dB.p, BF16, k, 0.0, other.p, BF16, m),
                "GemmEx eager")
        g.synchronize()
    del graph
    cap.close()
