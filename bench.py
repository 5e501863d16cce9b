#!/usr/bin/env python3
"""Benchmark of the grxBLAS / grxDNN hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--only NAME]

Prints ONE JSON line. The headline `value` is BASELINE config 2: bf16
grxblasGemmEx at M=N=K=8192 (row-major A x column-major B, i.e. transa=T,
transb=N; fp32 accumulate, bf16 C), in TFLOP/s of algorithmic work
2*M*N*K per launch. A "step" is one GemmEx call over resident HBM inputs.
The other BASELINE configs (bf16 4096^3, int8 GEMM + per-channel dequant,
RMSNorm / LayerNorm, causal attention) are reported under "ops", each with its
own roofline. Every kernel time is the HIP-event time of K back-to-back
launches on the library handle's stream divided by K, after W untimed
launches (default: as many as fill 0.25 s, at least 10; each line reports
its count as "warmup").

All inputs are generated and made resident in HBM first; the workloads then
run back to back with no host work between them (the extras -- fp32 Sgemm,
softmax, GELU -- first, the BASELINE configs after, the headline last), and
the CPU baselines run after all GPU timing. The GPU idles at ~157 MHz and
needs ~0.3 s of load to reach its operating clock (rocm-smi), so host work
between workloads would put the next workload's first launches in that ramp.
For the same reason the GPU is first brought out of idle: before the first
measurement every workload is launched in turn, one launch each, for
--preheat seconds (default 0.5; 0 turns it off). Measured on one box with 5
warm-up launches: the whole run otherwise sits in the ramp (causal attention
938 TFLOP/s after the other workloads, 846 alone, against 995 after 0.25 s of
its own launches). The line reports the pre-heat time as "preheat_s".

The CPU baseline (rank 0, N=1) times the oracle -- the reference's own CPU
GEMM loop restated in C (ref tests/libs/test_grxblas_ex.cpp:45-63) -- on a
bounded slice of the same workload on the host's cores. BASELINE config 1
(fp32 Sgemm 512^3) is the line "sgemm_fp32_512_config1": the GPU library's
grxblasSgemm, with its stated execution mode -- the CPU host backend
(oracle/libgrxblas_ref.so) -- timed beside it as that line's CPU baseline.

The matrix-core lines carry the shader clock their kernel ran at ("clock":
s_memtime spans from the kernels' cycle probe over one launch's event time)
and the fraction of peak at that clock ("roofline.frac_at_clock"). After the product's GPU timing, the same GEMM
problems run through torch (hipBLASLt) in a child process and are reported
beside the product lines ("vendor"); --no-vendor skips that.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import grxcp_amd as g  # noqa: E402
from grxcp_amd import synth  # noqa: E402

PEAK = {"bf16": 2500.0, "int8": 5000.0, "fp32": 157.3, "hbm": 8000.0}  # TFLOP/s, TOP/s, GB/s (MI355X dense)
BF16, I8, I32 = g.GRX_R_16BF, g.GRX_R_8I, g.GRX_R_32I


def log(msg: str) -> None:
    sys.stderr.write(f"[bench] {msg}\n")
    sys.stderr.flush()


WARM_SECONDS = 0.25   # auto warm-up: at least this much back-to-back work
PREHEAT_SECONDS = 0.5  # all workloads in turn before the first measurement
LAST_WARMUP = [0]     # warm-up launches of the latest measurement
LAST_CLOCK = [None]   # shader clock of the latest measurement (probed_clock)
NOMINAL_MHZ = 2400.0  # the clock MI355X's peak figures are quoted at


def probed_clock(set_probe, slots_needed: int, stream: g.Stream, launch, timed_ms: float) -> dict | None:
    """The shader clock one launch ran at, from the kernels' own cycle probe
    (grxCycleSlot: s_memtime at each wave's start and end, and the CU it ran
    on). The s_memtime counters of different CUs, even in one XCD, are not
    synchronized (measured: starts 1e8 ticks apart within one launch), so
    spans are taken per CU only: from the first wave's start to the last
    wave's end on that CU, over the workload's timed milliseconds per launch
    (timed_ms: back to back, so launch overhead is hidden and the figure
    stands for the kernel's duration). A CU is busy for at most the kernel's
    duration, so each figure errs low; the line reports the median over CUs.
    The probed launch's own HIP-event time is reported beside it
    ("launch_ms": it also holds that launch's fixed overhead, which matters
    for kernels of ~0.1 ms). Run right after the timed launches, with the GPU
    at their operating point."""
    n = int(slots_needed)
    if n <= 0:
        return None
    buf = g.DeviceBuffer(n * ctypes.sizeof(g.CycleSlot))
    buf.memset(0)
    try:
        if set_probe(buf.p, n) != 0:
            return None
        launch()                       # a first probed launch: warm the probe's lines
        g.synchronize()
        buf.memset(0)
        e0, e1 = g.Event(), g.Event()
        e0.record(stream.s)
        launch()
        e1.record(stream.s)
        ms = e0.elapsed_ms(e1)
        g.synchronize()
        e0.close()
        e1.close()
    finally:
        set_probe(None, 0)
    raw = buf.download(np.uint8, n * ctypes.sizeof(g.CycleSlot))
    buf.close()
    dt = np.dtype([("start", "<u8"), ("end", "<u8"), ("core", "<u4"), ("warp", "<u4")])
    sl = raw.view(dt)
    sl = sl[(sl["start"] != 0) | (sl["end"] != 0)]
    if sl.size == 0 or ms <= 0:
        return None
    spans = []
    for c in np.unique(sl["core"]):
        m = sl[sl["core"] == c]
        spans.append(int(m["end"].max()) - int(m["start"].min()))
    mhz = [sp / (timed_ms * 1e3) for sp in spans]
    return {"mhz": round(float(np.median(mhz)), 1), "min_mhz": round(min(mhz), 1),
            "max_mhz": round(max(mhz), 1), "cus": len(spans),
            "xcds": int(np.unique(sl["core"] >> 16).size), "launch_ms": round(ms, 4),
            "source": "s_memtime span per CU (cycle probe, one launch after the timed ones) / "
                      "the timed ms per launch; median over CUs (a lower bound per CU)"}


def time_launches(stream: g.Stream, launch, steps: int, warmup: int | None) -> float:
    """Mean milliseconds per launch over `steps` launches, measured with HIP
    events on the launching stream, after `warmup` untimed launches. With
    warmup None the count is chosen so that the warm-up runs for at least
    WARM_SECONDS (and at least 10 launches): the GPU idles while the host
    generates inputs, and a few launches after that sit in the clock ramp
    (measured: 4-13 % slower with 10 warm-up launches of these kernels)."""
    if warmup is None:
        e0, e1 = g.Event(), g.Event()
        e0.record(stream.s)
        for _ in range(3):
            launch()
        e1.record(stream.s)
        probe_ms = max(e0.elapsed_ms(e1) / 3, 1e-3)
        g.synchronize()
        e0.close()
        e1.close()
        warmup = max(10, int(np.ceil(WARM_SECONDS * 1e3 / probe_ms)))
    LAST_WARMUP[0] = warmup
    for _ in range(warmup):
        launch()
    g.synchronize()
    e0, e1 = g.Event(), g.Event()
    e0.record(stream.s)
    for _ in range(steps):
        launch()
    e1.record(stream.s)
    ms = e0.elapsed_ms(e1)
    g.synchronize()
    e0.close()
    e1.close()
    return ms / steps


def preheat(loads: list, seconds: float) -> int:
    """Launch every workload once in turn, synchronising after each round,
    until `seconds` have passed: takes the GPU from its idle clock to its
    operating point under this mix. Returns the number of rounds."""
    rounds = 0
    t_end = time.perf_counter() + seconds
    while loads and time.perf_counter() < t_end:
        for w in loads:
            w.launch()
        g.synchronize()
        rounds += 1
    return rounds


def traffic_from_profiles(name: str):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE, WRITE_SIZE),
    as committed under profiles/ by the profiling runs; None if not measured."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    try:
        return json.load(open(path)).get(name, {}).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


TRAFFIC_SOURCE = ("profiles/traffic.json: rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE, per dispatch "
                  "of this bench command (profiles/hbm_traffic.md), scaled by a plain copy kernel's "
                  "readings; these count L2-to-fabric bytes, which include Infinity Cache hits, so "
                  "they bound HBM traffic from above")


def roofline(bound: str, work: float, ms: float, peak_key: str, traffic_key: str):
    if bound == "hbm":
        achieved = work / (ms * 1e-3) / 1e9      # GB/s
        unit = "GB/s"
    else:
        achieved = work / (ms * 1e-3) / 1e12     # TFLOP/s (TOP/s for int8)
        unit = "TOP/s" if peak_key == "int8" else "TFLOP/s"
    peak = PEAK[peak_key]
    traffic = traffic_from_profiles(traffic_key)
    r = {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
         "frac": round(achieved / peak, 4), "traffic": traffic,
         "traffic_source": TRAFFIC_SOURCE if traffic is not None else None}
    clock = LAST_CLOCK[0]
    if bound == "mfma" and clock:
        # the matrix cores' peak scales with the shader clock: the fraction of
        # the peak at the clock the kernel actually ran at
        r["frac_at_clock"] = round(achieved / (peak * clock["mhz"] / NOMINAL_MHZ), 4)
    return r


# ---- CPU baseline -------------------------------------------------------------

def cpu_threads() -> int:
    n = os.cpu_count() or 1
    cap = int(os.environ.get("OMP_NUM_THREADS", n))
    return max(1, min(n, cap))


def cpu_model() -> str:
    """The host CPU's model name (what lscpu prints as "Model name")."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.lower().startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def with_host(d: dict) -> dict:
    d["cpu_model"] = cpu_model()
    d["host_cpus"] = os.cpu_count()
    return d


def cpu_gemm_baseline(A_bits, B_bits, M, N, K, target_s=10.0):
    """Oracle fp32-accumulate GemmEx loop on whole rows of M, slice by slice,
    until ~target_s of CPU time; returns TFLOP/s and the sample description."""
    import oracle as O
    threads = cpu_threads()
    O.set_threads(threads)
    Bf = O.bf16_to_f32(B_bits)                      # column-major K x N
    done, spent, rows_per = 0, 0.0, 16
    while spent < target_s and done < M:
        r = min(rows_per, M - done)
        a = O.bf16_to_f32(A_bits[done * K:(done + r) * K])
        t0 = time.perf_counter()
        O.gemm_f32acc(1, 0, r, N, K, 1.0, a, K, Bf, K, 0.0, np.zeros(r * N, np.float32), r)
        spent += time.perf_counter() - t0
        done += r
    flops = 2.0 * done * N * K
    return with_host({"value": round(flops / spent / 1e12, 6), "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": f"{done} of {M} rows of M ({flops / 1e9:.1f} GFLOP) through the oracle's "
                      f"fp32-accumulate GemmEx loop, {threads} OpenMP threads, {spent:.1f} s"})


def cpu_igemm_baseline(A, B, M, N, K, target_s=5.0):
    import oracle as O
    threads = cpu_threads()
    O.set_threads(threads)
    done, spent = 0, 0.0
    while spent < target_s and done < M:
        r = min(16, M - done)
        t0 = time.perf_counter()
        O.igemm(1, 0, r, N, K, 1, A[done * K:(done + r) * K], K, B, K, 0, np.zeros(r * N, np.int32), r)
        spent += time.perf_counter() - t0
        done += r
    ops = 2.0 * done * N * K
    return with_host({"value": round(ops / spent / 1e12, 6), "unit": "TOP/s", "cores": threads,
                      "kind": "port",
                      "sample": f"{done} of {M} rows ({ops / 1e9:.1f} GOP), oracle int32 GEMM, "
                                f"{threads} threads, {spent:.1f} s"})


def cpu_norm_baseline(x_bits, gamma_bits, beta_bits, rows, hidden, layer):
    import oracle as O
    threads = cpu_threads()
    O.set_threads(threads)
    r = min(rows, x_bits.size // hidden)   # config 4 runs in full on the CPU
    x = O.bf16_to_f32(x_bits[: r * hidden]).reshape(r, hidden)
    gf, bf = O.bf16_to_f32(gamma_bits), O.bf16_to_f32(beta_bits)
    t0 = time.perf_counter()
    if layer:
        O.layernorm(x, gf, bf, 1e-6)
    else:
        O.rmsnorm(x, gf, 1e-6)
    dt = time.perf_counter() - t0
    moved = r * hidden * 4 + hidden * 2 * (2 if layer else 1)   # bf16 in + bf16 out
    return with_host({"value": round(moved / dt / 1e9, 3), "unit": "GB/s", "cores": threads,
                      "kind": "port",
                      "sample": f"{r} of {rows} rows, oracle fp64 norm, {threads} threads"})


def cpu_attention_baseline(q, k, v, S, D, rows=256):
    import oracle as O
    threads = cpu_threads()
    O.set_threads(threads)
    t0 = time.perf_counter()
    r0 = S - rows
    O.attention_head(q, k, v, True, D ** -0.5, r0, S)
    dt = time.perf_counter() - t0
    flops = sum(4.0 * D * (i + 1) for i in range(r0, S))
    return with_host({"value": round(flops / dt / 1e12, 6), "unit": "TFLOP/s", "cores": threads,
                      "kind": "port",
                      "sample": f"one (b,h), last {rows} query rows ({flops / 1e9:.2f} GFLOP), "
                                f"oracle fp64, {threads} threads"})


# ---- GPU workloads --------------------------------------------------------------
#
# Each prepare_* generates its inputs (seeded, on the host), uploads them and
# returns a Workload: the launch closure, the algorithmic work per launch and
# a CPU-baseline closure over the host copies it keeps. main() prepares every
# selected workload first, then times them back to back (no host work between
# them, so the GPU does not fall back to its idle clock: it idles at ~157 MHz
# and takes ~0.3 s of load to reach its operating clock), then runs the CPU
# baselines.

class Workload:
    def __init__(self, name, unit, bound, peak_key, traffic_key, work, launch, buffers,
                 cpu=None, ms_digits=4, clock=None):
        self.name, self.unit, self.bound = name, unit, bound
        self.peak_key, self.traffic_key, self.work = peak_key, traffic_key, work
        self.launch, self.buffers, self.cpu, self.ms_digits = launch, buffers, cpu, ms_digits
        self.clock = clock   # (set_probe, slots) for probed_clock, or None

    def measure(self, stream, steps, warmup) -> dict:
        log(f"{self.name}: timing")
        ms = time_launches(stream, self.launch, steps, warmup)
        LAST_CLOCK[0] = probed_clock(*self.clock, stream, self.launch, ms) if self.clock else None
        scale = 1e6 if self.unit == "GB/s" else 1e9
        return {"name": self.name, "ms": round(ms, self.ms_digits), "warmup": LAST_WARMUP[0],
                "value": round(self.work / ms / scale, 2 if scale == 1e9 else 1), "unit": self.unit,
                "roofline": roofline(self.bound, self.work, ms, self.peak_key, self.traffic_key),
                "clock": LAST_CLOCK[0]}

    def close(self):
        for d in self.buffers:
            d.close()

    def release_device(self):
        """Free the device buffers once timed (the CPU baseline keeps host copies)."""
        self.close()
        self.buffers = []


def _checked(status, what):
    if status:
        raise g.GrxError(f"{what} status {status}")


def prepare_gemm_bf16(blas, M, cpu_seconds):
    N = K = M
    log(f"bf16 GemmEx {M}^3: generating inputs")
    A = synth.normal_bf16(M * K, 21)
    B = synth.normal_bf16(N * K, 22)
    dA, dB, dC = g.DeviceBuffer.from_array(A), g.DeviceBuffer.from_array(B), g.DeviceBuffer(M * N * 2)
    one, zero = g.fptr(1.0), g.fptr(0.0)

    def launch():
        _checked(blas.L.grxblasGemmEx(blas.h, 1, 0, M, N, K, one, dA.p, BF16, K, dB.p, BF16, K, zero,
                                      dC.p, BF16, M), "GemmEx")
    return Workload(f"gemm_bf16_{M}", "TFLOP/s", "mfma", "bf16", f"gemm_bf16_{M}", 2.0 * M * N * K,
                    launch, [dA, dB, dC], lambda: cpu_gemm_baseline(A, B, M, N, K, cpu_seconds),
                    clock=(blas.set_cycle_probe, blas.cycle_slots_needed(M, N)))


def prepare_sgemm(blas):
    """grxblasSgemm fp32 4096^3 (N, N, column-major), fp32 matrix-core roofline.
    The call copies A K-contiguous (transpose_k) and runs the 256x256-tile
    kernel; the timed region holds both."""
    M = N = K = 4096
    log("Sgemm 4096^3: generating inputs")
    A = synth.uniform_f32(M * K, 41, -1.0, 1.0)
    B = synth.uniform_f32(K * N, 42, -1.0, 1.0)
    dA, dB, dC = g.DeviceBuffer.from_array(A), g.DeviceBuffer.from_array(B), g.DeviceBuffer(M * N * 4)
    one, zero = g.fptr(1.0), g.fptr(0.0)

    def launch():
        _checked(blas.L.grxblasSgemm(blas.h, 0, 0, M, N, K, one, dA.p, M, dB.p, K, zero, dC.p, M), "Sgemm")
    return Workload("sgemm_fp32_4096", "TFLOP/s", "mfma", "fp32", "sgemm_fp32_4096", 2.0 * M * N * K,
                    launch, [dA, dB, dC])


_HOST_SGEMM = r"""
import ctypes, json, os, sys, time
import numpy as np
sys.path.insert(0, sys.argv[1])
import oracle as O
from grxcp_amd import synth
ctypes.CDLL(O.HOST_RT, mode=ctypes.RTLD_GLOBAL)
L = ctypes.CDLL(O.HOST_BLAS)
fp, vp, i = ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_int
L.grxblasCreate.argtypes = [ctypes.POINTER(vp)]
L.grxblasSgemm.argtypes = [vp, i, i, i, i, i, fp, vp, i, vp, i, fp, vp, i]
h = vp()
assert L.grxblasCreate(ctypes.byref(h)) == 0
M = N = K = 512
A = synth.uniform_f32(M * K, 1, -1.0, 1.0)
B = synth.uniform_f32(K * N, 2, -1.0, 1.0)
C = np.zeros(M * N, np.float32)
one, zero = ctypes.c_float(1.0), ctypes.c_float(0.0)
p = lambda a: a.ctypes.data_as(vp)
def call():
    # row-major C = A B as column-major C^T = B^T A^T (BASELINE config 1)
    assert L.grxblasSgemm(h, 0, 0, N, M, K, ctypes.byref(one), p(B), N, p(A), K,
                          ctypes.byref(zero), p(C), N) == 0
call()
n, t0 = 0, time.perf_counter()
while time.perf_counter() - t0 < float(sys.argv[2]):
    call()
    n += 1
dt = time.perf_counter() - t0
want = A.reshape(M, K).astype(np.float64) @ B.reshape(K, N).astype(np.float64)
err = float(np.max(np.abs(C.reshape(M, N) - want)) / np.max(np.abs(want)))
print(json.dumps({"calls": n, "seconds": dt, "rel_err_vs_fp64": err}))
"""


def cpu_host_sgemm_baseline(seconds=5.0):
    """BASELINE config 1 in its stated execution mode: grxblasSgemm 512^3 on
    the CPU host backend (oracle/libgrxblas_ref.so, the reference's CPU GEMM
    loop, ref tests/libs/test_grxblas.cpp:63-80, behind the grxblas.h ABI).
    Run in a child process: the host backend exports the same symbols as the
    GPU libraries this process has loaded."""
    import subprocess
    threads = cpu_threads()
    env = dict(os.environ, OMP_NUM_THREADS=str(threads))
    r = subprocess.run([sys.executable, "-c", _HOST_SGEMM, ROOT, str(seconds)], capture_output=True,
                       text=True, env=env, timeout=600)
    if r.returncode != 0:
        raise RuntimeError("host backend Sgemm failed: " + r.stderr[-1000:])
    v = json.loads(r.stdout.strip().splitlines()[-1])
    flops = 2.0 * 512 ** 3 * v["calls"]
    return with_host({"value": round(flops / v["seconds"] / 1e12, 6), "unit": "TFLOP/s",
                      "cores": threads, "kind": "port",
                      "sample": f"{v['calls']} calls of grxblasSgemm 512^3 (N,N) on the CPU host "
                                f"backend (oracle/libgrxblas_ref.so, OpenMP {threads} threads) in "
                                f"{v['seconds']:.1f} s; max rel err vs fp64 {v['rel_err_vs_fp64']:.2e}"})


def prepare_sgemm512(blas):
    """BASELINE config 1 on the GPU library: fp32 C = A*B, 512^3 row-major,
    alpha=1 beta=0, U[-1,1] from seeds 1 and 2, as column-major
    C^T = B^T A^T: Sgemm(N, N, m=512, n=512, k=512, B, 512, A, 512, C, 512)."""
    M = N = K = 512
    A = synth.uniform_f32(M * K, 1, -1.0, 1.0)
    B = synth.uniform_f32(K * N, 2, -1.0, 1.0)
    dA, dB, dC = g.DeviceBuffer.from_array(A), g.DeviceBuffer.from_array(B), g.DeviceBuffer(M * N * 4)
    one, zero = g.fptr(1.0), g.fptr(0.0)

    def launch():
        _checked(blas.L.grxblasSgemm(blas.h, 0, 0, N, M, K, one, dB.p, N, dA.p, K, zero, dC.p, N), "Sgemm")
    return Workload("sgemm_fp32_512_config1", "TFLOP/s", "mfma", "fp32", "sgemm_fp32_512",
                    2.0 * M * N * K, launch, [dA, dB, dC], cpu_host_sgemm_baseline, ms_digits=5)


def prepare_gemm_int8(blas):
    M, K, N = 4096, 8192, 28672
    log("int8 GEMM + dequant: generating inputs")
    A = synth.uniform_int8(M * K, 31)
    B = synth.uniform_int8(N * K, 32)
    scale = synth.uniform_f32(N, 33, 0.001, 0.01)
    dA, dB = g.DeviceBuffer.from_array(A), g.DeviceBuffer.from_array(B)
    dS, dY = g.DeviceBuffer.from_array(scale), g.DeviceBuffer(M * N * 2)

    def launch():
        _checked(blas.L.grxblasGemmExDequant(blas.h, 1, 0, M, N, K, dA.p, I8, K, dB.p, I8, K, dS.p,
                                             dY.p, BF16, M), "GemmExDequant")
    w = Workload("gemm_int8_dequant_4096x28672x8192", "TOP/s", "mfma", "int8", "gemm_int8_dequant",
                 2.0 * M * N * K, launch, [dA, dB, dS, dY], lambda: cpu_igemm_baseline(A, B, M, N, K),
                 clock=(blas.set_cycle_probe, blas.cycle_slots_needed(M, N)))
    return w


def prepare_norm(dnn, layer):
    rows, hidden = 16384, 8192
    name = "layernorm" if layer else "rmsnorm"
    log(f"{name}: generating inputs")
    xs = [synth.normal_bf16(rows * hidden, 41 + i) for i in range(2)]
    gb = synth.normal_bf16(hidden, 43, 1.0, 0.02)
    bb = synth.normal_bf16(hidden, 44, 0.0, 0.02)
    # two buffer sets, alternated, so reads stream from HBM rather than the
    # 256 MB Infinity Cache
    dx = [g.DeviceBuffer.from_array(x) for x in xs]
    dy = [g.DeviceBuffer(rows * hidden * 2) for _ in range(2)]
    dg, db = g.DeviceBuffer.from_array(gb), g.DeviceBuffer.from_array(bb)
    xd, wd = g.TensorDesc(BF16, [rows, hidden]), g.TensorDesc(BF16, [hidden])
    state = {"i": 0}

    def launch():
        i = state["i"] & 1
        state["i"] += 1
        _checked(dnn.layernorm(xd, dx[i].p, wd, dg.p, db.p, 1e-6, xd, dy[i].p) if layer
                 else dnn.rmsnorm(xd, dx[i].p, wd, dg.p, 1e-6, xd, dy[i].p), name)
    x0 = xs[0]                     # the CPU baseline's rows: all of them
    del xs
    moved = rows * hidden * 2 * 2 + hidden * 2 * (2 if layer else 1)
    return Workload(f"{name}_16384x8192", "GB/s", "hbm", "hbm", name, moved, launch,
                    dx + dy + [dg, db], lambda: cpu_norm_baseline(x0, gb, bb, rows, hidden, layer),
                    ms_digits=5)


def prepare_rowop(dnn, op):
    """grxdnnSoftmaxForward / grxdnnGeluForward(tanh) on [16384, 8192] bf16."""
    rows, hidden = 16384, 8192
    log(f"{op}: generating inputs")
    xs = [synth.normal_bf16(rows * hidden, 45 + i) for i in range(2)]
    dx = [g.DeviceBuffer.from_array(x) for x in xs]
    dy = [g.DeviceBuffer(rows * hidden * 2) for _ in range(2)]
    xd = g.TensorDesc(BF16, [rows, hidden])
    state = {"i": 0}

    def launch():
        i = state["i"] & 1
        state["i"] += 1
        _checked(dnn.softmax(xd, dx[i].p, xd, dy[i].p) if op == "softmax"
                 else dnn.gelu(g.GELU_TANH, xd, dx[i].p, xd, dy[i].p), op)
    return Workload(f"{op}_16384x8192", "GB/s", "hbm", "hbm", op, rows * hidden * 2 * 2, launch,
                    dx + dy, ms_digits=5)


def prepare_attention(dnn):
    B, H, S, D = 4, 32, 4096, 128
    n = B * H * S * D
    log("attention: generating inputs")
    qb, kb, vb = (synth.normal_bf16(n, s) for s in (51, 52, 53))
    dq, dk, dv = (g.DeviceBuffer.from_array(a) for a in (qb, kb, vb))
    do = g.DeviceBuffer(n * 2)
    desc = g.TensorDesc(BF16, [B, H, S, D])
    ad = g.AttnDesc(True, D ** -0.5)

    def launch():
        _checked(dnn.attention(ad, desc, dq.p, desc, dk.p, desc, dv.p, desc, do.p), "attention")
    q0, k0, v0 = (a[: S * D].copy() for a in (qb, kb, vb))   # the CPU baseline's head
    del qb, kb, vb

    def cpu():
        import oracle as O
        q, k, v = (O.bf16_to_f32(a).reshape(S, D) for a in (q0, k0, v0))
        return cpu_attention_baseline(q, k, v, S, D)
    return Workload("attention_causal_b4h32s4096d128", "TFLOP/s", "mfma", "bf16", "attention",
                    4.0 * D * B * H * S * (S + 1) / 2, launch, [dq, dk, dv, do], cpu,
                    clock=(dnn.set_cycle_probe, dnn.attention_cycle_slots_needed(B, H, S)))


SGEMM_SHAPES = [(1024, 1024, 1024), (2048, 2048, 2048), (3072, 3072, 3072), (4096, 4096, 4096),
                (4608, 4608, 4608), (5120, 5120, 5120), (6144, 6144, 6144), (8192, 8192, 4096),
                (1024, 1024, 8192), (2048, 2048, 8192), (4096, 4096, 1024), (6144, 6144, 2048),
                (4000, 4100, 1000)]


def vendor_lines(steps: int) -> int:
    """The same problems through the vendor libraries, for comparison in the
    same bench run (run by main() as a child process after its own GPU timing,
    so that torch's HIP runtime never hosts the product's measurements):
    torch.mm in bf16 at 8192^3 and 4096^3 with both operands K-contiguous
    (the product's TN layout; torch dispatches to hipBLASLt), torch._int_mm
    at config 3's int32 stage (4096 x 28672 x 8192, A row-major, B
    K-contiguous), and config 3's per-channel dequant as the unfused torch
    elementwise ops it would take (int32 * fp32 scale -> bf16), timed
    separately. Each after WARM_SECONDS of warm-up, torch events around
    `steps` calls. One JSON line per problem. (No clock figure: the vendor
    kernels carry no cycle probe.)"""
    import torch
    gen = torch.Generator(device="cuda").manual_seed(7)

    def timed(fn):
        t_end = time.perf_counter() + WARM_SECONDS
        while time.perf_counter() < t_end:
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps, None

    def emit(name, what, ms, work, unit, peak_key, clock):
        rate = work / ms / 1e9
        print(json.dumps({"vendor": name, "what": what, "ms": round(ms, 4), "value": round(rate, 2),
                          "unit": unit, "frac": round(rate / PEAK[peak_key], 4)}), flush=True)

    for M in (8192, 4096):
        a = torch.randn(M, M, device="cuda", generator=gen).to(torch.bfloat16)
        bt = torch.randn(M, M, device="cuda", generator=gen).to(torch.bfloat16)
        c = torch.empty(M, M, device="cuda", dtype=torch.bfloat16)
        ms, clk = timed(lambda: torch.mm(a, bt.t(), out=c))
        emit(f"gemm_bf16_{M}", f"torch.mm bf16 {M}^3, A row-major x B K-contiguous (hipBLASLt), bf16 out",
             ms, 2.0 * M ** 3, "TFLOP/s", "bf16", clk)
        del a, bt, c
    M, K, N = 4096, 8192, 28672
    a = torch.randint(-127, 128, (M, K), device="cuda", dtype=torch.int8, generator=gen)
    bt = torch.randint(-127, 128, (N, K), device="cuda", dtype=torch.int8, generator=gen)
    scale = torch.rand(N, device="cuda", generator=gen) * 0.009 + 0.001
    try:
        acc = torch._int_mm(a, bt.t())
        ms, clk = timed(lambda: torch._int_mm(a, bt.t()))
        emit("gemm_int8_int32", "torch._int_mm 4096x28672x8192, int32 out", ms, 2.0 * M * N * K,
             "TOP/s", "int8", clk)
        y = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
        ms, clk = timed(lambda: y.copy_(acc * scale))
        # the unfused dequant moves the int32 product in, an fp32 temporary out
        # and back in, and the bf16 result out
        moved = M * N * (4 + 4 + 4 + 2)
        print(json.dumps({"vendor": "dequant_int32_to_bf16", "what": "torch (acc * scale) -> bf16, "
                          "unfused elementwise", "ms": round(ms, 4),
                          "GB/s": round(moved / ms / 1e6, 1)}), flush=True)
    except RuntimeError as e:
        print(json.dumps({"vendor": "gemm_int8_int32", "error": str(e)[:300]}), flush=True)
    return 0


def run_vendor(steps: int) -> dict:
    """vendor_lines in a child process; {name: line}. Empty if torch is
    absent or the child fails."""
    import subprocess
    try:
        import importlib.util
        if importlib.util.find_spec("torch") is None:
            return {}
    except Exception:  # noqa: BLE001
        return {}
    log("vendor comparison (torch / hipBLASLt) in a child process")
    try:
        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--vendor-only", "--steps",
                            str(steps)], capture_output=True, text=True, timeout=900)
    except subprocess.TimeoutExpired:
        log("vendor comparison timed out")
        return {}
    if r.returncode != 0:
        log("vendor comparison failed: " + r.stderr[-500:])
        return {}
    out = {}
    for line in r.stdout.splitlines():
        try:
            d = json.loads(line)
        except ValueError:
            continue
        if "vendor" in d:
            out[d["vendor"]] = d
    return out


def sgemm_shapes(steps: int) -> int:
    """grxblasSgemm (N, N, column-major, alpha=1 beta=0, U[-0.5,0.5] inputs)
    against torch's fp32 matmul of the same product, each timed after the
    time-based warm-up, HIP/CUDA events around `steps` launches; the
    library's output is checked against an fp64 product."""
    import torch
    g.load()
    g.check_rt(g.load().rt.grxSetDevice(0), "grxSetDevice")
    stream = g.Stream()
    blas = g.Blas()
    blas.set_stream(stream.s)
    gen = torch.Generator(device="cuda").manual_seed(5)
    for (m, n, k) in SGEMM_SHAPES:
        a = torch.rand(k, m, device="cuda", generator=gen) - 0.5   # column-major m x k
        b = torch.rand(n, k, device="cuda", generator=gen) - 0.5   # column-major k x n
        c = torch.zeros(n, m, device="cuda")
        torch.cuda.synchronize()
        one, zero = g.fptr(1.0), g.fptr(0.0)
        pa, pb, pc = a.data_ptr(), b.data_ptr(), c.data_ptr()

        def launch():
            st = blas.L.grxblasSgemm(blas.h, 0, 0, m, n, k, one, pa, m, pb, k, zero, pc, m)
            if st != 0:
                raise g.GrxError(f"Sgemm status {st}")
        ms = time_launches(stream, launch, steps, None)
        err = (c.double() - b.double() @ a.double()).abs().max().item()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t_end = time.perf_counter() + WARM_SECONDS
        while time.perf_counter() < t_end:
            x = b @ a
        e0.record()
        for _ in range(steps):
            x = b @ a
        e1.record()
        torch.cuda.synchronize()
        tms = e0.elapsed_time(e1) / steps
        del x
        flops = 2.0 * m * n * k
        print(json.dumps({"sgemm": [m, n, k], "layout": "N,N", "ms": round(ms, 4),
                          "tflops": round(flops / ms / 1e9, 1), "torch_ms": round(tms, 4),
                          "torch_tflops": round(flops / tms / 1e9, 1), "max_abs_err_vs_fp64": err}),
              flush=True)
    return 0


def stream_ceiling(steps: int) -> int:
    """Streaming rates of plain device kernels on the norms' footprint
    (268 MB in, 268 MB out; two buffer sets alternated so reads come from
    HBM, not the 256 MB Infinity Cache), each after a 0.25 s warm-up, HIP
    events around `steps` launches: torch's copy_ (read + write), a read-only
    sum and a write-only fill. One JSON line per kernel."""
    import torch
    n = 16384 * 8192
    xs = [torch.randn(n, device="cuda").to(torch.bfloat16) for _ in range(2)]
    ys = [torch.empty_like(x) for x in xs]
    torch.cuda.synchronize()
    kernels = {
        "copy": (lambda i: ys[i].copy_(xs[i]), 2 * 2 * n),
        "read_sum": (lambda i: xs[i].sum(dtype=torch.float32), 2 * n),
        "write_fill": (lambda i: ys[i].fill_(1.0), 2 * n),
    }
    # the HIP runtime's device-to-device copy (its own copy kernel), on the
    # library's stream through grxMemcpyAsync
    rt = g.load().rt
    g.check_rt(rt.grxSetDevice(0), "grxSetDevice")
    cstream = torch.cuda.current_stream().cuda_stream

    def hip_copy(i):
        g.check_rt(rt.grxMemcpyAsync(ys[i].data_ptr(), xs[i].data_ptr(), ctypes.c_size_t(2 * n), 3,
                                     ctypes.c_void_p(cstream)), "grxMemcpyAsync")
    kernels["hip_memcpy_d2d"] = (hip_copy, 2 * 2 * n)
    for name, (fn, nbytes) in kernels.items():
        state = {"i": 0}

        def launch():
            fn(state["i"] & 1)
            state["i"] += 1
        t_end = time.perf_counter() + WARM_SECONDS
        while time.perf_counter() < t_end:
            launch()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            launch()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        print(json.dumps({"stream": name, "bytes": nbytes, "ms": round(ms, 5),
                          "GB/s": round(nbytes / ms / 1e6, 1),
                          "of_8TBps": round(nbytes / ms / 1e6 / PEAK["hbm"], 4)}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed launches before each measurement (default: enough for %.2f s)" % WARM_SECONDS)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--preheat", type=float, default=PREHEAT_SECONDS,
                    help="seconds of all workloads' launches in turn before the first measurement "
                         "(default %.1f; 0: none)" % PREHEAT_SECONDS)
    ap.add_argument("--only", default="", help="comma list: gemm,gemm4096,int8,rmsnorm,layernorm,attention,sgemm,softmax,gelu")
    ap.add_argument("--sgemm-shapes", action="store_true",
                    help="print one JSON line per fp32 Sgemm shape (N,N): this library and torch's fp32 matmul")
    ap.add_argument("--stream-ceiling", action="store_true",
                    help="print the streaming rates of plain device kernels (torch copy, read-only "
                         "sum, fill) on the norms' 16384x8192 bf16 footprint: the ceiling the "
                         "HBM-bound lines are compared against")
    ap.add_argument("--no-vendor", action="store_true",
                    help="skip the vendor comparison (torch / hipBLASLt in a child process)")
    ap.add_argument("--vendor-only", action="store_true",
                    help="only print the vendor comparison lines (what the child process runs)")
    ap.add_argument("--calibration-copy", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy kernel of MIB MiB (torch), "
                         "the reference for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE")
    args = ap.parse_args()
    if args.stream_ceiling:
        return stream_ceiling(args.steps)
    if args.vendor_only:
        return vendor_lines(args.steps)
    if args.calibration_copy:
        import torch
        n = args.calibration_copy * (1 << 20)
        src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration_copy_bytes": n, "launches": 3}))
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for {args.gpus}).",
              file=sys.stderr)
        return 2
    if args.sgemm_shapes:
        return sgemm_shapes(args.steps)
    only = set(filter(None, args.only.split(",")))
    want = lambda n: not only or n in only  # noqa: E731
    cpu = not args.no_cpu_baseline

    g.load()
    g.check_rt(g.load().rt.grxSetDevice(0), "grxSetDevice")
    stream = g.Stream()
    blas, dnn = g.Blas(), g.Dnn()
    blas.set_stream(stream.s)
    dnn.set_stream(stream.s)

    # Reported order of the lines (BASELINE configs first), and the order the
    # GPU runs them: the extras first, the BASELINE configs after, the
    # headline last, back to back.
    makers = {
        "gemm": lambda: prepare_gemm_bf16(blas, 8192, 10.0),
        "gemm4096": lambda: prepare_gemm_bf16(blas, 4096, 5.0),
        "int8": lambda: prepare_gemm_int8(blas),
        "rmsnorm": lambda: prepare_norm(dnn, False),
        "layernorm": lambda: prepare_norm(dnn, True),
        "attention": lambda: prepare_attention(dnn),
        "sgemm": lambda: prepare_sgemm(blas),
        "sgemm512": lambda: prepare_sgemm512(blas),
        "softmax": lambda: prepare_rowop(dnn, "softmax"),
        "gelu": lambda: prepare_rowop(dnn, "gelu"),
    }
    report_order = ["gemm", "gemm4096", "int8", "rmsnorm", "layernorm", "attention", "sgemm512",
                    "sgemm", "softmax", "gelu"]
    run_order = ["sgemm512", "sgemm", "softmax", "gelu", "gemm4096", "int8", "rmsnorm", "layernorm",
                 "attention", "gemm"]
    selected = [k for k in report_order if want(k)]
    loads = {k: makers[k]() for k in selected}          # inputs resident in HBM
    g.synchronize()
    if args.preheat > 0:
        rounds = preheat([loads[k] for k in run_order if k in loads], args.preheat)
        log(f"pre-heat: {rounds} rounds of every workload in {args.preheat} s")
    results = {}
    for k in run_order:
        if k in loads:
            results[k] = loads[k].measure(stream, args.steps, args.warmup)
    for w in loads.values():
        w.release_device()
    if not args.no_vendor and any(k in results for k in ("gemm", "gemm4096", "int8")):
        vendor = run_vendor(args.steps)
        for k, names in (("gemm", ["gemm_bf16_8192"]), ("gemm4096", ["gemm_bf16_4096"]),
                         ("int8", ["gemm_int8_int32", "dequant_int32_to_bf16"])):
            got = [vendor[n] for n in names if n in vendor]
            if k in results and got:
                results[k]["vendor"] = got
    if cpu:
        for k in run_order:
            w = loads.get(k)
            if w is not None and w.cpu is not None:
                log(f"{w.name}: CPU baseline")
                cb = w.cpu()
                # the whole workload at the sampled rate (the sample is a slice)
                scale = 1e9 if cb.get("unit") == "GB/s" else 1e12
                if cb.get("value"):
                    cb["full_problem_s_extrapolated"] = round(w.work / (cb["value"] * scale), 3)
                results[k]["cpu_baseline"] = cb
    for w in loads.values():
        w.close()
    headline = results.get("gemm")
    ops = [results[k] for k in report_order if k in results and k != "gemm"]

    config = {"workload": "grxblasGemmEx bf16 M=N=K=8192, transa=T transb=N (row-major A x "
                          "column-major B), fp32 accumulate, bf16 C, alpha=1 beta=0",
              "m": 8192, "n": 8192, "k": 8192}
    dtype = "bf16"
    if headline is None:   # --only without gemm: the first op stands in
        headline = ops.pop(0)
        config = {"workload": headline["name"]}
        dtype = ("f32" if headline["name"].startswith("sgemm") else
                 "int8" if "int8" in headline["name"] else "bf16")
    line = {
        "metric": "GEMM/attention TFLOP/s (bf16, int8), RMSNorm GB/s; % of MI355X peak",
        "value": headline["value"],
        "unit": headline["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": headline["warmup"],
        "preheat_s": args.preheat,
        "ms_per_step": headline["ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic: seeded N(0,1) bf16 (PCG64), resident in HBM before timing",
        "config": config,
        "roofline": headline["roofline"],
        "clock": headline.get("clock"),
        "vendor": headline.get("vendor"),
        "cpu_baseline": headline.get("cpu_baseline"),
        "ops": ops,
    }
    print(json.dumps(line))
    sys.stdout.flush()
    blas.close()
    dnn.close()
    stream.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
