"""gfx950 wait-state rules checked on the built kernels' assembly (CPU).

The kernels issue some instructions as inline assembly (gemm_tn_fast's
16x16 MFMAs, which accumulate in place in AGPRs, and the direct-to-LDS buffer
loads of attention and gemm_tn128). The compiler's hazard recognizer does not look inside inline
assembly, so those statements carry their own s_nop, and this test checks
the result on the code the build produces: every kernel source is compiled
to gfx950 assembly with the build's own flags, and the instruction stream of
every kernel is scanned, in program order, for the three rules that the
inline assembly could break, wherever the instruction the rule protects is
inline assembly (the compiler keeps the rules for its own instructions). The
wait states between two instructions count
one per instruction and n+1 per s_nop n (the compiler's own conservative
count). The limits are the ones the compiler applies to its own code on
gfx950, read off its output for builtin MFMAs (a dependent VALU read gets
s_nop 11 after a 32x32x16 MFMA; an MFMA reading a freshly VALU-written A or B
operand gets s_nop 1):

1. a VALU write of an SGPR (v_readlane / v_readfirstlane, as the compiler
   restores spilled SGPRs) needs 5 wait states before a memory instruction
   reads that SGPR (a buffer descriptor, an offset);
2. a VALU write of a VGPR needs 2 wait states before an MFMA reads it as its
   A or B operand;
3. an MFMA's result registers need 12 wait states before any instruction
   other than an MFMA accumulating into exactly those registers reads or
   writes them.

A fourth check holds the attention kernel to its own ordering contract: the
compiler does not count the inline-assembly DMA in its vmcnt bookkeeping, so
every s_barrier there must follow an s_waitcnt that drains it (vmcnt(0)) and
the wave's LDS reads (lgkmcnt(0)). An explicit waitcnt immediate with the
wrong vmcnt high bits (bits 15:14) reads as vmcnt(48): a wait that does not
wait.

Scanning in text order follows fall-through paths; a branch target's real
predecessors are not followed, which can only miss a hazard at a block entry,
where the compiler's own waits already sit.
"""
import os
import re
import subprocess
import tempfile

import pytest

from grxcp_amd import build as B

KERNELS = ["kernels/attention.hip", "kernels/gemm_mfma.hip", "kernels/sgemm.hip",
           "kernels/norms.hip", "kernels/softmax_gelu.hip"]

VMEM = ("buffer_", "global_", "flat_", "scratch_")


def _regs(text: str, kind: str) -> set:
    """Register numbers of one kind ('v', 'a' or 's') named in an operand
    string: single registers and ranges."""
    out = set()
    for a, b, c in re.findall(rf"\b{kind}\[(\d+):(\d+)\]|\b{kind}(\d+)\b", text):
        if c:
            out.add(int(c))
        else:
            out.update(range(int(a), int(b) + 1))
    return out


def _split(line: str):
    line = line.split(";")[0].strip()
    if not line or line.startswith(".") or line.endswith(":"):
        return None
    parts = line.split(None, 1)
    ops = [o.strip() for o in parts[1].split(",")] if len(parts) > 1 else []
    return parts[0], ops


def _kernels(asm: str):
    """(name, [(mnemonic, operands, from_inline_asm)]) of every kernel."""
    out = []
    for m in re.finditer(r"^(_Z\w+):", asm, re.M):
        start = m.end()
        end = asm.find("s_endpgm", start)
        body = []
        in_asm = False
        for line in asm[start:end].splitlines():
            if ";;#ASMSTART" in line:
                in_asm = True
                continue
            if ";;#ASMEND" in line:
                in_asm = False
                continue
            s = _split(line)
            if s:
                body.append((s[0], s[1], in_asm))
        out.append((m.group(1), body))
    return out


def _wait(ins) -> int:
    mn, ops, _ = ins
    if mn == "s_nop":
        return int(ops[0], 0) + 1
    return 1


def _check(body):
    """Hazards where the compiler cannot have placed the waits itself: the
    reading memory instruction (rule 1), the reading MFMA (rule 2) or the
    writing MFMA (rule 3) is inline assembly."""
    problems = []
    n = len(body)
    for i, (mn, ops, _) in enumerate(body):
        # rule 1: VALU writes an SGPR that an inline-assembly memory
        # instruction reads
        if mn in ("v_readlane_b32", "v_readfirstlane_b32") and ops and ops[0].startswith("s"):
            written = _regs(ops[0], "s")
            ws = 0
            for j in range(i + 1, n):
                if ws >= 5:
                    break
                mj, oj, aj = body[j]
                if aj and mj.startswith(VMEM) and written & _regs(", ".join(oj), "s"):
                    problems.append(f"SGPR {sorted(written)} from {mn} read by {mj} after {ws} wait states")
                ws += _wait(body[j])
        # rule 2: VALU writes a VGPR that an inline-assembly MFMA reads as A or B
        if mn.startswith("v_") and not mn.startswith(("v_mfma", "v_accvgpr", "v_readlane", "v_readfirstlane")) \
                and ops and re.match(r"v(\d+|\[)", ops[0]):
            written = _regs(ops[0], "v")
            ws = 0
            for j in range(i + 1, n):
                if ws >= 2:
                    break
                mj, oj, aj = body[j]
                if aj and mj.startswith("v_mfma") and len(oj) >= 3 \
                        and written & (_regs(oj[1], "v") | _regs(oj[2], "v")):
                    problems.append(f"VGPR {sorted(written)} from {mn} read by {mj} after {ws} wait states")
                ws += _wait(body[j])
        # rule 3: an inline-assembly MFMA's result touched by anything but an
        # accumulating MFMA
        if mn.startswith("v_mfma") and ops and body[i][2]:
            kind = "a" if ops[0].startswith("a") else "v"
            dst = _regs(ops[0], kind)
            ws = 0
            for j in range(i + 1, n):
                if ws >= 12:
                    break
                mj, oj, _ = body[j]
                touched = _regs(", ".join(oj), kind) & dst
                if touched:
                    if mj.startswith("v_mfma") and len(oj) >= 4 and oj[3] == ops[0] and oj[0] == ops[0]:
                        break          # the accumulator chain continues: fine
                    if mj.startswith("v_mfma") and oj[0] == ops[0] and oj[3] == "0":
                        break          # the next chain starts over the same registers
                    problems.append(f"{ops[0]} from {mn} touched by {mj} {', '.join(oj)} after {ws} wait states")
                    break
                ws += _wait(body[j])
    return problems


def _waits(ops) -> dict:
    """Counters an s_waitcnt waits on: {'vmcnt': n, 'lgkmcnt': n, ...}."""
    return {k: int(v) for k, v in re.findall(r"(\w+cnt)\((\d+)\)", " ".join(ops))}


def _is_dma(ins) -> bool:
    mn, ops, from_asm = ins
    return from_asm and mn.startswith("buffer_load") and bool(ops) and "lds" in ops[-1].split()


def _barrier_waits(body):
    """Barriers not preceded, since the last inline-assembly DMA, by a wait
    for vmcnt(0), or, since the last LDS instruction, by lgkmcnt(0)."""
    problems = []
    for i, (mn, _, _) in enumerate(body):
        if mn != "s_barrier":
            continue
        vm_ok = lgkm_ok = False
        vm_done = lgkm_done = False
        for j in range(i - 1, -1, -1):
            mj, oj, _ = body[j]
            if mj == "s_waitcnt":
                w = _waits(oj)
                if not vm_done and w.get("vmcnt") == 0:
                    vm_ok = vm_done = True
                if not lgkm_done and w.get("lgkmcnt") == 0:
                    lgkm_ok = lgkm_done = True
            elif _is_dma(body[j]):
                vm_done = True
            elif mj.startswith("ds_"):
                lgkm_done = True
            if vm_done and lgkm_done:
                break
        if not (vm_ok and lgkm_ok):
            problems.append(f"s_barrier #{i}: vmcnt(0) {'ok' if vm_ok else 'MISSING'}, "
                            f"lgkmcnt(0) {'ok' if lgkm_ok else 'MISSING'}")
    return problems


@pytest.fixture(scope="module")
def asm_files():
    out = {}
    with tempfile.TemporaryDirectory() as d:
        for src in KERNELS:
            path = os.path.join(B.CSRC, src)
            dst = os.path.join(d, os.path.basename(src) + ".s")
            cmd = [B.HIPCC, *B.HIP_FLAGS, *B.EXTRA.get(src, []), *B.INCLUDES, "--cuda-device-only",
                   "-S", path, "-o", dst]
            r = subprocess.run(cmd, capture_output=True, text=True)
            assert r.returncode == 0, r.stderr[-2000:]
            out[src] = open(dst).read()
    return out


@pytest.mark.parametrize("src", KERNELS)
def test_kernel_wait_states(asm_files, src):
    kernels = _kernels(asm_files[src])
    assert kernels, "no kernel found in " + src
    bad = []
    for name, body in kernels:
        for p in _check(body):
            bad.append(f"{name[:60]}: {p}")
    assert not bad, f"{len(bad)} hazards, first: " + "\n".join(bad[:10])


def test_attention_barriers_drain_dma(asm_files):
    kernels = _kernels(asm_files["kernels/attention.hip"])
    bad = []
    for name, body in kernels:
        assert any(_is_dma(ins) for ins in body), name
        assert any(mn == "s_barrier" for mn, _, _ in body), name
        bad += [f"{name[:60]}: {p}" for p in _barrier_waits(body)]
    assert not bad, "\n".join(bad[:10])


def _body(text: str, asm_lines=()):
    """A synthetic instruction stream; the 0-based lines in asm_lines are
    marked as inline assembly."""
    out = []
    for i, line in enumerate(text.strip().splitlines()):
        mn, ops = _split(line)
        out.append((mn, ops, i in asm_lines))
    return out


def test_checker_finds_planted_hazards():
    """Each rule catches its hazard one wait state short, and accepts it at
    the limit (the shapes of the bugs these rules were written for: a
    spilled descriptor restored right before a DMA, an MFMA operand zeroed
    right before the MFMA, an accumulator read right after its MFMA)."""
    dma = """
v_readlane_b32 s15, v185, 20
s_mov_b32 m0, s3
s_nop {n}
buffer_load_dwordx4 v118, s[12:15], s2 offen lds
"""
    assert _check(_body(dma.format(n=2), {3}))          # 4 wait states
    assert not _check(_body(dma.format(n=3), {3}))      # 5
    mf = """
v_mov_b64_e32 v[94:95], s[12:13]
s_nop {n}
v_mfma_f32_32x32x16_bf16 a[112:127], v[94:97], v[94:97], 0
"""
    assert _check(_body(mf.format(n=0), {2}))           # 1 wait state
    assert not _check(_body(mf.format(n=1), {2}))       # 2
    acc = """
v_mfma_f32_32x32x16_bf16 a[0:15], v[70:73], v[80:83], a[0:15]
s_nop {n}
v_accvgpr_read_b32 v5, a3
"""
    assert _check(_body(acc.format(n=10), {0}))         # 11 wait states
    assert not _check(_body(acc.format(n=11), {0}))     # 12
    chain = """
v_mfma_f32_32x32x16_bf16 a[0:15], v[70:73], v[80:83], a[0:15]
v_mfma_f32_32x32x16_bf16 a[0:15], v[74:77], v[80:83], a[0:15]
"""
    assert not _check(_body(chain, {0, 1}))             # an accumulator chain
    # the compiler's own instructions are its business
    assert not _check(_body(dma.format(n=0)))
    # a barrier after DMA: the wait must drain it; vmcnt(48) is the value an
    # explicit immediate with the vmcnt high bits set gives
    bar = """
buffer_load_dwordx4 v118, s[12:15], 0 offen lds
ds_read_b128 v[0:3], v4
s_waitcnt vmcnt({vm}) lgkmcnt(0)
s_barrier
"""
    assert _barrier_waits(_body(bar.format(vm=48), {0}))
    assert not _barrier_waits(_body(bar.format(vm=0), {0}))
    # the LDS read after the last wait is not drained
    late = """
s_waitcnt vmcnt(0) lgkmcnt(0)
ds_read_b128 v[0:3], v4
s_barrier
"""
    assert _barrier_waits(_body(late))
