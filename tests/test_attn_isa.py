"""The flash attention kernels, as compiled, never touch a V^T fragment
register before the read that fills it has completed, and use no scratch.

The transposing V^T reads (hk_vt_read in csrc/hk_attn.h) are inline
assembly whose completion the kernel waits for later, with an explicit
`s_waitcnt lgkmcnt(N)`, so that the next key tile's direct-to-LDS loads
keep flowing meanwhile.  The compiler takes an asm statement's outputs as
ready when the statement ends: under register pressure it has spilled such
an output to scratch, or copied it, before the read returned, which gave
wrong, run-to-run varying attention output.  This test compiles
csrc/hk_attn.hip with the Makefile's flags and walks every flash kernel
instance in program order.  LDS operations complete in issue order, so
`s_waitcnt lgkmcnt(N)` completes every LDS read but the last N issued; an
instruction that names a register of a read not yet completed fails the
test.  A straight-line walk is exact here: every wait that completes the
asm reads sits in the same block as the reads.  Scratch accesses fail the
test too (they are how the spill showed).  It needs hipcc, not a GPU.
"""
import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "h3.c_amd", "csrc", "hk_attn.hip")
HIPCC = "/opt/rocm/bin/hipcc"
# the Makefile's hk_attn.o rule
FLAGS = ["-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-mllvm", "-amdgpu-mfma-vgpr-form", "-fno-honor-nans",
         "-fno-signed-zeros", "-fno-trapping-math", "-fassociative-math",
         "-freciprocal-math"]
KERNEL = re.compile(r"^(_Z12hk_flash_fwdI\w+):")
REG = re.compile(r"\bv\[(\d+):(\d+)\]|\bv(\d+)\b")


def _regs(text):
    out = set()
    for m in REG.finditer(text):
        if m.group(3) is not None:
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def _instances():
    work = tempfile.mkdtemp(prefix="hk_attn_isa_")
    try:
        subprocess.run([HIPCC, *FLAGS, "--save-temps", "-c", SRC, "-o",
                        os.path.join(work, "hk_attn.o")], cwd=work,
                       check=True, capture_output=True)
        asm = [f for f in os.listdir(work)
               if f.endswith(".s") and "amdgcn" in f]
        assert asm, "no device assembly written"
        text = open(os.path.join(work, asm[0])).read().splitlines()
    finally:
        shutil.rmtree(work, ignore_errors=True)
    found, name, body = {}, None, []
    for line in text:
        m = KERNEL.match(line)
        if m:
            name, body = m.group(1), []
            continue
        if name and line.startswith(".Lfunc_end"):
            found[name] = body
            name = None
        elif name:
            body.append(line)
    return found


def _offenders(body):
    """(line, reason) for every early use of a pending V^T register."""
    lds = []           # per LDS op in issue order: registers it fills
    done = 0           # LDS ops known complete (a prefix of lds)
    bad = []
    for line in body:
        code = line.split(";")[0].strip()
        if not code or code.endswith(":") or code.startswith("."):
            continue
        op = code.split()[0]
        m = re.match(r"s_waitcnt\b.*lgkmcnt\((\d+)\)", code)
        if m:
            done = max(done, len(lds) - int(m.group(1)))
            continue
        if op.startswith("s_waitcnt"):
            continue
        pending = set()
        for regs in lds[done:]:
            pending |= regs
        if op.startswith("scratch_"):
            bad.append((code, "scratch access"))
        if op.startswith("ds_"):
            operands = code[len(op):]
            dst = _regs(operands.split(",")[0]) if op.startswith(
                "ds_read") else set()
            srcs = _regs(operands) - dst if op.startswith("ds_read") else \
                _regs(operands)
            if (srcs | dst) & pending:
                bad.append((code, "LDS op on a pending V^T register"))
            lds.append(dst if op == "ds_read_b64_tr_b16" else set())
            continue
        if _regs(code) & pending:
            bad.append((code, "uses a V^T register before its read "
                              "completed"))
    return bad


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_flash_kernels_wait_for_their_transposed_reads():
    found = _instances()
    assert len(found) >= 5, sorted(found)
    problems = {}
    for name, body in found.items():
        assert any("ds_read_b64_tr_b16" in l for l in body), name
        bad = _offenders(body)
        if bad:
            problems[name] = (len(bad), bad[:3])
    assert not problems, problems


def test_the_walk_sees_an_early_copy():
    """The checker flags a register copy taken before the wait, and passes
    the same sequence with the wait first."""
    early = ["\tds_read_b64_tr_b16 v[10:11], v3 offset:0",
             "\tds_read_b64_tr_b16 v[12:13], v3 offset:2048",
             "\tv_mov_b32_e32 v40, v11",
             "\ts_waitcnt lgkmcnt(0)"]
    late = [early[0], early[1], early[3], early[2]]
    spill = [early[0], "\tscratch_store_dwordx2 off, v[10:11], off",
             early[3]]
    partial = [early[0], early[1], "\ts_waitcnt lgkmcnt(1)",
               "\tv_mov_b32_e32 v40, v11", "\tv_mov_b32_e32 v41, v12"]
    assert _offenders(early)
    assert not _offenders(late)
    assert _offenders(spill)
    # lgkmcnt(1) completes the first read only
    assert [c for c, _ in _offenders(partial)] == ["v_mov_b32_e32 v41, v12"]
