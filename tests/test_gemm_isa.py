"""The MFMA GEMM's K loop, as compiled, moves no accumulator, touches no
scratch memory, and waits for its loads with vmcnt(2) only.

The 16x16x32 kernel holds 64 accumulator blocks in all 256 AGPRs.  Small
changes around the loop (an extra live value, a divergent branch in the
tile loop) have made the register allocator rotate those blocks through
`v_accvgpr_mov` / `v_accvgpr_write` copies inside the K loop, or spill into
scratch there, which cost the split-K instances 60-150% of their time with
correct results.  Every instance keeps two L2 prefetch loads in flight
across the stage wait; a vmcnt(0) there (which the compiler adds
for a barrier with a fence) quietly cancels the prefetch, and the cold-
weight launches of the forward lose 4-10%.  This test compiles
csrc/hk_gemm.hip as the Makefile does
(and as the phase-trace build does), takes the instructions between the
first and the last MFMA of every kernel instance, and requires none of
those.  It needs hipcc, not a GPU.
"""
import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "h3.c_amd", "csrc", "hk_gemm.hip")
HIPCC = "/opt/rocm/bin/hipcc"
FLAGS = ["-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
INSTANCES = {
    "hk_gemm_mfma<0>": "_Z12hk_gemm_mfmaILi0ELb0EEv12hk_gemm_args",
    "hk_gemm_mfma<1> (SwiGLU)": "_Z12hk_gemm_mfmaILi1ELb0EEv12hk_gemm_args",
    "hk_gemm_mfma<2> (GELU)": "_Z12hk_gemm_mfmaILi2ELb0EEv12hk_gemm_args",
    "hk_gemm_mfma<0, group>": "_Z12hk_gemm_mfmaILi0ELb1EEv12hk_gemm_args",
    "hk_gemm_mfma<3> (split-K)": "_Z12hk_gemm_mfmaILi3ELb0EEv12hk_gemm_args",
    "hk_gemm_mfma<4> (split-K SwiGLU)":
        "_Z12hk_gemm_mfmaILi4ELb0EEv12hk_gemm_args",
}
BAD = re.compile(r"\b(v_accvgpr_mov_b32|v_accvgpr_write_b32|scratch_\w+)\b")


def _k_loop_offenders(extra):
    work = tempfile.mkdtemp(prefix="hk_isa_")
    try:
        subprocess.run([HIPCC, *FLAGS, *extra, "--save-temps", "-c", SRC,
                        "-o", os.path.join(work, "hk_gemm.o")], cwd=work,
                       check=True, capture_output=True)
        asm = [f for f in os.listdir(work)
               if f.endswith(".s") and "amdgcn" in f]
        assert asm, "no device assembly written"
        text = open(os.path.join(work, asm[0])).read().splitlines()
    finally:
        shutil.rmtree(work, ignore_errors=True)
    found = {}
    for name, sym in INSTANCES.items():
        start = text.index(next(l for l in text if l.startswith(sym + ":")))
        end = next(i for i in range(start + 1, len(text))
                   if text[i].startswith(".Lfunc_end"))
        body = text[start:end]
        mfma = [i for i, l in enumerate(body) if "v_mfma_" in l]
        assert len(mfma) == 128, (name, len(mfma))
        loop = body[mfma[0]:mfma[-1]]
        found[name] = [l.strip() for l in loop if BAD.search(l)]
        waits = [int(m.group(1)) for l in loop
                 for m in [re.search(r"s_waitcnt\b.*vmcnt\((\d+)\)", l)]
                 if m]
        # the prefetch loads may follow the last MFMA: count them up to the
        # loop's back-edge branch
        back = next(i for i in range(mfma[-1], len(body))
                    if body[i].strip().startswith("s_cbranch"))
        pf = [l for l in body[mfma[0]:back]
              if re.search(r"buffer_load_dword\b.*\blds\b", l)]
        if waits != [2]:
            found[name].append(f"stage waits vmcnt{waits}, want [2]")
        if len(pf) != 2:
            found[name].append(f"{len(pf)} prefetch loads, want 2")
    return found


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
@pytest.mark.parametrize("extra", [[], ["-DHK_GEMM_TRACE"]],
                         ids=["product", "phase-trace"])
def test_gemm_k_loop_has_no_accumulator_copies_or_scratch(extra):
    offenders = _k_loop_offenders(extra)
    bad = {k: (len(v), v[:3]) for k, v in offenders.items() if v}
    assert not bad, bad
