"""Checks on the gfx950 assembly of the GEMM kernels (CPU: hipcc cross-compiles).

A matrix instruction issued while EXEC is narrowed (inside a lane-dependent
branch) does not read the inactive lanes' operands, so its result is wrong for
every lane. The compiler sinks MFMAs into such a branch when the branch holds
their only consumer; the kernels are written so that this never happens, and
this test keeps it that way for every instantiation in the library.

The tile schedule's outputs (16 to 32 values per lane) must go out as one run
of stores: a vmcnt wait between two stores (e.g. for an output-row lookup)
also waits for every store before it, which cost the config-1 GEMM 1.2 us.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "apus-deepseek-v4-flash_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

NARROW = re.compile(r"^(s_and_saveexec_b64|s_and_b64 exec|s_andn2_b64 exec|s_mov_b64 exec, s\[|"
                    r"s_xor_b64 exec|s_andn2_saveexec_b64|s_mov_b64 exec, vcc)")
RESTORE = re.compile(r"^(s_or_b64 exec, exec|s_mov_b64 exec, -1|s_or_saveexec_b64)")


def _asm(src, tmp_path):
    out = tmp_path / (os.path.basename(src) + ".s")
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "--cuda-device-only", "-S", src, "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True)
    return out.read_text()


def _mfma_under_narrowed_exec(asm):
    """{kernel: count} of MFMAs between an EXEC-narrowing instruction and the
    next restore, in program order (a linear approximation of the CFG that
    covers the structured branches the compiler emits here)."""
    bad = {}
    for m in re.finditer(r"^(_Z\S+):", asm, re.M):
        end = asm.find(".Lfunc_end", m.end())
        narrowed, n = False, 0
        for line in asm[m.end():end].split("\n"):
            line = line.strip()
            if NARROW.match(line):
                narrowed = True
            elif RESTORE.match(line):
                narrowed = False
            elif line.startswith("v_mfma") and narrowed:
                n += 1
        if n:
            bad[m.group(1)] = n
    return bad


def _longest_store_run(asm, prefix):
    """{kernel: longest run of global stores with no vmcnt wait between them}"""
    out = {}
    for m in re.finditer(r"^(" + prefix + r"\S*):", asm, re.M):
        end = asm.find(".Lfunc_end", m.end())
        run = best = 0
        for line in asm[m.end():end].split("\n"):
            line = line.strip()
            if line.startswith("global_store"):
                run += 1
                best = max(best, run)
            elif line.startswith("s_waitcnt") and "vmcnt" in line:
                run = 0
        out[m.group(1)] = best
    return out


@pytest.fixture(scope="module")
def gemm_asm(tmp_path_factory):
    if not os.path.exists(HIPCC) and not shutil.which("hipcc"):
        pytest.skip("no hipcc")
    return _asm(os.path.join(CSRC, "apus_gemm.hip"), tmp_path_factory.mktemp("asm"))


def test_no_mfma_under_narrowed_exec(gemm_asm):
    assert gemm_asm.count("v_mfma") > 1000          # every schedule was instantiated
    assert _mfma_under_narrowed_exec(gemm_asm) == {}


def test_tile_stores_not_serialised(gemm_asm):
    runs = _longest_store_run(gemm_asm, "_Z21apus_gemm_tile_kernel")
    assert len(runs) >= 8                           # FP4 and FP8, K 1024..8192
    assert all(v >= 16 for v in runs.values()), runs
