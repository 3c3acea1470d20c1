"""CPU check of the compiled matrix-core decode kernels (neon_mx.hip).

A select or branch on SCC placed right after a v_cmp that wrote VCC uses a
condition the v_cmp never set.  hipcc (ROCm 7.2) produced exactly that for a
serial loop of one thread over LDS counts (`slot = cnt ? y : -1`), leaving a
used expert without a slot; the routing kernel now computes slots with a
lane-parallel ballot prefix.  This test compiles the source to gfx950
assembly with the library's flags and checks that no s_cselect /
s_cbranch_scc follows a v_cmp directly (waits, nops and moves skipped)."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SKIP = re.compile(r"^\s*(s_waitcnt|s_nop|v_mov|s_mov|;|$)")


def suspicious(asm: str):
    lines = asm.split("\n")
    out = []
    for i, line in enumerate(lines):
        if re.match(r"^\s*(s_cselect|s_cbranch_scc)", line):
            j = i - 1
            while j > 0 and SKIP.match(lines[j]):
                j -= 1
            if re.match(r"^\s*v_cmp", lines[j]):
                out.append((line.strip(), lines[j].strip()))
    return out


def test_pattern_detector():
    bad = "\tv_cmp_eq_u32_e32 vcc, 0, v4\n\ts_waitcnt lgkmcnt(0)\n\ts_cselect_b32 s15, -1, s14\n"
    good = "\ts_cmp_eq_u32 s4, 0\n\tv_cmp_eq_u32_e32 vcc, 0, v4\n\tv_mov_b32 v1, v2\n" \
           "\ts_cbranch_vccz .L1\n\ts_cmp_lg_u32 s2, 1\n\ts_cselect_b32 s3, 1, 0\n"
    assert len(suspicious(bad)) == 1 and suspicious(good) == []


def test_matrix_kernels_select_on_their_own_compares(tmp_path):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    from neonengine_amd import _build
    flags = [f for f in _build.HIPCC_FLAGS if f != "-shared"]
    src = os.path.join(ROOT, "neonengine_amd", "csrc", "neon_mx.hip")
    out = tmp_path / "neon_mx.s"
    subprocess.run([hipcc] + flags + ["--cuda-device-only", "-S", src, "-o", str(out)],
                   check=True, capture_output=True, timeout=600)
    found = suspicious(out.read_text())
    assert found == [], found[:4]
