"""CPU check of the compiled route-list kernel (k_topk_route in
neon_kernels.hip, which ranks every row's experts and lists each used
expert's (row, slot) pairs for the matrix-core expert kernels).

A select or branch on SCC placed after a v_cmp that wrote VCC, with no
scalar instruction of the same block having set SCC first, uses a condition
nobody computed.  hipcc (ROCm 7.2) produced exactly that for an earlier,
serial form of the route lists (`slot = cnt ? y : -1` in a one-thread loop),
which left a used expert without a slot; the slots now come from a
lane-parallel ballot prefix.  This test compiles the source to gfx950
assembly with the library's flags and checks k_topk_route for the pattern
(waits, nops and moves skipped).  tests/test_gpu_mx.py::
test_route_lists_match_host checks the route table itself on the GPU."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SKIP = re.compile(r"^\s*(s_waitcnt|s_nop|v_mov|s_mov|;|$)")
# scalar ALU instructions that write SCC
SCC_WRITER = re.compile(r"^\s*s_(cmp|cmpk|and|or|xor|andn2|orn2|nand|nor|xnor|add|sub|addc|"
                        r"subb|lshl|lshr|ashr|bfe|bitcmp|min|max|abs|not|bcnt|ff1|flbit)")
BLOCK_START = re.compile(r"^[.\w]+:")


def suspicious(asm: str):
    lines = asm.split("\n")
    out = []
    for i, line in enumerate(lines):
        if not re.match(r"^\s*(s_cselect|s_cbranch_scc)", line):
            continue
        j = i - 1
        while j > 0 and SKIP.match(lines[j]):
            j -= 1
        if not re.match(r"^\s*v_cmp", lines[j]):
            continue
        # an SCC writer earlier in the same block: SCC holds a real condition
        k = j - 1
        set_before = False
        while k >= 0 and not BLOCK_START.match(lines[k]):
            if SCC_WRITER.match(lines[k]):
                set_before = True
                break
            k -= 1
        if not set_before:
            out.append((line.strip(), lines[j].strip()))
    return out


def function_asm(asm: str, name_part: str) -> str:
    """The assembly of the (first) kernel whose mangled name contains name_part."""
    m = re.search(r"^(_Z\w*" + name_part + r"\w*):", asm, flags=re.M)
    assert m, f"no kernel matching {name_part}"
    start = m.end()
    end = asm.index(".Lfunc_end", start)
    return asm[start:end]


def test_pattern_detector():
    bad = "\tv_cmp_eq_u32_e32 vcc, 0, v4\n\ts_waitcnt lgkmcnt(0)\n\ts_cselect_b32 s15, -1, s14\n"
    good = "\ts_cmp_eq_u32 s4, 0\n\tv_cmp_eq_u32_e32 vcc, 0, v4\n\tv_mov_b32 v1, v2\n" \
           "\ts_cbranch_vccz .L1\n\ts_cmp_lg_u32 s2, 1\n\ts_cselect_b32 s3, 1, 0\n"
    # SCC set by a compare earlier in the block, then a v_cmp, then the select
    set_earlier = ".LBB0_3:\n\ts_cmp_lg_u32 s91, 0\n\tv_cmp_gt_i32_e32 vcc, s4, v2\n" \
                  "\ts_cselect_b64 s[6:7], -1, 0\n"
    # a compare in an earlier block does not count
    other_block = "\ts_cmp_lg_u32 s91, 0\n.LBB0_4:\n\tv_cmp_gt_i32_e32 vcc, s4, v2\n" \
                  "\ts_cselect_b64 s[6:7], -1, 0\n"
    assert len(suspicious(bad)) == 1 and suspicious(good) == []
    assert suspicious(set_earlier) == [] and len(suspicious(other_block)) == 1


def test_route_list_kernel_selects_on_its_own_compares(tmp_path):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    from neonengine_amd import _build
    flags = [f for f in _build.HIPCC_FLAGS if f != "-shared"]
    src = os.path.join(ROOT, "neonengine_amd", "csrc", "neon_kernels.hip")
    out = tmp_path / "neon_kernels.s"
    subprocess.run([hipcc] + flags + ["-I", os.path.join(ROOT, "include"), "--cuda-device-only",
                                      "-S", src, "-o", str(out)],
                   check=True, capture_output=True, timeout=900)
    found = suspicious(function_asm(out.read_text(), "k_topk_route"))
    assert found == [], found[:4]
