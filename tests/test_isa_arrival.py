"""CPU check of the in-launch arrival protocols of the split attention kernel
(k_attn_split) and the batched router kernels (k_router_route,
k_router_logits) in neon_kernels.hip, in their compiled gfx950 assembly.

With several key splits, each block stores its partial softmax state with
relaxed agent-scope stores, waits for them (s_waitcnt vmcnt(0)), meets its
block at a barrier, and one thread then arrives on the (row, kv head)
counter with a relaxed agent-scope fetch_add; the block that arrives last
reads every split's partials with agent-scope loads and merges them.  The
protocol is correct when (1) every partial store is written through to the
device's coherence point (agent scope: the sc1 bit on gfx950), (2) no
arrival atomic is issued before the stores of every wave of its block have
completed, and (3) the merging loads bypass this XCD's L2 (sc1 as well).
The HIP memory model does not promise (2) for relaxed atomics, so this test
pins the order the compiler actually emits: between the last partial store
and each returning atomic add there must be an s_waitcnt vmcnt(0) and then
an s_barrier, and the loads after the atomic that read partials carry sc1.
The bit-exact GPU tests of the merge (tests/test_gpu_kernels.py) check the
results; this checks the ordering they rely on."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
STORE = re.compile(r"^\s*global_store_\w+")
ARRIVE = re.compile(r"^\s*global_atomic_add\b.*\bsc0\b")  # returning add
WAIT0 = re.compile(r"^\s*s_waitcnt\s+vmcnt\(0\)")
BARRIER = re.compile(r"^\s*s_barrier\b")
LOAD = re.compile(r"^\s*global_load_dword\w*\b")


def arrival_problems(asm: str, barrier: bool = True):
    """Ordering faults of the arrival protocol in one kernel's assembly
    (barrier False: one-wave blocks, whose arrival needs only the wave's own
    stores completed)."""
    lines = [l for l in asm.split("\n") if l.strip() and not l.strip().startswith(";")]
    out = []
    arrivals = [i for i, l in enumerate(lines) if ARRIVE.match(l)]
    if not arrivals:
        return ["no returning atomic add (arrival) found"]
    for a in arrivals:
        s = a - 1
        while s >= 0 and not STORE.match(lines[s]):
            s -= 1
        if s < 0:
            out.append(f"arrival at {a}: no partial store before it")
            continue
        between = lines[s + 1:a]
        w = next((k for k, l in enumerate(between) if WAIT0.match(l)), None)
        b = next((k for k, l in enumerate(between) if BARRIER.match(l)), None)
        if w is None:
            out.append(f"arrival at {a}: no s_waitcnt vmcnt(0) after the last store")
        elif barrier and (b is None or b < w):
            out.append(f"arrival at {a}: no s_barrier after the wait")
        # the stores of the partials just before: agent scope (sc1)
        k = s
        while k >= 0 and a - k < 60:
            if STORE.match(lines[k]) and "sc1" not in lines[k]:
                out.append(f"store at {k} before arrival {a} lacks sc1: {lines[k].strip()}")
            k -= 1
        loads = [l for l in lines[a + 1:] if LOAD.match(l)]
        if not loads or any("sc1" not in l for l in loads):
            out.append(f"after arrival {a}: partial loads missing or without sc1")
    return out


def kernel_asm(asm: str, name_part: str) -> str:
    m = re.search(r"^(_Z\w*" + name_part + r"\w*):", asm, flags=re.M)
    assert m, f"no kernel matching {name_part}"
    start = m.end()
    return asm[start:asm.index(".Lfunc_end", start)]


def test_detector_catches_misorderings():
    good = ("\tglobal_store_dwordx2 v[1:2], v[3:4], off sc1\n\ts_waitcnt vmcnt(0)\n"
            "\ts_barrier\n\tglobal_atomic_add v1, v1, v2, s[6:7] sc0\n"
            "\tglobal_load_dwordx2 v[5:6], v[7:8], off sc1\n")
    no_wait = good.replace("\ts_waitcnt vmcnt(0)\n", "")
    wait_after_barrier = good.replace("\ts_waitcnt vmcnt(0)\n\ts_barrier\n",
                                      "\ts_barrier\n\ts_waitcnt vmcnt(0)\n")
    plain_store = good.replace("off sc1\n\ts_waitcnt", "off\n\ts_waitcnt")
    cached_load = good.replace("v[7:8], off sc1", "v[7:8], off")
    assert arrival_problems(good) == []
    for bad in (no_wait, wait_after_barrier, plain_store, cached_load):
        assert arrival_problems(bad), bad
    # one-wave form: the barrier is not required, the wait and scopes are
    assert arrival_problems(good.replace("\ts_barrier\n", ""), barrier=False) == []
    for bad in (no_wait, plain_store, cached_load):
        assert arrival_problems(bad.replace("\ts_barrier\n", ""), barrier=False), bad


@pytest.fixture(scope="module")
def kernels_asm(tmp_path_factory):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    from neonengine_amd import _build
    flags = [f for f in _build.HIPCC_FLAGS if f != "-shared"]
    src = os.path.join(ROOT, "neonengine_amd", "csrc", "neon_kernels.hip")
    out = tmp_path_factory.mktemp("isa") / "neon_kernels.s"
    subprocess.run([hipcc] + flags + ["-I", os.path.join(ROOT, "include"), "--cuda-device-only",
                                      "-S", src, "-o", str(out)],
                   check=True, capture_output=True, timeout=900)
    return out.read_text()


def test_attention_merge_arrival_order(kernels_asm):
    problems = arrival_problems(kernel_asm(kernels_asm, "k_attn_split"))
    assert problems == [], problems[:4]


def test_router_route_arrival_order(kernels_asm):
    """k_router_route (router logits + top-k + route lists, one block per
    row): each row's expert ids are stored at agent scope, waited for and
    met at a barrier before the row's arrival; the last block reads every
    row's ids with agent-scope loads."""
    problems = arrival_problems(kernel_asm(kernels_asm, "k_router_route"))
    assert problems == [], problems[:4]


def test_router_logits_row_arrival_order(kernels_asm):
    """k_router_logits with row counters (the top-k in the logits launch):
    each one-wave block stores its logit at agent scope and waits for it
    before its row's arrival; the row's last block reads the row's logits
    with agent-scope loads."""
    problems = arrival_problems(kernel_asm(kernels_asm, "k_router_logits"), barrier=False)
    assert problems == [], problems[:4]
