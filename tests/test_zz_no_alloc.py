"""neon_moe_layer_noalloc (scratch in the library's fixed per-GPU array, no
allocation) against neon_moe_layer (scratch allocated per call): identical
ids, weights and outputs, on two calls in a row, the second smaller (the
array keeps the first call's contents, which the second must not see)."""
import sys

import numpy as np
import pytest

import neonengine_amd as ne
from tests.gpu_util import empty_dev, to_dev, to_host, torch_cuda

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def inputs(orc, E, H, I, B, seed):
    return dict(
        x=orc.fill_bf16(seed, 51, B * H, 0.0, 1.0),
        rw=orc.fill_bf16(seed, 52, E * H, 0.0, 0.02),
        rb=orc.fill_bf16(seed, 53, E, 0.0, 0.02),
        guc=orc.fill_bytes(seed, 54, E * 2 * I * H // 2),
        gus=orc.fill_scales(seed, 55, E * 2 * I * H // 32, 119, 6),
        gub=orc.fill_bf16(seed, 56, E * 2 * I, 0.0, 0.02),
        dnc=orc.fill_bytes(seed, 57, E * H * I // 2),
        dns=orc.fill_scales(seed, 58, E * H * I // 32, 119, 6),
        dnb=orc.fill_bf16(seed, 59, E * H, 0.0, 0.02),
        res=orc.fill_bf16(seed, 60, B * H, 0.0, 4.0),
    )


def run(fn, dv, B, E, H, I, k, residual):
    out = empty_dev((B, H), np.uint16)
    idx, sc = empty_dev((B, k), np.int32), empty_dev((B, k), np.float32)
    fn(dv["x"], dv["rw"], dv["rb"], dv["guc"], dv["gus"], dv["gub"], dv["dnc"], dv["dns"],
       dv["dnb"], dv["res"] if residual else None, out, idx, sc, B, E, H, I, k)
    return to_host(out), to_host(idx), to_host(sc)


def test_moe_layer_noalloc_matches_allocating_entry_point(orc):
    torch_cuda()
    E, H, I, k = 32, 2880, 2880, 4
    for B, seed, residual in ((64, 11, False), (3, 12, True)):
        say(f"noalloc vs neon_moe_layer: B={B} seed={seed} residual={residual}")
        dv = {n: to_dev(v) for n, v in inputs(orc, E, H, I, B, seed).items()}
        got = run(ne.moe_layer_noalloc, dv, B, E, H, I, k, residual)
        want = run(ne.moe_layer, dv, B, E, H, I, k, residual)
        assert np.array_equal(got[1], want[1])
        assert np.array_equal(got[2].view(np.uint32), want[2].view(np.uint32))
        assert np.array_equal(got[0], want[0])


def test_moe_layer_noalloc_rejects_oversized_scratch(orc):
    torch_cuda()
    E, H, I, k, B = 32, 2880, 2880, 4, 200  # 4.6 MB of activations > 4 MiB
    dv = {n: to_dev(v) for n, v in inputs(orc, E, 64, 64, 1, 1).items()}
    out = empty_dev((1, 64), np.uint16)
    with pytest.raises(ne.NeonError) as e:
        ne.moe_layer_noalloc(dv["x"], dv["rw"], dv["rb"], dv["guc"], dv["gus"], dv["gub"],
                             dv["dnc"], dv["dns"], dv["dnb"], None, out, None, None, B, E, H, I,
                             k)
    assert e.value.status == ne.NEON_EINVAL
    assert "scratch" in str(e.value)
