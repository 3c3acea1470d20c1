"""GPU parity of the kernel-level C-ABI entry points against the CPU oracle
(same seeded inputs).

Every kernel evaluates one canonical fp32 operation order that the oracle's
or_c_* functions restate, so the bar is bit-exact equality throughout:
MXFP4 dequantisation, GEMVs, RMSNorm, RoPE, router logits / top-k / scores,
the MoE block and split-KV sink attention.  The fp64 oracle functions are
checked too, within the stated fp32 bounds, so a mistake shared by kernel and
mirror would still fail.
"""
import sys

import numpy as np
import pytest

import neonengine_amd as ne
from tests import rounding_cases
from tests.gpu_util import bf16_err_ok, empty_dev, to_dev, to_host, torch_cuda

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


# config 0/1 distributions: E2M1 codes uniform, E8M0 exponents uniform in
# [-8, -3] (bytes 119..124), bf16 activations ~N(0, 1), seed 0
def mx_weights(orc, N, K, stream):
    codes = orc.fill_bytes(0, stream, N * K // 2)
    scales = orc.fill_scales(0, stream + 1, N * K // 32, 119, 6)
    return codes, scales


def test_dequant_exhaustive_bitexact(orc):
    torch_cuda()
    blocks = np.tile(np.arange(256, dtype=np.uint8), 256)
    scales = np.repeat(np.arange(256, dtype=np.uint8), 16)
    out = empty_dev((256 * 512,), np.float32)
    say("dequant exhaustive 16x256")
    ne.mxfp4_dequant(to_dev(blocks), to_dev(scales), out)
    got = to_host(out)
    want = orc.mxfp4_dequant(blocks, scales)
    nan_g, nan_w = np.isnan(got), np.isnan(want)
    assert np.array_equal(nan_g, nan_w)
    assert np.array_equal(got[~nan_g].view(np.uint32), want[~nan_w].view(np.uint32))


@pytest.mark.parametrize("N", [2880, 5760, 4096])
@pytest.mark.parametrize("B", [1, 4, 16, 64])
def test_mxfp4_gemv_config1(orc, N, B):
    K = 2880
    codes, scales = mx_weights(orc, N, K, 1000 + N)
    x = orc.fill_bf16(0, 2000 + B, B * K, 0.0, 1.0)
    bias = orc.fill_bf16(0, 3000 + N, N, 0.0, 0.02)
    say(f"mxfp4_gemv N={N} K={K} B={B}")
    y = empty_dev((B, N), np.uint16)
    ne.mxfp4_gemv(to_dev(codes), to_dev(scales), to_dev(bias), to_dev(x), y, N, K, B)
    got = to_host(y)
    want, _ = orc.c_mxfp4_gemv(codes, scales, bias, x, N, K)
    if B < 16:  # the exact kernels: the canonical fp32 order
        assert np.array_equal(got, want), f"{(got != want).sum()} mismatches"
    _, ref = orc.mxfp4_gemv(codes, scales, bias, x, N, K)
    Wabs = np.abs(orc.mxfp4_dequant(codes, scales).reshape(N, K))
    abs_sum = np.abs(orc.bf16_to_f32(x)).reshape(B, K) @ Wabs.T
    ok, ratio = bf16_err_ok(got, ref, abs_sum)
    say(f"  {'bit-exact' if B < 16 else f'matrix cores, {(got == want).mean():.3f} bit-equal'}; "
        f"worst error / fp64 bound = {ratio.max():.3f}")
    assert ok.all()


@pytest.mark.parametrize("N,K,B", [(37, 2880, 17), (130, 4096, 65), (5, 8192, 20), (16, 32, 16),
                                   (21, 5760, 40), (2880, 2880, 64), (40, 2880, 130)])
def test_mxfp4_gemv_matrix_cores_ragged(orc, N, K, B):
    """B >= 16 runs on the matrix cores: ragged N, B past one 64-row block,
    K = 8192, and the smallest K (the register-fed kernel), and K = 2880 /
    4096 / 5760 (the kernel that shares the input rows through LDS: ragged N
    and B, a partial last K chunk, three 64-row blocks); each output within
    one bf16 rounding plus the fp32-accumulation slack of the fp64 result."""
    codes, scales = mx_weights(orc, N, K, 79)
    x = orc.fill_bf16(0, 80, B * K, 0.0, 1.0)
    bias = orc.fill_bf16(0, 81, N, 0.0, 0.02)
    say(f"mxfp4_gemv matrix cores N={N} K={K} B={B}")
    y = empty_dev((B, N), np.uint16)
    ne.mxfp4_gemv(to_dev(codes), to_dev(scales), to_dev(bias), to_dev(x), y, N, K, B)
    got = to_host(y)
    _, ref = orc.mxfp4_gemv(codes, scales, bias, x, N, K)
    Wabs = np.abs(orc.mxfp4_dequant(codes, scales).reshape(N, K))
    abs_sum = np.abs(orc.bf16_to_f32(x)).reshape(B, K) @ Wabs.T
    ok, ratio = bf16_err_ok(got, ref, abs_sum)
    say(f"  worst error / fp64 bound = {ratio.max():.3f}")
    assert ok.all()


@pytest.mark.parametrize("K", [64, 2880])
def test_mxfp4_gemv_matrix_cores_nan_scale(orc, K):
    N, B = 20, 16
    codes, scales = mx_weights(orc, N, K, 82)
    scales = scales.copy()
    scales[3 * (K // 32) + 1] = 0xFF  # row 3, second block
    x = orc.fill_bf16(0, 83, B * K, 0.0, 1.0)
    y = empty_dev((B, N), np.uint16)
    ne.mxfp4_gemv(to_dev(codes), to_dev(scales), None, to_dev(x), y, N, K, B)
    got = orc.bf16_to_f32(to_host(y))
    assert np.isnan(got[:, 3]).all()
    assert np.isfinite(np.delete(got, 3, axis=1)).all()


@pytest.mark.parametrize("N,K,B", [(5, 32, 1), (3, 64, 2), (130, 4096, 3), (17, 8192, 1),
                                   (37, 2880, 5), (9, 8192, 2), (6, 96, 7)])
def test_mxfp4_gemv_ragged(orc, N, K, B):
    codes, scales = mx_weights(orc, N, K, 77)
    x = orc.fill_bf16(0, 78, B * K, 0.0, 1.0)
    say(f"mxfp4_gemv ragged N={N} K={K} B={B}")
    y = empty_dev((B, N), np.uint16)
    ne.mxfp4_gemv(to_dev(codes), to_dev(scales), None, to_dev(x), y, N, K, B)
    want, _ = orc.c_mxfp4_gemv(codes, scales, None, x, N, K)
    assert np.array_equal(to_host(y), want)


def test_mxfp4_gemv_nan_scale_propagates(orc):
    N, K = 4, 64
    codes, scales = mx_weights(orc, N, K, 5)
    scales = scales.copy()
    scales[2 * (K // 32)] = 0xFF  # row 2, first block
    x = orc.fill_bf16(0, 6, K, 0.0, 1.0)
    y = empty_dev((1, N), np.uint16)
    ne.mxfp4_gemv(to_dev(codes), to_dev(scales), None, to_dev(x), y, N, K, 1)
    got = orc.bf16_to_f32(to_host(y))[0]
    assert np.isnan(got[2]) and np.all(np.isfinite(got[[0, 1, 3]]))


@pytest.mark.parametrize("N,K,B", [(5120, 2880, 1), (2880, 4096, 1), (7001, 2880, 2), (32, 2880, 4),
                                   (9, 8, 1)])
def test_gemv_bf16(orc, N, K, B):
    W = orc.fill_bf16(0, 11, N * K, 0.0, 0.02)
    bias = orc.fill_bf16(0, 12, N, 0.0, 0.02)
    x = orc.fill_bf16(0, 13, B * K, 0.0, 1.0)
    say(f"gemv_bf16 N={N} K={K} B={B}")
    y = empty_dev((B, N), np.uint16)
    ne.gemv_bf16(to_dev(W), to_dev(bias), to_dev(x), y, N, K, B)
    got = to_host(y)
    want, _ = orc.c_gemv_bf16(W, bias, x, N, K)
    assert np.array_equal(got, want), f"{(got != want).sum()} mismatches"
    _, ref = orc.gemv_bf16(W, bias, x, N, K)
    abs_sum = np.abs(orc.bf16_to_f32(x)).reshape(B, K) @ np.abs(orc.bf16_to_f32(W)).reshape(N, K).T
    ok, ratio = bf16_err_ok(got, ref, abs_sum)
    say(f"  bit-exact; worst error / fp64 bound = {ratio.max():.3f}")
    assert ok.all()


def test_gemv_bf16_output_rounding(orc):
    """The kernels' fp32 -> bf16 output rounding at its edge cases (ties to
    even both ways, overflow to inf, subnormal ties, NaN): hand-derived bits,
    see tests/rounding_cases.py."""
    Wb, x, bias, want, N, K = rounding_cases.gemv_inputs(orc)
    y = empty_dev((1, N), np.uint16)
    ne.gemv_bf16(to_dev(Wb.reshape(-1)), to_dev(bias), to_dev(x), y, N, K, 1)
    got = to_host(y)[0]
    assert np.array_equal(got[: N - 1], want), [hex(v) for v in got]
    assert np.isnan(orc.bf16_to_f32(got[N - 1:]))[0]


@pytest.mark.parametrize("B,H", [(1, 2880), (3, 2880), (2, 64)])
def test_rmsnorm(orc, B, H):
    x = orc.fill_bf16(0, 21, B * H, 0.0, 30.0)
    w = orc.fill_bf16(0, 22, H, 1.0, 0.05)
    out = empty_dev((B, H), np.uint16)
    ne.rmsnorm(to_dev(x), to_dev(w), out, B, H, 1e-5)
    got = to_host(out)
    assert np.array_equal(got, orc.c_rmsnorm(x, w, 1e-5))
    # and within one bf16 ulp of the fp64 form
    assert np.abs(got.astype(np.int32) - orc.rmsnorm(x, w, 1e-5).astype(np.int32)).max() <= 1


def test_rope_yarn(orc):
    cfg = ne.config_preset("gpt-oss-20b", max_seq=40000)
    ocfg = orc.make_config(max_seq=40000)
    pos = np.array([0, 1, 127, 128, 2047, 4096, 32767, 39999], np.int32)
    nh = 9
    x = orc.fill_bf16(0, 31, len(pos) * nh * 64, 0.0, 1.0)
    xd = to_dev(x)
    torch = torch_cuda()
    table = torch.empty(2 * 40000 * 32, dtype=torch.float32, device="cuda")
    ne.rope_table(cfg, 40000, table)
    ne.rope_yarn(xd, to_dev(pos), len(pos), nh, 64, table, 40000)
    got = to_host(xd).reshape(len(pos), nh * 64).astype(np.int32)
    c, s = orc.rope_table(ocfg, 40000)
    for t, p in enumerate(pos):
        want = orc.rope_apply(x.reshape(len(pos), -1)[t], nh, 64, c[p], s[p]).astype(np.int32)
        assert np.array_equal(got[t], want), p


@pytest.mark.parametrize("B,E,k", [(1, 32, 4), (5, 128, 4), (2, 8, 8)])
def test_router_bitexact(orc, B, E, k):
    H = 2880
    x = orc.fill_bf16(0, 41, B * H, 0.0, 1.0)
    W = orc.fill_bf16(0, 42, E * H, 0.0, 0.02)
    b = orc.fill_bf16(0, 43, E, 0.0, 0.02)
    idx, sc, lg = empty_dev((B, k), np.int32), empty_dev((B, k), np.float32), empty_dev((B, E), np.float32)
    ne.router_topk(to_dev(x), to_dev(W), to_dev(b), idx, sc, lg, B, E, H, k)
    ridx, rsc, rlg = orc.router(x, W, b, E, H, k)
    assert np.array_equal(to_host(lg).view(np.uint32), rlg.view(np.uint32))  # canonical order
    assert np.array_equal(to_host(idx), ridx)
    assert np.array_equal(to_host(sc).view(np.uint32), rsc.view(np.uint32))


def test_router_tie_break_lower_index(orc):
    H, E, k = 64, 8, 4
    x = orc.f32_to_bf16(np.ones(H, np.float32))
    Wf = np.zeros((E, H), np.float32)
    Wf[[1, 2, 3, 5, 6]] = 0.5
    W = orc.f32_to_bf16(Wf)
    b = orc.f32_to_bf16(np.zeros(E, np.float32))
    idx, sc = empty_dev((1, k), np.int32), empty_dev((1, k), np.float32)
    ne.router_topk(to_dev(x), to_dev(W), to_dev(b), idx, sc, None, 1, E, H, k)
    assert list(to_host(idx)[0]) == [1, 2, 3, 5]


@pytest.mark.parametrize("k", [4, 6, 8])
def test_router_total_order_with_nan(orc, k):
    """NaN and -inf logits: the GPU ranks experts exactly like the oracle."""
    H, E = 64, 8
    x = orc.f32_to_bf16(np.ones(H, np.float32))
    W = orc.f32_to_bf16(np.zeros((E, H), np.float32))
    b = orc.f32_to_bf16(np.array([2, np.nan, 5, 5, -np.inf, np.nan, 1, 5], np.float32))
    idx, sc = empty_dev((1, k), np.int32), empty_dev((1, k), np.float32)
    say(f"router total order with NaN, k={k}")
    ne.router_topk(to_dev(x), to_dev(W), to_dev(b), idx, sc, None, 1, E, H, k)
    ridx, rsc, _ = orc.router(x.reshape(1, H), W, b, E, H, k)
    assert np.array_equal(to_host(idx), ridx)
    got = to_host(sc)
    assert np.array_equal(np.isnan(got), np.isnan(rsc))  # NaN payloads may differ
    ok = ~np.isnan(rsc)
    assert np.array_equal(got[ok].view(np.uint32), rsc[ok].view(np.uint32))


def moe_inputs(orc, E, H, I, B, seed=0):
    """config 0: E2M1 uniform, E8M0 exponent uniform in [-8,-3], router std
    0.02, x ~ N(0, 1) bf16, seed 0."""
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
    )


@pytest.mark.parametrize("B", [1, 3])
def test_moe_layer_config0(orc, B):
    E, H, I, k = 32, 2880, 2880, 4
    d = moe_inputs(orc, E, H, I, B)
    say(f"moe_layer config0 B={B}")
    out = empty_dev((B, H), np.uint16)
    idx, sc = empty_dev((B, k), np.int32), empty_dev((B, k), np.float32)
    dv = {n: to_dev(v) for n, v in d.items()}
    ne.moe_layer(dv["x"], dv["rw"], dv["rb"], dv["guc"], dv["gus"], dv["gub"], dv["dnc"],
                 dv["dns"], dv["dnb"], None, out, idx, sc, B, E, H, I, k)
    ref, ridx, rsc = orc.moe_layer(d["x"], d["rw"], d["rb"], d["guc"], d["gus"], d["gub"],
                                   d["dnc"], d["dns"], d["dnb"], E, H, I, k)
    assert np.array_equal(to_host(idx), ridx)  # bit-exact top-k indices
    assert np.array_equal(to_host(sc).view(np.uint32), rsc.view(np.uint32))
    got = to_host(out)
    say(f"  moe mismatches vs canonical oracle: {(got != ref).sum()}/{got.size}")
    assert np.array_equal(got, ref)


def test_moe_layer_one_launch(orc, monkeypatch):
    """neon_moe_layer at batch 1 with the opt-in one-launch expert kernel
    (NEON_MOE_FUSED=1): ids, weights and outputs bit-identical to the oracle,
    with and without the residual."""
    monkeypatch.setenv("NEON_MOE_FUSED", "1")
    E, H, I, k, B = 32, 2880, 2880, 4, 1
    d = moe_inputs(orc, E, H, I, B, seed=8)
    res = orc.fill_bf16(8, 60, B * H, 0.0, 10.0)
    dv = {n: to_dev(v) for n, v in d.items()}
    ref, ridx, rsc = orc.moe_layer(d["x"], d["rw"], d["rb"], d["guc"], d["gus"], d["gub"],
                                   d["dnc"], d["dns"], d["dnb"], E, H, I, k)
    for residual in (None, res):
        out = empty_dev((B, H), np.uint16)
        idx, sc = empty_dev((B, k), np.int32), empty_dev((B, k), np.float32)
        ne.moe_layer(dv["x"], dv["rw"], dv["rb"], dv["guc"], dv["gus"], dv["gub"], dv["dnc"],
                     dv["dns"], dv["dnb"], None if residual is None else to_dev(residual), out,
                     idx, sc, B, E, H, I, k)
        ne.device_check()
        assert np.array_equal(to_host(idx), ridx)
        assert np.array_equal(to_host(sc).view(np.uint32), rsc.view(np.uint32))
        want = ref if residual is None else orc.f32_to_bf16(
            orc.bf16_to_f32(residual) + orc.bf16_to_f32(ref).reshape(-1)).reshape(B, H)
        assert np.array_equal(to_host(out), want)


def test_moe_layer_residual(orc):
    E, H, I, k, B = 8, 256, 512, 2, 2
    d = moe_inputs(orc, E, H, I, B, seed=3)
    res = orc.fill_bf16(3, 60, B * H, 0.0, 10.0)
    dv = {n: to_dev(v) for n, v in d.items()}
    out = empty_dev((B, H), np.uint16)
    out2 = empty_dev((B, H), np.uint16)
    ne.moe_layer(dv["x"], dv["rw"], dv["rb"], dv["guc"], dv["gus"], dv["gub"], dv["dnc"],
                 dv["dns"], dv["dnb"], to_dev(res), out, None, None, B, E, H, I, k)
    ne.moe_layer(dv["x"], dv["rw"], dv["rb"], dv["guc"], dv["gus"], dv["gub"], dv["dnc"],
                 dv["dns"], dv["dnb"], None, out2, None, None, B, E, H, I, k)
    m = to_host(out2)
    want = orc.f32_to_bf16(orc.bf16_to_f32(res) + orc.bf16_to_f32(m).reshape(-1))
    assert np.array_equal(to_host(out).reshape(-1), want)


@pytest.mark.parametrize("B", [1, 4, 16, 20])
def test_moe_experts_config0(orc, B):
    """Caller-given ids / weights (the router's) through neon_moe_experts:
    B = 1 runs the per-row kernels, 4 and 16 the grouped kernels (each used
    expert read once for its rows), 20 (80 pairs) the per-row kernels again;
    all bit-identical to the canonical per-row oracle."""
    E, H, I, k = 32, 2880, 2880, 4
    d = moe_inputs(orc, E, H, I, B, seed=4)
    _, ridx, rsc = orc.moe_layer(d["x"], d["rw"], d["rb"], d["guc"], d["gus"], d["gub"],
                                 d["dnc"], d["dns"], d["dnb"], E, H, I, k)
    say(f"moe_experts config0 B={B}")
    dv = {n: to_dev(v) for n, v in d.items()}
    out = empty_dev((B, H), np.uint16)
    act = empty_dev((B * k * I,), np.uint16)
    ne.moe_experts(dv["x"], to_dev(ridx), to_dev(rsc), dv["guc"], dv["gus"], dv["gub"],
                   dv["dnc"], dv["dns"], dv["dnb"], None, out, act, B, E, H, I, k)
    ne.device_check()
    want = orc.moe_experts(d["x"], ridx, rsc, d["guc"], d["gus"], d["gub"], d["dnc"], d["dns"],
                           d["dnb"], E, H, I, k)
    got = to_host(out)
    say(f"  mismatches vs canonical oracle: {(got != want).sum()}/{got.size}")
    assert np.array_equal(got, want)


@pytest.mark.parametrize("B", [1, 3])
def test_moe_experts_drops_out_of_range_ids(orc, B):
    """An expert id outside [0, E) in device memory: the slot is dropped (adds
    0, no read past the expert arrays) and neon_device_check reports
    NEON_EINVAL once; the other slots are unchanged."""
    E, H, I, k = 8, 256, 512, 2
    d = moe_inputs(orc, E, H, I, B, seed=5)
    _, ridx, rsc = orc.moe_layer(d["x"], d["rw"], d["rb"], d["guc"], d["gus"], d["gub"],
                                 d["dnc"], d["dns"], d["dnb"], E, H, I, k)
    ridx = ridx.copy()
    ridx[0, 1] = E          # one past the last expert
    if B > 1:
        ridx[B - 1, 0] = -1  # negative
    dv = {n: to_dev(v) for n, v in d.items()}
    out = empty_dev((B, H), np.uint16)
    act = empty_dev((B * k * I,), np.uint16)
    ne.device_check()  # clean start
    ne.moe_experts(dv["x"], to_dev(ridx), to_dev(rsc), dv["guc"], dv["gus"], dv["gub"],
                   dv["dnc"], dv["dns"], dv["dnb"], None, out, act, B, E, H, I, k)
    with pytest.raises(ne.NeonError) as e:
        ne.device_check()
    assert e.value.status == ne.NEON_EINVAL
    ne.device_check()  # the status word was cleared
    want = orc.moe_experts(d["x"], ridx, rsc, d["guc"], d["gus"], d["gub"], d["dnc"], d["dns"],
                           d["dnb"], E, H, I, k)
    assert np.array_equal(to_host(out), want)


@pytest.mark.parametrize("B", [1, 16, 64])
def test_moe_layer_config4(orc, B):
    """BASELINE config 4's MoE: 128 experts, H = I = 2880, top-4, at batch 1,
    16 and 64 (router + experts through neon_moe_layer): ids, weights and
    outputs bit-identical to the canonical oracle."""
    E, H, I, k = 128, 2880, 2880, 4
    d = moe_inputs(orc, E, H, I, B, seed=6)
    say(f"moe_layer config4 E={E} B={B}")
    out = empty_dev((B, H), np.uint16)
    idx, sc = empty_dev((B, k), np.int32), empty_dev((B, k), np.float32)
    dv = {n: to_dev(v) for n, v in d.items()}
    ne.moe_layer(dv["x"], dv["rw"], dv["rb"], dv["guc"], dv["gus"], dv["gub"], dv["dnc"],
                 dv["dns"], dv["dnb"], None, out, idx, sc, B, E, H, I, k)
    ref, ridx, rsc = orc.moe_layer(d["x"], d["rw"], d["rb"], d["guc"], d["gus"], d["gub"],
                                   d["dnc"], d["dns"], d["dnb"], E, H, I, k)
    say(f"  distinct experts used: {len(np.unique(ridx))}")
    assert np.array_equal(to_host(idx), ridx)
    assert np.array_equal(to_host(sc).view(np.uint32), rsc.view(np.uint32))
    got = to_host(out)
    say(f"  mismatches vs canonical oracle: {(got != ref).sum()}/{got.size}")
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("T,B,window,Tm", [
    (1, 1, 0, 1), (5, 2, 128, 5), (1024, 1, 0, 1024), (1024, 8, 128, 1024), (8192, 1, 0, 8192),
    (8192, 8, 128, 8192), (8192, 8, 0, 8192), (32768, 1, 0, 32768), (32768, 4, 128, 32768),
    (300, 3, 0, 300), (1, 2, 128, 256), (3, 1, 0, 2048), (200, 2, 128, 4096),
    # config 2 at batch 32
    (1024, 32, 0, 1024), (1024, 32, 128, 1024), (8192, 32, 0, 8192), (8192, 32, 128, 8192),
    (32768, 32, 0, 32768), (32768, 32, 128, 32768),
    # config 2 at batch 8: T = 32768 both windows, T = 1024 full
    (32768, 8, 0, 32768), (32768, 8, 128, 32768), (1024, 8, 0, 1024)])
def test_attn_decode_config2(orc, T, B, window, Tm):
    """64 q / 8 kv heads, d=64, Q/K/V and sinks ~N(0,1) bf16 (T keys live in a
    cache of Tm rows; small T in a large cache leaves empty splits)."""
    Hq, Hkv, D = 64, 8, 64
    q = orc.fill_bf16(0, 71, B * Hq * D, 0.0, 1.0)
    kc = orc.fill_bf16(0, 72, B * Hkv * Tm * D, 0.0, 1.0)
    vc = orc.fill_bf16(0, 73, B * Hkv * Tm * D, 0.0, 1.0)
    sinks = orc.fill_bf16(0, 74, Hq, 0.0, 1.0)
    pos = np.array([T - 1 - (b % 3) for b in range(B)], np.int32).clip(0)
    say(f"attn T={T} B={B} window={window}")
    out = empty_dev((B, Hq * D), np.uint16)
    ne.attn_decode(to_dev(q), to_dev(kc), to_dev(vc), to_dev(sinks), to_dev(pos), out, B, Hq,
                   Hkv, D, Tm, window)
    got = to_host(out)
    want, _ = orc.c_attn_decode(q, kc, vc, sinks, B, Hq, Hkv, D, Tm, pos, window)
    say(f"  splits {orc.attn_splits(Tm, window)}; mismatches vs canonical oracle "
        f"{(got != want).sum()}/{got.size}")
    assert np.array_equal(got, want)
    _, ref = orc.attn_decode(q, kc, vc, sinks, B, Hq, Hkv, D, Tm, pos, window)
    g = orc.bf16_to_f32(got).astype(np.float64)
    r = ref.astype(np.float64)
    bound = np.abs(r) * 2.0 ** -8 + 2e-5 * np.abs(r).max()  # one bf16 rounding + fp32 slack
    assert np.all(np.abs(g - r) <= bound)
