"""GPU checks of the matrix-core batched decode steps (NEON_DECODE_MATRIX).

The matrix cores add the fp32 products of each dot product in their own order,
so these steps are not bit-identical to the exact batched steps.  The bars:
  - the projection kernel (neon_gemv_bf16_mfma): within one bf16 rounding of
    the fp64 product plus fp32-accumulation slack (2^-17 of the sum of
    |terms|), per element;
  - whole steps: the first step's logits within north_star's 2e-2 relative
    bound of the exact step's (the prompt runs through the exact kernels in
    both modes), the same first token wherever the exact top-2 margin
    exceeds that bound, and the greedy ids of the following steps reported.
"""
import sys

import numpy as np
import pytest

import neonengine_amd as ne
from tests.gpu_util import bf16_err_ok, empty_dev, fix_routing, to_dev, to_host, torch_cuda

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def orc():
    from oracle import oracle
    return oracle


@pytest.mark.parametrize("N,K,B,with_bias", [(5120, 2880, 16, True), (2880, 4096, 64, True),
                                             (32, 2880, 5, True), (4096, 64, 33, False),
                                             (201088, 2880, 2, False)])
def test_gemv_bf16_mfma(orc, N, K, B, with_bias):
    torch_cuda()
    say(f"gemv_bf16_mfma N={N} K={K} B={B} bias={with_bias}")
    W = orc.fill_bf16(5, 71, N * K, 0.0, 0.02)
    x = orc.fill_bf16(5, 72, B * K, 0.0, 1.0)
    bias = orc.fill_bf16(5, 73, N, 0.0, 0.5) if with_bias else None
    y = empty_dev((B, N), np.uint16)
    ne.gemv_bf16_mfma(to_dev(W), to_dev(bias) if with_bias else None, to_dev(x), y, N, K, B)
    got = to_host(y)
    Wf = orc.bf16_to_f32(W).reshape(N, K).astype(np.float64)
    xf = orc.bf16_to_f32(x).reshape(B, K).astype(np.float64)
    bf = orc.bf16_to_f32(bias).astype(np.float64) if with_bias else np.zeros(N)
    ref = xf @ Wf.T + bf
    abs_sum = np.abs(xf) @ np.abs(Wf).T + np.abs(bf)
    ok, ratio = bf16_err_ok(got, ref, abs_sum)
    say(f"  worst error / bound = {ratio.max():.3f}")
    assert ok.all()


def run(cfg, seed, prompt, n_steps, mode, fixed_routing=False):
    eng = ne.Engine(cfg)
    eng.init_random(seed)
    if fixed_routing:
        fix_routing(eng, cfg)
    eng.set_decode_mode(mode)
    eng.prefill(prompt)
    first = eng.read_logits()
    eng.decode(n_steps)
    toks = eng.read_tokens()[:, len(prompt[0]):]
    eng.close()
    return first, toks


def compare(cfg, seed, B, plen, n_steps, fixed_routing=False, mode=ne.DECODE_MATRIX):
    torch_cuda()
    say(f"decode modes layers={cfg.n_layers} hidden={cfg.hidden} E={cfg.n_experts} B={B} "
        f"prompt={plen} fixed_routing={fixed_routing} mode={mode}")
    rng = np.random.default_rng(seed)
    prompt = rng.integers(0, cfg.vocab, size=(B, plen)).tolist()
    lg_e, tok_e = run(cfg, seed, prompt, n_steps, ne.DECODE_EXACT, fixed_routing)
    lg_m, tok_m = run(cfg, seed, prompt, n_steps, mode, fixed_routing)
    rel = np.abs(lg_m - lg_e).max() / np.abs(lg_e).max()
    top2 = np.sort(lg_e, axis=1)[:, -2:]
    margin = (top2[:, 1] - top2[:, 0]) / np.abs(lg_e).max(axis=1)
    agree = (tok_m == tok_e).all(axis=1)
    say(f"  first-step logits rel max err {rel:.3e}; rows with identical ids over "
        f"{n_steps + 1} tokens: {agree.sum()}/{B}")
    assert rel < 2e-2
    for b in range(B):
        if margin[b] > 2e-2:
            assert tok_m[b, 0] == tok_e[b, 0]
    return rel, agree


SMALL = dict(n_layers=4, hidden=512, n_heads=16, n_kv_heads=2, head_dim=64, n_experts=8,
             top_k=4, intermediate=512, vocab=4096, sliding_window=128, max_seq=256)


@pytest.mark.parametrize("B", [2, 5, 16, 33, 64])
def test_small_model_matrix_steps(B):
    cfg = ne.config_preset("gpt-oss-20b", **dict(SMALL, max_batch=B))
    compare(cfg, 3, B, 20, 24)


def test_small_model_matrix_long_context():
    """600-token prompts in a 1024-row cache: the full layers' attention spans
    10 chunks in 16 key splits (partials + merge), the sliding layers' ring
    wraps."""
    cfg = ne.config_preset("gpt-oss-20b", **dict(SMALL, max_seq=1024, max_batch=4))
    compare(cfg, 6, 4, 600, 8)


def test_small_model_128_experts_matrix():
    """128 experts (the route lists of 64 used-expert slots), 16 rows, one
    layer.  With 128 experts, a row's 4th and 5th router logits are often
    within rounding of each other, so the two modes may route a row
    differently; the step's expert ids are read back, and every row routed
    the same way must agree within 2e-2 (at most 4 of 16 may differ)."""
    cfg = ne.config_preset("gpt-oss-20b", **dict(SMALL, n_layers=1, n_experts=128, max_batch=16))
    say("matrix mode, 128 experts, one layer, 16 rows")
    routed_alike_compare(cfg, 5, 16, 12, 12)


def routed_alike_compare(cfg, seed, B, plen, min_same, mode=ne.DECODE_MATRIX):
    """First-step logits of both modes for rows whose experts agree (the
    step's moe_idx is read back); returns (rows alike, worst rel error)."""
    torch_cuda()
    prompt = np.random.default_rng(seed).integers(0, cfg.vocab, size=(B, plen)).tolist()
    got = {}
    for m in (ne.DECODE_EXACT, mode):
        eng = ne.Engine(cfg)
        eng.init_random(seed)
        eng.set_decode_mode(m)
        eng.prefill(prompt)
        got[m] = (eng.read_logits(), eng.read_activation("moe_idx"))
        eng.close()
    (lg_e, id_e), (lg_m, id_m) = got[ne.DECODE_EXACT], got[mode]
    same = (np.sort(id_e, axis=1) == np.sort(id_m, axis=1)).all(axis=1)
    rel = np.abs(lg_m - lg_e).max(axis=1) / np.abs(lg_e).max(axis=1)
    say(f"  rows routed alike {same.sum()}/{B}; worst rel error among them {rel[same].max():.3e}")
    assert same.sum() >= min_same
    assert (rel[same] < 2e-2).all()


def test_gpt_oss_120b_width_matrix_one_layer():
    """The 120b shape's width (128 experts, 2880 hidden, vocab 201088), one
    layer, 16 rows: the matrix-core step against the exact one, row by row
    wherever the routing agrees."""
    cfg = ne.config_preset("gpt-oss-120b", n_layers=1, max_seq=64, max_batch=16)
    say("matrix mode, 120b width, one layer, 16 rows")
    routed_alike_compare(cfg, 8, 16, 10, 12)


def test_gpt_oss_20b_width_matrix_steps():
    """Full 20b width (2880 hidden, 64 / 8 heads, 32 experts, vocab 201088),
    16 sequences: one layer with free routing, then four layers with the
    routing fixed (router weights 0, distinct biases).  With random weights
    and 32 experts, some rows' 4th and 5th router logits lie within rounding
    of each other; across 16 rows and several layers one of them picks the
    other expert in one mode, and that row's logits then differ by far more
    than rounding (0.61 measured at four layers with free routing, while
    every buffer of a one-layer step agrees to 2e-3)."""
    cfg = ne.config_preset("gpt-oss-20b", n_layers=1, max_seq=64, max_batch=16)
    compare(cfg, 1, 16, 24, 16)
    cfg = ne.config_preset("gpt-oss-20b", n_layers=4, max_seq=64, max_batch=16)
    compare(cfg, 1, 16, 24, 16, fixed_routing=True)


@pytest.mark.parametrize("B,plen", [(5, 250), (16, 20)])
def test_matrix_attention_rope_append_fused_bit_identical(monkeypatch, B, plen):
    """The matrix-core attention rotates q, and in the block that holds the
    new position rotates k and appends k and v, instead of a separate
    launch before it: the logits and ids of every step equal the separate
    launch's bit for bit (B = 5 crosses the 256-row ring of the sliding
    layers)."""
    torch_cuda()
    cfg = ne.config_preset("gpt-oss-20b", **dict(SMALL, max_batch=B, max_seq=512))
    rng = np.random.default_rng(11)
    prompt = rng.integers(0, cfg.vocab, size=(B, plen)).tolist()
    out = []
    for fuse in ("0", "1"):
        monkeypatch.setenv("NEON_MX_FUSE_ROPE", fuse)
        eng = ne.Engine(cfg)
        eng.init_random(4)
        eng.set_decode_mode(ne.DECODE_MATRIX)
        eng.prefill(prompt)
        lg = []
        for _ in range(12):
            eng.decode(1)
            lg.append(eng.read_logits())
        out.append((np.stack(lg), eng.read_tokens()))
        eng.close()
    say(f"fused rope/append B={B} prompt={plen}: ids {out[1][1][0, plen:plen + 6].tolist()}")
    assert np.array_equal(out[0][0].view(np.uint32), out[1][0].view(np.uint32))
    assert np.array_equal(out[0][1], out[1][1])


@pytest.mark.parametrize("mode", ["matrix", "mx8"])
@pytest.mark.parametrize("shape,B", [("small", 5), ("small", 33), ("20b", 16), ("20b", 7),
                                     ("20b", 64)])
def test_combine_norm_fused_bit_identical(monkeypatch, shape, B, mode):
    """The expert combine writes the next layer's (and after the last layer
    the final) RMSNorm into the packed layout in the same launch: the logits
    and ids of every step equal those of the separate combine and norm
    launches (NEON_MX_COMBINE_NORM=0) bit for bit, at hidden 512 (one pass
    per lane) and at the 20b width (six), with padding rows in the tile."""
    torch_cuda()
    if shape == "small":
        cfg = ne.config_preset("gpt-oss-20b", **dict(SMALL, max_batch=B, max_seq=64))
    else:
        cfg = ne.config_preset("gpt-oss-20b", n_layers=2, max_batch=B, max_seq=64)
    rng = np.random.default_rng(B)
    prompt = rng.integers(0, cfg.vocab, size=(B, 4)).tolist()
    out = []
    for fused in ("1", "0"):
        monkeypatch.setenv("NEON_MX_COMBINE_NORM", fused)
        eng = ne.Engine(cfg)
        eng.init_random(8)
        eng.set_decode_mode(ne.DECODE_MATRIX if mode == "matrix" else ne.DECODE_MATRIX_MX8)
        eng.prefill(prompt)
        lg = []
        for _ in range(3):
            eng.decode(1)
            lg.append(eng.read_logits())
        out.append((np.stack(lg), eng.read_tokens(), eng.read_activation("hidden")))
        eng.close()
    say(f"combine + norm {shape} B={B} {mode}: ids {out[0][1][0, 4:].tolist()}")
    assert np.array_equal(out[0][0].view(np.uint32), out[1][0].view(np.uint32))
    assert np.array_equal(out[0][1], out[1][1])
    assert np.array_equal(out[0][2], out[1][2])


# ---- the expert GEMMs on the scaled fp8 x fp4 instruction (DECODE_MATRIX_MX8)
@pytest.mark.parametrize("B", [2, 16, 33, 64])
def test_small_model_matrix_mx8_steps(B):
    """Each expert input carried as two MXFP8 terms (within half a bf16 unit
    of each 32-block's maximum): the same 2e-2 bar against the exact steps."""
    cfg = ne.config_preset("gpt-oss-20b", **dict(SMALL, max_batch=B))
    compare(cfg, 3, B, 20, 24, mode=ne.DECODE_MATRIX_MX8)


def test_small_model_matrix_mx8_long_context():
    cfg = ne.config_preset("gpt-oss-20b", **dict(SMALL, max_seq=1024, max_batch=4))
    compare(cfg, 6, 4, 600, 8, mode=ne.DECODE_MATRIX_MX8)


def test_gpt_oss_20b_width_matrix_mx8_steps():
    """Full 20b width, 16 sequences: one layer with free routing, four with the
    routing fixed (the reasons of test_gpt_oss_20b_width_matrix_steps)."""
    cfg = ne.config_preset("gpt-oss-20b", n_layers=1, max_seq=64, max_batch=16)
    compare(cfg, 1, 16, 24, 16, mode=ne.DECODE_MATRIX_MX8)
    cfg = ne.config_preset("gpt-oss-20b", n_layers=4, max_seq=64, max_batch=16)
    compare(cfg, 1, 16, 24, 16, fixed_routing=True, mode=ne.DECODE_MATRIX_MX8)


def test_gpt_oss_120b_width_matrix_mx8_one_layer():
    cfg = ne.config_preset("gpt-oss-120b", n_layers=1, max_seq=64, max_batch=16)
    say("matrix mode with MXFP8 experts, 120b width, one layer, 16 rows")
    routed_alike_compare(cfg, 8, 16, 10, 12, mode=ne.DECODE_MATRIX_MX8)


def test_decode_mode_validation():
    torch_cuda()
    eng = ne.Engine(ne.config_preset("gpt-oss-20b", **dict(SMALL, max_batch=1)))
    with pytest.raises(ne.NeonError) as e:
        eng.set_decode_mode(ne.DECODE_MATRIX)  # one sequence only
    assert e.value.status == ne.NEON_EINVAL
    with pytest.raises(ne.NeonError) as e:
        eng.set_decode_mode(3)
    assert e.value.status == ne.NEON_EINVAL
    eng.set_decode_mode(ne.DECODE_EXACT)
    eng.close()
    eng = ne.Engine(ne.config_preset("gpt-oss-20b", **dict(SMALL, max_batch=65)))
    with pytest.raises(ne.NeonError) as e:
        eng.set_decode_mode(ne.DECODE_MATRIX)
    assert e.value.status == ne.NEON_EINVAL
    eng.close()


def test_matrix_mode_follows_weight_changes():
    """The packed weight copy is refreshed after neon_load_tensor: a context
    that selected the matrix mode before its weights changed gives the logits
    of an exact context holding the same weights."""
    torch_cuda()
    cfg = ne.config_preset("gpt-oss-20b", **dict(SMALL, max_batch=4))
    say("matrix mode after a weight change")
    rng = np.random.default_rng(7)
    prompt = rng.integers(0, cfg.vocab, size=(4, 9)).tolist()
    from oracle import oracle as orc
    new_lm = orc.fill_bf16(9, 81, cfg.vocab * cfg.hidden, 0.0, 0.05)
    eng = ne.Engine(cfg)
    eng.set_decode_mode(ne.DECODE_MATRIX)  # before any weights
    eng.init_random(3)
    eng.prefill(prompt)
    before = eng.read_logits()
    eng.load_tensor("lm_head.weight", new_lm)
    eng.prefill(prompt)
    after = eng.read_logits()
    eng.close()
    ref = ne.Engine(cfg)
    ref.init_random(3)
    ref.load_tensor("lm_head.weight", new_lm)
    ref.prefill(prompt)
    want = ref.read_logits()
    ref.close()
    changed = np.abs(after - before).max() / np.abs(before).max()
    rel = np.abs(after - want).max() / np.abs(want).max()
    say(f"  change from the new lm_head {changed:.3e}; matrix vs exact {rel:.3e}")
    assert changed > 0.1
    assert rel < 2e-2


def test_matrix_mode_sampling_reproducible():
    """Temperature / nucleus sampling on top of the matrix-core steps: ids in
    range and the same draw for the same seed."""
    torch_cuda()
    cfg = ne.config_preset("gpt-oss-20b", **dict(SMALL, max_batch=8))
    rng = np.random.default_rng(11)
    prompt = rng.integers(0, cfg.vocab, size=(8, 6)).tolist()
    runs = []
    for _ in range(2):
        eng = ne.Engine(cfg)
        eng.init_random(5)
        eng.set_decode_mode(ne.DECODE_MATRIX)
        eng.set_sampling(0.8, 0.9, 1234)
        eng.prefill(prompt)
        eng.decode(12)
        runs.append(eng.read_tokens())
        eng.close()
    say(f"matrix-mode sampling: {runs[0][0, 6:].tolist()}")
    assert np.array_equal(runs[0], runs[1])
    assert (runs[0] >= 0).all() and (runs[0] < cfg.vocab).all()


@pytest.mark.parametrize("table", ["0", "1"])
@pytest.mark.parametrize("E,B", [(32, 16), (128, 16), (8, 5), (8, 64), (32, 64)])
def test_route_lists_match_host(monkeypatch, E, B, table):
    """The route table the matrix-core steps write when one is asked for
    (NEON_ROUTER_ROUTE=0: k_topk_route after the router logits, =1: the last
    block of the router launch) -- used experts in ascending order, their pair
    counts and ascending pair lists, and the work items -- equals one built
    on the host from the same step's expert ids."""
    torch_cuda()
    monkeypatch.setenv("NEON_ROUTER_ROUTE", table)
    cfg = ne.config_preset("gpt-oss-20b", **dict(SMALL, n_experts=E, max_batch=B, max_seq=32))
    eng = ne.Engine(cfg)
    eng.init_random(3)
    eng.set_decode_mode(ne.DECODE_MATRIX)
    eng.prefill([[(37 * b + 11 * t + 1) % cfg.vocab for t in range(3)] for b in range(B)])
    eng.decode(2)
    idx = eng.read_activation("moe_idx").reshape(-1)
    route = eng.read_activation("mx_route")
    items = eng.read_activation("mx_items")
    eng.close()
    k = cfg.top_k
    S = min(E, B * k)
    used = sorted(set(int(e) for e in idx))
    say(f"route lists E={E} B={B}: {len(used)} used experts of {S} slots")
    for y in range(S):
        if y < len(used):
            e = used[y]
            pairs = [q for q in range(B * k) if idx[q] == e]
            assert route[y] == e and route[S + y] == len(pairs), y
            assert list(route[2 * S + 64 * y: 2 * S + 64 * y + len(pairs)]) == pairs, y
        else:
            assert route[y] == -1 and route[S + y] == 0, y
    # work items: (slot, group of 16 pairs), group 0 of every used slot, then
    # group 1 of the slots with more than 16 pairs, ...
    want = []
    for q in range(4):
        for y, e in enumerate(used):
            n = int((idx == e).sum())
            if n > 16 * q:
                want.append(y | (q << 8) | (e << 10) | (min(n, 64) << 19))
    assert items[0] == len(want)
    assert list(items[1:1 + len(want)]) == want
    assert len(want) <= (B * k + 15 * S) // 16  # the launch's block rows


@pytest.mark.parametrize("mode", ["matrix", "mx8"])
@pytest.mark.parametrize("E,B", [(32, 16), (128, 16), (8, 5), (8, 64), (32, 64), (128, 64)])
def test_route_from_ids_bit_identical(monkeypatch, E, B, mode):
    """By default every expert block of a matrix-core step builds its work
    item and pair rows from the step's expert ids (mx_route_item) instead of
    reading a route table: the logits and ids of every step equal those of
    the table path (test_route_lists_match_host pins the table to the host)
    bit for bit, with the table built in either launch form, and so do those
    of the one-launch router without a table (NEON_ROUTER_ROUTE=2) and of a
    top-k launch of its own instead of the router's last wave per row
    (NEON_ROUTER_RANK=0)."""
    torch_cuda()
    cfg = ne.config_preset("gpt-oss-20b", **dict(SMALL, n_experts=E, max_batch=B, max_seq=64))
    rng = np.random.default_rng(E + B)
    prompt = rng.integers(0, cfg.vocab, size=(B, 5)).tolist()
    out = {}
    for table in (None, "0", "1", "2", "rank0"):
        monkeypatch.delenv("NEON_ROUTER_RANK", raising=False)
        if table is None:
            monkeypatch.delenv("NEON_ROUTER_ROUTE", raising=False)
        elif table == "rank0":
            monkeypatch.delenv("NEON_ROUTER_ROUTE", raising=False)
            monkeypatch.setenv("NEON_ROUTER_RANK", "0")
        else:
            monkeypatch.setenv("NEON_ROUTER_ROUTE", table)
        eng = ne.Engine(cfg)
        eng.init_random(6)
        eng.set_decode_mode(ne.DECODE_MATRIX if mode == "matrix" else ne.DECODE_MATRIX_MX8)
        eng.prefill(prompt)
        lg = []
        for _ in range(4):
            eng.decode(1)
            lg.append(eng.read_logits())
        ids = eng.read_activation("moe_idx").reshape(-1)
        out[table] = (np.stack(lg), eng.read_tokens(), ids)
        eng.close()
    used = len(set(int(e) for e in out[None][2]))
    say(f"route from ids E={E} B={B} {mode}: {used} used experts in the last step")
    for table in ("0", "1", "2", "rank0"):
        assert np.array_equal(out[None][0].view(np.uint32), out[table][0].view(np.uint32)), table
        assert np.array_equal(out[None][1], out[table][1]), table
        assert np.array_equal(out[None][2], out[table][2]), table
