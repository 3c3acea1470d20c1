"""GPU parity of the whole token loop (context-level C-ABI) against the CPU
oracle: bit-identical random-init weights, identical greedy token ids for 64
steps, and logits that are bit-identical (the bar north_star sets is 2e-2
relative max error on bf16 logits; the canonical fp32 order gives equality).
The prompt runs stepwise here (every token through the decode kernels); the
batched matrix-core prompt pass is checked in test_gpu_prefill.py.
"""
import sys

import numpy as np
import pytest

import neonengine_amd as ne
from tests.gpu_util import d2h, torch_cuda

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


SMALL = dict(n_layers=4, hidden=512, n_heads=16, n_kv_heads=2, head_dim=64, n_experts=8,
             top_k=4, intermediate=512, vocab=4096, sliding_window=128, max_seq=512,
             max_batch=2)


def pair(orc, **kw):
    cfg = ne.config_preset("gpt-oss-20b", **kw)
    ocfg = orc.make_config(**cfg.as_dict())
    return cfg, ocfg


def logits_close(g, r):
    gb = orc_bf(g)
    rb = orc_bf(r)
    return np.abs(gb - rb).max() / np.abs(rb).max()


def orc_bf(a):
    from oracle import oracle as orc
    return orc.bf16_to_f32(orc.f32_to_bf16(a)).astype(np.float64)


def run_parity(orc, cfg, ocfg, seed, prompt, n_steps, batch=1, mode=ne.PREFILL_STEPWISE):
    torch_cuda()
    eng = ne.Engine(cfg)
    eng.init_random(seed)
    say(f"model parity layers={cfg.n_layers} hidden={cfg.hidden} E={cfg.n_experts} "
        f"vocab={cfg.vocab} batch={batch} prompt={len(prompt[0])} steps={n_steps}")
    m = orc.Model(ocfg, seed=seed, batch=batch)
    # oracle: teacher-forced prompt, then its own greedy ids
    ids_o = np.array([p[0] for p in prompt], np.int32)
    for t in range(len(prompt[0])):
        ids_o = np.array([p[t] for p in prompt], np.int32)
        nxt, lg_o = m.step(ids_o)
    o_tokens = [nxt.copy()]
    o_logits = [lg_o]
    for _ in range(n_steps):
        nxt, lg_o = m.step(nxt)
        o_tokens.append(nxt.copy())
        o_logits.append(lg_o)
    m.close()
    # margins[b, t]: top-2 gap of the logits that produced generated token t
    margins = np.stack([np.diff(np.sort(lg, axis=1)[:, -2:], axis=1)[:, 0] for lg in o_logits], 1)
    eng.set_prefill_mode(mode)  # both modes run the exact decode kernels
    eng.prefill(prompt)
    g_first_logits = eng.read_logits()
    eng.decode(n_steps)
    toks = eng.read_tokens()
    g_last_logits = eng.read_logits()
    eng.close()
    n = len(prompt[0])
    gen_g = toks[:, n:]
    gen_o = np.stack(o_tokens, 1)[:, : n_steps + 1]
    same = gen_g == gen_o
    if not same.all():
        b, t = np.argwhere(~same)[0]
        say(f"first divergence row {b} step {t}: gpu {gen_g[b, t]} oracle {gen_o[b, t]}, "
            f"oracle top-2 margin there {margins[b, t]:.4g}")
    say(f"  min oracle top-2 margin over the run: {margins.min():.4g}")
    e1 = logits_close(g_first_logits, o_logits[0])
    e2 = logits_close(g_last_logits, o_logits[n_steps]) if same.all() else 0.0
    x1 = np.array_equal(g_first_logits.view(np.uint32), o_logits[0].view(np.uint32))
    x2 = same.all() and np.array_equal(g_last_logits.view(np.uint32), o_logits[n_steps].view(np.uint32))
    say(f"  logits rel max err: first {e1:.3e} last {e2:.3e}; bit-identical first {x1} last {x2}")
    assert x1 and x2, "fp32 logits differ from the canonical oracle"
    return same, e1, e2


def test_init_random_matches_oracle_bits(orc):
    torch_cuda()
    cfg, ocfg = pair(orc, **SMALL)
    eng = ne.Engine(cfg)
    eng.init_random(11)
    m = orc.Model(ocfg, seed=11, batch=1)
    H, E, I = cfg.hidden, cfg.n_experts, cfg.intermediate
    qkv = (cfg.n_heads + 2 * cfg.n_kv_heads) * 64
    checks = [
        ("model.embed_tokens.weight", -1, orc.T_EMBED, cfg.vocab * H, np.uint16),
        ("lm_head.weight", -1, orc.T_LM_HEAD, cfg.vocab * H, np.uint16),
        ("model.norm.weight", -1, orc.T_FINAL_NORM, H, np.uint16),
        ("model.layers.0.input_layernorm.weight", 0, orc.T_ATTN_NORM, H, np.uint16),
        ("model.layers.3.self_attn.sinks", 3, orc.T_SINKS, cfg.n_heads, np.uint16),
        ("model.layers.1.mlp.router.weight", 1, orc.T_ROUTER_W, E * H, np.uint16),
        ("model.layers.2.mlp.experts.gate_up_proj_blocks", 2, orc.T_GU_CODES, E * 2 * I * H // 2, np.uint8),
        ("model.layers.2.mlp.experts.gate_up_proj_scales", 2, orc.T_GU_SCALES, E * 2 * I * H // 32, np.uint8),
        ("model.layers.3.mlp.experts.down_proj_blocks", 3, orc.T_DN_CODES, E * H * I // 2, np.uint8),
        ("model.layers.3.mlp.experts.down_proj_bias", 3, orc.T_DN_BIAS, E * H, np.uint16),
    ]
    for name, layer, kind, count, dt in checks:
        ptr, nbytes = eng.tensor_ptr(name)
        got = d2h(ptr, nbytes, dt)
        want = m.tensor(layer, kind, count, dt)
        assert np.array_equal(got, want), name
    # fused q/k/v: the checkpoint's q_proj rows come first, then k, then v
    ptr, nbytes = eng.tensor_ptr("model.layers.1.self_attn.v_proj.weight")
    got = d2h(ptr, nbytes, np.uint16)
    want = m.tensor(1, orc.T_WQKV, qkv * H)[(cfg.n_heads + cfg.n_kv_heads) * 64 * H:]
    assert np.array_equal(got, want)
    m.close()
    eng.close()


def test_small_model_greedy_64(orc):
    cfg, ocfg = pair(orc, **SMALL)
    same, e1, e2 = run_parity(orc, cfg, ocfg, 5, [[1, 2, 3, 4000, 17, 9, 9, 300]], 64)
    assert same.all()
    assert e1 < 2e-2 and e2 < 2e-2


def test_small_model_batch2_and_sliding_wrap(orc):
    """Two rows; 160 positions so the 128-key sliding window moves."""
    cfg, ocfg = pair(orc, **SMALL)
    prompt = [[(7 * i + 3) % 4096 for i in range(100)], [(11 * i + 5) % 4096 for i in range(100)]]
    same, e1, e2 = run_parity(orc, cfg, ocfg, 9, prompt, 60, batch=2)
    assert same.all()
    assert e1 < 2e-2 and e2 < 2e-2


@pytest.mark.parametrize("batch", [5, 16])
def test_small_model_batched_decode(orc, batch):
    """Batch 5 (a padded 8-row input block) and 16 (a full one): the batched
    projections read each weight row once for all rows and must give every
    row the batch-1 bits."""
    cfg, ocfg = pair(orc, **dict(SMALL, max_batch=batch, max_seq=160))
    prompt = [[(13 * i + 7 * b + 1) % 4096 for i in range(9 + b)][:9] for b in range(batch)]
    same, e1, e2 = run_parity(orc, cfg, ocfg, 21, prompt, 24, batch=batch)
    assert same.all()
    assert e1 < 2e-2 and e2 < 2e-2


@pytest.mark.parametrize("batch", [1, 8])
def test_small_model_128_experts(orc, batch):
    """E = 128 (the 120b router width): the two-quarter top-k ranking and, at
    batch 8, the expert grouping over 128 candidate experts."""
    cfg, ocfg = pair(orc, **dict(SMALL, n_experts=128, intermediate=256, max_batch=batch,
                                 max_seq=64))
    prompt = [[(17 * i + 3 * b + 2) % 4096 for i in range(6)] for b in range(batch)]
    same, e1, e2 = run_parity(orc, cfg, ocfg, 29, prompt, 16, batch=batch)
    assert same.all()
    assert e1 < 2e-2 and e2 < 2e-2


def test_small_model_batch32(orc):
    """Batch 32: two 16-row input blocks per projection, and the per-row expert
    kernels (32 rows x 4 slots is past the grouped kernels' 64 pairs)."""
    cfg, ocfg = pair(orc, **dict(SMALL, max_batch=32, max_seq=48))
    prompt = [[(7 * i + 5 * b + 1) % 4096 for i in range(5)] for b in range(32)]
    same, e1, e2 = run_parity(orc, cfg, ocfg, 31, prompt, 10, batch=32)
    assert same.all()
    assert e1 < 2e-2 and e2 < 2e-2


def test_gpt_oss_20b_batch4(orc):
    """20b shape, 4 rows: the batched projections at K = 2880 and 4096."""
    cfg, ocfg = pair(orc, max_seq=64, max_batch=4)
    prompt = [[101 + b, 2002, 30003 + 7 * b, 200000 - b] for b in range(4)]
    same, e1, e2 = run_parity(orc, cfg, ocfg, 3, prompt, 8, batch=4)
    assert same.all()
    assert e1 < 2e-2 and e2 < 2e-2


def test_small_model_chunked_prompt(orc):
    """Two 40-token prompts in passes of 16, 16 and 7 rows (the last pass
    partial), then 24 greedy steps: bit-identical to the oracle."""
    cfg, ocfg = pair(orc, **dict(SMALL, max_seq=96))
    prompt = [[(5 * i + 1) % 4096 for i in range(40)], [(9 * i + 2) % 4096 for i in range(40)]]
    same, e1, e2 = run_parity(orc, cfg, ocfg, 17, prompt, 24, batch=2, mode=ne.PREFILL_CHUNKED)
    assert same.all()
    assert e1 < 2e-2 and e2 < 2e-2


def test_small_model_sliding_ring_wraps(orc):
    """max_seq 700: the sliding layers keep a 256-row ring (window 128 + one
    prompt pass of 16 rows, rounded up to a power of two).  A 600-token prompt
    and 40 steps wrap it twice; every id and the logits must still equal the
    oracle's, which keeps every position."""
    cfg, ocfg = pair(orc, **dict(SMALL, max_seq=700, max_batch=1))
    prompt = [[(31 * i + 11) % 4096 for i in range(600)]]
    same, e1, e2 = run_parity(orc, cfg, ocfg, 23, prompt, 40, mode=ne.PREFILL_CHUNKED)
    assert same.all()
    assert e1 < 2e-2 and e2 < 2e-2


def test_gpt_oss_20b_chunked_prompt(orc):
    """20b shape, a 150-token prompt in 10 passes: the 128-key sliding window
    moves inside the prompt."""
    cfg, ocfg = pair(orc, max_seq=192)
    prompt = [[(1009 * i + 17) % 201088 for i in range(150)]]
    same, e1, e2 = run_parity(orc, cfg, ocfg, 2, prompt, 8, mode=ne.PREFILL_CHUNKED)
    assert same.all()
    assert e1 < 2e-2 and e2 < 2e-2


def test_gpt_oss_20b_greedy_64(orc):
    """Full gpt-oss-20b shape (24 layers, 32 experts, vocab 201088)."""
    cfg, ocfg = pair(orc, max_seq=256)
    same, e1, e2 = run_parity(orc, cfg, ocfg, 0, [[101, 2002, 30003, 200000]], 64)
    assert same.all()
    assert e1 < 2e-2 and e2 < 2e-2


def test_gpt_oss_20b_greedy_one_launch_experts(orc, monkeypatch):
    """The opt-in one-launch expert kernel (NEON_MOE_FUSED=1: gate_up and down
    with a grid-wide wait between them) gives the same bits as the oracle."""
    monkeypatch.setenv("NEON_MOE_FUSED", "1")
    cfg, ocfg = pair(orc, max_seq=64)
    same, e1, e2 = run_parity(orc, cfg, ocfg, 4, [[7, 2002, 30003, 200001]], 24)
    assert same.all()


@pytest.mark.parametrize("fuse", ["1", "0"])
def test_gpt_oss_20b_greedy_tail_fusions(orc, monkeypatch, fuse):
    """The launch forms of the step's follow-up work give the oracle's bits:
    NEON_FUSE_TAILS=1 runs the router logits in tail blocks of the O
    projection (opt-in) as well as the attention merge in the split kernel
    (the default); 0 runs both as separate launches.  max_seq 320 gives the
    full layers 5 key splits, so the merge runs."""
    monkeypatch.setenv("NEON_FUSE_TAILS", fuse)
    cfg, ocfg = pair(orc, max_seq=320)
    same, e1, e2 = run_parity(orc, cfg, ocfg, 6, [[5, 2002, 30003, 200002]], 40)
    assert same.all()


def test_engine_errors_on_gpu(orc):
    torch_cuda()
    cfg, _ = pair(orc, **dict(SMALL, max_seq=16))
    eng = ne.Engine(cfg)
    with pytest.raises(ne.NeonError) as e:
        eng.prefill([[1, 2]])
    assert e.value.status == ne.NEON_ESTATE  # no weights yet
    eng.init_random(1)
    with pytest.raises(ne.NeonError) as e:
        eng.prefill([[1, 4096]])
    assert e.value.status == ne.NEON_ERANGE_TOKEN
    with pytest.raises(ne.NeonError) as e:
        eng.decode(1)
    assert e.value.status == ne.NEON_ESTATE
    with pytest.raises(ne.NeonError) as e:
        eng.prefill([[1] * 17])
    assert e.value.status == ne.NEON_EKV_FULL
    eng.prefill([[1] * 10])
    with pytest.raises(ne.NeonError) as e:
        eng.decode(7)
    assert e.value.status == ne.NEON_EKV_FULL
    eng.decode(6)  # exactly fills the cache
    assert eng.seq_len() == 17
    bad = np.zeros(cfg.n_experts * 2 * cfg.intermediate * cfg.hidden // 32, np.uint8)
    bad[5] = 0xFF
    with pytest.raises(ne.NeonError) as e:
        eng.load_tensor("model.layers.0.mlp.experts.gate_up_proj_scales", bad.tobytes())
    assert e.value.status == ne.NEON_ENAN_SCALE
    with pytest.raises(ne.NeonError) as e:
        eng.load_tensor("model.layers.0.mlp.experts.gate_up_proj_scales", bad[:10].tobytes())
    assert e.value.status == ne.NEON_EINVAL
    eng.close()
