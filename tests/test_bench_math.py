"""CPU checks of the algorithmic byte counts bench.py divides by: they are
recomputed here from the checkpoint tensor shapes (Hugging Face gpt-oss
layout), so a dropped term or a wrong factor in the roofline denominators
fails."""
import numpy as np

import bench
import neonengine_amd as ne
from neonengine_amd import loader


def tensor_bytes(shape, dt):
    return int(np.prod(shape)) * (1 if dt == "u8" else 2)


def test_moe_bytes_per_launch_pair():
    cfg = ne.config_preset("gpt-oss-20b")
    shapes = loader.checkpoint_shapes(cfg)
    p = "model.layers.0.mlp.experts."
    per_expert = sum(tensor_bytes(*shapes[p + n]) for n in (
        "gate_up_proj_blocks", "gate_up_proj_scales", "gate_up_proj_bias",
        "down_proj_blocks", "down_proj_scales", "down_proj_bias")) // cfg.n_experts
    want = cfg.top_k * per_expert + 2 * cfg.hidden * 2  # + the input and output rows
    assert bench.moe_bytes(cfg) == want == 52_957_440


def test_step_bytes_match_the_checkpoint():
    cfg = ne.config_preset("gpt-oss-20b")
    shapes = loader.checkpoint_shapes(cfg)
    weights = 0
    for name, (shape, dt) in shapes.items():
        b = tensor_bytes(shape, dt)
        if ".mlp.experts." in name:
            b = b * cfg.top_k // cfg.n_experts  # k of E experts per token
        elif name == "model.embed_tokens.weight":
            b = cfg.hidden * 2  # one row
        weights += b
    kv_row = 2 * cfg.n_kv_heads * cfg.head_dim * 2
    # an empty cache: only the new K/V row is written in every layer
    assert bench.step_bytes(cfg, 0) == weights + cfg.n_layers * kv_row
    # past the window only the full layers read one more cached row per position
    n_full = sum(1 for l in range(cfg.n_layers) if l % 2 == 1)
    t = 4 * cfg.sliding_window
    assert bench.step_bytes(cfg, t + 1) - bench.step_bytes(cfg, t) == n_full * kv_row


def test_prefill_flops_small_case():
    cfg = ne.config_preset("gpt-oss-20b", n_layers=2, sliding_window=2)
    H, D, Hq, Hkv = cfg.hidden, cfg.head_dim, cfg.n_heads, cfg.n_kv_heads
    per_row = (2 * H * (Hq + 2 * Hkv) * D + 2 * Hq * D * H + 2 * H * cfg.n_experts
               + cfg.top_k * (2 * H * 2 * cfg.intermediate + 2 * cfg.intermediate * H))
    M = 3  # a 4-token prompt: rows 0, 1, 2 attend to 1, 2, 3 keys (full) or 1, 2, 2 (window 2)
    keys = (1 + 2 + 2) + (1 + 2 + 3)
    want = 2 * M * per_row + keys * Hq * D * 2 * 2
    assert bench.prefill_flops(cfg, M + 1) == want
