"""Load a gpt-oss checkpoint from local safetensors files into an Engine.

The files hold the Hugging Face gpt-oss layout (HF integrations/mxfp4.py:
111-123, 298-304): bf16 attention / router / norm / embedding tensors, and
the experts as MXFP4 `*_blocks` (uint8 [E][N][K/32][16], low nibble = even
element) with E8M0 `*_scales` (uint8 [E][N][K/32]) and bf16 biases.  Every
tensor goes to the context through neon_load_tensor under its checkpoint
name, which checks its size and (for scales) the NaN byte 0xFF.  Only local
paths are read; nothing is fetched.
"""
from __future__ import annotations

import glob
import os

import numpy as np


def tensor_data(name: str, t) -> np.ndarray:
    """The tensor as a C-contiguous numpy array in the library's layout:
    uint8 MXFP4 blocks/scales as they are, every float tensor as bf16 bits."""
    import torch
    if name.endswith("_blocks") or name.endswith("_scales"):
        if t.dtype != torch.uint8:
            raise ValueError(f"{name}: MXFP4 tensor must be uint8, got {t.dtype}")
        return np.ascontiguousarray(t.numpy())
    if not t.is_floating_point():
        raise ValueError(f"{name}: expected a floating-point tensor, got {t.dtype}")
    if t.dtype != torch.bfloat16:
        t = t.to(torch.bfloat16)  # round to nearest even
    return np.ascontiguousarray(t.contiguous().view(torch.int16).numpy().view(np.uint16))


def checkpoint_files(path: str) -> list[str]:
    """The *.safetensors files of a local file or directory, in name order."""
    if os.path.isdir(path):
        files = sorted(glob.glob(os.path.join(path, "*.safetensors")))
    else:
        files = [path]
    if not files or not all(os.path.isfile(f) for f in files):
        raise FileNotFoundError(f"no safetensors file at {path!r}")
    return files


def check_tensor(name: str, t, expected) -> None:
    """Raises ValueError when a checkpoint tensor's shape or element type is
    not the one the engine's config gives for that name (a transposed q_proj
    or o_proj, or experts stored in another order, has the right byte count
    but the wrong shape)."""
    import torch
    shape, kind = expected
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: shape {tuple(t.shape)}, the model expects {tuple(shape)}")
    if kind == "u8" and t.dtype != torch.uint8:
        raise ValueError(f"{name}: MXFP4 tensor must be uint8, got {t.dtype}")
    if kind == "bf16" and not t.is_floating_point():
        raise ValueError(f"{name}: expected a floating-point tensor, got {t.dtype}")


def load_checkpoint(engine, path: str, strict: bool = True) -> int:
    """Loads every tensor of the checkpoint at `path` into `engine` and returns
    how many it loaded.  A known tensor whose shape or element type differs
    from the engine's config raises ValueError before anything of it is
    copied; a name the model does not have, or a size that does not match,
    raises NeonError (from neon_load_tensor); with `strict`, a checkpoint that
    lacks one of the model's tensors raises KeyError after the others were
    loaded."""
    from safetensors import safe_open
    shapes = checkpoint_shapes(engine.cfg)
    seen = set()
    for f in checkpoint_files(path):
        with safe_open(f, framework="pt") as sf:
            for name in sf.keys():
                t = sf.get_tensor(name)
                if name in shapes:
                    check_tensor(name, t, shapes[name])
                engine.load_tensor(name, tensor_data(name, t))
                seen.add(name)
    if strict:
        missing = [n for n in checkpoint_names(engine.cfg) if n not in seen]
        if missing:
            raise KeyError(f"checkpoint {path!r} lacks {len(missing)} tensors, "
                           f"first {missing[:4]}")
    return len(seen)


def checkpoint_names(cfg) -> list[str]:
    """Every tensor name a gpt-oss checkpoint of shape `cfg` holds."""
    names = ["model.embed_tokens.weight", "lm_head.weight", "model.norm.weight"]
    per_layer = [
        "input_layernorm.weight", "post_attention_layernorm.weight",
        "self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
        "self_attn.q_proj.bias", "self_attn.k_proj.bias", "self_attn.v_proj.bias",
        "self_attn.o_proj.weight", "self_attn.o_proj.bias", "self_attn.sinks",
        "mlp.router.weight", "mlp.router.bias",
        "mlp.experts.gate_up_proj_blocks", "mlp.experts.gate_up_proj_scales",
        "mlp.experts.gate_up_proj_bias", "mlp.experts.down_proj_blocks",
        "mlp.experts.down_proj_scales", "mlp.experts.down_proj_bias",
    ]
    for layer in range(cfg.n_layers):
        names += [f"model.layers.{layer}.{r}" for r in per_layer]
    return names


def checkpoint_shapes(cfg) -> dict[str, tuple[tuple[int, ...], str]]:
    """(shape, dtype) of every checkpoint tensor of shape `cfg` (HF layout)."""
    H, D, Hq, Hkv = cfg.hidden, cfg.head_dim, cfg.n_heads, cfg.n_kv_heads
    E, I, V = cfg.n_experts, cfg.intermediate, cfg.vocab
    out = {"model.embed_tokens.weight": ((V, H), "bf16"), "lm_head.weight": ((V, H), "bf16"),
           "model.norm.weight": ((H,), "bf16")}
    per = {
        "input_layernorm.weight": ((H,), "bf16"),
        "post_attention_layernorm.weight": ((H,), "bf16"),
        "self_attn.q_proj.weight": ((Hq * D, H), "bf16"),
        "self_attn.k_proj.weight": ((Hkv * D, H), "bf16"),
        "self_attn.v_proj.weight": ((Hkv * D, H), "bf16"),
        "self_attn.q_proj.bias": ((Hq * D,), "bf16"),
        "self_attn.k_proj.bias": ((Hkv * D,), "bf16"),
        "self_attn.v_proj.bias": ((Hkv * D,), "bf16"),
        "self_attn.o_proj.weight": ((H, Hq * D), "bf16"),
        "self_attn.o_proj.bias": ((H,), "bf16"),
        "self_attn.sinks": ((Hq,), "bf16"),
        "mlp.router.weight": ((E, H), "bf16"),
        "mlp.router.bias": ((E,), "bf16"),
        "mlp.experts.gate_up_proj_blocks": ((E, 2 * I, H // 32, 16), "u8"),
        "mlp.experts.gate_up_proj_scales": ((E, 2 * I, H // 32), "u8"),
        "mlp.experts.gate_up_proj_bias": ((E, 2 * I), "bf16"),
        "mlp.experts.down_proj_blocks": ((E, H, I // 32, 16), "u8"),
        "mlp.experts.down_proj_scales": ((E, H, I // 32), "u8"),
        "mlp.experts.down_proj_bias": ((E, H), "bf16"),
    }
    for layer in range(cfg.n_layers):
        for r, v in per.items():
            out[f"model.layers.{layer}.{r}"] = v
    return out
