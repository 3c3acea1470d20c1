"""Writes tests/golden/hf_gptoss_fixtures.npz: input/output vectors from the
gpt-oss modules of HuggingFace transformers 5.15.0 (the installed third-party
package whose source states the model maths; NOT the reference repository,
which has no implementation of this path).

Run in the build container only (needs transformers + torch; no network:
every module is built from a local GptOssConfig, never from a model name):
    python tests/golden/make_golden.py

Everything runs in fp32 on the CPU, on inputs that are exactly representable
in bf16 so the same inputs can be fed to the oracle.  Fixtures:
  mxfp4_*     HF _convert_moe_packed_tensors (integrations/mxfp4.py:257-313)
              on all 16 codes x 255 non-NaN scales
  yarn_*      HF _compute_yarn_parameters (modeling_rope_utils.py:345-483)
  rope_*      GptOssRotaryEmbedding + apply_rotary_pos_emb (HFM:165-231)
  rms_*       GptOssRMSNorm (HFM:48-62)
  router_*    GptOssTopKRouter (HFM:117-130)
  experts_*   GptOssExperts (HFM:65-114), weights dequantised from MXFP4
  attn_*      eager_attention_forward with sinks (HFM:235-263), full and
              sliding masks
  model_*     GptOssForCausalLM, 2 layers, logits for a 10-token prompt, with
              the oracle's random-init weights (oracle/libneon_oracle.so)
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as orc  # noqa: E402

from transformers import GptOssConfig  # noqa: E402
from transformers.integrations.mxfp4 import _convert_moe_packed_tensors  # noqa: E402
from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS  # noqa: E402
from transformers.models.gpt_oss import modeling_gpt_oss as M  # noqa: E402

torch.manual_seed(0)
rng = np.random.default_rng(1234)


def bf16_exact(a):
    """fp32 array rounded to bf16 (so both sides see identical inputs)."""
    return orc.bf16_to_f32(orc.f32_to_bf16(np.asarray(a, np.float32)))


def tiny_config(**kw):
    d = dict(num_hidden_layers=2, num_local_experts=4, num_experts_per_tok=2, vocab_size=128,
             hidden_size=64, intermediate_size=64, head_dim=64, num_attention_heads=8,
             num_key_value_heads=2, sliding_window=4, max_position_embeddings=4096,
             rms_norm_eps=1e-5)
    d.update(kw)
    cfg = GptOssConfig(**d)
    cfg._attn_implementation = "eager"
    return cfg


out = {}

# ---- MXFP4 dequantisation ------------------------------------------------------
codes = np.arange(256, dtype=np.uint8)                 # every byte = every nibble pair
scales = np.arange(255, dtype=np.uint8)                # every non-NaN E8M0 byte
blocks = np.tile(codes.reshape(1, 16, 16), (255, 1, 1))  # [255 rows][16 blocks][16 B]
sc = np.tile(scales.reshape(255, 1), (1, 16))          # [255][16]
deq = _convert_moe_packed_tensors(torch.from_numpy(blocks[None]), torch.from_numpy(sc[None]),
                                  dtype=torch.float32)  # -> [1][K=512][N=255]
out["mxfp4_blocks"] = blocks
out["mxfp4_scales"] = sc
out["mxfp4_deq"] = deq[0].transpose(0, 1).contiguous().numpy()  # [N][K]

# ---- YaRN ------------------------------------------------------------------------
cfg20 = tiny_config()
inv, af = ROPE_INIT_FUNCTIONS["yarn"](cfg20, "cpu")
out["yarn_inv_freq"] = inv.numpy().astype(np.float32)
out["yarn_attn_factor"] = np.array([af], np.float64)

# ---- rotary embedding + application ---------------------------------------------
rot = M.GptOssRotaryEmbedding(cfg20)
positions = np.array([0, 1, 7, 127, 128, 2047, 4095, 30000], np.int64)
xq = bf16_exact(rng.standard_normal((len(positions), 3, 64)))
cos, sin = rot(torch.zeros(1, dtype=torch.float32), torch.from_numpy(positions)[None])
q_t = torch.from_numpy(xq).transpose(0, 1)[None]  # [1, heads, T, D]
k_t = q_t.clone()
q_emb, _ = M.apply_rotary_pos_emb(q_t, k_t, cos, sin)
out["rope_positions"] = positions.astype(np.int32)
out["rope_cos"] = cos[0].numpy()
out["rope_sin"] = sin[0].numpy()
out["rope_x"] = xq
out["rope_out"] = q_emb[0].transpose(0, 1).contiguous().numpy()

# ---- RMSNorm ----------------------------------------------------------------------
rms = M.GptOssRMSNorm(64, eps=1e-5)
w = bf16_exact(1.0 + 0.1 * rng.standard_normal(64))
rms.weight.data = torch.from_numpy(w)
xr = bf16_exact(3.0 * rng.standard_normal((4, 64)))
out["rms_x"], out["rms_w"] = xr, w
out["rms_out"] = rms(torch.from_numpy(xr)).detach().numpy()

# ---- router ------------------------------------------------------------------------
rcfg = tiny_config(num_local_experts=8, num_experts_per_tok=4)
router = M.GptOssTopKRouter(rcfg)
rw = bf16_exact(0.2 * rng.standard_normal((8, 64)))
rb = bf16_exact(0.2 * rng.standard_normal(8))
router.weight.data = torch.from_numpy(rw)
router.bias.data = torch.from_numpy(rb)
xrt = bf16_exact(rng.standard_normal((5, 64)))
logits, scores, idx = router(torch.from_numpy(xrt))
out["router_x"], out["router_w"], out["router_b"] = xrt, rw, rb
out["router_logits"] = logits.detach().numpy()
out["router_scores"] = scores.detach().numpy()
out["router_idx"] = idx.numpy().astype(np.int32)

# ---- experts (MXFP4 weights dequantised by HF) ---------------------------------------
E, H, I = 4, 64, 64
gu_blocks = rng.integers(0, 256, (E, 2 * I, H // 32, 16), dtype=np.uint8)
gu_scales = rng.integers(119, 125, (E, 2 * I, H // 32), dtype=np.uint8)
dn_blocks = rng.integers(0, 256, (E, H, I // 32, 16), dtype=np.uint8)
dn_scales = rng.integers(119, 125, (E, H, I // 32), dtype=np.uint8)
gu_bias = bf16_exact(0.5 * rng.standard_normal((E, 2 * I)))
dn_bias = bf16_exact(0.5 * rng.standard_normal((E, H)))
ex = M.GptOssExperts(tiny_config(num_local_experts=E))
ex.gate_up_proj.data = _convert_moe_packed_tensors(torch.from_numpy(gu_blocks), torch.from_numpy(gu_scales), dtype=torch.float32)
ex.down_proj.data = _convert_moe_packed_tensors(torch.from_numpy(dn_blocks), torch.from_numpy(dn_scales), dtype=torch.float32)
ex.gate_up_proj_bias.data = torch.from_numpy(gu_bias)
ex.down_proj_bias.data = torch.from_numpy(dn_bias)
xe = bf16_exact(rng.standard_normal((3, H)))
e_idx = np.array([[0, 2], [3, 1], [1, 0]], np.int64)
e_w = np.array([[0.7, 0.3], [0.55, 0.45], [0.9, 0.1]], np.float32)
with torch.no_grad():
    ye = ex(torch.from_numpy(xe), torch.from_numpy(e_idx), torch.from_numpy(e_w)).numpy()
    gu_full = torch.from_numpy(xe) @ ex.gate_up_proj[0] + ex.gate_up_proj_bias[0]
    out["experts_gate_up_e0"] = gu_full.numpy()
    out["experts_glu_e0"] = ex._apply_gate(gu_full).numpy()
out.update(experts_gu_blocks=gu_blocks, experts_gu_scales=gu_scales, experts_dn_blocks=dn_blocks,
           experts_dn_scales=dn_scales, experts_gu_bias=gu_bias, experts_dn_bias=dn_bias,
           experts_x=xe, experts_idx=e_idx.astype(np.int32), experts_w=e_w, experts_out=ye)


# ---- attention with sinks ----------------------------------------------------------------
class _AttnStub(torch.nn.Module):
    def __init__(self, hq, hkv):
        super().__init__()
        self.num_key_value_groups = hq // hkv
        self.sinks = torch.nn.Parameter(torch.zeros(hq))


Hq, Hkv, D, T = 8, 2, 64, 37
stub = _AttnStub(Hq, Hkv)
sinks = bf16_exact(rng.standard_normal(Hq))
stub.sinks.data = torch.from_numpy(sinks)
qa = bf16_exact(rng.standard_normal((1, Hq, 1, D)))
ka = bf16_exact(rng.standard_normal((1, Hkv, T, D)))
va = bf16_exact(rng.standard_normal((1, Hkv, T, D)))
res = {}
for name, window in (("full", 0), ("sliding", 16)):
    mask = np.zeros((1, 1, 1, T), np.float32)
    if window:
        mask[..., : T - window] = -np.inf  # keys j with j <= q - window are masked
    o, _ = M.eager_attention_forward(stub, torch.from_numpy(qa), torch.from_numpy(ka),
                                     torch.from_numpy(va), torch.from_numpy(mask),
                                     scaling=D ** -0.5)
    out[f"attn_out_{name}"] = o.detach().numpy().reshape(Hq, D)
out.update(attn_q=qa.reshape(Hq, D), attn_k=ka.reshape(Hkv, T, D), attn_v=va.reshape(Hkv, T, D),
           attn_sinks=sinks, attn_window=np.array([16], np.int32))

# ---- full tiny model with the oracle's random-init weights --------------------------------
mc = dict(n_layers=2, hidden=64, n_heads=8, n_kv_heads=2, head_dim=64, n_experts=4, top_k=2,
          intermediate=64, vocab=128, sliding_window=4, max_seq=32, max_batch=1)
ocfg = orc.make_config(**mc)
om = orc.Model(ocfg, seed=7, batch=1)
hcfg = tiny_config()
model = M.GptOssForCausalLM(hcfg).float().eval()
QKV = (8 + 2 * 2) * 64


def t_bf(layer, kind, n, shape):
    return torch.from_numpy(orc.bf16_to_f32(om.tensor(layer, kind, n)).reshape(shape))


def t_u8(layer, kind, n, shape):
    return torch.from_numpy(om.tensor(layer, kind, n, np.uint8).reshape(shape))


with torch.no_grad():
    model.model.embed_tokens.weight.copy_(t_bf(-1, orc.T_EMBED, 128 * 64, (128, 64)))
    model.lm_head.weight.copy_(t_bf(-1, orc.T_LM_HEAD, 128 * 64, (128, 64)))
    model.model.norm.weight.copy_(t_bf(-1, orc.T_FINAL_NORM, 64, (64,)))
    for l, layer in enumerate(model.model.layers):
        wqkv = t_bf(l, orc.T_WQKV, QKV * 64, (QKV, 64))
        bqkv = t_bf(l, orc.T_BQKV, QKV, (QKV,))
        a = layer.self_attn
        a.q_proj.weight.copy_(wqkv[:512]); a.q_proj.bias.copy_(bqkv[:512])
        a.k_proj.weight.copy_(wqkv[512:640]); a.k_proj.bias.copy_(bqkv[512:640])
        a.v_proj.weight.copy_(wqkv[640:768]); a.v_proj.bias.copy_(bqkv[640:768])
        a.o_proj.weight.copy_(t_bf(l, orc.T_WO, 64 * 512, (64, 512)))
        a.o_proj.bias.copy_(t_bf(l, orc.T_BO, 64, (64,)))
        a.sinks.copy_(t_bf(l, orc.T_SINKS, 8, (8,)))
        layer.input_layernorm.weight.copy_(t_bf(l, orc.T_ATTN_NORM, 64, (64,)))
        layer.post_attention_layernorm.weight.copy_(t_bf(l, orc.T_MLP_NORM, 64, (64,)))
        layer.mlp.router.weight.copy_(t_bf(l, orc.T_ROUTER_W, 4 * 64, (4, 64)))
        layer.mlp.router.bias.copy_(t_bf(l, orc.T_ROUTER_B, 4, (4,)))
        exm = layer.mlp.experts
        exm.gate_up_proj.copy_(_convert_moe_packed_tensors(
            t_u8(l, orc.T_GU_CODES, 4 * 128 * 32, (4, 128, 2, 16)),
            t_u8(l, orc.T_GU_SCALES, 4 * 128 * 2, (4, 128, 2)), dtype=torch.float32))
        exm.down_proj.copy_(_convert_moe_packed_tensors(
            t_u8(l, orc.T_DN_CODES, 4 * 64 * 32, (4, 64, 2, 16)),
            t_u8(l, orc.T_DN_SCALES, 4 * 64 * 2, (4, 64, 2)), dtype=torch.float32))
        exm.gate_up_proj_bias.copy_(t_bf(l, orc.T_GU_BIAS, 4 * 128, (4, 128)))
        exm.down_proj_bias.copy_(t_bf(l, orc.T_DN_BIAS, 4 * 64, (4, 64)))
    ids = np.array([5, 17, 99, 3, 3, 64, 127, 0, 42, 8], np.int64)
    router_logits = []
    hooks = [layer.mlp.router.register_forward_hook(
        lambda mod, inp, outp: router_logits.append(outp[0].detach().numpy().copy()))
        for layer in model.model.layers]
    logits = model(input_ids=torch.from_numpy(ids)[None]).logits[0].numpy()
    for hk in hooks:
        hk.remove()
out["model_router_logits"] = np.stack(router_logits).astype(np.float32)  # [L][T][E]
out["model_cfg"] = np.array([mc[k] for k in ("n_layers", "hidden", "n_heads", "n_kv_heads",
                                             "head_dim", "n_experts", "top_k", "intermediate",
                                             "vocab", "sliding_window", "max_seq")], np.int32)
out["model_seed"] = np.array([7], np.int64)
out["model_ids"] = ids.astype(np.int32)
out["model_logits"] = logits.astype(np.float32)
om.close()

path = os.path.join(HERE, "hf_gptoss_fixtures.npz")
np.savez_compressed(path, **out)
print("wrote", path, os.path.getsize(path), "bytes,", len(out), "arrays")
