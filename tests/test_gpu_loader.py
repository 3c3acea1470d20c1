"""GPU checks of the local safetensors loader.

- Oracle checkpoint: the CPU oracle's random-init tensors are written as a
  gpt-oss checkpoint in the HF layout -- q / k / v split out of the fused
  projection, experts as [E][N][K/32][16] blocks, shapes from this file's own
  table (not the loader's) -- and loaded into a context that never ran
  neon_init_random; its greedy ids and logits must equal the oracle's.
- HF fixture: the same for the weights behind the HF GptOssForCausalLM
  fixture (tests/golden/hf_gptoss_fixtures.npz: the oracle's seed-7 tensors
  in a 2-layer HF model); the loaded model's logits must match HF's own at
  the oracle's HF bar.
- Round trip: one context's weights written out and loaded into a fresh one
  give identical bytes, logits and greedy ids; and the error paths of
  neon_load_tensor (unknown name, wrong size, NaN scale byte)."""
import sys

import numpy as np
import pytest

import neonengine_amd as ne
from neonengine_amd import loader
from tests.gpu_util import d2h, torch_cuda

pytestmark = pytest.mark.gpu

SMALL = dict(n_layers=4, hidden=512, n_heads=16, n_kv_heads=2, head_dim=64, n_experts=8,
             top_k=4, intermediate=512, vocab=4096, sliding_window=128, max_seq=256,
             max_batch=1)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def dump_checkpoint(eng, cfg, out_dir):
    import torch
    from safetensors.torch import save_file
    shapes = loader.checkpoint_shapes(cfg)
    files = [{}, {}]
    host = {}
    for i, (name, (shape, dt)) in enumerate(shapes.items()):
        ptr, nbytes = eng.tensor_ptr(name)
        a = d2h(ptr, nbytes, np.uint8 if dt == "u8" else np.uint16)
        assert a.size == int(np.prod(shape)), name
        host[name] = a
        if dt == "u8":
            t = torch.from_numpy(a.reshape(shape))
        else:
            t = torch.from_numpy(a.view(np.int16).reshape(shape)).view(torch.bfloat16)
            if name.endswith("self_attn.sinks"):
                t = t.float()  # exact; the loader rounds it back to the same bf16
        files[i % 2][name] = t
    for j, f in enumerate(files):
        save_file(f, str(out_dir / f"model-0000{j + 1}-of-00002.safetensors"))
    return host


def hf_tensors_from_oracle(orc, m, c):
    """The oracle model's tensors under gpt-oss checkpoint names, in the HF
    layout (HFM:83 interleaved gate/up rows; HFX:111-123 blocks/scales),
    shapes written out here from the HF module definitions."""
    import torch
    H, D, Hq, Hkv = c["hidden"], 64, c["n_heads"], c["n_kv_heads"]
    E, I, V = c["n_experts"], c["intermediate"], c["vocab"]
    Q, KV = Hq * D, Hkv * D

    def bf(layer, kind, shape, as_f32=False):
        a = m.tensor(layer, kind, int(np.prod(shape)))
        t = torch.from_numpy(a.view(np.int16).reshape(shape)).view(torch.bfloat16)
        return t.float() if as_f32 else t  # fp32 is exact; the loader rounds it back

    def u8(layer, kind, shape):
        return torch.from_numpy(m.tensor(layer, kind, int(np.prod(shape)), np.uint8).reshape(shape))

    out = {"model.embed_tokens.weight": bf(-1, orc.T_EMBED, (V, H)),
           "lm_head.weight": bf(-1, orc.T_LM_HEAD, (V, H)),
           "model.norm.weight": bf(-1, orc.T_FINAL_NORM, (H,), as_f32=True)}
    for l in range(c["n_layers"]):
        p = f"model.layers.{l}."
        wqkv = bf(l, orc.T_WQKV, (Q + 2 * KV, H))
        bqkv = bf(l, orc.T_BQKV, (Q + 2 * KV,))
        out.update({
            p + "input_layernorm.weight": bf(l, orc.T_ATTN_NORM, (H,)),
            p + "post_attention_layernorm.weight": bf(l, orc.T_MLP_NORM, (H,)),
            p + "self_attn.q_proj.weight": wqkv[:Q].clone(),
            p + "self_attn.k_proj.weight": wqkv[Q:Q + KV].clone(),
            p + "self_attn.v_proj.weight": wqkv[Q + KV:].clone(),
            p + "self_attn.q_proj.bias": bqkv[:Q].clone(),
            p + "self_attn.k_proj.bias": bqkv[Q:Q + KV].clone(),
            p + "self_attn.v_proj.bias": bqkv[Q + KV:].clone(),
            p + "self_attn.o_proj.weight": bf(l, orc.T_WO, (H, Q)),
            p + "self_attn.o_proj.bias": bf(l, orc.T_BO, (H,)),
            p + "self_attn.sinks": bf(l, orc.T_SINKS, (Hq,), as_f32=True),
            p + "mlp.router.weight": bf(l, orc.T_ROUTER_W, (E, H)),
            p + "mlp.router.bias": bf(l, orc.T_ROUTER_B, (E,)),
            p + "mlp.experts.gate_up_proj_blocks": u8(l, orc.T_GU_CODES, (E, 2 * I, H // 32, 16)),
            p + "mlp.experts.gate_up_proj_scales": u8(l, orc.T_GU_SCALES, (E, 2 * I, H // 32)),
            p + "mlp.experts.gate_up_proj_bias": bf(l, orc.T_GU_BIAS, (E, 2 * I)),
            p + "mlp.experts.down_proj_blocks": u8(l, orc.T_DN_CODES, (E, H, I // 32, 16)),
            p + "mlp.experts.down_proj_scales": u8(l, orc.T_DN_SCALES, (E, H, I // 32)),
            p + "mlp.experts.down_proj_bias": bf(l, orc.T_DN_BIAS, (E, H)),
        })
    return out


def save_split(tensors, out_dir):
    from safetensors.torch import save_file
    names = sorted(tensors)
    for j, part in enumerate((names[0::2], names[1::2])):
        save_file({n: tensors[n] for n in part}, str(out_dir / f"model-0000{j + 1}-of-00002.safetensors"))


def test_oracle_checkpoint_loads_to_oracle_bits(orc, tmp_path):
    torch_cuda()
    seed = 41
    cfg = ne.config_preset("gpt-oss-20b", **SMALL)
    c = cfg.as_dict()
    m = orc.Model(orc.make_config(**c), seed=seed, batch=1)
    save_split(hf_tensors_from_oracle(orc, m, c), tmp_path)
    say(f"oracle checkpoint layers={cfg.n_layers} hidden={cfg.hidden}: loading")
    eng = ne.Engine(cfg)
    assert eng.load_checkpoint(str(tmp_path)) == 3 + 19 * cfg.n_layers
    prompt = [5, 900, 17, 4001]
    eng.prefill([prompt])
    eng.decode(24)
    toks = eng.read_tokens()[0, len(prompt):]
    lg = eng.read_logits()[0]
    eng.close()
    for t in prompt:
        nxt, _ = m.step(np.array([t], np.int32), want_logits=False)
    want = [int(nxt[0])]
    for _ in range(24):
        nxt, lo = m.step(nxt)
        want.append(int(nxt[0]))
    m.close()
    say(f"  ids equal: {list(map(int, toks)) == want}")
    assert list(map(int, toks)) == want
    assert np.array_equal(lg.view(np.uint32), lo[0].view(np.uint32))


def test_hf_fixture_checkpoint_matches_hf(orc, golden, tmp_path):
    """The weights behind the HF fixture model, loaded as a checkpoint: each
    prompt position's logits against HF's fp32 GptOssForCausalLM (the bar and
    the router-margin excusal of tests/test_oracle.py::test_model_matches_hf)
    and, bit for bit, against the oracle."""
    torch_cuda()
    g = golden
    names = ("n_layers", "hidden", "n_heads", "n_kv_heads", "head_dim", "n_experts", "top_k",
             "intermediate", "vocab", "sliding_window", "max_seq")
    c = dict(zip(names, (int(v) for v in g["model_cfg"])))
    cfg = ne.config_preset("gpt-oss-20b", **c, max_batch=1)
    seed = int(g["model_seed"][0])
    m = orc.Model(orc.make_config(**cfg.as_dict()), seed=seed, batch=1)
    save_split(hf_tensors_from_oracle(orc, m, cfg.as_dict()), tmp_path)
    ids = [int(t) for t in g["model_ids"]]
    ours, oracle = [], []
    for t in range(len(ids)):
        eng = ne.Engine(cfg)
        eng.load_checkpoint(str(tmp_path))
        eng.set_prefill_mode(ne.PREFILL_STEPWISE)
        eng.prefill([ids[:t + 1]])
        ours.append(eng.read_logits()[0])
        eng.close()
        oracle.append(m.step(np.array([ids[t]], np.int32))[1][0])
    m.close()
    ours, oracle = np.stack(ours), np.stack(oracle)
    assert np.array_equal(ours.view(np.uint32), oracle.view(np.uint32))
    ref = g["model_logits"]
    k = c["top_k"]
    rs = np.sort(g["model_router_logits"], axis=-1)
    ok = (rs[..., -k] - rs[..., -k - 1]).min(axis=0) >= 1e-2
    err = np.abs(ours - ref).max(axis=1) / np.abs(ref).max(axis=1)
    say(f"loaded HF fixture model: rel max err per position {np.round(err, 4)}")
    assert ok.sum() >= len(ok) - 2
    assert np.all(err[ok] < 3e-2)


def greedy(eng, prompt, n):
    eng.set_prefill_mode(ne.PREFILL_STEPWISE)
    eng.prefill(prompt)
    eng.decode(n)
    return eng.read_tokens(), eng.read_logits()


def test_checkpoint_round_trip(tmp_path):
    torch_cuda()
    cfg = ne.config_preset("gpt-oss-20b", **SMALL)
    say(f"loader round trip layers={cfg.n_layers} hidden={cfg.hidden} E={cfg.n_experts}")
    src = ne.Engine(cfg)
    src.init_random(23)
    host = dump_checkpoint(src, cfg, tmp_path)
    dst = ne.Engine(cfg)
    n = dst.load_checkpoint(str(tmp_path))
    assert n == len(host)
    for name, a in host.items():
        ptr, nbytes = dst.tensor_ptr(name)
        assert np.array_equal(d2h(ptr, nbytes, a.dtype), a), name
    prompt = [[3, 99, 4000, 17, 256]]
    t_src, lg_src = greedy(src, prompt, 32)
    t_dst, lg_dst = greedy(dst, prompt, 32)
    say(f"  greedy ids equal: {np.array_equal(t_src, t_dst)}")
    assert np.array_equal(t_src, t_dst)
    assert np.array_equal(lg_src.view(np.uint32), lg_dst.view(np.uint32))
    src.close()
    dst.close()


def test_load_tensor_rejects_bad_input():
    torch_cuda()
    cfg = ne.config_preset("gpt-oss-20b", **SMALL)
    eng = ne.Engine(cfg)
    H = cfg.hidden
    with pytest.raises(ne.NeonError) as e:
        eng.load_tensor("model.layers.0.self_attn.not_a_tensor", np.zeros(H, np.uint16))
    assert e.value.status == ne.NEON_EINVAL
    with pytest.raises(ne.NeonError) as e:
        eng.load_tensor(f"model.layers.{cfg.n_layers}.input_layernorm.weight",
                        np.zeros(H, np.uint16))
    assert e.value.status == ne.NEON_EINVAL
    with pytest.raises(ne.NeonError) as e:
        eng.load_tensor("model.norm.weight", np.zeros(H + 1, np.uint16))
    assert e.value.status == ne.NEON_EINVAL
    name = "model.layers.2.mlp.experts.down_proj_scales"
    scales = np.full(cfg.n_experts * H * cfg.intermediate // 32, 127, np.uint8)
    scales[1234] = 0xFF
    with pytest.raises(ne.NeonError) as e:
        eng.load_tensor(name, scales)
    assert e.value.status == ne.NEON_ENAN_SCALE
    scales[1234] = 126
    eng.load_tensor(name, scales)
    ptr, nbytes = eng.tensor_ptr(name)
    assert np.array_equal(d2h(ptr, nbytes, np.uint8), scales)
    eng.close()
