"""GPU round trip of the local safetensors loader: the weights of one context
are written out as a gpt-oss checkpoint in the HF layout (split over two
files, one float tensor stored as fp32), loaded into a fresh context through
neon_load_tensor, and the two contexts must then hold identical bytes and
produce bit-identical logits and identical greedy ids.  The error paths of
neon_load_tensor (unknown name, wrong size, NaN scale byte) are checked on
the same context."""
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
