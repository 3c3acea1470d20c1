"""CPU checks of the local safetensors loader: file discovery, the bytes each
checkpoint tensor becomes (bf16 bits, float tensors rounded to nearest even),
the name list against the HF gpt-oss layout, and strict-mode reporting.  The
engine is a stand-in that records what neon_load_tensor would receive."""
import numpy as np
import pytest

import neonengine_amd as ne
from neonengine_amd import loader

torch = pytest.importorskip("torch")
st = pytest.importorskip("safetensors.torch")


class Recorder:
    def __init__(self, cfg):
        self.cfg = cfg
        self.got = {}

    def load_tensor(self, name, data):
        assert isinstance(data, np.ndarray) and data.flags.c_contiguous
        self.got[name] = data.copy()


TINY = dict(n_layers=2, hidden=64, n_heads=4, n_kv_heads=2, head_dim=16, n_experts=4,
            top_k=2, intermediate=64, vocab=128, max_seq=32, max_batch=1)


def test_float_tensors_become_bf16_bits(tmp_path):
    # 1 + 2^-8 is the tie between bf16 1.0 and 1 + 2^-7: even mantissa wins (0x3F80);
    # 1 + 3 * 2^-9 rounds up to 1 + 2^-7 (0x3F81); -2.5 is exact (0xC020)
    f32 = torch.tensor([1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -9, -2.5, 0.0], dtype=torch.float32)
    bf = torch.tensor([0.5, -1.0], dtype=torch.bfloat16)
    blocks = torch.arange(32, dtype=torch.uint8).reshape(1, 1, 2, 16)
    st.save_file({"a.sinks": f32, "b.bias": bf, "c_blocks": blocks}, str(tmp_path / "m.safetensors"))
    eng = Recorder(ne.config_preset("gpt-oss-20b", **TINY))
    n = loader.load_checkpoint(eng, str(tmp_path), strict=False)
    assert n == 3
    assert eng.got["a.sinks"].dtype == np.uint16
    assert eng.got["a.sinks"].tolist() == [0x3F80, 0x3F81, 0xC020, 0x0000]
    assert eng.got["b.bias"].tolist() == [0x3F00, 0xBF80]
    assert eng.got["c_blocks"].ravel().tolist() == list(range(32))  # raw, row-major [E][N][K/32][16]


def test_mxfp4_tensor_must_be_uint8(tmp_path):
    st.save_file({"x.down_proj_scales": torch.zeros(4, dtype=torch.float32)},
                 str(tmp_path / "m.safetensors"))
    with pytest.raises(ValueError, match="uint8"):
        loader.load_checkpoint(Recorder(ne.config_preset("gpt-oss-20b", **TINY)),
                               str(tmp_path), strict=False)


def test_files_in_name_order_and_missing_path(tmp_path):
    st.save_file({"z": torch.zeros(2, dtype=torch.bfloat16)}, str(tmp_path / "b.safetensors"))
    st.save_file({"y": torch.zeros(2, dtype=torch.bfloat16)}, str(tmp_path / "a.safetensors"))
    (tmp_path / "notes.txt").write_text("not a checkpoint")
    files = loader.checkpoint_files(str(tmp_path))
    assert [f.rsplit("/", 1)[1] for f in files] == ["a.safetensors", "b.safetensors"]
    with pytest.raises(FileNotFoundError):
        loader.checkpoint_files(str(tmp_path / "absent.safetensors"))
    with pytest.raises(FileNotFoundError):
        loader.checkpoint_files(str(tmp_path / "nowhere"))


def test_names_and_shapes_follow_hf_layout():
    cfg = ne.config_preset("gpt-oss-20b")
    names = loader.checkpoint_names(cfg)
    shapes = loader.checkpoint_shapes(cfg)
    assert set(names) == set(shapes) and len(names) == len(set(names))
    assert len(names) == 3 + 19 * 24
    # 20b: 2880 hidden, 32 experts, 64 q heads, 8 kv heads of 64, vocab 201088
    assert shapes["model.layers.0.mlp.experts.gate_up_proj_blocks"] == ((32, 5760, 90, 16), "u8")
    assert shapes["model.layers.23.mlp.experts.down_proj_scales"] == ((32, 2880, 90), "u8")
    assert shapes["model.layers.5.self_attn.q_proj.weight"] == ((4096, 2880), "bf16")
    assert shapes["model.layers.5.self_attn.k_proj.weight"] == ((512, 2880), "bf16")
    assert shapes["model.layers.5.self_attn.o_proj.weight"] == ((2880, 4096), "bf16")
    assert shapes["model.layers.5.self_attn.sinks"] == ((64,), "bf16")
    assert shapes["lm_head.weight"] == ((201088, 2880), "bf16")
    # the on-disk sizes add up to the 20b parameter count (about 20.9 B values)
    values = sum(int(np.prod(s)) * (2 if n.endswith("_blocks") else 1)
                 for n, (s, _) in shapes.items() if not n.endswith("_scales"))
    assert 20.8e9 < values < 21.0e9


def test_strict_reports_missing_tensors(tmp_path):
    cfg = ne.config_preset("gpt-oss-20b", **TINY)
    shapes = loader.checkpoint_shapes(cfg)
    full = {}
    for n, (s, dt) in shapes.items():
        full[n] = torch.zeros(s, dtype=torch.uint8 if dt == "u8" else torch.bfloat16)
    drop = "model.layers.1.self_attn.sinks"
    st.save_file({n: t for n, t in full.items() if n != drop}, str(tmp_path / "m.safetensors"))
    eng = Recorder(cfg)
    with pytest.raises(KeyError, match="lacks 1 tensors"):
        loader.load_checkpoint(eng, str(tmp_path / "m.safetensors"))
    assert len(eng.got) == len(shapes) - 1
    for n, a in eng.got.items():  # every tensor arrived whole
        s, dt = shapes[n]
        assert a.size == int(np.prod(s)) and a.dtype == (np.uint8 if dt == "u8" else np.uint16)


@pytest.mark.parametrize("name,bad", [
    ("model.layers.0.self_attn.q_proj.weight", lambda s: (s[1], s[0])),   # transposed
    ("model.layers.1.self_attn.o_proj.weight", lambda s: (s[1], s[0])),   # transposed
    ("model.layers.0.mlp.experts.gate_up_proj_blocks", lambda s: (s[1], s[0], s[2], s[3])),
    ("model.layers.1.mlp.experts.down_proj_scales", lambda s: (s[0] * s[1] * s[2],)),
])
def test_shape_mismatch_of_equal_size_is_rejected(tmp_path, name, bad):
    """A tensor with the right number of elements in the wrong layout (HF's
    q_proj stored transposed, experts in another order, a flattened scale
    tensor) is refused before anything of it reaches the engine."""
    cfg = ne.config_preset("gpt-oss-20b", **dict(TINY, head_dim=32))  # q / o not square
    shape, dt = loader.checkpoint_shapes(cfg)[name]
    assert bad(shape) != shape
    t = torch.zeros(bad(shape), dtype=torch.uint8 if dt == "u8" else torch.bfloat16)
    st.save_file({name: t}, str(tmp_path / "m.safetensors"))
    eng = Recorder(cfg)
    with pytest.raises(ValueError, match="shape"):
        loader.load_checkpoint(eng, str(tmp_path), strict=False)
    assert name not in eng.got


def test_expert_tensor_dtype_is_checked(tmp_path):
    cfg = ne.config_preset("gpt-oss-20b", **TINY)
    name = "model.layers.0.mlp.experts.down_proj_blocks"
    shape, _ = loader.checkpoint_shapes(cfg)[name]
    st.save_file({name: torch.zeros(shape, dtype=torch.float16)}, str(tmp_path / "m.safetensors"))
    with pytest.raises(ValueError, match="uint8"):
        loader.load_checkpoint(Recorder(cfg), str(tmp_path), strict=False)
