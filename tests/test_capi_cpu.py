"""C-ABI checks that need no GPU: the library loads, exports every symbol the
header declares, and rejects bad arguments on the host before touching a
device (status codes of include/neon_gptoss.h)."""
import ctypes as C
import os
import re

import pytest

import neonengine_amd as ne

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, "include", "neon_gptoss.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(neon_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_header_symbol():
    L = ne.lib()
    declared = header_functions()
    assert declared, "no declarations parsed"
    assert sorted(ne.EXPORTS) == declared
    for name in declared:
        assert hasattr(L, name), name


def test_presets():
    c = ne.config_preset("gpt-oss-20b")
    assert (c.n_layers, c.hidden, c.n_heads, c.n_kv_heads, c.head_dim) == (24, 2880, 64, 8, 64)
    assert (c.n_experts, c.top_k, c.intermediate, c.vocab) == (32, 4, 2880, 201088)
    assert c.sliding_window == 128 and abs(c.rope_theta - 150000.0) < 1e-3
    c2 = ne.config_preset("gpt-oss-120b")
    assert (c2.n_layers, c2.n_experts) == (36, 128)
    with pytest.raises(ne.NeonError) as e:
        ne.config_preset("llama")
    assert e.value.status == ne.NEON_EINVAL


@pytest.mark.parametrize("field,value", [
    ("head_dim", 128), ("hidden", 100), ("n_kv_heads", 3), ("top_k", 0), ("top_k", 40),
    ("n_experts", 1000), ("max_batch", 0), ("max_seq", 0), ("rms_eps", 0.0),
    ("intermediate", 33), ("n_heads", 12),
])
def test_ctx_create_rejects_bad_config(field, value):
    cfg = ne.config_preset("gpt-oss-20b")
    setattr(cfg, field, value)
    ctx = C.c_void_p()
    st = ne.lib().neon_ctx_create(C.byref(cfg), 0, C.byref(ctx))
    assert st == ne.NEON_EINVAL
    assert not ctx.value
    assert ne.lib().neon_last_error(None)


def test_ctx_create_null_args():
    assert ne.lib().neon_ctx_create(None, 0, None) == ne.NEON_EINVAL


def test_context_calls_reject_null_context():
    L = ne.lib()
    assert L.neon_init_random(None, 0, None) == ne.NEON_EINVAL
    assert L.neon_load_tensor(None, b"lm_head.weight", None, 0) == ne.NEON_EINVAL
    assert L.neon_prefill(None, None, 1, 1, None) == ne.NEON_EINVAL
    assert L.neon_decode(None, 1, None) == ne.NEON_EINVAL
    assert L.neon_read_tokens(None, 0, 1, None, None) == ne.NEON_EINVAL
    assert L.neon_read_logits(None, None, None) == ne.NEON_EINVAL
    assert L.neon_read_activation(None, b"hidden", None, 0, None) == ne.NEON_EINVAL
    assert L.neon_seq_len(None, None) == ne.NEON_EINVAL
    assert L.neon_prefill_ragged(None, None, None, 1, None) == ne.NEON_EINVAL
    assert L.neon_seq_lens(None, None) == ne.NEON_EINVAL
    assert L.neon_set_sampling(None, 1.0, 0.9, 0) == ne.NEON_EINVAL
    L.neon_ctx_destroy(None)  # no-op


def test_kernel_entry_points_validate_on_host():
    L = ne.lib()
    p = C.c_void_p(16)  # never dereferenced: validation fails first
    assert L.neon_sample(None, 1, 8, 1.0, 1.0, 0, p, p, p, 1 << 20, None) == ne.NEON_EINVAL
    assert L.neon_sample(p, 1, 8, 0.0, 1.0, 0, p, p, p, 1 << 20, None) == ne.NEON_EINVAL   # temperature
    assert L.neon_sample(p, 1, 8, 1.0, 0.0, 0, p, p, p, 1 << 20, None) == ne.NEON_EINVAL   # top_p
    assert L.neon_sample(p, 1, 8, 1.0, 1.5, 0, p, p, p, 1 << 20, None) == ne.NEON_EINVAL
    assert L.neon_sample(p, 0, 8, 1.0, 1.0, 0, p, p, p, 1 << 20, None) == ne.NEON_EINVAL
    assert L.neon_mxfp4_gemv(None, p, None, p, p, 8, 64, 1, None) == ne.NEON_EINVAL
    assert L.neon_mxfp4_gemv(p, p, None, p, p, 8, 48, 1, None) == ne.NEON_EINVAL   # K % 32
    assert L.neon_mxfp4_gemv(p, p, None, p, p, 0, 64, 1, None) == ne.NEON_EINVAL
    assert L.neon_mxfp4_gemv(p, p, None, p, p, 8, 16384, 1, None) == ne.NEON_EINVAL
    assert L.neon_gemv_bf16(p, None, p, p, 8, 12, 1, None) == ne.NEON_EINVAL       # K % 8
    assert L.neon_gemv_bf16_mfma(p, None, p, p, 24, 64, 1, None) == ne.NEON_EINVAL  # N % 16
    assert L.neon_gemv_bf16_mfma(p, None, p, p, 32, 48, 1, None) == ne.NEON_EINVAL  # K % 32
    assert L.neon_gemv_bf16_mfma(p, None, p, p, 32, 8192, 1, None) == ne.NEON_EINVAL  # K > 4096
    assert L.neon_gemv_bf16_mfma(p, None, p, p, 32, 64, 65, None) == ne.NEON_EINVAL  # B > 64
    assert L.neon_gemv_bf16_mfma(None, None, p, p, 32, 64, 1, None) == ne.NEON_EINVAL
    assert L.neon_rmsnorm(p, p, p, 1, 2880, 0.0, None) == ne.NEON_EINVAL
    assert L.neon_router_topk(p, p, p, p, p, None, 1, 32, 2880, 40, None) == ne.NEON_EINVAL
    assert L.neon_moe_layer(*([p] * 9), None, p, None, None, 1, 32, 2880, 2880, 0, 1.702, 7.0,
                            p, 1 << 30, None) == ne.NEON_EINVAL
    # a workspace smaller than neon_moe_layer_workspace's figure
    need = L.neon_moe_layer_workspace(1, 32, 2880, 4)
    assert need >= 4 * 2880 * 2 + 32 * 4
    assert L.neon_moe_layer(*([p] * 9), None, p, None, None, 1, 32, 2880, 2880, 4, 1.702, 7.0,
                            p, need - 1, None) == ne.NEON_EINVAL
    assert L.neon_moe_layer(*([p] * 9), None, p, None, None, 1, 32, 2880, 2880, 4, 1.702, 7.0,
                            None, need, None) == ne.NEON_EINVAL
    assert L.neon_attn_decode(p, p, p, p, p, p, 1, 64, 8, 128, 64, 0, p, 1 << 30, p, 1 << 30,
                              None) == ne.NEON_EINVAL  # D
    assert L.neon_attn_decode(p, p, p, p, p, p, 1, 64, 5, 64, 64, 0, p, 1 << 30, p, 1 << 30,
                              None) == ne.NEON_EINVAL  # Hq % Hkv
    # split partials and arrival counters sized by the queries: one split
    # (the 128-key window) needs neither, 32 splits need both
    assert L.neon_attn_decode_workspace(4, 64, 8, 64, 32768, 128) == 0
    ws = L.neon_attn_decode_workspace(4, 64, 8, 64, 32768, 0)
    assert ws == 4 * 64 * 32 * 66 * 4
    cn = L.neon_attn_decode_counters(4, 8)
    assert cn >= 4 * 8 * 4
    assert L.neon_attn_decode(p, p, p, p, p, p, 4, 64, 8, 64, 32768, 0, p, ws - 4, p, cn,
                              None) == ne.NEON_EINVAL
    assert L.neon_attn_decode(p, p, p, p, p, p, 4, 64, 8, 64, 32768, 0, p, ws, p, cn - 4,
                              None) == ne.NEON_EINVAL
    assert L.neon_attn_decode(p, p, p, p, p, p, 4, 64, 8, 64, 32768, 0, None, ws, p, cn,
                              None) == ne.NEON_EINVAL
    assert L.neon_sample_workspace(3, 1000) == 3 * 1000 * 4
    assert L.neon_sample(p, 3, 1000, 1.0, 0.9, 0, p, p, p, 3 * 1000 * 4 - 4,
                         None) == ne.NEON_EINVAL
    assert L.neon_router_topk(p, p, p, p, p, None, 1, 32, 2880, 4, None) == ne.NEON_EINVAL
    assert L.neon_gemm_bf16(None, p, None, p, 8, 8, 64, 0, None) == ne.NEON_EINVAL
    assert L.neon_gemm_bf16(p, p, None, p, 8, 8, 48, 0, None) == ne.NEON_EINVAL     # K % 32
    assert L.neon_gemm_bf16(p, p, None, p, 0, 8, 64, 0, None) == ne.NEON_EINVAL
    assert L.neon_moe_prefill(*([p] * 10), 4, 32, 2880, 2880, 0, 1.702, 7.0, p, 1 << 30,
                              None) == ne.NEON_EINVAL                              # k = 0
    assert L.neon_moe_prefill(*([p] * 10), 4, 32, 2880, 2872, 4, 1.702, 7.0, p, 1 << 30,
                              None) == ne.NEON_EINVAL                              # I % 32
    need = L.neon_moe_prefill_workspace(64, 32, 2880, 2880, 4, 0)
    need8 = L.neon_moe_prefill_workspace(64, 32, 2880, 2880, 4, 1)
    assert need >= 64 * 4 * 2880 * 4 and need8 > need
    assert L.neon_moe_prefill_workspace(64, 32, 2880, 2880, 4, 1) == need8
    assert L.neon_moe_prefill(*([p] * 10), 64, 32, 2880, 2880, 4, 1.702, 7.0, p, need - 1,
                              None) == ne.NEON_EINVAL
    assert L.neon_attn_prefill(p, p, p, p, p, 16, 64, 8, 128, 64, 0, None) == ne.NEON_EINVAL  # D
    assert L.neon_attn_prefill(p, p, p, p, p, 65, 64, 8, 64, 64, 0, None) == ne.NEON_EINVAL   # T_max < M
    # the allocation-free MoE layer: same shape checks, plus its fixed 4 MiB
    # scratch (B = 200 rows of 4 x 2880 activations need 4.6 MB); rejected on
    # the host before any device call
    assert L.neon_moe_layer_noalloc(*([p] * 9), None, p, None, None, 1, 32, 2880, 2880, 0,
                                    1.702, 7.0, None) == ne.NEON_EINVAL
    assert L.neon_moe_layer_noalloc(*([p] * 9), None, p, None, None, 200, 32, 2880, 2880, 4,
                                    1.702, 7.0, None) == ne.NEON_EINVAL
    assert b"scratch" in L.neon_last_error(None)
    assert L.neon_set_prefill_mode(None, 0) == ne.NEON_EINVAL
    assert L.neon_mxfp4_dequant(None, p, 1, p, None) == ne.NEON_EINVAL
    assert L.neon_mxfp4_dequant(p, p, 0, p, None) == ne.NEON_OK  # empty is a no-op
    assert b"K" in L.neon_last_error(None) or L.neon_last_error(None)


def test_no_device_reports_ehip():
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    cfg = ne.config_preset("gpt-oss-20b")
    ctx = C.c_void_p()
    assert ne.lib().neon_ctx_create(C.byref(cfg), 0, C.byref(ctx)) == ne.NEON_EHIP
    assert b"device" in ne.lib().neon_last_error(None)


def test_cpp_host_program_reports_no_device():
    """tests/cpp/engine_greedy (neon::Engine over the C-ABI) builds with g++
    and, without a GPU, fails at construction with neon::Error(NEON_EHIP)."""
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is present (tests/test_gpu_cpp_host.py runs it)")
    import subprocess
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "tests", "cpp")], check=True)
    r = subprocess.run([os.path.join(ROOT, "tests", "cpp", "engine_greedy"), "small", "2", "1"],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 3, (r.stdout, r.stderr)
    assert "neon::Error 3" in r.stderr and "device" in r.stderr


def test_engine_header_is_self_contained_cpp(tmp_path):
    """include/neon_engine.hpp compiles standalone against the C header."""
    import shutil
    import ast
    import subprocess
    gxx = shutil.which("g++")
    if not gxx:
        pytest.skip("no g++")
    src = tmp_path / "t.cpp"
    src.write_text('#include "neon_engine.hpp"\nint main(){ neon::Config c = neon::Config::preset("gpt-oss-20b"); return c.raw().n_layers == 24 ? 0 : 1; }\n')
    r = subprocess.run([gxx, "-std=c++17", "-fsyntax-only", "-I", os.path.join(ROOT, "include"),
                        str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_one_hip_runtime_per_process():
    """Loading the library before torch must not map a second HIP runtime:
    torch bundles libamdhip64.so.7 under its own path, and a process holding
    both copies sees no device through the library's."""
    import ast
    import subprocess
    import sys
    pytest.importorskip("torch")
    code = ("import neonengine_amd as ne; ne.lib(); import torch; "
            "print(sorted({l.split()[-1] for l in open('/proc/self/maps') "
            "if 'libamdhip64' in l or 'libhsa-runtime64' in l}))")
    out = subprocess.run([sys.executable, "-c", code], cwd=ROOT, capture_output=True,
                         text=True, timeout=300, check=True).stdout
    maps = ast.literal_eval(out.strip().splitlines()[-1])
    assert sum("libamdhip64" in m for m in maps) == 1, maps
    assert sum("libhsa-runtime64" in m for m in maps) == 1, maps


def test_kernel_tier_allocates_nothing():
    """No kernel-level entry point allocates device memory: the library's
    sources hold no stream-ordered allocation at all, and every hipMalloc
    fills a member of the context (weights, KV cache, work and prompt
    buffers, the matrix-core copies), allocated at set-up like the
    reference's System buffers.  The kernel tier's scratch is caller-owned
    (the *_workspace queries) and its status word a file-scope device array."""
    import re
    src = os.path.join(ROOT, "neonengine_amd", "csrc")
    for name in os.listdir(src):
        text = open(os.path.join(src, name)).read()
        assert "hipMallocAsync" not in text and "hipFreeAsync" not in text, name
        for m in re.finditer(r"hipMalloc\(([^,]*),", text):
            assert m.group(1).strip().startswith("&ctx->"), (name, m.group(0))
