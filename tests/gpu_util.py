"""Helpers for the GPU parity tests (device memory via torch, raw copies via
the HIP runtime)."""
import ctypes as C

import numpy as np
import pytest

_hip = None


def torch_cuda():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch


def to_dev(a):
    torch = torch_cuda()
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).to("cuda")


def empty_dev(shape, dtype):
    torch = torch_cuda()
    tmap = {np.uint16: torch.int16, np.uint8: torch.uint8, np.float32: torch.float32,
            np.int32: torch.int32}
    return torch.empty(shape, dtype=tmap[dtype], device="cuda")


def to_host(t, dtype=None):
    torch = torch_cuda()
    torch.cuda.synchronize()
    a = t.cpu().numpy()
    if a.dtype == np.int16:
        a = a.view(np.uint16)
    return a if dtype is None else a.view(dtype)


def d2h(ptr, nbytes, dtype):
    """Copy nbytes from a raw device pointer into a numpy array."""
    global _hip
    if _hip is None:
        import neonengine_amd as ne
        ne.lib()  # torch first, then the library: their HIP runtime is this one
        _hip = C.CDLL("libamdhip64.so.7")
        _hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        _hip.hipMemcpy.restype = C.c_int
    out = np.empty(nbytes // np.dtype(dtype).itemsize, dtype)
    rc = _hip.hipMemcpy(out.ctypes.data_as(C.c_void_p), C.c_void_p(ptr), nbytes, 2)  # D2H
    assert rc == 0, rc
    return out


def fix_routing(eng, cfg):
    """Router weights 0 and distinct biases: every row of layer l picks the
    same 4 experts, so no near-tied router logit can flip between modes."""
    E = cfg.n_experts
    for layer in range(cfg.n_layers):
        p = f"model.layers.{layer}.mlp.router."
        eng.load_tensor(p + "weight", np.zeros(E * cfg.hidden, np.uint16))
        bias = np.array([1.0 - 0.25 * ((e + 3 * layer) % E) for e in range(E)], np.float32)
        eng.load_tensor(p + "bias", (bias.view(np.uint32) >> 16).astype(np.uint16))  # exact


def bf16_err_ok(gpu_bf16, ref_f32, abs_sum, k_eps=2.0 ** -17):
    """|gpu - ref| <= one bf16 rounding of ref + fp32-accumulation slack."""
    from oracle import oracle as orc
    g = orc.bf16_to_f32(gpu_bf16).astype(np.float64)
    r = ref_f32.astype(np.float64)
    bound = np.abs(r) * 2.0 ** -8 + k_eps * abs_sum + 1e-30
    return np.abs(g - r) <= bound, np.abs(g - r) / np.maximum(bound, 1e-30)
