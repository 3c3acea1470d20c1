"""neonengine_amd -- ctypes view of the gfx950 gpt-oss token-loop library.

The product is libneon_gptoss.so (hand-written HIP kernels for gfx950 behind
the C-ABI in include/neon_gptoss.h).  This module binds that ABI for Python
callers (tests, bench.py): every call goes straight into the shared library;
there is no Python or CPU fallback, and loading fails loudly when the library
has not been built.

Device memory for the kernel-level entry points comes from torch tensors on
``cuda`` (HIP) devices; only their data pointers cross the boundary.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# NEON_GPTOSS_LIB selects another build of the library (e.g. the host-
# sanitizer build neonengine_amd/_asan/libneon_gptoss.so)
LIB_PATH = os.environ.get("NEON_GPTOSS_LIB") or os.path.join(HERE, "libneon_gptoss.so")

NEON_OK, NEON_EINVAL, NEON_ENOMEM, NEON_EHIP = 0, 1, 2, 3
NEON_ENAN_SCALE, NEON_EKV_FULL, NEON_ERANGE_TOKEN, NEON_ESTATE = 4, 5, 6, 7
STATUS_NAMES = {0: "NEON_OK", 1: "NEON_EINVAL", 2: "NEON_ENOMEM", 3: "NEON_EHIP",
                4: "NEON_ENAN_SCALE", 5: "NEON_EKV_FULL", 6: "NEON_ERANGE_TOKEN",
                7: "NEON_ESTATE"}

# Every symbol include/neon_gptoss.h declares (tests check the exports).
EXPORTS = (
    "neon_config_preset", "neon_ctx_create", "neon_ctx_destroy", "neon_last_error",
    "neon_init_random", "neon_load_tensor", "neon_prefill", "neon_decode",
    "neon_read_tokens", "neon_read_logits", "neon_read_activation", "neon_seq_len",
    "neon_tensor_ptr",
    "neon_mxfp4_dequant", "neon_mxfp4_gemv", "neon_gemv_bf16", "neon_rmsnorm",
    "neon_rope_yarn", "neon_router_topk", "neon_moe_layer", "neon_moe_experts",
    "neon_attn_decode", "neon_set_prefill_mode", "neon_gemm_bf16", "neon_moe_prefill",
    "neon_attn_prefill", "neon_set_sampling", "neon_sample", "neon_set_decode_mode",
    "neon_gemv_bf16_mfma", "neon_device_check", "neon_moe_layer_noalloc",
    "neon_prefill_ragged", "neon_seq_lens", "neon_moe_prefill_mx8", "neon_mx8_quant",
    "neon_rope_table", "neon_moe_layer_workspace", "neon_attn_decode_workspace",
    "neon_attn_decode_counters", "neon_sample_workspace", "neon_moe_prefill_workspace",
    "neon_seq_add", "neon_seq_remove",
)


class NeonError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {msg}")
        self.status = status


class Config(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "n_layers", "hidden", "n_heads", "n_kv_heads", "head_dim",
        "n_experts", "top_k", "intermediate", "vocab",
        "sliding_window", "max_seq", "max_batch")] + [
        (n, C.c_float) for n in ("rope_theta", "rope_factor", "rope_beta_fast", "rope_beta_slow")] + [
        ("rope_orig_max_pos", C.c_int32)] + [
        (n, C.c_float) for n in ("rms_eps", "swiglu_limit", "swiglu_alpha")]

    def as_dict(self):
        return {n: getattr(self, n) for n, _ in self._fields_}


_lib = None
_P, _I, _I64, _U64, _F, _SZ = C.c_void_p, C.c_int, C.c_int64, C.c_uint64, C.c_float, C.c_size_t


def lib():
    """Load libneon_gptoss.so (raises if it is not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m neonengine_amd._build` "
                "(the gfx950 HIP library is required; there is no fallback)")
        # One HIP runtime per process: torch bundles its own libamdhip64 (same
        # soname, libamdhip64.so.7), and a process that loads /opt/rocm's copy
        # through this library first and torch's afterwards holds two runtimes,
        # of which ours then sees no device.  Loading torch first makes the
        # library's libamdhip64.so.7 dependency resolve to torch's copy.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = C.CDLL(LIB_PATH)
        sig = {
            "neon_config_preset": [C.c_char_p, _P],
            "neon_ctx_create": [_P, _I, _P],
            "neon_ctx_destroy": [_P],
            "neon_last_error": [_P],
            "neon_init_random": [_P, _U64, _P],
            "neon_load_tensor": [_P, C.c_char_p, _P, _SZ],
            "neon_prefill": [_P, _P, _I, _I, _P],
            "neon_prefill_ragged": [_P, _P, _P, _I, _P],
            "neon_decode": [_P, _I, _P],
            "neon_read_tokens": [_P, _I, _I, _P, _P],
            "neon_read_logits": [_P, _P, _P],
            "neon_read_activation": [_P, C.c_char_p, _P, _SZ, _P],
            "neon_seq_len": [_P, _P],
            "neon_seq_lens": [_P, _P],
            "neon_seq_add": [_P, _P, _I, _P, _P],
            "neon_seq_remove": [_P, _I, _P],
            "neon_tensor_ptr": [_P, C.c_char_p, _P, _P],
            "neon_mxfp4_dequant": [_P, _P, _I64, _P, _P],
            "neon_mxfp4_gemv": [_P, _P, _P, _P, _P, _I, _I, _I, _P],
            "neon_gemv_bf16": [_P, _P, _P, _P, _I, _I, _I, _P],
            "neon_rmsnorm": [_P, _P, _P, _I, _I, _F, _P],
            "neon_rope_table": [_P, _I, _P, _P],
            "neon_rope_yarn": [_P, _P, _I, _I, _I, _P, _I, _P],
            "neon_router_topk": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P],
            "neon_moe_layer": [_P] * 13 + [_I] * 5 + [_F, _F, _P, _SZ, _P],
            "neon_moe_experts": [_P] * 12 + [_I] * 5 + [_F, _F, _P],
            "neon_attn_decode": [_P] * 6 + [_I] * 6 + [_P, _SZ, _P, _SZ, _P],
            "neon_set_prefill_mode": [_P, _I],
            "neon_gemm_bf16": [_P] * 4 + [_I] * 4 + [_P],
            "neon_moe_prefill": [_P] * 10 + [_I] * 5 + [_F, _F, _P, _SZ, _P],
            "neon_moe_prefill_mx8": [_P] * 10 + [_I] * 5 + [_F, _F, _P, _SZ, _P],
            "neon_mx8_quant": [_P, _I64, _I, _P, _P, _P, _P, _P],
            "neon_attn_prefill": [_P] * 5 + [_I] * 6 + [_P],
            "neon_set_sampling": [_P, _F, _F, _U64],
            "neon_sample": [_P, _I, _I, _F, _F, _U64, _P, _P, _P, _SZ, _P],
            "neon_set_decode_mode": [_P, _I],
            "neon_gemv_bf16_mfma": [_P, _P, _P, _P, _I, _I, _I, _P],
            "neon_device_check": [_P],
            "neon_moe_layer_noalloc": [_P] * 13 + [_I] * 5 + [_F, _F, _P],
        }
        for name, args in sig.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = C.c_int
        # workspace-size queries (size_t results)
        for name, args in {"neon_moe_layer_workspace": [_I] * 4,
                           "neon_attn_decode_workspace": [_I] * 6,
                           "neon_attn_decode_counters": [_I] * 2,
                           "neon_sample_workspace": [_I] * 2,
                           "neon_moe_prefill_workspace": [_I] * 6}.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = _SZ
        L.neon_ctx_destroy.restype = None
        L.neon_last_error.restype = C.c_char_p
        _lib = L
    return _lib


def _check(status: int, ctx=None):
    if status != NEON_OK:
        msg = lib().neon_last_error(ctx)
        raise NeonError(status, msg.decode() if msg else "")


def device_check(stream=None):
    """Synchronise and raise NeonError(NEON_EINVAL) if a kernel-level call on
    the current device saw an expert id outside [0, E) since the last check."""
    _check(lib().neon_device_check(stream))


def config_preset(name: str = "gpt-oss-20b", **overrides) -> Config:
    cfg = Config()
    _check(lib().neon_config_preset(name.encode(), C.byref(cfg)))
    for k, v in overrides.items():
        setattr(cfg, k, v)
    return cfg


def _ptr(t):
    """Device pointer of a torch tensor (None -> NULL)."""
    if t is None:
        return None
    if hasattr(t, "data_ptr"):
        if not t.is_contiguous():
            raise ValueError("tensor must be contiguous")
        return C.c_void_p(t.data_ptr())
    return C.c_void_p(int(t))


def _nbytes(t):
    """Size in bytes of a torch tensor (None -> 0)."""
    if t is None:
        return 0
    return t.numel() * t.element_size()


def _stream(stream):
    if stream is None:
        try:
            import torch
            if torch.cuda.is_available():
                return C.c_void_p(torch.cuda.current_stream().cuda_stream)
        except Exception:
            pass
        return None
    if hasattr(stream, "cuda_stream"):
        return C.c_void_p(stream.cuda_stream)
    return C.c_void_p(int(stream))


# ---------------------------------------------------------------------------
# kernel-level entry points (torch tensors on the HIP device; bf16 tensors may
# be torch.bfloat16 or int16/uint16 views of the bit patterns)
# ---------------------------------------------------------------------------
def mxfp4_dequant(codes, scales, out, stream=None):
    _check(lib().neon_mxfp4_dequant(_ptr(codes), _ptr(scales), scales.numel(), _ptr(out),
                                    _stream(stream)))


def mxfp4_gemv(codes, scales, bias, x, y, N, K, B, stream=None):
    _check(lib().neon_mxfp4_gemv(_ptr(codes), _ptr(scales), _ptr(bias), _ptr(x), _ptr(y),
                                 N, K, B, _stream(stream)))


def gemv_bf16(W, bias, x, y, N, K, B, stream=None):
    _check(lib().neon_gemv_bf16(_ptr(W), _ptr(bias), _ptr(x), _ptr(y), N, K, B,
                                _stream(stream)))


def gemv_bf16_mfma(W, bias, x, y, N, K, B, stream=None):
    _check(lib().neon_gemv_bf16_mfma(_ptr(W), _ptr(bias), _ptr(x), _ptr(y), N, K, B,
                                     _stream(stream)))


def rmsnorm(x, w, out, B, H, eps=1e-5, stream=None):
    _check(lib().neon_rmsnorm(_ptr(x), _ptr(w), _ptr(out), B, H, eps, _stream(stream)))


def rope_table(cfg: Config, n_pos, table, stream=None):
    """table: device fp32 [2][n_pos][head_dim / 2] (cos, then sin)."""
    _check(lib().neon_rope_table(C.byref(cfg), n_pos, _ptr(table), _stream(stream)))


def rope_yarn(x, pos, n_tok, n_heads, head_dim, table, n_pos, stream=None):
    _check(lib().neon_rope_yarn(_ptr(x), _ptr(pos), n_tok, n_heads, head_dim, _ptr(table),
                                n_pos, _stream(stream)))


def _workspace(nbytes, zero=False):
    """A caller-side device buffer of nbytes (torch), for callers that do not
    keep their own workspace; the library itself allocates nothing."""
    import torch
    n = max(int(nbytes), 1)
    return torch.zeros(n, dtype=torch.uint8, device="cuda") if zero else \
        torch.empty(n, dtype=torch.uint8, device="cuda")


def router_topk(x, W, b, idx, score, logits, B, E, H, k, stream=None):
    if logits is None:  # the C-ABI takes the logits buffer from the caller
        logits = _workspace(B * E * 4)
    _check(lib().neon_router_topk(_ptr(x), _ptr(W), _ptr(b), _ptr(idx), _ptr(score),
                                  _ptr(logits), B, E, H, k, _stream(stream)))


def moe_layer_workspace(B, E, I, k):
    return lib().neon_moe_layer_workspace(B, E, I, k)


def moe_layer(x, router_w, router_b, gu_codes, gu_scales, gu_bias, dn_codes, dn_scales,
              dn_bias, residual, out, idx, score, B, E, H, I, k, alpha=1.702, limit=7.0,
              stream=None, workspace=None):
    if workspace is None:
        workspace = _workspace(moe_layer_workspace(B, E, I, k))
    _check(lib().neon_moe_layer(
        _ptr(x), _ptr(router_w), _ptr(router_b), _ptr(gu_codes), _ptr(gu_scales),
        _ptr(gu_bias), _ptr(dn_codes), _ptr(dn_scales), _ptr(dn_bias), _ptr(residual),
        _ptr(out), _ptr(idx), _ptr(score), B, E, H, I, k, alpha, limit, _ptr(workspace),
        _nbytes(workspace), _stream(stream)))


def moe_layer_noalloc(x, router_w, router_b, gu_codes, gu_scales, gu_bias, dn_codes,
                      dn_scales, dn_bias, residual, out, idx, score, B, E, H, I, k,
                      alpha=1.702, limit=7.0, stream=None):
    """neon_moe_layer with its scratch in the library's fixed per-GPU array
    (no allocation; overlapping calls on one GPU race)."""
    _check(lib().neon_moe_layer_noalloc(
        _ptr(x), _ptr(router_w), _ptr(router_b), _ptr(gu_codes), _ptr(gu_scales),
        _ptr(gu_bias), _ptr(dn_codes), _ptr(dn_scales), _ptr(dn_bias), _ptr(residual),
        _ptr(out), _ptr(idx), _ptr(score), B, E, H, I, k, alpha, limit, _stream(stream)))


def moe_experts(x, idx, score, gu_codes, gu_scales, gu_bias, dn_codes, dn_scales, dn_bias,
                residual, out, act, B, E, H, I, k, alpha=1.702, limit=7.0, stream=None):
    _check(lib().neon_moe_experts(
        _ptr(x), _ptr(idx), _ptr(score), _ptr(gu_codes), _ptr(gu_scales), _ptr(gu_bias),
        _ptr(dn_codes), _ptr(dn_scales), _ptr(dn_bias), _ptr(residual), _ptr(out), _ptr(act),
        B, E, H, I, k, alpha, limit, _stream(stream)))


def attn_decode_workspace(B, Hq, Hkv, D, T_max, window):
    """(workspace bytes, counter bytes) of neon_attn_decode."""
    L = lib()
    return (L.neon_attn_decode_workspace(B, Hq, Hkv, D, T_max, window),
            L.neon_attn_decode_counters(B, Hkv))


def attn_decode(q, k_cache, v_cache, sinks, pos, out, B, Hq, Hkv, D, T_max, window,
                stream=None, workspace=None, counters=None):
    """counters: zero-filled once by the caller (each call leaves it zero)."""
    wb, cb = attn_decode_workspace(B, Hq, Hkv, D, T_max, window)
    if workspace is None and wb:
        workspace = _workspace(wb)
    if counters is None:
        counters = _workspace(cb, zero=True)
    _check(lib().neon_attn_decode(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(sinks),
                                  _ptr(pos), _ptr(out), B, Hq, Hkv, D, T_max, window,
                                  _ptr(workspace), _nbytes(workspace), _ptr(counters),
                                  _nbytes(counters), _stream(stream)))


def gemm_bf16(A, W, bias, C_, M, N, K, accumulate=False, stream=None):
    _check(lib().neon_gemm_bf16(_ptr(A), _ptr(W), _ptr(bias), _ptr(C_), M, N, K,
                                1 if accumulate else 0, _stream(stream)))


def moe_prefill_workspace(M, E, H, I, k, mx8=False):
    return lib().neon_moe_prefill_workspace(M, E, H, I, k, 1 if mx8 else 0)


def moe_prefill(x, idx, score, gu_codes, gu_scales, gu_bias, dn_codes, dn_scales, dn_bias,
                h, M, E, H, I, k, alpha=1.702, limit=7.0, stream=None, workspace=None):
    if workspace is None:
        workspace = _workspace(moe_prefill_workspace(M, E, H, I, k))
    _check(lib().neon_moe_prefill(
        _ptr(x), _ptr(idx), _ptr(score), _ptr(gu_codes), _ptr(gu_scales), _ptr(gu_bias),
        _ptr(dn_codes), _ptr(dn_scales), _ptr(dn_bias), _ptr(h), M, E, H, I, k, alpha, limit,
        _ptr(workspace), _nbytes(workspace), _stream(stream)))


def moe_prefill_mx8(x, idx, score, gu_codes, gu_scales, gu_bias, dn_codes, dn_scales, dn_bias,
                    h, M, E, H, I, k, alpha=1.702, limit=7.0, stream=None, workspace=None):
    if workspace is None:
        workspace = _workspace(moe_prefill_workspace(M, E, H, I, k, mx8=True))
    _check(lib().neon_moe_prefill_mx8(
        _ptr(x), _ptr(idx), _ptr(score), _ptr(gu_codes), _ptr(gu_scales), _ptr(gu_bias),
        _ptr(dn_codes), _ptr(dn_scales), _ptr(dn_bias), _ptr(h), M, E, H, I, k, alpha, limit,
        _ptr(workspace), _nbytes(workspace), _stream(stream)))


def mx8_quant(x, rows, K, hi, lo, s_hi, s_lo, stream=None):
    _check(lib().neon_mx8_quant(_ptr(x), rows, K, _ptr(hi), _ptr(lo), _ptr(s_hi), _ptr(s_lo),
                                _stream(stream)))


def attn_prefill(q, k_cache, v_cache, sinks, out, M, Hq, Hkv, D, T_max, window, stream=None):
    _check(lib().neon_attn_prefill(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(sinks),
                                   _ptr(out), M, Hq, Hkv, D, T_max, window, _stream(stream)))


def sample_workspace(B, V):
    return lib().neon_sample_workspace(B, V)


def sample_logits(logits, B, V, temperature, top_p, seed, pos, out_ids, stream=None,
                  workspace=None):
    if workspace is None:
        workspace = _workspace(sample_workspace(B, V))
    _check(lib().neon_sample(_ptr(logits), B, V, temperature, top_p, seed, _ptr(pos),
                             _ptr(out_ids), _ptr(workspace), _nbytes(workspace),
                             _stream(stream)))


PREFILL_BATCHED, PREFILL_STEPWISE, PREFILL_CHUNKED, PREFILL_MX8 = 0, 1, 2, 3
DECODE_EXACT, DECODE_MATRIX, DECODE_MATRIX_MX8 = 0, 1, 2


# ---------------------------------------------------------------------------
# context-level API
# ---------------------------------------------------------------------------
class Engine:
    """One model context on one device (weights, KV cache, captured step)."""

    def __init__(self, cfg: Config | str = "gpt-oss-20b", device: int = 0, **overrides):
        if isinstance(cfg, str):
            cfg = config_preset(cfg, **overrides)
        self.cfg = cfg
        self._ctx = C.c_void_p()
        _check(lib().neon_ctx_create(C.byref(cfg), device, C.byref(self._ctx)))
        self.batch = 0

    def close(self):
        if self._ctx:
            lib().neon_ctx_destroy(self._ctx)
            self._ctx = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _chk(self, status):
        _check(status, self._ctx)

    def init_random(self, seed: int = 0, stream=None):
        self._chk(lib().neon_init_random(self._ctx, seed, _stream(stream)))

    def load_tensor(self, name: str, data):
        """data: bytes, memoryview or a C-contiguous numpy array (read in place)."""
        import numpy as np
        a = np.frombuffer(data, dtype=np.uint8) if not isinstance(data, np.ndarray) else data
        if not a.flags.c_contiguous:
            raise ValueError(f"load_tensor({name!r}): data must be contiguous")
        self._chk(lib().neon_load_tensor(self._ctx, name.encode(), C.c_void_p(a.ctypes.data),
                                         a.nbytes))

    def load_checkpoint(self, path: str, strict: bool = True) -> int:
        """Loads a local gpt-oss safetensors checkpoint (file or directory)."""
        from .loader import load_checkpoint
        return load_checkpoint(self, path, strict=strict)

    def tensor_ptr(self, name: str):
        p, n = C.c_void_p(), C.c_size_t()
        self._chk(lib().neon_tensor_ptr(self._ctx, name.encode(), C.byref(p), C.byref(n)))
        return p.value, n.value

    def set_decode_mode(self, mode: int):
        """DECODE_EXACT (default: batched steps bit-identical to batch 1) or
        DECODE_MATRIX (steps of 2+ sequences on the matrix cores; equal to
        the exact steps up to the order of fp32 additions)."""
        self._chk(lib().neon_set_decode_mode(self._ctx, mode))

    def set_prefill_mode(self, mode: int):
        """PREFILL_CHUNKED (default: 16 prompt rows per pass), PREFILL_STEPWISE
        (every prompt token as a decode step) or PREFILL_BATCHED (all prompt rows at
        once on the matrix cores; equal to the others up to bf16 rounding)."""
        self._chk(lib().neon_set_prefill_mode(self._ctx, mode))

    def set_sampling(self, temperature: float = 0.0, top_p: float = 1.0, seed: int = 0):
        """temperature 0: greedy; else softmax(logits / temperature) within the
        top-p nucleus, reproducible for a given seed."""
        self._chk(lib().neon_set_sampling(self._ctx, temperature, top_p, seed))

    def prefill(self, ids, stream=None):
        """ids: nested list / array [batch][n_tokens] of int, or a list of
        prompts of different lengths (neon_prefill_ragged)."""
        import numpy as np
        if isinstance(ids, (list, tuple)) and ids and not np.isscalar(ids[0]) and \
                len({len(p) for p in ids}) > 1:
            return self.prefill_ragged(ids, stream)
        a = np.ascontiguousarray(ids, dtype=np.int32)
        if a.ndim == 1:
            a = a[None, :]
        self._chk(lib().neon_prefill(self._ctx, a.ctypes.data_as(C.c_void_p), a.shape[0],
                                     a.shape[1], _stream(stream)))
        self.batch = a.shape[0]

    def prefill_ragged(self, prompts, stream=None):
        """prompts: one sequence of int ids per sequence, lengths free."""
        import numpy as np
        lens = np.ascontiguousarray([len(p) for p in prompts], dtype=np.int32)
        flat = np.ascontiguousarray(np.concatenate([np.asarray(p, np.int64) for p in prompts])
                                    if len(prompts) else np.zeros(0), dtype=np.int32)
        self._chk(lib().neon_prefill_ragged(self._ctx, flat.ctypes.data_as(C.c_void_p),
                                            lens.ctypes.data_as(C.c_void_p), len(prompts),
                                            _stream(stream)))
        self.batch = len(prompts)

    def seq_add(self, prompt, stream=None) -> int:
        """A sequence joins the running batch (neon_seq_add): returns its row."""
        import numpy as np
        ids = np.ascontiguousarray(prompt, dtype=np.int32)
        slot = C.c_int(-1)
        self._chk(lib().neon_seq_add(self._ctx, ids.ctypes.data_as(C.c_void_p), len(ids),
                                     C.byref(slot), _stream(stream)))
        self.batch = max(self.batch, slot.value + 1)
        return slot.value

    def seq_remove(self, slot: int, stream=None):
        """A sequence leaves (neon_seq_remove): its row and KV block are free;
        free rows at the end of the batch leave it."""
        import numpy as np
        held = self.seq_lens() if self.batch else np.zeros(0, np.int32)
        self._chk(lib().neon_seq_remove(self._ctx, slot, _stream(stream)))
        held[slot] = 0
        nz = np.nonzero(held)[0]
        self.batch = int(nz[-1]) + 1 if len(nz) else 0

    def seq_lens(self):
        """Tokens held by each sequence (prompt + generated), int32 [batch]."""
        import numpy as np
        out = np.empty(max(self.batch, 1), np.int32)
        self._chk(lib().neon_seq_lens(self._ctx, out.ctypes.data_as(C.c_void_p)))
        return out[:self.batch]

    def decode(self, n_steps: int, stream=None):
        self._chk(lib().neon_decode(self._ctx, n_steps, _stream(stream)))

    def seq_len(self) -> int:
        n = C.c_int()
        self._chk(lib().neon_seq_len(self._ctx, C.byref(n)))
        return n.value

    def read_tokens(self, start=0, count=None, stream=None):
        import numpy as np
        if count is None:
            count = self.seq_len() - start
        out = np.empty((self.batch, count), np.int32)
        self._chk(lib().neon_read_tokens(self._ctx, start, count,
                                         out.ctypes.data_as(C.c_void_p), _stream(stream)))
        return out

    def read_activation(self, name: str, stream=None):
        """One activation buffer of the last step (see neon_read_activation)."""
        import numpy as np
        c = self.cfg
        if name == "mx_route":
            S = min(c.n_experts, self.batch * c.top_k)
            out = np.empty(66 * S, np.int32)
            self._chk(lib().neon_read_activation(self._ctx, name.encode(),
                                                 out.ctypes.data_as(C.c_void_p), out.nbytes,
                                                 _stream(stream)))
            return out
        if name == "mx_items":  # count, then up to 256 packed work items
            out = np.empty(257, np.int32)
            self._chk(lib().neon_read_activation(self._ctx, name.encode(),
                                                 out.ctypes.data_as(C.c_void_p), out.nbytes,
                                                 _stream(stream)))
            return out
        width = {"hidden": c.hidden, "moe_in": c.hidden, "moe_idx": c.top_k,
                 "moe_score": c.top_k, "qkv": (c.n_heads + 2 * c.n_kv_heads) * c.head_dim,
                 "attn_out": c.n_heads * c.head_dim}[name]
        dt = {"moe_idx": np.int32, "moe_score": np.float32}.get(name, np.uint16)
        out = np.empty((self.batch, width), dt)
        self._chk(lib().neon_read_activation(self._ctx, name.encode(),
                                             out.ctypes.data_as(C.c_void_p), out.nbytes,
                                             _stream(stream)))
        return out

    def read_hidden(self, stream=None):
        return self.read_activation("hidden", stream)

    def read_logits(self, stream=None):
        import numpy as np
        out = np.empty((self.batch, self.cfg.vocab), np.float32)
        self._chk(lib().neon_read_logits(self._ctx, out.ctypes.data_as(C.c_void_p),
                                         _stream(stream)))
        return out
