"""ctypes view of the CPU oracle (oracle/libneon_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py as the checker.  The product never imports it.

Every function takes and returns numpy arrays; bf16 tensors travel as uint16
bit patterns.  See neon_oracle.h for the semantics and what pins each one.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# NEON_ORACLE_LIB selects another build (the host-sanitizer build in _asan/)
_LIB_PATH = os.environ.get("NEON_ORACLE_LIB") or os.path.join(_HERE, "libneon_oracle.so")


def build() -> None:
    """Compile the oracle with its Makefile (gcc, seconds)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _load():
    if not os.path.exists(_LIB_PATH):
        raise RuntimeError(
            f"{_LIB_PATH} is not built; run `make -C oracle` (or __graft_entry__.build())")
    return C.CDLL(_LIB_PATH)


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load()
        _declare(_lib)
    return _lib


class OrConfig(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "n_layers", "hidden", "n_heads", "n_kv_heads", "head_dim",
        "n_experts", "top_k", "intermediate", "vocab",
        "sliding_window", "max_seq", "max_batch")] + [
        (n, C.c_float) for n in ("rope_theta", "rope_factor", "rope_beta_fast", "rope_beta_slow")] + [
        ("rope_orig_max_pos", C.c_int32)] + [
        (n, C.c_float) for n in ("rms_eps", "swiglu_limit", "swiglu_alpha")]


GPT_OSS_20B = dict(n_layers=24, hidden=2880, n_heads=64, n_kv_heads=8, head_dim=64,
                   n_experts=32, top_k=4, intermediate=2880, vocab=201088,
                   sliding_window=128, max_seq=4096, max_batch=1,
                   rope_theta=150000.0, rope_factor=32.0, rope_beta_fast=32.0,
                   rope_beta_slow=1.0, rope_orig_max_pos=4096, rms_eps=1e-5,
                   swiglu_limit=7.0, swiglu_alpha=1.702)
GPT_OSS_120B = dict(GPT_OSS_20B, n_layers=36, n_experts=128)


def make_config(**kw) -> OrConfig:
    d = dict(GPT_OSS_20B)
    d.update(kw)
    return OrConfig(**d)


# tensor kinds (match OR_T_* / the product's init streams)
T_ATTN_NORM, T_WQKV, T_BQKV, T_WO, T_BO, T_SINKS, T_MLP_NORM = 0, 1, 2, 3, 4, 5, 6
T_ROUTER_W, T_ROUTER_B, T_GU_CODES, T_GU_SCALES, T_GU_BIAS = 7, 8, 9, 10, 11
T_DN_CODES, T_DN_SCALES, T_DN_BIAS = 12, 13, 14
T_EMBED, T_LM_HEAD, T_FINAL_NORM = 100, 101, 102

_P = C.c_void_p
_I = C.c_int
_I64 = C.c_int64
_U64 = C.c_uint64
_F = C.c_float
_D = C.c_double


def _declare(L):
    sig = {
        "or_hash": (_U64, [_U64, _U64, _U64]),
        "or_gauss_mul": (_F, [_D]),
        "or_fill_bf16": (None, [_U64, _U64, _I64, _F, _D, _P]),
        "or_fill_bytes": (None, [_U64, _U64, _I64, _P]),
        "or_fill_scales": (None, [_U64, _U64, _I64, _I, _I, _P]),
        "or_stream_id": (_U64, [_I, _I]),
        "or_bf16_to_f32": (_F, [C.c_uint16]),
        "or_f32_to_bf16": (C.c_uint16, [_F]),
        "or_mxfp4_dequant": (None, [_P, _P, _I64, _P]),
        "or_e4m3_decode": (_F, [C.c_uint8]),
        "or_e4m3_encode": (C.c_uint8, [_F]),
        "or_ilog2f": (_I, [_F]),
        "or_mx8_quant": (None, [_P, _I64, _I, _P, _P, _P, _P]),
        "or_mxfp4_gemv": (None, [_P, _P, _P, _P, _I, _I, _I, _P, _P]),
        "or_gemv_bf16": (None, [_P, _P, _P, _I, _I, _I, _P, _P]),
        "or_rmsnorm": (None, [_P, _P, _I, _I, _F, _P]),
        "or_yarn_inv_freq": (None, [_P, _P, _P]),
        "or_rope_table": (None, [_P, _I, _P, _P]),
        "or_rope_apply": (None, [_P, _I, _I, _P, _P, _P]),
        "or_router": (None, [_P, _P, _P, _I, _I, _I, _I, _P, _P, _P]),
        "or_swiglu": (None, [_P, _I, _F, _F, _P]),
        "or_moe_layer": (None, [_P] * 9 + [_I] * 5 + [_F, _F, _P, _P, _P]),
        "or_moe_experts": (None, [_P] * 9 + [_I] * 5 + [_F, _F, _P]),
        "or_attn_decode": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _I, _P, _P]),
        "or_model_create": (_P, [_P, _U64, _I]),
        "or_model_create_ex": (_P, [_P, _U64, _I, _I]),
        "or_model_fill_kv": (None, [_P, _I, _U64]),
        "or_model_set_tensor": (_I, [_P, _I, _I, _P, C.c_size_t]),
        "or_set_accumulation": (None, [_I]),
        "or_fill_bytes_at": (None, [_U64, _U64, _I64, _I64, _P]),
        "or_fill_scales_at": (None, [_U64, _U64, _I64, _I64, _I, _I, _P]),
        "or_model_free": (None, [_P]),
        "or_model_step": (None, [_P, _P, _P, _P]),
        "or_model_prompt": (None, [_P, _P, C.c_int]),
        "or_sample": (None, [_P, _I, _I, _F, _F, _U64, _P, _P]),
        "or_model_hidden": (_P, [_P]),
        "or_model_pos": (C.c_int32, [_P, _I]),
        "or_model_tensor": (_P, [_P, _I, _I]),
        "or_num_threads": (_I, []),
        "or_model_trace": (_P, [_P, _I]),
        "or_expf": (_F, [_F]),
        "or_c_gemv_bf16": (None, [_P, _P, _P, _I, _I, _I, _P, _P]),
        "or_c_mxfp4_gemv": (None, [_P, _P, _P, _P, _I, _I, _I, _P, _P]),
        "or_c_rmsnorm": (None, [_P, _P, _I, _I, _F, _P]),
        "or_c_gemv_bf16_ref": (None, [_P, _P, _P, _I, _I, _I, _P, _P]),
        "or_c_mxfp4_gemv_ref": (None, [_P, _P, _P, _P, _I, _I, _I, _P, _P]),
        "or_attn_splits": (_I, [_I, _I]),
        "or_c_attn_decode": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _I, _I, _P, _P]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---- numeric helpers -------------------------------------------------------
def bf16_to_f32(a) -> np.ndarray:
    a = np.asarray(a, dtype=np.uint16)
    return (a.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(a) -> np.ndarray:
    """Round-to-nearest-even (same rule as the oracle and the device)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


# ---- RNG --------------------------------------------------------------------
def hash64(seed, stream, i) -> int:
    return lib().or_hash(seed, stream, i)


def fill_bf16(seed, stream, n, mean=0.0, std=1.0) -> np.ndarray:
    out = np.empty(n, np.uint16)
    lib().or_fill_bf16(seed, stream, n, mean, std, _p(out))
    return out


def fill_bytes(seed, stream, n) -> np.ndarray:
    out = np.empty(n, np.uint8)
    lib().or_fill_bytes(seed, stream, n, _p(out))
    return out


def fill_scales(seed, stream, n, lo=119, rng=6) -> np.ndarray:
    out = np.empty(n, np.uint8)
    lib().or_fill_scales(seed, stream, n, lo, rng, _p(out))
    return out


def fill_bytes_at(seed, stream, start, n) -> np.ndarray:
    out = np.empty(n, np.uint8)
    lib().or_fill_bytes_at(seed, stream, start, n, _p(out))
    return out


def fill_scales_at(seed, stream, start, n, lo=119, rng=6) -> np.ndarray:
    out = np.empty(n, np.uint8)
    lib().or_fill_scales_at(seed, stream, start, n, lo, rng, _p(out))
    return out


def set_accumulation(mode: int) -> None:
    """0: canonical fp32 orders (default); 1: fp64 accumulation (for measuring
    the model's sensitivity to summation order)."""
    lib().or_set_accumulation(mode)


def num_threads() -> int:
    return lib().or_num_threads()


def stream_id(layer, kind) -> int:
    return lib().or_stream_id(layer, kind)


# ---- kernels ----------------------------------------------------------------
def mxfp4_dequant(codes, scales) -> np.ndarray:
    codes = _c(codes, np.uint8)
    scales = _c(scales, np.uint8)
    nb = scales.size
    assert codes.size == nb * 16
    out = np.empty(nb * 32, np.float32)
    lib().or_mxfp4_dequant(_p(codes), _p(scales), nb, _p(out))
    return out


def e4m3_decode(code) -> float:
    return lib().or_e4m3_decode(int(code))


def e4m3_encode(v) -> int:
    return int(lib().or_e4m3_encode(float(v)))


def mx8_quant(x):
    """bf16 bits [rows][K] -> (hi, lo uint8 [rows][K], s_hi, s_lo uint8
    [rows][K/32]): the two-term MXFP8 image of the rows."""
    x = _c(x, np.uint16)
    rows, K = x.shape
    hi, lo = np.empty((rows, K), np.uint8), np.empty((rows, K), np.uint8)
    sh, sl = np.empty((rows, K // 32), np.uint8), np.empty((rows, K // 32), np.uint8)
    lib().or_mx8_quant(_p(x), rows, K, _p(hi), _p(lo), _p(sh), _p(sl))
    return hi, lo, sh, sl


def mx8_dequant(hi, lo, s_hi, s_lo) -> np.ndarray:
    """float64 [rows][K] = dec(hi) 2^(s_hi-127) + dec(lo) 2^(s_lo-127)."""
    table = np.array([lib().or_e4m3_decode(c) for c in range(256)], np.float64)
    sh = np.repeat(np.asarray(s_hi, np.int64), 32, axis=1) - 127
    sl = np.repeat(np.asarray(s_lo, np.int64), 32, axis=1) - 127
    return table[hi] * np.exp2(sh) + table[lo] * np.exp2(sl)


def mxfp4_gemv(codes, scales, bias, x, N, K):
    """x: uint16 [B][K] -> (bf16 [B][N], f32 [B][N])."""
    codes, scales, x = _c(codes, np.uint8), _c(scales, np.uint8), _c(x, np.uint16)
    B = x.size // K
    bias = None if bias is None else _c(bias, np.uint16)
    y = np.empty((B, N), np.uint16)
    yf = np.empty((B, N), np.float32)
    lib().or_mxfp4_gemv(_p(codes), _p(scales), _p(bias), _p(x), B, N, K, _p(y), _p(yf))
    return y, yf


def gemv_bf16(W, bias, x, N, K):
    W, x = _c(W, np.uint16), _c(x, np.uint16)
    B = x.size // K
    bias = None if bias is None else _c(bias, np.uint16)
    y = np.empty((B, N), np.uint16)
    yf = np.empty((B, N), np.float32)
    lib().or_gemv_bf16(_p(W), _p(bias), _p(x), B, N, K, _p(y), _p(yf))
    return y, yf


def rmsnorm(x, w, eps=1e-5):
    x, w = _c(x, np.uint16), _c(w, np.uint16)
    H = w.size
    B = x.size // H
    out = np.empty((B, H), np.uint16)
    lib().or_rmsnorm(_p(x), _p(w), B, H, eps, _p(out))
    return out


def yarn_inv_freq(cfg: OrConfig):
    inv = np.empty(cfg.head_dim // 2, np.float64)
    af = C.c_double()
    lib().or_yarn_inv_freq(C.byref(cfg), _p(inv), C.byref(af))
    return inv, af.value


def rope_table(cfg: OrConfig, n_pos):
    half = cfg.head_dim // 2
    c = np.empty((n_pos, half), np.float32)
    s = np.empty((n_pos, half), np.float32)
    lib().or_rope_table(C.byref(cfg), n_pos, _p(c), _p(s))
    return c, s


def rope_apply(x, n_heads, D, cos_row, sin_row):
    x = _c(x, np.uint16)
    out = np.empty(n_heads * D, np.uint16)
    lib().or_rope_apply(_p(x), n_heads, D, _p(_c(cos_row, np.float32)),
                        _p(_c(sin_row, np.float32)), _p(out))
    return out


def router(x, W, b, E, H, k):
    x, W, b = _c(x, np.uint16), _c(W, np.uint16), _c(b, np.uint16)
    B = x.size // H
    idx = np.empty((B, k), np.int32)
    sc = np.empty((B, k), np.float32)
    lg = np.empty((B, E), np.float32)
    lib().or_router(_p(x), _p(W), _p(b), B, E, H, k, _p(idx), _p(sc), _p(lg))
    return idx, sc, lg


def swiglu(gate_up, alpha=1.702, limit=7.0):
    gu = _c(gate_up, np.float32)
    I = gu.size // 2
    out = np.empty(I, np.float32)
    lib().or_swiglu(_p(gu), I, alpha, limit, _p(out))
    return out


def moe_layer(x, rw, rb, gu_codes, gu_scales, gu_bias, dn_codes, dn_scales, dn_bias,
              E, H, I, k, alpha=1.702, limit=7.0):
    x = _c(x, np.uint16)
    B = x.size // H
    out = np.empty((B, H), np.uint16)
    idx = np.empty((B, k), np.int32)
    sc = np.empty((B, k), np.float32)
    args = [_c(rw, np.uint16), _c(rb, np.uint16), _c(gu_codes, np.uint8),
            _c(gu_scales, np.uint8), _c(gu_bias, np.uint16), _c(dn_codes, np.uint8),
            _c(dn_scales, np.uint8), _c(dn_bias, np.uint16)]
    lib().or_moe_layer(_p(x), *[_p(a) for a in args], B, E, H, I, k, alpha, limit,
                       _p(out), _p(idx), _p(sc))
    return out, idx, sc


def moe_experts(x, idx, score, gu_codes, gu_scales, gu_bias, dn_codes, dn_scales, dn_bias,
                E, H, I, k, alpha=1.702, limit=7.0):
    """Given ids/weights [B][k]; a slot whose id lies outside [0, E) adds nothing."""
    x = _c(x, np.uint16)
    B = x.size // H
    out = np.empty((B, H), np.uint16)
    args = [_c(idx, np.int32), _c(score, np.float32), _c(gu_codes, np.uint8),
            _c(gu_scales, np.uint8), _c(gu_bias, np.uint16), _c(dn_codes, np.uint8),
            _c(dn_scales, np.uint8), _c(dn_bias, np.uint16)]
    lib().or_moe_experts(_p(x), *[_p(a) for a in args], B, E, H, I, k, alpha, limit, _p(out))
    return out


def attn_decode(q, kc, vc, sinks, B, Hq, Hkv, D, T_max, pos, window):
    q, kc, vc, sinks = _c(q, np.uint16), _c(kc, np.uint16), _c(vc, np.uint16), _c(sinks, np.uint16)
    pos = _c(pos, np.int32)
    out = np.empty((B, Hq * D), np.uint16)
    outf = np.empty((B, Hq * D), np.float32)
    lib().or_attn_decode(_p(q), _p(kc), _p(vc), _p(sinks), B, Hq, Hkv, D, T_max,
                         _p(pos), window, _p(out), _p(outf))
    return out, outf


# ---- canonical fp32 forms (bit-identical to the device kernels) -------------
def expf(x: float) -> float:
    return lib().or_expf(x)


def c_gemv_bf16(W, bias, x, N, K):
    W, x = _c(W, np.uint16), _c(x, np.uint16)
    B = x.size // K
    bias = None if bias is None else _c(bias, np.uint16)
    y = np.empty((B, N), np.uint16)
    yf = np.empty((B, N), np.float32)
    lib().or_c_gemv_bf16(_p(W), _p(bias), _p(x), B, N, K, _p(y), _p(yf))
    return y, yf


def c_mxfp4_gemv(codes, scales, bias, x, N, K):
    codes, scales, x = _c(codes, np.uint8), _c(scales, np.uint8), _c(x, np.uint16)
    B = x.size // K
    bias = None if bias is None else _c(bias, np.uint16)
    y = np.empty((B, N), np.uint16)
    yf = np.empty((B, N), np.float32)
    lib().or_c_mxfp4_gemv(_p(codes), _p(scales), _p(bias), _p(x), B, N, K, _p(y), _p(yf))
    return y, yf


def c_gemv_bf16_ref(W, bias, x, N, K):
    """Scalar statement of c_gemv_bf16 (same bits, one lane at a time)."""
    W, x = _c(W, np.uint16), _c(x, np.uint16)
    B = x.size // K
    bias = None if bias is None else _c(bias, np.uint16)
    y = np.empty((B, N), np.uint16)
    yf = np.empty((B, N), np.float32)
    lib().or_c_gemv_bf16_ref(_p(W), _p(bias), _p(x), B, N, K, _p(y), _p(yf))
    return y, yf


def c_mxfp4_gemv_ref(codes, scales, bias, x, N, K):
    """Scalar statement of c_mxfp4_gemv (same bits, one lane at a time)."""
    codes, scales, x = _c(codes, np.uint8), _c(scales, np.uint8), _c(x, np.uint16)
    B = x.size // K
    bias = None if bias is None else _c(bias, np.uint16)
    y = np.empty((B, N), np.uint16)
    yf = np.empty((B, N), np.float32)
    lib().or_c_mxfp4_gemv_ref(_p(codes), _p(scales), _p(bias), _p(x), B, N, K, _p(y), _p(yf))
    return y, yf


def c_rmsnorm(x, w, eps=1e-5):
    x, w = _c(x, np.uint16), _c(w, np.uint16)
    H = w.size
    B = x.size // H
    out = np.empty((B, H), np.uint16)
    lib().or_c_rmsnorm(_p(x), _p(w), B, H, eps, _p(out))
    return out


def attn_splits(T_max, window) -> int:
    return lib().or_attn_splits(T_max, window)


def c_attn_decode(q, kc, vc, sinks, B, Hq, Hkv, D, T_max, pos, window, S=None):
    q, kc, vc, sinks = _c(q, np.uint16), _c(kc, np.uint16), _c(vc, np.uint16), _c(sinks, np.uint16)
    pos = _c(pos, np.int32)
    if S is None:
        S = attn_splits(T_max, window)
    out = np.empty((B, Hq * D), np.uint16)
    outf = np.empty((B, Hq * D), np.float32)
    lib().or_c_attn_decode(_p(q), _p(kc), _p(vc), _p(sinks), B, Hq, Hkv, D, T_max,
                           _p(pos), window, S, _p(out), _p(outf))
    return out, outf


def sample(logits, temperature, top_p, seed, pos):
    """Ids [B] drawn from logits [B][V] in the device's exact order."""
    lg = _c(logits, np.float32)
    B, V = lg.shape
    pos = _c(pos, np.int32).reshape(B)
    out = np.empty(B, np.int32)
    lib().or_sample(_p(lg), B, V, temperature, top_p, seed, _p(pos), _p(out))
    return out


class Model:
    """Random-init gpt-oss model (bit-identical weights to neon_init_random)."""

    LAZY_EXPERTS = 1

    def __init__(self, cfg: OrConfig, seed: int, batch: int = 1, lazy_experts: bool = False):
        """lazy_experts: keep no MXFP4 expert tensors; regenerate the chosen
        experts each step (same bits; needed where the experts exceed host
        memory, e.g. the 120b shape)."""
        self.cfg = cfg
        self.batch = batch
        flags = self.LAZY_EXPERTS if lazy_experts else 0
        self._h = lib().or_model_create_ex(C.byref(cfg), seed, batch, flags)
        if not self._h:
            raise MemoryError("or_model_create failed")

    def close(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.or_model_free(self._h)
        self._h = None

    def __del__(self):
        self.close()

    def step(self, ids, want_logits=True):
        ids = _c(ids, np.int32).reshape(self.batch)
        out = np.empty(self.batch, np.int32)
        lg = np.empty((self.batch, self.cfg.vocab), np.float32) if want_logits else None
        lib().or_model_step(self._h, _p(ids), _p(lg), _p(out))
        return out, lg

    def prompt_step(self, ids):
        """A teacher-forced prompt row for every sequence: fills the KV cache
        at each sequence's position and advances it, without lm_head."""
        ids = _c(ids, np.int32).reshape(self.batch)
        lib().or_model_step(self._h, _p(ids), None, None)

    def prompt(self, ids):
        """Teacher-forced prompt rows ids [B][n] in layer-major order
        (or_model_prompt): the same KV cache, positions and hidden state as
        n prompt_step calls, with each weight row read once per layer."""
        ids = _c(ids, np.int32).reshape(self.batch, -1)
        lib().or_model_prompt(self._h, _p(ids), ids.shape[1])

    def set_tensor(self, layer, kind, data):
        a = np.ascontiguousarray(data)
        if lib().or_model_set_tensor(self._h, layer, kind, _p(a), a.nbytes) != 0:
            raise ValueError(f"set_tensor(layer {layer}, kind {kind}): bad kind or size")

    def fill_kv(self, n_pos, seed=1234):
        """Synthetic N(0,1) KV history at positions 0..n_pos-1 (timing only)."""
        lib().or_model_fill_kv(self._h, n_pos, seed)

    def hidden(self):
        p = lib().or_model_hidden(self._h)
        n = self.batch * self.cfg.hidden
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint16)), shape=(n,)).copy()

    def trace(self):
        """Last step's last-layer activations of row 0 (same names as
        neon_read_activation)."""
        c = self.cfg
        qkv = (c.n_heads + 2 * c.n_kv_heads) * c.head_dim

        def arr(what, ctype, n):
            p = lib().or_model_trace(self._h, what)
            return np.ctypeslib.as_array(C.cast(p, C.POINTER(ctype)), shape=(n,)).copy()
        return {"qkv": arr(0, C.c_uint16, qkv), "attn_out": arr(1, C.c_uint16, c.n_heads * c.head_dim),
                "moe_in": arr(2, C.c_uint16, c.hidden), "moe_idx": arr(3, C.c_int32, c.top_k),
                "moe_score": arr(4, C.c_float, c.top_k)}

    def tensor(self, layer, kind, count, dtype=np.uint16):
        p = lib().or_model_tensor(self._h, layer, kind)
        ct = C.c_uint16 if dtype == np.uint16 else C.c_uint8
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(ct)), shape=(count,)).copy()
