"""One kernel-level configuration launched repeatedly, for counter profiles.

    python3 -m neonengine_amd.kernel_points attn T B WINDOW [--reps R]
    python3 -m neonengine_amd.kernel_points gemv N B [--reps R]
    python3 -m neonengine_amd.kernel_points gemm M N K RESID [--reps R]

`attn` runs neon_attn_decode (64 q / 8 kv heads, d = 64, N(0, 1) bf16 q, K,
V and sinks; every row at position T - 1; full layer when WINDOW is 0) and
`gemv` runs neon_mxfp4_gemv on an [N x 2880] MXFP4 matrix (codes uniform,
E8M0 exponents in [-8, -3]) with a batch of B bf16 rows.  Inputs rotate over
copies holding >= 1 GB of distinct weights or caches (at most 4 GB), so the
256 MB last-level cache cannot serve them, as in bench.py's sweeps (`gemm`,
the prompt pass's projection, runs neon_gemm_bf16 on one N(0, 1) bf16 A and
one W; RESID 1 adds into C as the O projection does); the
workspace and the zeroed arrival counters are allocated once.  Each launch's
duration and counters come from rocprofv3 around this program; it prints the
configuration and the number of launches.
"""
from __future__ import annotations

import argparse
import sys


def rotation(nbytes_one, want=1 << 30, cap=4 << 30):
    n = max(1, -(-want // nbytes_one))
    return max(1, min(n, cap // nbytes_one))


def run_attn(ne, torch, T, B, window, reps):
    Hq, Hkv, D = 64, 8, 64
    n = rotation(2 * B * Hkv * T * D * 2)
    kc = torch.randn(n, B * Hkv * T * D, device="cuda").to(torch.bfloat16).view(torch.int16)
    vc = torch.randn(n, B * Hkv * T * D, device="cuda").to(torch.bfloat16).view(torch.int16)
    q = torch.randn(B, Hq * D, device="cuda").to(torch.bfloat16).view(torch.int16)
    sinks = torch.randn(Hq, device="cuda").to(torch.bfloat16).view(torch.int16)
    out = torch.empty(B, Hq * D, dtype=torch.int16, device="cuda")
    pos = torch.full((B,), T - 1, dtype=torch.int32, device="cuda")
    wb, cb = ne.attn_decode_workspace(B, Hq, Hkv, D, T, window)
    ws = torch.empty(max(wb, 4), dtype=torch.uint8, device="cuda")
    cnt = torch.zeros(max(cb, 4), dtype=torch.uint8, device="cuda")
    for r in range(reps):
        ne.attn_decode(q, kc[r % n], vc[r % n], sinks, pos, out, B, Hq, Hkv, D, T, window,
                       workspace=ws, counters=cnt)
    torch.cuda.synchronize()
    return f"attn T={T} B={B} window={window}: {reps} launches over {n} cache copies"


def run_gemv(ne, torch, N, B, reps):
    K = 2880
    n = rotation(N * K * 17 // 32)
    codes = torch.randint(0, 256, (n, N * K // 2), dtype=torch.uint8, device="cuda")
    scales = torch.randint(119, 125, (n, N * K // 32), dtype=torch.uint8, device="cuda")
    x = torch.randn(B, K, device="cuda").to(torch.bfloat16).view(torch.int16)
    y = torch.empty(B, N, dtype=torch.int16, device="cuda")
    for r in range(reps):
        ne.mxfp4_gemv(codes[r % n], scales[r % n], None, x, y, N, K, B)
    torch.cuda.synchronize()
    return f"gemv N={N} K={K} B={B}: {reps} launches over {n} weight copies"


def run_gemm(ne, torch, M, N, K, resid, reps):
    A = torch.randn(M, K, device="cuda").to(torch.bfloat16).view(torch.int16)
    W = (0.02 * torch.randn(N, K, device="cuda")).to(torch.bfloat16).view(torch.int16)
    b = (0.02 * torch.randn(N, device="cuda")).to(torch.bfloat16).view(torch.int16)
    C = torch.zeros(M, N, dtype=torch.int16, device="cuda")
    for _ in range(reps):
        ne.gemm_bf16(A, W, b, C, M, N, K, accumulate=bool(resid))
    torch.cuda.synchronize()
    return f"gemm M={M} N={N} K={K} resid={resid}: {reps} launches"


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("kind", choices=["attn", "gemv", "gemm"])
    ap.add_argument("args", nargs="+", type=int)
    ap.add_argument("--reps", type=int, default=16)
    a = ap.parse_args(argv)
    import torch
    import neonengine_amd as ne
    assert torch.cuda.is_available(), "needs a HIP device"
    if a.kind == "attn":
        T, B, window = a.args
        msg = run_attn(ne, torch, T, B, window, a.reps)
    elif a.kind == "gemv":
        N, B = a.args
        msg = run_gemv(ne, torch, N, B, a.reps)
    else:
        M, N, K, resid = a.args
        msg = run_gemm(ne, torch, M, N, K, resid, a.reps)
    print(msg, flush=True)


if __name__ == "__main__":
    sys.exit(main())
