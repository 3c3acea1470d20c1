#!/usr/bin/env python3
"""Benchmark: gpt-oss-20b-shaped greedy decode at batch 1 on one MI355X.

Workload (one GPU): random-init gpt-oss-20b weights
(24 layers alternating sliding-128 / full attention, 32 experts top-4 in
MXFP4, bf16 attention / router / embeddings, vocab 201088, untied lm_head),
a 2048-token prompt of ids uniform over the vocabulary (teacher-forced
through the decode graph, untimed), W untimed warm-up decode steps, then K
timed greedy decode steps.  One "step" = one token for the one sequence.
Weights, KV cache and token ids stay in HBM throughout.

Printed: one JSON line with tokens/s (`value`), the whole-step fraction of
the HBM roofline, and a `roofline` object for the MoE expert FFN (the MXFP4
gate_up+SwiGLU and down+combine kernels), timed live with HIP events over
graph replays of the 24 layers' launch pairs with the experts their routers
pick (1.27 GB of distinct weights, beyond the 256 MB last-level cache), next
to a device-copy figure for the achievable HBM rate.  `cpu_baseline` times
the CPU oracle (oracle/, test infrastructure) on a bounded sample of the same
workload at the same KV length.  `--sweep gemv` / `--sweep attn` measure
BASELINE configs 1 and 2 instead.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X vendor HBM3E peak, GB/s
METRIC = "decode tokens/s bs=1 gpt-oss-20b shape; MoE GEMV HBM GB/s as % of peak"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def step_bytes(cfg, kv_len: int) -> int:
    """Algorithmic HBM bytes of one decode step at batch 1 with kv_len cached
    positions: every weight byte read once, KV rows read/written once."""
    H, D, L = cfg.hidden, cfg.head_dim, cfg.n_layers
    Hq, Hkv, E, k, I, V = cfg.n_heads, cfg.n_kv_heads, cfg.n_experts, cfg.top_k, cfg.intermediate, cfg.vocab
    qkv = (Hq + 2 * Hkv) * D
    per_layer = (qkv * H * 2 + qkv * 2          # QKV weight + bias
                 + H * Hq * D * 2 + H * 2        # O weight + bias
                 + 2 * H * 2 + Hq * 2            # two norms, sinks
                 + E * H * 2 + E * 2             # router
                 + k * (2 * I * H + H * I) * 17 // 32  # 4 experts, MXFP4
                 + k * (2 * I + H) * 2)          # expert biases
    kv_row = 2 * Hkv * D * 2                     # K and V of one position
    total = L * per_layer + V * H * 2 + H * 2 + H * 2  # + lm_head, final norm, embed row
    for layer in range(L):
        sliding = layer % 2 == 0 and cfg.sliding_window > 0
        t_eff = min(kv_len, cfg.sliding_window) if sliding else kv_len
        total += t_eff * kv_row + kv_row        # read cached rows, write the new one
    return total


def moe_bytes(cfg) -> int:
    H, I, k = cfg.hidden, cfg.intermediate, cfg.top_k
    weights = k * (2 * I * H + H * I) * 17 // 32
    biases = k * (2 * I + H) * 2
    return weights + biases + 2 * H * 2  # + x in, out


def time_moe(ne, torch, eng, cfg, reps: int):
    """Average duration of one expert-FFN launch pair (gate_up+SwiGLU, down+
    combine), batch 1, over all layers' experts (1.27 GB of distinct weights
    per rotation, beyond the 256 MB last-level cache).  Each layer's experts
    are the ones its own router picks for an N(0, 1) activation row
    (neon_rmsnorm + neon_router_topk), and the 24 launch pairs are captured in
    one graph, so consecutive kernels meet the same launch boundaries as in the
    decode graph; the replays are timed with HIP events on the replay stream."""
    H, I, k, E, L = cfg.hidden, cfg.intermediate, cfg.top_k, cfg.n_experts, cfg.n_layers
    dev = "cuda"
    g = torch.Generator(device="cpu").manual_seed(0)
    x = torch.randn(H, generator=g).to(torch.bfloat16).view(torch.int16).to(dev)
    act = torch.empty(k * I, dtype=torch.int16, device=dev)
    out = torch.empty(H, dtype=torch.int16, device=dev)
    lg = torch.empty(E, dtype=torch.float32, device=dev)
    ptrs, xn, idx, score = [], [], [], []
    for l in range(L):
        p = "model.layers.%d." % l
        w = {n: eng.tensor_ptr(p + n)[0] for n in (
            "post_attention_layernorm.weight", "mlp.router.weight", "mlp.router.bias",
            "mlp.experts.gate_up_proj_blocks", "mlp.experts.gate_up_proj_scales",
            "mlp.experts.gate_up_proj_bias", "mlp.experts.down_proj_blocks",
            "mlp.experts.down_proj_scales", "mlp.experts.down_proj_bias")}
        xn.append(torch.empty(H, dtype=torch.int16, device=dev))
        idx.append(torch.empty(k, dtype=torch.int32, device=dev))
        score.append(torch.empty(k, dtype=torch.float32, device=dev))
        ne.rmsnorm(x, w["post_attention_layernorm.weight"], xn[l], 1, H, cfg.rms_eps)
        ne.router_topk(xn[l], w["mlp.router.weight"], w["mlp.router.bias"], idx[l], score[l],
                       lg, 1, E, H, k)
        ptrs.append([w["mlp.experts." + n] for n in (
            "gate_up_proj_blocks", "gate_up_proj_scales", "gate_up_proj_bias",
            "down_proj_blocks", "down_proj_scales", "down_proj_bias")])
    ne.device_check()  # also sets up the status word before the capture

    def launch_all():
        for l in range(L):
            gc, gs, gb, dc, ds, db = ptrs[l]
            ne.moe_experts(xn[l], idx[l], score[l], gc, gs, gb, dc, ds, db, None, out, act,
                           1, E, H, I, k, cfg.swiglu_alpha, cfg.swiglu_limit)

    launch_all()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch_all()
    stream = torch.cuda.current_stream()
    for _ in range(2):
        graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        graph.replay()
    e1.record(stream)
    e1.synchronize()
    return e0.elapsed_time(e1) / (reps * L) * 1e-3  # seconds per launch pair


def cpu_info():
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count()
    return dict(cpu_model=model, nproc=os.cpu_count(), usable_cpus=usable)


def cpu_baseline(seed: int, kv_len: int, steps: int):
    """The build's CPU oracle (C, OpenMP over the rows of each GEMV) decoding
    the same 20b-shaped model at the GPU line's KV length: a synthetic
    N(0, 1) KV history of kv_len positions in every layer, then `steps`
    greedy decode steps (one warm-up step untimed)."""
    import numpy as np
    from oracle import oracle as orc
    if not os.path.exists(orc._LIB_PATH):
        orc.build()
    cfg = orc.make_config(max_seq=kv_len + steps + 2)
    t0 = time.perf_counter()
    m = orc.Model(cfg, seed=seed, batch=1)
    m.fill_kv(kv_len)
    gen_s = time.perf_counter() - t0
    ids, _ = m.step(np.array([101], np.int32), want_logits=False)
    t0 = time.perf_counter()
    for _ in range(steps):
        ids, _ = m.step(ids, want_logits=False)
    dt = time.perf_counter() - t0
    m.close()
    info = cpu_info()
    return dict(value=round(steps / dt, 4), unit="tokens/s", cores=orc.num_threads(),
                kind="port",
                sample=f"build's CPU oracle, gpt-oss-20b shape, {steps} greedy decode steps at "
                       f"KV length {kv_len + 1}..{kv_len + steps} (synthetic KV history; weight "
                       f"generation {gen_s:.1f}s untimed); label: build's CPU oracle, not the "
                       f"reference", **info)


def hbm_copy_peak(torch, nbytes=1 << 30, reps=5):
    """Achievable HBM bandwidth: a plain device copy of nbytes (read + write)."""
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    e1.synchronize()
    t = e0.elapsed_time(e1) * 1e-3 / reps
    del src, dst
    return round(2 * nbytes / t / 1e9, 1)


def graph_time(torch, calls, reps):
    """Seconds per call: the calls captured once into a graph (so host launch
    overhead does not gap the kernels), replayed `reps` times between HIP
    events on the replay stream."""
    for c in calls:
        c()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for c in calls:
            c()
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        graph.replay()
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) * 1e-3 / (reps * len(calls))


def eager_time(torch, calls, reps):
    for c in calls:
        c()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        for c in calls:
            c()
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) * 1e-3 / (reps * len(calls))


def rotation(nbytes_one, want=1 << 30, cap=4 << 30):
    """Copies of a working set so that one rotation reads >= `want` distinct
    bytes (past the 256 MB last-level cache), at most `cap` bytes in all."""
    n = max(1, -(-want // nbytes_one))
    return max(1, min(n, cap // nbytes_one))


def sweep_gemv(ne, torch, reps=20):
    """MXFP4 GEMV [N x 2880] (codes uniform, E8M0 exponent
    uniform in [-8, -3]) times a bf16 batch, N in {2880, 5760, 4096}, batch
    in {1, 4, 16, 64}, rotating >= 1 GB of distinct weight copies."""
    K, out = 2880, []
    for N in (2880, 5760, 4096):
        mb = N * K * 17 // 32
        n = rotation(mb)
        codes = torch.randint(0, 256, (n, N * K // 2), dtype=torch.uint8, device="cuda")
        scales = torch.randint(119, 125, (n, N * K // 32), dtype=torch.uint8, device="cuda")
        for B in (1, 4, 16, 64):
            x = torch.randn(B, K, device="cuda").to(torch.bfloat16).view(torch.int16)
            y = torch.empty(B, N, dtype=torch.int16, device="cuda")

            calls = [lambda i=i: ne.mxfp4_gemv(codes[i], scales[i], None, x, y, N, K, B)
                     for i in range(n)]
            t = graph_time(torch, calls, reps)
            byt = mb + 2 * B * (K + N)
            out.append(dict(N=N, K=K, B=B, us=round(t * 1e6, 3), bytes=byt,
                            gbs=round(byt / t / 1e9, 1), frac=round(byt / t / 1e9 / HBM_PEAK_GBS, 4),
                            tflops=round(2 * N * K * B / t / 1e12, 3), copies=n))
            log(f"[bench] gemv N={N} B={B}: {t * 1e6:.2f} us, {byt / t / 1e9:.0f} GB/s "
                f"({n} weight copies)")
        del codes, scales
    return out


def sweep_attn(ne, torch, reps=10):
    """sink attention decode, 64 q / 8 kv heads, d = 64,
    bf16 q / k / v / sinks ~ N(0, 1), KV length T in {1024, 8192, 32768},
    batch in {1, 8, 32}, sliding-128 and full layers; >= 1 GB of distinct
    caches per rotation where it fits in 4 GB (sliding windows move with the
    position, so consecutive launches read different keys)."""
    Hq, Hkv, D, out = 64, 8, 64, []
    for T in (1024, 8192, 32768):
        for B in (1, 8, 32):
            cache = B * Hkv * T * D * 2  # one of K / V
            n = rotation(2 * cache)
            kc = torch.randn(n, B * Hkv * T * D, device="cuda").to(torch.bfloat16).view(torch.int16)
            vc = torch.randn(n, B * Hkv * T * D, device="cuda").to(torch.bfloat16).view(torch.int16)
            q = torch.randn(B, Hq * D, device="cuda").to(torch.bfloat16).view(torch.int16)
            sinks = torch.randn(Hq, device="cuda").to(torch.bfloat16).view(torch.int16)
            o = torch.empty(B, Hq * D, dtype=torch.int16, device="cuda")
            for window in (128, 0):
                npos = 16 if window else 1
                pos = [torch.full((B,), T - 1 - 129 * j if window else T - 1, dtype=torch.int32,
                                  device="cuda") for j in range(npos)]

                # one caller workspace and one zeroed counter array for every
                # call (the library allocates nothing per call)
                wb, cb = ne.attn_decode_workspace(B, Hq, Hkv, D, T, window)
                ws = torch.empty(max(wb, 4), dtype=torch.uint8, device="cuda")
                cnt = torch.zeros(max(cb, 4), dtype=torch.uint8, device="cuda")
                calls = [lambda c=c: ne.attn_decode(q, kc[c % n], vc[c % n], sinks, pos[c % npos],
                                                    o, B, Hq, Hkv, D, T, window, workspace=ws,
                                                    counters=cnt)
                         for c in range(max(n, npos))]
                try:
                    t, how = graph_time(torch, calls, reps), "graph"
                except Exception as exc:  # capture refused: time eager launches
                    log(f"[bench] graph capture of attn_decode failed ({exc}); eager timing")
                    t, how = eager_time(torch, calls, reps), "eager"
                t_eff = min(T, window) if window else T
                byt = B * t_eff * 2048 + 2 * B * Hq * D * 2
                out.append(dict(T=T, B=B, window=window, us=round(t * 1e6, 3), bytes=byt,
                                gbs=round(byt / t / 1e9, 1),
                                frac=round(byt / t / 1e9 / HBM_PEAK_GBS, 4), copies=n,
                                timing=how))
                log(f"[bench] attn T={T} B={B} window={window}: {t * 1e6:.2f} us, "
                    f"{byt / t / 1e9:.0f} GB/s ({n} cache copies)")
            del kc, vc
    return out


COPY_BYTES = 256 << 20


def moe_only(ne, torch, args):
    """MoE launch pairs over all layers' experts, then three passes of a plain
    elementwise kernel over a 256 MiB buffer (known traffic: 256 MiB read and
    256 MiB written per dispatch), the yardstick for the traffic counters."""
    cfg = ne.config_preset("gpt-oss-20b", max_seq=64, max_batch=1)
    eng = ne.Engine(cfg, device=0)
    stream = torch.cuda.current_stream()
    eng.init_random(args.seed, stream)
    torch.cuda.synchronize()
    moe_s = time_moe(ne, torch, eng, cfg, max(args.moe_reps, 1))
    eng.close()
    src = torch.ones(COPY_BYTES, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):  # one elementwise dispatch each: 256 MiB in, 256 MiB out
        torch.bitwise_not(src, out=dst)
    torch.cuda.synchronize()
    log(f"[bench] MoE expert FFN: {moe_s * 1e6:.2f} us per launch pair, "
        f"{moe_bytes(cfg) / moe_s / 1e9:.0f} GB/s; copy kernel {COPY_BYTES} B x3 done")


MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 matrix-core peak


def prefill_flops(cfg, P):
    """Matrix work of the batched prompt pass over rows 0..P-2 (2 flop per
    multiply-add): projections, router, the k experts of every row, and the
    causal / sliding attention (QK and PV); the last row runs as a decode step."""
    M = P - 1
    H, D, Hq, Hkv = cfg.hidden, cfg.head_dim, cfg.n_heads, cfg.n_kv_heads
    qkv = (Hq + 2 * Hkv) * D
    per_row = 2 * H * qkv + 2 * Hq * D * H + 2 * H * cfg.n_experts + \
        cfg.top_k * (2 * H * 2 * cfg.intermediate + 2 * cfg.intermediate * H)
    total = 0
    for layer in range(cfg.n_layers):
        sliding = layer % 2 == 0 and cfg.sliding_window > 0
        keys = sum(min(t + 1, cfg.sliding_window) if sliding else t + 1 for t in range(M))
        total += M * per_row + 4 * Hq * D * keys
    return total


def load_traffic():
    path = os.path.join(ROOT, "profiles", "moe_experts_traffic.json")
    if os.path.exists(path):
        with open(path) as f:
            d = json.load(f)
        return d.get("bytes_per_launch")
    return None


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=2048)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--model", default="gpt-oss-20b", choices=["gpt-oss-20b", "gpt-oss-120b"],
                    help="model shape (the headline metric is quoted on gpt-oss-20b)")
    ap.add_argument("--batch", type=int, default=1,
                    help="sequences decoded together (the headline metric is batch 1; "
                         "larger batches are reported as a separate line)")
    ap.add_argument("--matrix", action="store_true",
                    help="run steps of 2+ sequences on the matrix cores (NEON_DECODE_MATRIX)")
    ap.add_argument("--matrix-mx8", action="store_true",
                    help="as --matrix, with the expert GEMMs on the scaled fp8 x fp4 "
                         "instruction (NEON_DECODE_MATRIX_MX8)")
    ap.add_argument("--moe-reps", type=int, default=20)
    ap.add_argument("--cpu-steps", type=int, default=12)
    ap.add_argument("--sweep", choices=["gemv", "attn"],
                    help="BASELINE config 1 (MXFP4 GEMV) or config 2 (sink attention) sweep "
                         "instead of the decode benchmark; prints one JSON line")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--prompt-only", type=int, default=0, metavar="N",
                    help="profiling aid: run the matrix-core prompt pass N times and exit")
    ap.add_argument("--mx8", action="store_true",
                    help="with --prompt-only: the MXFP8 x MXFP4 expert GEMMs (NEON_PREFILL_MX8)")
    ap.add_argument("--moe-only", action="store_true",
                    help="only the MoE launch-pair timing plus a plain 256 MiB device copy "
                         "(the reference kernel for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build runs on exactly one GPU (the token loop is measured on "
              "one MI355X; multi-GPU sharding is a design note only). Use --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    import neonengine_amd as ne

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)
    if args.moe_only:
        moe_only(ne, torch, args)
        return
    if args.sweep:
        pts = sweep_gemv(ne, torch) if args.sweep == "gemv" else sweep_attn(ne, torch)
        print(json.dumps({"sweep": args.sweep, "config": 1 if args.sweep == "gemv" else 2,
                          "peak_gbs": HBM_PEAK_GBS, "points": pts}), flush=True)
        return
    if args.prompt_only:
        cfg = ne.config_preset(args.model, max_seq=args.prompt + 8, max_batch=1)
        eng = ne.Engine(cfg, device=0)
        eng.init_random(args.seed)
        eng.set_prefill_mode(ne.PREFILL_MX8 if args.mx8 else ne.PREFILL_BATCHED)
        prompt = np.random.default_rng(args.seed).integers(0, cfg.vocab, size=(1, args.prompt))
        for i in range(args.prompt_only):
            eng.prefill(prompt)
            torch.cuda.synchronize()
            log(f"[bench] matrix-core prompt pass {i + 1}/{args.prompt_only} done")
        eng.close()
        return
    B = args.batch
    max_seq = args.prompt + args.warmup + args.steps + 8
    cfg = ne.config_preset(args.model, max_seq=max_seq, max_batch=B)
    log(f"[bench] creating {args.model} context (max_seq {max_seq})")
    eng = ne.Engine(cfg, device=0)
    stream = torch.cuda.current_stream()
    eng.init_random(args.seed, stream)
    if args.matrix_mx8:
        eng.set_decode_mode(ne.DECODE_MATRIX_MX8)
    elif args.matrix:
        eng.set_decode_mode(ne.DECODE_MATRIX)
    rng = np.random.default_rng(args.seed)
    prompt = rng.integers(0, cfg.vocab, size=(B, args.prompt), dtype=np.int64)
    t0 = time.perf_counter()
    eng.prefill(prompt, stream)  # first pass: allocates prefill scratch, captures the step
    torch.cuda.synchronize()
    log(f"[bench] prompt of {args.prompt} tokens (first, untimed pass): "
        f"{time.perf_counter() - t0:.2f}s")
    prefill = None

    def timed_prefill():
        p0, p1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        pt0 = time.perf_counter()
        p0.record(stream)
        eng.prefill(prompt, stream)
        p1.record(stream)
        torch.cuda.synchronize()
        return max(time.perf_counter() - pt0, p0.elapsed_time(p1) * 1e-3)

    if B == 1:
        # the matrix-core prompt pass (all rows at once; equal to the exact
        # modes up to bf16 rounding), first once untimed for its scratch
        eng.set_prefill_mode(ne.PREFILL_BATCHED)
        eng.prefill(prompt, stream)
        mfma_s = timed_prefill()
        log(f"[bench] matrix-core prompt pass: {mfma_s * 1e3:.1f} ms = "
            f"{args.prompt / mfma_s:.0f} tok/s")
        # the same with the expert GEMMs on the scaled fp8 x fp4 instruction
        eng.set_prefill_mode(ne.PREFILL_MX8)
        eng.prefill(prompt, stream)
        mx8_s = timed_prefill()
        log(f"[bench] matrix-core prompt pass, MXFP8 x MXFP4 experts: {mx8_s * 1e3:.1f} ms = "
            f"{args.prompt / mx8_s:.0f} tok/s")
        # then the library's default mode, whose cache the decode steps use:
        # prompt rows 16 at a time through the batched decode kernels
        # (bit-identical to running every prompt token as a decode step)
        eng.set_prefill_mode(ne.PREFILL_CHUNKED)
        pre_s = timed_prefill()
        flops = prefill_flops(cfg, args.prompt)
        prefill = {"tokens": args.prompt, "ms": round(pre_s * 1e3, 3),
                   "tokens_per_s": round(args.prompt / pre_s, 1),
                   "mode": "chunked (16 prompt rows per pass through the batched decode kernels)",
                   "matrix_core_pass": {
                       "ms": round(mfma_s * 1e3, 3),
                       "tokens_per_s": round(args.prompt / mfma_s, 1),
                       "tflop_per_s": round(flops / mfma_s / 1e12, 1),
                       "frac_of_bf16_mfma_peak": round(flops / mfma_s / 1e12
                                                       / MFMA_BF16_PEAK_TFLOPS, 4)},
                   "matrix_core_pass_mx8_experts": {
                       "ms": round(mx8_s * 1e3, 3),
                       "tokens_per_s": round(args.prompt / mx8_s, 1),
                       "tflop_per_s": round(flops / mx8_s / 1e12, 1)},
                   "flop_batched_form": flops}
        log(f"[bench] prompt pass: {pre_s * 1e3:.1f} ms = {args.prompt / pre_s:.0f} tok/s")
    eng.decode(args.warmup, stream)
    torch.cuda.synchronize()
    log(f"[bench] warm-up {args.warmup} steps done")

    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    eng.decode(args.steps, stream)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_s = e0.elapsed_time(e1) * 1e-3
    elapsed = max(wall, gpu_s)
    tok_s = B * args.steps / elapsed  # whole-job tokens (B sequences)
    kv0 = args.prompt + args.warmup
    kv_mid = kv0 + args.steps // 2
    bpt = step_bytes(cfg, kv_mid)
    log(f"[bench] {args.steps} steps x batch {B} in {elapsed * 1e3:.1f} ms -> {tok_s:.1f} tok/s"
        + (f" ({bpt * tok_s / 1e9:.0f} GB/s algorithmic)" if B == 1 else ""))
    toks = eng.read_tokens(args.prompt, min(8, args.warmup + args.steps + 1))
    log(f"[bench] first generated ids {toks[0].tolist()}")

    mb = moe_bytes(cfg)
    moe_s = moe_gbs = None
    headline = B == 1 and args.model == "gpt-oss-20b"
    if args.moe_reps > 0 and headline:  # 0 skips it (profiling runs that want only the decode loop)
        moe_s = time_moe(ne, torch, eng, cfg, args.moe_reps)
        moe_gbs = mb / moe_s / 1e9
        log(f"[bench] MoE expert FFN: {moe_s * 1e6:.2f} us per launch pair, {moe_gbs:.0f} GB/s")
    eng.close()

    copy_gbs = hbm_copy_peak(torch) if headline else None
    if copy_gbs:
        log(f"[bench] device copy (1 GiB read + 1 GiB write): {copy_gbs:.0f} GB/s")
    cpu = None
    if not args.no_cpu_baseline and headline:
        log("[bench] CPU baseline (build's oracle) ...")
        cpu = cpu_baseline(args.seed, kv_mid, args.cpu_steps)
        log(f"[bench] CPU baseline {cpu['value']} tok/s on {cpu['cores']} threads "
            f"({cpu['cpu_model']}, {cpu['usable_cpus']} usable of {cpu['nproc']})")

    line = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 activations, mxfp4 experts, fp32 accumulate",
        "data": "synthetic (random-init weights, uniform random prompt ids)",
        "config": {"workload": f"{args.model}-shaped greedy decode, batch {B}, after a "
                               f"{args.prompt}-token prompt (BASELINE config "
                               f"{3 if args.model == 'gpt-oss-20b' else 4})",
                   "batch": B, "prompt": args.prompt,
                   "decode_mode": ("matrix-mx8" if args.matrix_mx8 and B > 1 else
                                   "matrix" if args.matrix and B > 1 else "exact"),
                   "kv_len": [kv0, kv0 + args.steps], "parallelism": "none (1 GPU)"},
        # bytes per token of a batch-1 step (at batch > 1 weights are shared)
        "step_bytes_per_token": bpt if B == 1 else None,
        "step_hbm_gbs": round(bpt * tok_s / 1e9, 1) if B == 1 else None,
        "step_hbm_frac": round(bpt * tok_s / 1e9 / HBM_PEAK_GBS, 4) if B == 1 else None,
        "roofline": {"kernel": "MoE expert FFN (k_moe_gate_up + k_moe_down), batch 1, 4 experts",
                     "bound": "hbm", "achieved": moe_gbs and round(moe_gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": moe_gbs and round(moe_gbs / HBM_PEAK_GBS, 4),
                     "traffic": load_traffic() if moe_gbs else None, "bytes_per_launch": mb,
                     "us_per_launch": moe_s and round(moe_s * 1e6, 3),
                     "achievable_copy_gbs": copy_gbs,
                     "frac_of_copy": moe_gbs and copy_gbs and round(moe_gbs / copy_gbs, 4)},
        "cpu_baseline": cpu,
        "prefill": prefill,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
