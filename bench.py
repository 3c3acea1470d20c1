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
launches that rotate through all 24 layers' expert weights (1.27 GB, beyond
the 256 MB last-level cache).  `cpu_baseline` times the CPU oracle
(oracle/, test infrastructure) on a bounded sample of the same workload.
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
    combine) measured with HIP events on the launch stream."""
    H, I, k, E, L = cfg.hidden, cfg.intermediate, cfg.top_k, cfg.n_experts, cfg.n_layers
    dev = "cuda"
    g = torch.Generator(device="cpu").manual_seed(0)
    x = (torch.randn(H, generator=g) ).to(torch.bfloat16).to(dev)
    act = torch.empty(k * I, dtype=torch.int16, device=dev)
    out = torch.empty(H, dtype=torch.int16, device=dev)
    score = torch.full((k,), 1.0 / k, dtype=torch.float32, device=dev)
    idx = [torch.tensor([(l * 7 + s * (E // k)) % E for s in range(k)], dtype=torch.int32,
                        device=dev) for l in range(L)]
    ptrs = []
    for l in range(L):
        p = "model.layers.%d.mlp.experts." % l
        ptrs.append([eng.tensor_ptr(p + n)[0] for n in (
            "gate_up_proj_blocks", "gate_up_proj_scales", "gate_up_proj_bias",
            "down_proj_blocks", "down_proj_scales", "down_proj_bias")])
    stream = torch.cuda.current_stream()

    def launch(l):
        gc, gs, gb, dc, ds, db = ptrs[l]
        ne.moe_experts(x, idx[l], score, gc, gs, gb, dc, ds, db, None, out, act,
                       1, E, H, I, k, cfg.swiglu_alpha, cfg.swiglu_limit, stream)

    for l in range(L):
        launch(l)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        for l in range(L):
            launch(l)
    e1.record(stream)
    e1.synchronize()
    return e0.elapsed_time(e1) / (reps * L) * 1e-3  # seconds per launch pair


def cpu_baseline(seed: int, prompt_len: int, steps: int):
    """Build's CPU oracle (scalar C + OpenMP) on a bounded sample: a short
    prompt then `steps` greedy decode steps of the same 20b-shaped model."""
    import numpy as np
    from oracle import oracle as orc
    if not os.path.exists(orc._LIB_PATH):
        orc.build()
    cfg = orc.make_config(max_seq=prompt_len + steps + 1)
    t0 = time.perf_counter()
    m = orc.Model(cfg, seed=seed, batch=1)
    gen_s = time.perf_counter() - t0
    ids = np.array([101], np.int32)
    for t in range(prompt_len):
        ids, _ = m.step(np.array([(7919 * t + 101) % cfg.vocab], np.int32), want_logits=False)
    t0 = time.perf_counter()
    for _ in range(steps):
        ids, _ = m.step(ids, want_logits=False)
    dt = time.perf_counter() - t0
    m.close()
    return dict(value=round(steps / dt, 4), unit="tokens/s", cores=orc.num_threads(),
                kind="port",
                sample=f"build's CPU oracle, gpt-oss-20b shape, {steps} greedy decode steps "
                       f"after a {prompt_len}-token prompt (KV length <= {prompt_len + steps}; "
                       f"weight generation {gen_s:.1f}s untimed); label: build's CPU oracle, "
                       f"not the reference")


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
    ap.add_argument("--moe-reps", type=int, default=20)
    ap.add_argument("--cpu-steps", type=int, default=48)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--prompt-only", type=int, default=0, metavar="N",
                    help="profiling aid: run the matrix-core prompt pass N times and exit")
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
    if args.prompt_only:
        cfg = ne.config_preset(args.model, max_seq=args.prompt + 8, max_batch=1)
        eng = ne.Engine(cfg, device=0)
        eng.init_random(args.seed)
        eng.set_prefill_mode(ne.PREFILL_BATCHED)
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
    if args.matrix:
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
    toks = eng.read_tokens(args.prompt, 8)
    log(f"[bench] first generated ids {toks[0].tolist()}")

    mb = moe_bytes(cfg)
    moe_s = moe_gbs = None
    headline = B == 1 and args.model == "gpt-oss-20b"
    if args.moe_reps > 0 and headline:  # 0 skips it (profiling runs that want only the decode loop)
        moe_s = time_moe(ne, torch, eng, cfg, args.moe_reps)
        moe_gbs = mb / moe_s / 1e9
        log(f"[bench] MoE expert FFN: {moe_s * 1e6:.2f} us per launch pair, {moe_gbs:.0f} GB/s")
    eng.close()

    cpu = None
    if not args.no_cpu_baseline and headline:
        log("[bench] CPU baseline (build's oracle) ...")
        cpu = cpu_baseline(args.seed, 4, args.cpu_steps)
        log(f"[bench] CPU baseline {cpu['value']} tok/s on {cpu['cores']} threads")

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
                   "decode_mode": "matrix" if args.matrix and B > 1 else "exact",
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
                     "us_per_launch": moe_s and round(moe_s * 1e6, 3)},
        "cpu_baseline": cpu,
        "prefill": prefill,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
