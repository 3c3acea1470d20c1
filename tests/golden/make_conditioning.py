"""Measures how far a change of summation order alone moves the outputs of
the random-init gpt-oss-20b shape, and writes tests/golden/conditioning.npz.

The CPU oracle runs the same inputs twice: once in the canonical fp32 orders
(what the exact GPU path reproduces bit for bit) and once with every dot
product, norm and attention accumulated in fp64 and rounded once (a more
accurate order, with the same bf16 rounding points).  Both runs take the same
tokens (the canonical run's greedy ids).  The per-row relative max logit error
between them, max|a - b| / max|b|, is what any implementation that sums in a
different order must expect; the matrix-core tests set their bars from it.

Cases: batch 16, the seed and prompt of tests/test_gpu_configs.py, depth
2, 6, 12 and 24 layers, router as initialised ("free") and fixed (router
weight 0, distinct biases: every row picks the same 4 experts); and the
gpt-oss-120b shape (36 layers, 128 experts, lazy experts) with the routing
fixed ("fixed_36").

Run: python tests/golden/make_conditioning.py [key ...]   (CPU only, ~15
minutes for the 20b keys; keys already in the file and not named are kept.)
Test infrastructure: it runs the oracle, never the product.
"""
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import oracle as orc  # noqa: E402

OUT = os.path.join(ROOT, "tests", "golden", "conditioning.npz")
SEED, B, STEPS = 7, 16, 2
DEPTHS = (2, 6, 12, 24)


def fixed_bias(E, layer):
    b = np.array([1.0 - 0.25 * ((e + 3 * layer) % E) for e in range(E)], np.float32)
    return (b.view(np.uint32) >> 16).astype(np.uint16)


def run(depth, fixed, mode, tokens=None, shape=None):
    cfg = orc.make_config(**dict(shape or {}, n_layers=depth, max_seq=32, max_batch=B))
    rng = np.random.default_rng(SEED)
    prompt = rng.integers(0, cfg.vocab, (B, 2), dtype=np.int32)
    m = orc.Model(cfg, seed=SEED, batch=B, lazy_experts=shape is not None)
    if fixed:
        for layer in range(depth):
            m.set_tensor(layer, orc.T_ROUTER_W, np.zeros(cfg.n_experts * cfg.hidden, np.uint16))
            m.set_tensor(layer, orc.T_ROUTER_B, fixed_bias(cfg.n_experts, layer))
    orc.set_accumulation(mode)
    try:
        m.step(prompt[:, 0], want_logits=False)
        ids = prompt[:, 1]
        logits, out_ids = [], []
        for s in range(STEPS + 1):
            nxt, lg = m.step(ids)
            logits.append(lg)
            out_ids.append(nxt)
            ids = nxt if tokens is None else tokens[s]
    finally:
        orc.set_accumulation(0)
        m.close()
    return np.stack(logits), np.stack(out_ids)


CASES = {f"{'fixed' if fixed else 'free'}_{depth}": (depth, fixed, None)
         for fixed in (True, False) for depth in DEPTHS}
CASES["fixed_36"] = (36, True, orc.GPT_OSS_120B)


def main(keys):
    data = {}
    if os.path.exists(OUT):
        with np.load(OUT, allow_pickle=False) as z:
            data = {k: z[k] for k in z.files}
    t0 = time.time()
    for key in keys:
        depth, fixed, shape = CASES[key]
        lg_c, ids_c = run(depth, fixed, 0, shape=shape)
        lg_f, ids_f = run(depth, fixed, 1, tokens=ids_c, shape=shape)
        scale = np.abs(lg_c).max(axis=2)
        rel = np.abs(lg_f.astype(np.float64) - lg_c).max(axis=2) / scale
        flips = (ids_c != ids_f).sum()
        data[key] = rel
        print(f"{key}: rel max err max {rel.max():.3e} median {np.median(rel):.3e}; "
              f"greedy ids differ {flips}/{ids_c.size}  ({time.time() - t0:.0f}s)", flush=True)
        np.savez_compressed(OUT, **data)


if __name__ == "__main__":
    main(sys.argv[1:] or list(CASES))
