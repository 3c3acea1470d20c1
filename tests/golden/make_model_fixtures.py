"""Writes tests/golden/model_fixtures.npz: the CPU oracle's greedy runs at the
BASELINE shapes that take the oracle minutes (too long to run inside a GPU
test).  Each case stores its inputs (seed, prompt ids) and, per generated
token, the oracle's greedy id, the SHA-256 of its fp32 logits row (the GPU
exact path is bit-identical to the oracle, so a digest is the whole check),
the top-2 margin and the top-8 (id, value) pairs for diagnosis.

Cases:
  long20b   config 3: gpt-oss-20b shape, a 2048-token prompt uniform over the
            vocab, then 64 greedy steps (batch 1).
  b16_20b   config 3: gpt-oss-20b shape, 16 sequences of 8 prompt tokens,
            then 32 greedy steps at batch 16.
  l120b     config 4: gpt-oss-120b shape (36 layers, 128 experts; the oracle
            regenerates each chosen expert from the counter RNG, so the
            65 GB of experts never sit in host memory), 4 prompt tokens, then
            24 greedy steps.
  ragged20b gpt-oss-20b shape, four sequences with prompts of 5, 77, 300
            and 1000 tokens decoding together (neon_prefill_ragged), then 16
            greedy steps; the oracle runs each sequence alone at batch 1.
  long120b  config 4: gpt-oss-120b shape, a 2048-token prompt uniform over
            the vocab, then 64 greedy steps (batch 1, lazy experts).

Prompt rows go through the oracle's layer-major or_model_prompt (bit-identical
to one teacher-forced step per row, tests/test_oracle.py; the long20b digests
written row by row are reproduced by it), which generates a lazy model's
experts once per layer instead of once per row.

Run: python tests/golden/make_model_fixtures.py [case ...]   (CPU only).
`--check case` recomputes a stored case and compares it with the file.  Test infrastructure: it
runs the oracle, never the product.
"""
import hashlib
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import oracle as orc  # noqa: E402

OUT = os.path.join(ROOT, "tests", "golden", "model_fixtures.npz")

CASES = {
    "long20b": dict(shape="20b", seed=0, batch=1, prompt_len=2048, steps=64, max_seq=2176,
                    prompt_seed=2048),
    "b16_20b": dict(shape="20b", seed=1, batch=16, prompt_len=8, steps=32, max_seq=64,
                    prompt_seed=16),
    "l120b": dict(shape="120b", seed=2, batch=1, prompt_len=4, steps=24, max_seq=64,
                  prompt_seed=120),
    "ragged20b": dict(shape="20b", seed=4, lens=(5, 77, 300, 1000), steps=16, max_seq=1040,
                      prompt_seed=1382),
    "long120b": dict(shape="120b", seed=3, batch=1, prompt_len=2048, steps=64, max_seq=2176,
                     prompt_seed=4096),
}


def prompt_ids(case):
    rng = np.random.default_rng(case["prompt_seed"])
    return rng.integers(0, orc.GPT_OSS_20B["vocab"], (case["batch"], case["prompt_len"]),
                        dtype=np.int32)


def digest(row):
    return np.frombuffer(hashlib.sha256(np.ascontiguousarray(row, np.float32).tobytes()).digest(),
                         np.uint8)


def run_ragged_case(name):
    """Each sequence alone through a batch-1 oracle: teacher-forced prompt rows
    (no lm_head), then the last prompt token and `steps` greedy steps."""
    case = CASES[name]
    lens = case["lens"]
    B, n = len(lens), case["steps"] + 1
    rng = np.random.default_rng(case["prompt_seed"])
    flat = rng.integers(0, orc.GPT_OSS_20B["vocab"], sum(lens), dtype=np.int32)
    cfg = orc.make_config(**dict(orc.GPT_OSS_20B, max_seq=case["max_seq"], max_batch=1))
    out_ids = np.zeros((B, n), np.int32)
    sha = np.zeros((B, n, 32), np.uint8)
    margin = np.zeros((B, n), np.float32)
    top_id = np.zeros((B, n, 8), np.int32)
    top_val = np.zeros((B, n, 8), np.float32)
    t0 = time.time()
    start = 0
    for b, L in enumerate(lens):
        prompt = flat[start:start + L]
        start += L
        m = orc.Model(cfg, seed=case["seed"], batch=1)
        for t in range(L - 1):
            m.prompt_step(prompt[t:t + 1])
            if t % 128 == 0:
                print(f"[{name}] sequence {b} prompt {t}/{L} {time.time() - t0:.0f}s", flush=True)
        ids = prompt[-1:]
        for s in range(n):
            ids, lg = m.step(ids)
            order = np.argsort(-lg[0], kind="stable")[:8]
            top_id[b, s] = order
            top_val[b, s] = lg[0, order]
            margin[b, s] = lg[0, order[0]] - lg[0, order[1]]
            sha[b, s] = digest(lg[0])
            out_ids[b, s] = ids[0]
        print(f"[{name}] sequence {b} ids {out_ids[b, :6]} {time.time() - t0:.0f}s", flush=True)
        m.close()
    return {f"{name}__{k}": v for k, v in dict(
        prompt=flat, lens=np.array(lens, np.int32), ids=out_ids, sha=sha, margin=margin,
        top_id=top_id, top_val=top_val,
        meta=np.array([case["seed"], B, 0, case["steps"], case["max_seq"], 24],
                      np.int64)).items()}


def run_case(name):
    if "lens" in CASES[name]:
        return run_ragged_case(name)
    case = CASES[name]
    shape = orc.GPT_OSS_20B if case["shape"] == "20b" else orc.GPT_OSS_120B
    B = case["batch"]
    cfg = orc.make_config(**dict(shape, max_seq=case["max_seq"], max_batch=B))
    prompt = prompt_ids(case)
    t0 = time.time()
    m = orc.Model(cfg, seed=case["seed"], batch=B, lazy_experts=case["shape"] == "120b")
    print(f"[{name}] model ready in {time.time() - t0:.0f}s", flush=True)
    m.prompt(prompt[:, :-1])
    print(f"[{name}] prompt of {case['prompt_len'] - 1} rows {time.time() - t0:.0f}s", flush=True)
    ids = prompt[:, -1]
    n = case["steps"] + 1
    out_ids = np.zeros((B, n), np.int32)
    sha = np.zeros((B, n, 32), np.uint8)
    margin = np.zeros((B, n), np.float32)
    top_id = np.zeros((B, n, 8), np.int32)
    top_val = np.zeros((B, n, 8), np.float32)
    for s in range(n):
        ids, lg = m.step(ids)
        for b in range(B):
            order = np.argsort(-lg[b], kind="stable")[:8]
            top_id[b, s] = order
            top_val[b, s] = lg[b, order]
            margin[b, s] = lg[b, order[0]] - lg[b, order[1]]
            sha[b, s] = digest(lg[b])
        out_ids[:, s] = ids
        print(f"[{name}] step {s}/{n} ids {ids[:4]} {time.time() - t0:.0f}s", flush=True)
    m.close()
    return {f"{name}__{k}": v for k, v in dict(
        prompt=prompt, ids=out_ids, sha=sha, margin=margin, top_id=top_id, top_val=top_val,
        meta=np.array([case["seed"], B, case["prompt_len"], case["steps"], case["max_seq"],
                       36 if case["shape"] == "120b" else 24], np.int64)).items()}


def check(name):
    """Recompute a stored case and compare every array with the file."""
    with np.load(OUT, allow_pickle=False) as z:
        want = {k: z[k] for k in z.files if k.startswith(name + "__")}
    got = run_case(name)
    bad = [k for k in want if not np.array_equal(want[k], got[k])]
    print(f"[{name}] {'identical' if not bad else 'DIFFERS in ' + ', '.join(bad)}", flush=True)
    return not bad


def main(names):
    data = {}
    if os.path.exists(OUT):
        with np.load(OUT, allow_pickle=False) as z:
            data = {k: z[k] for k in z.files}
    for name in names:
        data = {k: v for k, v in data.items() if not k.startswith(name + "__")}
        data.update(run_case(name))
        np.savez_compressed(OUT, **data)
        print(f"[{name}] written to {OUT}", flush=True)


if __name__ == "__main__":
    if sys.argv[1:2] == ["--check"]:
        sys.exit(0 if all(check(n) for n in sys.argv[2:]) else 1)
    main(sys.argv[1:] or list(CASES))
