"""Sequences of different prompt lengths decoding together
(neon_prefill_ragged): every sequence keeps its own position, and in the
exact modes each sequence's fp32 logits are bit-identical to the CPU oracle
running that sequence alone.  Prompt lengths 5, 77, 300 and 1000 cross the
16-row chunk boundaries at different offsets, put rows of several sequences
into one chunked pass, and wrap the sliding layers' 256-row ring cache
(1000 > 256) while the shorter sequences do not.
"""
import sys

import numpy as np
import pytest

import neonengine_amd as ne
from tests.gpu_util import torch_cuda

pytestmark = pytest.mark.gpu

LENS = (5, 77, 300, 1000)
SMALL = dict(n_layers=4, hidden=512, n_heads=16, n_kv_heads=2, head_dim=64, n_experts=8,
             top_k=4, intermediate=512, vocab=4096, sliding_window=128, max_seq=1100,
             max_batch=4)


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def prompts_for(lens, vocab, seed):
    rng = np.random.default_rng(seed)
    return [rng.integers(0, vocab, n, dtype=np.int32).tolist() for n in lens]


def oracle_alone(orc, cfg, seed, prompt, n_steps):
    """The oracle on one sequence at batch 1: teacher-forced prompt rows, then
    the last prompt token and n_steps greedy steps.  Returns the fp32 logits of
    the n_steps + 1 generating steps and their greedy ids."""
    ocfg = orc.make_config(**dict(cfg.as_dict(), max_batch=1))
    m = orc.Model(ocfg, seed=seed, batch=1)
    for t in prompt[:-1]:
        m.prompt_step([t])
    nxt = np.array([prompt[-1]], np.int32)
    lgs, ids = [], []
    for _ in range(n_steps + 1):
        nxt, lg = m.step(nxt)
        lgs.append(lg[0])
        ids.append(int(nxt[0]))
    m.close()
    return np.stack(lgs), np.array(ids, np.int32)


def gpu_ragged(cfg, seed, prompts, n_steps, mode=None, decode_mode=None):
    """Logits [steps+1][B][V], tokens [B][max_len + n_steps + 1], seq_lens."""
    torch_cuda()
    eng = ne.Engine(cfg)
    eng.init_random(seed)
    if mode is not None:
        eng.set_prefill_mode(mode)
    if decode_mode is not None:
        eng.set_decode_mode(decode_mode)
    eng.prefill_ragged(prompts)
    lgs = [eng.read_logits()]
    for _ in range(n_steps):
        eng.decode(1)
        lgs.append(eng.read_logits())
    toks = eng.read_tokens()
    lens = eng.seq_lens()
    eng.close()
    return np.stack(lgs), toks, lens


def check_tokens(prompts, toks, lens, want_ids, n_steps):
    for b, p in enumerate(prompts):
        n = len(p)
        assert lens[b] == n + 1 + n_steps
        assert np.array_equal(toks[b, :n], p)
        assert np.array_equal(toks[b, n:n + n_steps + 1], want_ids[b]), \
            f"sequence {b}: gpu {toks[b, n:n + n_steps + 1]} oracle {want_ids[b]}"
        assert not toks[b, n + n_steps + 1:].any()  # past the sequence's length


@pytest.mark.parametrize("mode", [ne.PREFILL_CHUNKED, ne.PREFILL_STEPWISE])
def test_ragged_prompts_bit_identical_to_oracle(orc, mode):
    cfg = ne.config_preset("gpt-oss-20b", **SMALL)
    seed, n_steps = 5, 12
    prompts = prompts_for(LENS, cfg.vocab, 77)
    say(f"ragged prompts {LENS} mode {mode}, {n_steps} steps")
    g_lg, toks, lens = gpu_ragged(cfg, seed, prompts, n_steps, mode)
    want = []
    for b, p in enumerate(prompts):
        o_lg, o_ids = oracle_alone(orc, cfg, seed, p, n_steps)
        bad = [s for s in range(n_steps + 1) if not np.array_equal(g_lg[s, b], o_lg[s])]
        if bad:
            s = bad[0]
            say(f"  sequence {b} (length {len(p)}): logits differ first at step {s}, "
                f"max abs {np.abs(g_lg[s, b] - o_lg[s]).max():.3e}")
        assert not bad
        want.append(o_ids)
    check_tokens(prompts, toks, lens, want, n_steps)
    say(f"  all {len(prompts)} sequences bit-identical; seq_lens {lens}")


def test_ragged_equals_each_sequence_alone_on_gpu():
    """The same four prompts prefilled one at a time (batch 1, chunked): the
    ragged batch gives the same logits bit for bit."""
    cfg = ne.config_preset("gpt-oss-20b", **SMALL)
    seed, n_steps = 3, 6
    prompts = prompts_for(LENS, cfg.vocab, 13)
    g_lg, toks, _ = gpu_ragged(cfg, seed, prompts, n_steps)
    for b, p in enumerate(prompts):
        a_lg, a_toks, _ = gpu_ragged(ne.config_preset("gpt-oss-20b", **SMALL), seed, [p], n_steps)
        assert np.array_equal(g_lg[:, b], a_lg[:, 0])
        assert np.array_equal(toks[b, :len(p) + n_steps + 1], a_toks[0])


def test_ragged_lengths_with_single_token_prompts(orc):
    """Prompts of 1 token (no prompt rows, only the first decode step) next to
    longer ones, and one sequence exactly one chunk long."""
    cfg = ne.config_preset("gpt-oss-20b", **dict(SMALL, max_seq=64))
    seed, n_steps = 8, 5
    prompts = prompts_for((1, 17, 1, 2), cfg.vocab, 21)
    g_lg, toks, lens = gpu_ragged(cfg, seed, prompts, n_steps)
    want = []
    for b, p in enumerate(prompts):
        o_lg, o_ids = oracle_alone(orc, cfg, seed, p, n_steps)
        assert np.array_equal(g_lg[:, b], o_lg)
        want.append(o_ids)
    check_tokens(prompts, toks, lens, want, n_steps)


def test_ragged_batched_prompt_pass_and_matrix_decode(orc):
    """The matrix-core prompt pass (one pass per sequence) and matrix-core
    decode steps on ragged prompts: within the 2e-2 relative bar of the
    oracle at this depth (4 layers), with the same greedy ids wherever the
    oracle's top-2 margin exceeds the bar."""
    cfg = ne.config_preset("gpt-oss-20b", **SMALL)
    seed, n_steps = 5, 8
    prompts = prompts_for(LENS, cfg.vocab, 77)
    g_lg, toks, lens = gpu_ragged(cfg, seed, prompts, n_steps, ne.PREFILL_BATCHED,
                                  ne.DECODE_MATRIX)
    for b, p in enumerate(prompts):
        o_lg, o_ids = oracle_alone(orc, cfg, seed, p, 0)
        scale = np.abs(o_lg[0]).max()
        rel = np.abs(g_lg[0, b] - o_lg[0]).max() / scale
        top2 = np.sort(o_lg[0])[-2:]
        say(f"  sequence {b} (length {len(p)}): first-step logits rel err {rel:.3e}, "
            f"oracle margin {(top2[1] - top2[0]) / scale:.3e}")
        assert rel < 2e-2
        if (top2[1] - top2[0]) / scale > 2e-2:
            assert toks[b, len(p)] == o_ids[0]
    assert np.array_equal(lens, np.array(LENS) + 1 + n_steps)


def test_ragged_validation():
    torch_cuda()
    cfg = ne.config_preset("gpt-oss-20b", **dict(SMALL, max_seq=32))
    eng = ne.Engine(cfg)
    eng.init_random(1)
    with pytest.raises(ne.NeonError) as e:
        eng.prefill_ragged([[1, 2], []])
    assert e.value.status == ne.NEON_EINVAL
    with pytest.raises(ne.NeonError) as e:
        eng.prefill_ragged([[1] * 33, [2]])
    assert e.value.status == ne.NEON_EKV_FULL
    with pytest.raises(ne.NeonError) as e:
        eng.prefill_ragged([[1, 2], [cfg.vocab]])
    assert e.value.status == ne.NEON_ERANGE_TOKEN
    eng.prefill_ragged([[1, 2, 3], [4]])
    with pytest.raises(ne.NeonError) as e:  # the longest sequence reaches max_seq
        eng.decode(30)
    assert e.value.status == ne.NEON_EKV_FULL
    eng.decode(28)
    assert list(eng.seq_lens()) == [32, 30]
    eng.close()
