"""GPU checks of temperature / nucleus sampling.  The draw is bit-exact
against the oracle's or_sample, which restates the kernel's operation order
(itself pinned on the CPU against an fp64 inverse-CDF restatement,
tests/test_oracle.py): every id over a grid of temperatures, top_p, seeds and
positions, rows with ties, and a 201088-entry row; and the context's sampled
steps against the oracle's logits fed through or_sample.  What the
mathematics fixes is checked as well: the draw frequencies against
softmax(logits / T) (chi-square over thousands of rows, each row its own RNG
stream), the nucleus (only the top-p set ever appears, in the ratio of its
probabilities), the limits (T -> 0 and top_p -> 0 give the argmax),
reproducibility for a seed, and that temperature 0 keeps the exact greedy
path."""
import sys

import numpy as np
import pytest

import neonengine_amd as ne
from tests.gpu_util import empty_dev, to_dev, to_host, torch_cuda

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def draws(logits_row, n, temperature, top_p, seed, pos0=0):
    V = len(logits_row)
    lg = np.tile(np.asarray(logits_row, np.float32), (n, 1))
    pos = np.full(n, pos0, np.int32)
    out = empty_dev((n,), np.int32)
    ne.sample_logits(to_dev(lg), n, V, temperature, top_p, seed, to_dev(pos), out)
    return to_host(out).astype(np.int64)


def test_sample_bit_exact_vs_oracle(orc):
    """neon_sample against or_sample: identical ids over temperature x top_p x
    seed x position, on rows with a block of tied values, flat rows, rows with
    -inf entries, and the 201088-entry vocabulary."""
    torch_cuda()
    rng = np.random.default_rng(17)
    cases = [(1000, 48), (4099, 24), (201088, 4)]
    total = 0
    for V, B in cases:
        lg = (rng.normal(size=(B, V)) * rng.uniform(0.5, 4.0, (B, 1))).astype(np.float32)
        lg[1, rng.integers(0, V, V // 3)] = lg[1, 0]  # ties
        lg[2] = 0.0                                   # flat
        lg[3, : V // 2] = -np.inf                     # masked half
        dl = to_dev(lg)
        for temperature in (0.3, 1.0, 2.0):
            for top_p in (0.1, 0.5, 0.95, 1.0):
                for seed in (0, 99, 2 ** 50 + 1):
                    pos = rng.integers(0, 30000, B).astype(np.int32)
                    out = empty_dev((B,), np.int32)
                    ne.sample_logits(dl, B, V, temperature, top_p, seed, to_dev(pos), out)
                    got = to_host(out)
                    want = orc.sample(lg, temperature, top_p, seed, pos)
                    assert np.array_equal(got, want), (V, temperature, top_p, seed, got, want)
                    total += B
    say(f"{total} draws identical to the oracle")


def test_engine_sampled_steps_match_oracle(orc):
    """The context's sampled steps (neon_set_sampling): each step's fp32
    logits are the exact path's, and the id drawn from them at the row's
    position equals or_sample's on the oracle's logits."""
    torch_cuda()
    cfg = ne.config_preset("gpt-oss-20b", **SMALL)
    T, top_p, seed = 0.9, 0.8, 31
    prompt = np.array([[5, 6, 7, 8], [9, 10, 11, 12]], np.int32)
    eng = ne.Engine(cfg)
    eng.init_random(4)
    eng.set_sampling(T, top_p, seed)
    eng.prefill(prompt)
    m = orc.Model(orc.make_config(**cfg.as_dict()), seed=4, batch=2)
    for t in range(prompt.shape[1] - 1):
        m.prompt_step(prompt[:, t])
    ids = prompt[:, -1]
    n = 20
    for s in range(n):
        if s:
            eng.decode(1)
        pos = np.array([m_pos(m, b) for b in range(2)], np.int32)
        _, lg = m.step(ids)
        ids = orc.sample(lg, T, top_p, seed, pos)
        got = eng.read_tokens(start=4 + s, count=1)[:, 0]
        assert np.array_equal(got, ids), (s, got, ids)
    m.close()
    eng.close()


def m_pos(m, b):
    from oracle import oracle as orc_mod
    return orc_mod.lib().or_model_pos(m._h, b)


def chi2(counts, probs):
    exp = probs * counts.sum()
    return float((((counts - exp) ** 2) / exp).sum())


def test_frequencies_follow_softmax():
    torch_cuda()
    logits = np.array([0.3, -1.0, 2.0, 0.0, 1.1, -0.4, 0.7, -2.5], np.float32)
    T = 1.3
    ids = draws(logits, 6000, T, 1.0, seed=11)
    p = np.exp(logits.astype(np.float64) / T)
    p /= p.sum()
    c = np.bincount(ids, minlength=8)
    stat = chi2(c, p)
    say(f"counts {c.tolist()} expected {(p * 6000).round(1).tolist()} chi2 {stat:.2f}")
    assert stat < 29.9  # 0.9999 quantile of chi-square with 7 degrees of freedom


def test_nucleus_keeps_only_the_top_set():
    torch_cuda()
    # probabilities 1/2, 1/4, 1/8, ... : top_p 0.7 keeps {0, 1} (mass 0.75)
    logits = np.log(np.array([0.5, 0.25, 0.125, 0.0625, 0.03125, 0.03125], np.float64)).astype(np.float32)
    ids = draws(logits, 6000, 1.0, 0.7, seed=5)
    c = np.bincount(ids, minlength=6)
    say(f"top_p 0.7 counts {c.tolist()}")
    assert c[2:].sum() == 0
    stat = chi2(c[:2], np.array([2 / 3, 1 / 3]))
    assert stat < 15.1  # 0.9999 quantile, 1 degree of freedom


def test_limits_give_the_argmax():
    torch_cuda()
    logits = np.array([0.3, -1.0, 2.0, 0.0, 1.9, -0.4], np.float32)
    assert (draws(logits, 512, 0.001, 1.0, seed=3) == 2).all()   # exp(-100) underflows
    assert (draws(logits, 512, 1.0, 1e-6, seed=3) == 2).all()    # nucleus of one token


def test_large_vocab_and_reproducible():
    torch_cuda()
    rng = np.random.default_rng(0)
    logits = rng.normal(0, 3, 201088).astype(np.float32)
    a = draws(logits, 16, 0.8, 0.95, seed=123, pos0=40)
    b = draws(logits, 16, 0.8, 0.95, seed=123, pos0=40)
    c = draws(logits, 16, 0.8, 0.95, seed=124, pos0=40)
    assert np.array_equal(a, b)
    assert not np.array_equal(a, c)
    # every draw lies in the top-0.95 nucleus of softmax(logits / 0.8)
    p = np.exp((logits.astype(np.float64) - logits.max()) / 0.8)
    order = np.argsort(-p)
    cum = np.cumsum(p[order]) / p.sum()
    nucleus = set(order[: int(np.searchsorted(cum, 0.95)) + 2].tolist())
    assert all(int(i) in nucleus for i in a)


SMALL = dict(n_layers=2, hidden=256, n_heads=8, n_kv_heads=2, head_dim=64, n_experts=8,
             top_k=4, intermediate=256, vocab=1024, sliding_window=128, max_seq=96, max_batch=2)


def run(temperature, top_p, seed, n=32):
    cfg = ne.config_preset("gpt-oss-20b", **SMALL)
    eng = ne.Engine(cfg)
    eng.init_random(4)
    eng.set_sampling(temperature, top_p, seed)
    eng.prefill([[5, 6, 7, 8], [9, 10, 11, 12]])
    eng.decode(n)
    t = eng.read_tokens()
    eng.close()
    return t


def test_engine_sampling_reproducible_and_greedy_default():
    torch_cuda()
    a = run(0.9, 0.9, 7)
    b = run(0.9, 0.9, 7)
    c = run(0.9, 0.9, 8)
    g1 = run(0.0, 1.0, 7)
    g2 = run(0.0, 1.0, 99)  # temperature 0: the seed is not used
    say(f"sampled row 0 {a[0, 4:16].tolist()} greedy row 0 {g1[0, 4:16].tolist()}")
    assert np.array_equal(a, b)
    assert not np.array_equal(a, c)
    assert np.array_equal(g1, g2)
    assert (a[:, :4] == [[5, 6, 7, 8], [9, 10, 11, 12]]).all()  # prompt kept


def test_engine_sampling_validation():
    torch_cuda()
    cfg = ne.config_preset("gpt-oss-20b", **SMALL)
    eng = ne.Engine(cfg)
    for bad in [(-1.0, 0.9), (1.0, 0.0), (1.0, 1.5), (float("nan"), 1.0), (float("inf"), 1.0)]:
        with pytest.raises(ne.NeonError) as e:
            eng.set_sampling(*bad, 0)
        assert e.value.status == ne.NEON_EINVAL
    eng.close()
