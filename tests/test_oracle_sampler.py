"""CPU checks that pin the sampler oracle (oracle/sampler.py).

* the reference's one-hot ``batch_accept`` cases (tests/test_spec_accept.py:29-73);
* the reference's sampler properties (tests/test_sampler.py:18-64);
* the library identity ``torch.multinomial(p, 1, g) == argmax(p / E)`` with ``E``
  drawn by ``exponential_`` from a clone of ``g`` (same generator state after);
* golden vectors written by running the reference's ``batch_accept`` with a
  live generator (tests/golden/batch_accept_golden.json): same tokens, same
  amount of randomness consumed;
* exact enumeration on a vocab-8 toy: the accept / residual rule reproduces the
  target distribution (Leviathan et al. 2023, Thm 1) -- a wrong residual sign,
  a missing clamp or an inverted ratio breaks it.
"""

from __future__ import annotations

import json
import os

import pytest
import torch

from oracle import sampler as S

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "batch_accept_golden.json")


def _one_hot(t, v=8):
    x = torch.zeros(v)
    x[t] = 1.0
    return x


def test_batch_accept_full_acceptance_with_bonus():
    g = torch.Generator().manual_seed(0)
    p = {0: torch.stack([_one_hot(3)] * 3)}
    q = {0: [_one_hot(3), _one_hot(3)]}
    assert S.batch_accept(p, q, {0: [3, 3]}, g)[0] == [3, 3, 3]


def test_batch_accept_rejection_resamples_residual():
    g = torch.Generator().manual_seed(0)
    p = {0: torch.stack([_one_hot(5), _one_hot(5)])}
    q = {0: [_one_hot(2)]}
    assert S.batch_accept(p, q, {0: [2]}, g)[0] == [5]


def test_batch_accept_rejects_then_stops():
    g = torch.Generator().manual_seed(0)
    p = {0: torch.stack([_one_hot(1), _one_hot(4), _one_hot(4)])}
    q = {0: [_one_hot(1), _one_hot(7)]}
    assert S.batch_accept(p, q, {0: [1, 7]}, g)[0] == [1, 4]


def test_greedy_mode_is_one_hot():
    probs = S.logits_to_probs(torch.tensor([[0.1, 2.0, -1.0, 0.5]]), 0.0)
    assert float(probs.sum()) == 1.0 and int(probs.argmax()) == 1


def test_greedy_ties_take_first_index():
    probs = S.logits_to_probs(torch.tensor([1.0, 3.0, 3.0, 0.0]), 0.0)
    assert probs.tolist() == [0.0, 1.0, 0.0, 0.0]


def test_temperature_sharpens_distribution():
    z = torch.tensor([[1.0, 2.0, 3.0]])
    cold, warm = S.logits_to_probs(z, 0.5), S.logits_to_probs(z, 2.0)
    assert float(cold.max()) > float(warm.max())
    assert abs(float(cold.sum()) - 1.0) < 1e-6


def test_residual_distribution_is_normalised_and_non_negative():
    r = S.residual_distribution(torch.tensor([0.5, 0.3, 0.2]), torch.tensor([0.1, 0.4, 0.5]))
    assert abs(float(r.sum()) - 1.0) < 1e-6 and float(r.min()) >= 0.0 and float(r[2]) == 0.0


def test_residual_falls_back_to_p_when_identical():
    p = torch.tensor([0.2, 0.8])
    assert torch.allclose(S.residual_distribution(p, p.clone()), p, atol=1e-6)


def test_acceptance_probability_branches():
    p = torch.tensor([0.5, 0.0, 0.3, 1e-13])
    q = torch.tensor([0.25, 0.5, 0.0, 0.0])
    assert S.acceptance_probability(p, q, 0) == 1.0            # min(1, 2)
    assert S.acceptance_probability(p, q, 1) == 0.0            # p = 0
    assert S.acceptance_probability(p, q, 2) == 1.0            # q <= eps, p > eps
    assert S.acceptance_probability(p, q, 3) == 0.0            # q <= eps, p <= eps
    assert S.acceptance_probability(q, p, 0) == float(torch.tensor(0.25)) / float(torch.tensor(0.5))


@pytest.mark.parametrize("vocab,seed", [(8, 0), (8, 1), (1000, 2), (151936, 3)])
def test_multinomial_is_exponential_race(vocab, seed):
    g = torch.Generator().manual_seed(seed)
    probs = torch.softmax(torch.randn(vocab, generator=g) * 2.0, 0)
    g1 = torch.Generator().manual_seed(100 + seed)
    g2 = torch.Generator()
    g2.set_state(g1.get_state())
    for _ in range(5):
        a = S.sample_token(probs, g1)
        b = S.race_argmax(probs, S.draw_race_noise(vocab, g2))
        assert a == b
    assert torch.equal(g1.get_state(), g2.get_state())


def _golden_cases():
    with open(GOLDEN) as f:
        return json.load(f)["cases"]


@pytest.mark.parametrize("case", _golden_cases(), ids=lambda c: "v{}s{}".format(c["vocab"], c["seed"]))
def test_batch_accept_matches_reference_golden(case):
    B, gm, V = case["batch"], case["gamma"], case["vocab"]
    p = torch.tensor(case["p"], dtype=torch.float32).reshape(B, gm + 1, V)
    q = torch.tensor(case["q"], dtype=torch.float32).reshape(B, gm, V)
    sids = case["sids"]
    p_by = {s: p[b] for b, s in enumerate(sids)}
    q_by = {s: [q[b, j] for j in range(gm)] for b, s in enumerate(sids)}
    x_by = {s: case["proposals"][b] for b, s in enumerate(sids)}
    gen = torch.Generator().manual_seed(case["gen_seed"])
    record = {}
    out = S.batch_accept(p_by, q_by, x_by, gen, record=record)
    assert [out[s] for s in sids] == case["accepted"]
    assert float(torch.rand(1, generator=gen).item()) == case["next_uniform"]
    # the same decisions from the recorded noise through the batched form
    u = torch.full((B, gm), 2.0)
    noise = torch.empty(B, V)
    for b, s in enumerate(sids):
        us, e = record[s]
        u[b, : len(us)] = torch.tensor(us)
        noise[b] = e
    x = torch.tensor(case["proposals"])
    assert S.batch_accept_noise(p, q, x, u, noise) == case["accepted"]


@pytest.mark.parametrize("seed", range(4))
def test_accept_rule_reproduces_target_exactly(seed):
    # P(out = t) = sum_x q(x) [a(x) 1{t = x} + (1 - a(x)) rhat(t)] must equal p(t).
    g = torch.Generator().manual_seed(seed)
    V = 8
    p = torch.softmax(torch.randn(V, generator=g) * 1.5, 0)
    q = torch.softmax(torch.randn(V, generator=g) * 1.5, 0)
    r = S.residual_distribution(p, q).double()
    dist = torch.zeros(V, dtype=torch.float64)
    for x in range(V):
        a = S.acceptance_probability(p, q, x)
        dist[x] += float(q[x]) * a
        dist += float(q[x]) * (1.0 - a) * r
    assert torch.allclose(dist, p.double(), atol=2e-7)


def test_accept_rule_sampled_chi_square():
    # Monte Carlo over the noise inputs of the batched form: first emitted token ~ p_0.
    g = torch.Generator().manual_seed(11)
    V, N = 8, 20000
    p = torch.softmax(torch.randn(1, 2, V, generator=g) * 1.5, -1)
    q = torch.softmax(torch.randn(1, 1, V, generator=g) * 1.5, -1)
    counts = torch.zeros(V)
    for _ in range(N):
        x = torch.multinomial(q[0, 0], 1, generator=g).reshape(1, 1)
        u = torch.rand(1, 1, generator=g)
        e = torch.empty(1, V).exponential_(1, generator=g)
        counts[S.batch_accept_noise(p, q, x, u, e)[0][0]] += 1
    expected = p[0, 0] * N
    chi2 = float(((counts - expected) ** 2 / expected).sum())
    assert chi2 < 24.3  # chi^2_{7} at p = 0.001


# ------------------------------------------------------------- top-k / top-p
def test_top_k_keeps_exactly_k_tokens():
    # reference tests/test_sampler.py:34-39
    filtered = S.apply_top_k(torch.tensor([[5.0, 4.0, 3.0, 2.0, 1.0]]), 2)
    assert torch.isfinite(filtered).sum().item() == 2 and float(filtered[0, 0]) == 5.0


def test_top_p_truncates_tail():
    # reference tests/test_sampler.py:42-48
    filtered = S.apply_top_p(torch.log(torch.tensor([[0.5, 0.3, 0.15, 0.05]])), 0.8)
    probs = torch.softmax(filtered, dim=-1)
    assert float(probs[0, 3]) == 0.0 and float(probs.sum()) >= 0.8 - 1e-6


def test_top_p_ignored_when_one():
    # reference tests/test_sampler.py:76-78
    logits = torch.randn(1, 8)
    assert torch.allclose(S.apply_top_p(logits, 1.0), logits)


def _brute_keep(x, top_k, top_p):
    """float64 brute force on a row without ties: top-k keeps a value when
    fewer than k values are larger; top-p (on what top-k kept) keeps a value
    when the mass of the kept values larger than it is below p times their
    total mass."""
    x = x.double()
    keep = torch.ones_like(x, dtype=torch.bool)
    if 0 < top_k < x.numel():
        for i in range(x.numel()):
            keep[i] = int((x > x[i]).sum()) < top_k
    if 0.0 < top_p < 1.0:
        w = torch.where(keep, torch.exp(x - x[keep].max()), torch.zeros_like(x))
        tot = float(w.sum())
        keep2 = keep.clone()
        for i in range(x.numel()):
            if keep[i]:
                keep2[i] = float(w[(x > x[i]) & keep].sum()) < top_p * tot
        keep = keep2
    return keep


@pytest.mark.parametrize("top_k,top_p", [(5, 1.0), (0, 0.9), (40, 0.5), (3, 0.99), (0, 0.05)])
def test_filters_match_the_brute_force(top_k, top_p):
    g = torch.Generator().manual_seed(top_k + int(100 * top_p))
    for _ in range(3):
        x = torch.randn(200, generator=g) * 2
        got = torch.isfinite(S.filter_logits(x, 1.0, top_k, top_p))
        assert torch.equal(got, _brute_keep(x, top_k, top_p))


def test_brute_force_catches_an_unshifted_nucleus_mask():
    # dropping the value that crosses p (mask cum >= p instead of cum - p >= p)
    # keeps one value fewer
    x = torch.log(torch.tensor([0.5, 0.3, 0.15, 0.05]))
    keep = _brute_keep(x, 0, 0.6)
    assert keep.tolist() == [True, True, False, False]
    sorted_p = torch.softmax(x, -1)
    assert (torch.cumsum(sorted_p, -1) < 0.6).tolist() == [True, False, False, False]
