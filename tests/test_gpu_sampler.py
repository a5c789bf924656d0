"""GPU parity of the rejection-sampling kernels against the oracle.

Token ids, accept lengths and commit outputs must be identical (bit-exact):

* the reference's one-hot ``batch_accept`` cases (tests/test_spec_accept.py:29-73);
* the golden vectors recorded from the reference's ``batch_accept`` with a live
  generator -- same tokens and the same generator state afterwards;
* the fused-sampler workload (B = 64, gamma = 5, V = 151,936, target logits
  ~ N(0, 2^2), draft = target + N(0, 1), T = 1, 0.25 and 0) against the
  oracle's logits_to_probs + batch_accept on the same logits, uniforms and
  Exp(1) rows;
* the commit cut (budget with Python slice semantics, eos) against the oracle.

Given logits, p and q are the kernel's own fp32 softmax, a few 1e-6 from
torch's CPU softmax; the kernel reports every result that rounding could have
decided otherwise in the sequence's flag word (``VerifyResult.flags``). Every
unflagged sequence must equal the oracle and every sequence that differs must
be flagged; the tests print how many were flagged. Crafted cases must raise the
flag: a uniform within 1e-7 of ``min(1, p/q)``, and a residual race whose
winner is within the probabilities' rounding of a cancelling token (p ~ q)
that is not among the two best fast keys. With probabilities as inputs the
arithmetic is exactly the reference's: crafted near-ties (race keys equal, or
one fp32 ulp apart, at the residual and bonus rows) take the exact re-race and
must return torch's own argmax (flagged as within a few ulp).
"""

from __future__ import annotations

import json
import os

import pytest
import torch

from engine import _hip
from engine import spec_scheduler as es
from oracle import sampler as S
from oracle import spec_step as ref_step
from specdec import sampler as gs
from specdec.config import SamplingConfig

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "batch_accept_golden.json")


def _one_hot(t, dev, v=8):
    x = torch.zeros(v, device=dev)
    x[t] = 1.0
    return x


def test_one_hot_cases(cuda):
    g = torch.Generator().manual_seed(0)
    p = {0: torch.stack([_one_hot(3, cuda)] * 3)}
    assert es.batch_accept(p, {0: [_one_hot(3, cuda)] * 2}, {0: [3, 3]}, g)[0] == [3, 3, 3]
    p = {0: torch.stack([_one_hot(5, cuda)] * 2)}
    assert es.batch_accept(p, {0: [_one_hot(2, cuda)]}, {0: [2]}, g)[0] == [5]
    p = {0: torch.stack([_one_hot(1, cuda), _one_hot(4, cuda), _one_hot(4, cuda)])}
    q = {0: [_one_hot(1, cuda), _one_hot(7, cuda)]}
    assert es.batch_accept(p, q, {0: [1, 7]}, g)[0] == [1, 4]


def _golden_cases():
    with open(GOLDEN) as f:
        return json.load(f)["cases"]


@pytest.mark.parametrize("case", _golden_cases(), ids=lambda c: "v{}s{}".format(c["vocab"], c["seed"]))
def test_batch_accept_golden(cuda, case):
    B, gm, V = case["batch"], case["gamma"], case["vocab"]
    p = torch.tensor(case["p"], dtype=torch.float32).reshape(B, gm + 1, V).to(cuda)
    q = torch.tensor(case["q"], dtype=torch.float32).reshape(B, gm, V).to(cuda)
    sids = case["sids"]
    gen = torch.Generator().manual_seed(case["gen_seed"])
    out = es.batch_accept({s: p[b] for b, s in enumerate(sids)},
                          {s: [q[b, j] for j in range(gm)] for b, s in enumerate(sids)},
                          {s: case["proposals"][b] for b, s in enumerate(sids)}, gen)
    assert [out[s] for s in sids] == case["accepted"]
    assert float(torch.rand(1, generator=gen).item()) == case["next_uniform"]


def test_sampler_primitives_match_oracle(cuda):
    g = torch.Generator().manual_seed(3)
    z = torch.randn(4, 1000, generator=g) * 2
    for T in (0.0, 0.7, 1.0):
        got = gs.logits_to_probs(z.to(cuda), SamplingConfig(temperature=T)).cpu()
        want = S.logits_to_probs(z, T)
        if T == 0.0:
            assert torch.equal(got, want)
        else:
            assert torch.allclose(got, want, rtol=2e-6, atol=1e-9)
    p, q = S.logits_to_probs(z[0], 1.0), S.logits_to_probs(z[1], 1.0)
    assert torch.allclose(gs.residual_distribution(p.to(cuda), q.to(cuda)).cpu(),
                          S.residual_distribution(p, q), rtol=1e-6, atol=1e-9)
    assert torch.allclose(gs.residual_distribution(p.to(cuda), p.to(cuda)).cpu(), p, atol=1e-7)
    for x in (0, 5, 999):
        assert gs.acceptance_probability(p.to(cuda), q.to(cuda), x) == S.acceptance_probability(p, q, x)
    for seed in range(5):
        g1 = torch.Generator().manual_seed(seed)
        g2 = torch.Generator().manual_seed(seed)
        assert gs.sample_token(p.to(cuda), g1) == S.sample_token(p, g2)
        assert torch.equal(g1.get_state(), g2.get_state())


def _workload(seed, B=64, gamma=5, V=151936, sigma=2.0):
    g = torch.Generator().manual_seed(seed)
    target = torch.randn(B, gamma + 1, V, generator=g) * sigma
    draft = target[:, :gamma] + torch.randn(B, gamma, V, generator=g)
    u = torch.rand(B, gamma, generator=g)
    noise = torch.empty(B, V).exponential_(1, generator=g)
    return g, target, draft, u, noise


def _proposals(draft, T, g):
    q = S.logits_to_probs(draft, T)
    B, gamma, V = q.shape
    return torch.multinomial(q.reshape(-1, V), 1, generator=g).reshape(B, gamma)


def _decision_margins(target, draft, x, u, noise, T):
    """Smallest |u - a| over the examined positions and smallest relative gap
    between the two best race keys over the sequences, as the oracle computes
    them (T > 0)."""
    p, q = S.logits_to_probs(target, T), S.logits_to_probs(draft, T)
    B, gamma = x.shape
    min_u, min_gap = float("inf"), float("inf")
    for b in range(B):
        k = gamma
        for j in range(gamma):
            a = S.acceptance_probability(p[b, j], q[b, j], int(x[b, j]))
            min_u = min(min_u, abs(float(u[b, j]) - a))
            if not float(u[b, j]) < a:
                k = j
                break
        r = S.residual_distribution(p[b, k], q[b, k]) if k < gamma else p[b, gamma]
        top = torch.topk(r / noise[b], 2).values
        min_gap = min(min_gap, float((top[0] - top[1]) / top[0]))
    return min_u, min_gap


def _check_flagged(res, want, what=""):
    """Unflagged sequences equal the oracle; any that differs is flagged.
    Returns the number of flagged sequences."""
    got = res.accepted_lists()
    flags = res.flags.tolist()
    for b, (g, w, f) in enumerate(zip(got, want, flags)):
        assert g == w or f != 0, (what, b, g, w)
    n = sum(1 for f in flags if f)
    print("{}: {} of {} sequences flagged {}".format(what, n, len(flags),
                                                   [(b, f) for b, f in enumerate(flags) if f]))
    return n


@pytest.mark.parametrize("T", [1.0, 0.25, 0.0])
def test_fused_sampler_workload(cuda, T):
    g, target, draft, u, noise = _workload({1.0: 42, 0.25: 44, 0.0: 43}[T])
    x = _proposals(draft, T, g)
    want = S.verify_from_logits(target, draft, x, u, noise, T)
    if T > 0:
        min_u, min_gap = _decision_margins(target, draft, x, u, noise, T)
        print("decision margins: min |u - a| = {:.3e}, min race top-2 gap = {:.3e}".format(min_u, min_gap))
    res = es.verify_sample(target.to(cuda), draft.to(cuda), x.to(cuda), u.to(cuda),
                           noise.to(cuda) if T > 0 else None, T)
    n = _check_flagged(res, want, "T={}".format(T))
    if T == 0:
        assert n == 0  # one-hot rows are exact
    assert n <= 2  # a flag is a near coincidence, at most a handful per workload
    lens = res.accept_len.tolist()
    assert [len(w) - 1 for w, f in zip(want, res.flags.tolist()) if not f] == \
        [n_ for n_, f in zip(lens, res.flags.tolist()) if not f]
    if T == 1.0:
        assert 0 < sum(lens) < 5 * 64  # both accepts and rejections occur


def test_decision_inside_the_band_is_flagged(cuda):
    """Logits mode at V = 151,936: position 0's uniform placed within 5e-8
    (relative) of the oracle's acceptance probability a must raise
    SPV_FLAG_ACCEPT_BAND; placed 1e-3 away it must not, and the result must
    be the oracle's."""
    B, gamma, V = 8, 3, 151936
    g, target, draft, _, noise = _workload(90, B=B, gamma=gamma, V=V)
    p = S.logits_to_probs(target, 1.0)
    q = S.logits_to_probs(draft, 1.0)
    # position 0's proposal: a token with 0.2 < p/q < 0.9, so a < 1
    x = torch.zeros(B, gamma, dtype=torch.int64)
    a0 = []
    for b in range(B):
        ratio = p[b, 0] / q[b, 0]
        cand = ((ratio > 0.2) & (ratio < 0.9) & (q[b, 0] > 1e-5)).nonzero().flatten()
        x[b, 0] = int(cand[b])
        x[b, 1:] = torch.multinomial(q[b, 1:], 1, generator=g).flatten()
        a0.append(S.acceptance_probability(p[b, 0], q[b, 0], int(x[b, 0])))
    for rel, inside in ((5e-8, True), (-5e-8, True), (1e-3, False), (-1e-3, False)):
        u = torch.rand(B, gamma, generator=g)
        for b in range(B):
            u[b, 0] = float(torch.tensor(a0[b] * (1.0 + rel), dtype=torch.float32))
        want = S.verify_from_logits(target, draft, x, u, noise, 1.0)
        res = es.verify_sample(target.to(cuda), draft.to(cuda), x.to(cuda), u.to(cuda), noise.to(cuda), 1.0)
        flags = res.flags.tolist()
        if inside:
            assert all(f & _hip.FLAG_ACCEPT_BAND for f in flags), (rel, flags)
            _check_flagged(res, want, "u = a (1 {:+.0e})".format(rel))
        else:
            assert flags == [0] * B, (rel, flags)
            assert res.accepted_lists() == want


def _tie_case(seed, V, reject_at, relation, gamma=3):
    """One sequence whose race has two keys tied at fp32 level: ``relation`` 0
    makes the keys of indices a < b equal (torch.argmax takes a), +1 puts b one
    ulp above a, -1 one ulp below. ``reject_at`` < gamma races the residual of
    that row (u = 1 rejects it), gamma races the bonus row (u = 0 accepts all)."""
    g = torch.Generator().manual_seed(seed)
    p = torch.softmax(torch.randn(gamma + 1, V, generator=g) * 2, -1)
    q = torch.softmax(torch.randn(gamma, V, generator=g) * 2, -1)
    x = torch.randint(0, V, (1, gamma), generator=g)
    u = torch.zeros(1, gamma)
    if reject_at < gamma:
        u[0, reject_at] = 1.0
    noise = torch.empty(V).exponential_(1, generator=g)
    k = reject_at
    cand = torch.randperm(V, generator=g)[:64].tolist()
    a = min(cand[:2])
    if k < gamma:
        q[k, cand] = 0.0  # residual mass at every candidate index
        r = S.residual_distribution(p[k], q[k])
    else:
        r = p[gamma]
    noise[a] = r[a] * 1e-10  # a's key ~1e10: above every other key by far
    key_a = r[a] / noise[a]
    want = key_a if relation == 0 else torch.nextafter(key_a, key_a * (1 + relation))
    for b in cand:
        if b <= a:
            continue
        # E_b such that r_b / E_b is exactly `want` (not every quotient is reachable)
        e_b = (r[b] / want).to(torch.float32)
        for _ in range(16):
            kb = r[b] / e_b
            if kb == want:
                break
            e_b = torch.nextafter(e_b, e_b * (2.0 if kb > want else 0.5))
        if r[b] / e_b == want:
            noise[b] = e_b
            break
    else:
        raise AssertionError("could not place the tie")
    assert S.race_argmax(r, noise) == (b if relation > 0 else a)
    return p.unsqueeze(0), q.unsqueeze(0), x.to(torch.int32), u, noise.unsqueeze(0)


@pytest.mark.parametrize("reject_at", [0, 2, 3])
@pytest.mark.parametrize("relation", [0, 1, -1])
def test_near_tie_race_takes_the_exact_path(cuda, reject_at, relation):
    p, q, x, u, noise = _tie_case(100 + 3 * reject_at + relation, 151936, reject_at, relation)
    want = S.batch_accept_noise(p, q, x, u, noise)
    res = es.verify_sample(p.to(cuda), q.to(cuda), x.to(cuda), u.to(cuda), noise.to(cuda), 1.0,
                           is_probs=True)
    assert res.accepted_lists() == want
    # keys equal or one ulp apart: within rounding of the reference's own
    # residual normalisation, so the draw is reported
    assert res.flags.tolist() == [_hip.FLAG_DRAW_BAND]


def _cancelling_residual_case(seed, V, gap, gamma=3):
    """Logits mode, row 0 rejected (u = 1): the draft row is the target row with
    the logits of two tokens a < b lowered by 0.01, so only a and b keep a
    residual r = p - q, about 1% of p (p and q nearly cancel). Their Exp(1)
    entries make them the two best keys, key_b = key_a (1 + gap) on the
    oracle's arithmetic."""
    g = torch.Generator().manual_seed(seed)
    target = torch.randn(1, gamma + 1, V, generator=g) * 2.0
    draft = target[:, :gamma].clone()
    a, b = sorted(torch.randperm(V, generator=g)[:2].tolist())
    draft[0, 0, a] -= 0.01
    draft[0, 0, b] -= 0.01
    x = torch.randint(0, V, (1, gamma), generator=g).to(torch.int32)
    u = torch.ones(1, gamma)
    noise = torch.empty(1, V).exponential_(1, generator=g)
    p = S.logits_to_probs(target, 1.0)[0, 0]
    q = S.logits_to_probs(draft, 1.0)[0, 0]
    d = torch.clamp(p - q, min=0)  # the residual before its normalisation
    assert float(d[a]) > 0 and float(d[b]) > 0 and int((d > 0).sum()) == 2
    assert float(d[a] / p[a]) < 0.02  # the residual is a near cancellation
    r = S.residual_distribution(p, q)
    noise[0, a] = float(r[a]) * 1e-3  # key_a ~ 1000, far above the rest (r = 0 elsewhere)
    noise[0, b] = float(r[b]) * 1e-3 / (1.0 + gap)
    return target, draft, x, u, noise, (b if gap > 0 else a)


@pytest.mark.parametrize("gap", [2e-4, -2e-4])
def test_cancelling_residual_near_tie_in_logits_mode(cuda, gap):
    """Two residual keys 2e-4 apart where r = p - q cancels to ~1% of p: the
    fast race's keys carry up to ~8e-4 of relative error there (p and q each
    up to 4e-6 off torch's), beyond the fixed 1e-6 tie window, so the kernel's
    tie test adds the keys' own bound and re-races exactly; the token must be
    the oracle's, and since the bound exceeds the gap the draw is flagged."""
    target, draft, x, u, noise, tok = _cancelling_residual_case(7 if gap > 0 else 8, 151936, gap)
    want = S.verify_from_logits(target, draft, x, u, noise, 1.0)
    assert want[0][-1] == tok
    res = es.verify_sample(target.to(cuda), draft.to(cuda), x.to(cuda), u.to(cuda), noise.to(cuda), 1.0)
    assert res.accepted_lists() == want
    # r is ~1% of p, so the probabilities' 4e-6 error is ~8e-4 of the keys:
    # beyond the 2e-4 gap, the draw is reported
    assert res.flags.tolist() == [_hip.FLAG_DRAW_BAND]


def test_cancelling_token_outside_the_top_two_is_flagged(cuda):
    """Logits mode, row 0 rejected: the draft row equals the target row except
    token d, lowered by 0.5, so the true residual sits at d alone and every
    other token's p - q is a near cancellation (the normalisers differ by
    ~p_d 0.4), which fp32 rounding can leave slightly positive on either side.
    Token c, the row's most probable, gets an Exp(1) entry small enough that
    its residual's rounding error over E_c reaches twice d's key: c never
    leads the fast race (its computed residual is ~0), but the reference's
    rounding could make it win, so the draw must carry SPV_FLAG_DRAW_BAND (and
    match the oracle if it does not)."""
    V, gamma = 151936, 3
    g = torch.Generator().manual_seed(11)
    target = torch.randn(1, gamma + 1, V, generator=g) * 2.0
    draft = target[:, :gamma].clone()
    p0 = S.logits_to_probs(target, 1.0)[0, 0]
    c = int(p0.argmax())
    order = torch.argsort(p0)
    d = int(order[V // 2])  # a token of median probability
    draft[0, 0, d] -= 0.5
    x = torch.randint(0, V, (1, gamma), generator=g).to(torch.int32)
    u = torch.ones(1, gamma)
    noise = torch.empty(1, V).exponential_(1, generator=g)
    p = S.logits_to_probs(target, 1.0)[0, 0]
    q = S.logits_to_probs(draft, 1.0)[0, 0]
    r_d = float(p[d] - q[d])
    assert r_d > 0
    key_d = r_d / float(noise[0, d])
    # c's fast-key bound is about 4e-6 (p_c + q_c) / E_c: make it 2 key_d
    noise[0, c] = 4e-6 * float(p[c] + q[c]) / (2.0 * key_d)
    want = S.verify_from_logits(target, draft, x, u, noise, 1.0)
    res = es.verify_sample(target.to(cuda), draft.to(cuda), x.to(cuda), u.to(cuda), noise.to(cuda), 1.0)
    flags = res.flags.tolist()
    print("cancelling token: oracle draws {}, kernel {}, flags {}".format(want[0][-1], res.accepted_lists()[0][-1],
                                                                          flags))
    assert flags[0] & _hip.FLAG_DRAW_BAND
    _check_flagged(res, want, "cancelling token outside the top two")


def test_fused_sampler_probs_mode_matches_batch_accept(cuda):
    g, target, draft, u, noise = _workload(7, B=8, gamma=3, V=5000)
    p, q = S.logits_to_probs(target, 1.0), S.logits_to_probs(draft, 1.0)
    x = _proposals(draft, 1.0, g)
    want = S.batch_accept_noise(p, q, x, u, noise)
    res = es.verify_sample(p.to(cuda), q.to(cuda), x.to(cuda), u.to(cuda), noise.to(cuda), 1.0,
                           is_probs=True)
    assert res.accepted_lists() == want


def test_identical_rows_take_the_p_fallback(cuda):
    # p == q: every proposal drawn from q is accepted w.p. 1 unless u >= 1;
    # force a rejection with u = 1.0 so the residual is empty and p is raced.
    g, target, _, _, noise = _workload(9, B=4, gamma=2, V=3000)
    draft = target[:, :2].clone()
    x = _proposals(draft, 1.0, g)
    u = torch.ones(4, 2)
    want = S.verify_from_logits(target, draft, x, u, noise, 1.0)
    res = es.verify_sample(target.to(cuda), draft.to(cuda), x.to(cuda), u.to(cuda), noise.to(cuda), 1.0)
    assert res.accepted_lists() == want


@pytest.mark.parametrize("eos", [None, 3])
def test_commit_cut_matches_oracle(cuda, eos):
    B, gamma, V = 16, 4, 8
    g = torch.Generator().manual_seed(5)
    target = torch.randn(B, gamma + 1, V, generator=g)
    draft = target[:, :gamma] + 0.3 * torch.randn(B, gamma, V, generator=g)
    x = _proposals(draft, 0.0, g)
    u = torch.rand(B, gamma, generator=g)
    start = torch.randint(10, 100, (B,), generator=g)
    remaining = torch.randint(-2, 7, (B,), generator=g)
    want = S.verify_from_logits(target, draft, x, u, torch.ones(B, V), 0.0)
    res = es.verify_sample(target.to(cuda), draft.to(cuda), x.to(cuda), u.to(cuda), None, 0.0,
                           start_pos=start.to(cuda), remaining=remaining.to(cuda), eos_id=eos)
    assert res.accepted_lists() == want
    n_commit, fin, new_len = res.n_commit.tolist(), res.finished.tolist(), res.new_len.tolist()
    for b in range(B):
        kept, eos_hit = ref_step.cut_accepted(want[b], int(remaining[b]), eos)
        k = len(kept)
        assert n_commit[b] == k
        assert fin[b] == int(eos_hit or k == 0 or k >= int(remaining[b]))
        assert new_len[b] == (int(start[b]) + k if k > 0 else -1)


SAMPLE_COUNTER_BYTES = 1 << 19  # SPV_SAMPLE_COUNTER_BYTES


@pytest.mark.parametrize("T", [1.0, 0.0])
def test_repeated_calls_are_identical_and_leave_counters_zero(cuda, T):
    g, target, draft, u, noise = _workload(21, B=16, gamma=5, V=20000)
    x = _proposals(draft, T, g)
    want = S.verify_from_logits(target, draft, x, u, noise, T)
    args = (target.to(cuda), draft.to(cuda), x.to(cuda), u.to(cuda), noise.to(cuda) if T > 0 else None, T)
    outs = []
    for _ in range(3):
        res = es.verify_sample(*args)
        assert res.accepted_lists() == want
        outs.append((res.accept_len.clone(), res.out_tokens.clone()))
        torch.cuda.synchronize()
        assert int(torch.count_nonzero(es._workspace.current(cuda)[:SAMPLE_COUNTER_BYTES])) == 0
    for a, o in outs[1:]:
        assert torch.equal(a, outs[0][0]) and torch.equal(o, outs[0][1])


def test_workspace_reused_across_batch_sizes(cuda):
    # One workspace serves calls of growing and shrinking B; the counters sit
    # at fixed offsets, so no call reads another call's partials as counters.
    es._workspace.get(4 << 20, cuda)
    for i, B in enumerate([4, 24, 8, 40]):
        # odd vocabularies take the element-wise paths
        g, target, draft, u, noise = _workload(30 + i, B=B, gamma=4, V=12000 + i % 2)
        x = _proposals(draft, 1.0, g)
        want = S.verify_from_logits(target, draft, x, u, noise, 1.0)
        res = es.verify_sample(target.to(cuda), draft.to(cuda), x.to(cuda), u.to(cuda), noise.to(cuda), 1.0)
        assert res.accepted_lists() == want, B
