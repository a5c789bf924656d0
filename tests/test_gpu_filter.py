"""GPU parity of top-k / top-p filtering (specdec/sampler.py:19-56) against the oracle.

* ``spv_filter_logits``: over rows of V = 151,936 logits ~ N(0, 2^2) at T = 1
  and 0.7, with top_k in {50, 1000}, top_p in {0.9, 0.5} and their
  combinations, the kept values are identical to the oracle's
  ``apply_top_p(apply_top_k(z / T))`` (-inf everywhere else) and so is the
  kept set, except where the nucleus rule is decided within rounding. The
  kernel sums masses in fp64 against the exact total; torch's fp32 softmax of
  a 151,936-entry row sums to 1 +- eps (its normalisation rounds), which
  shifts every preceding mass it compares with top_p by up to eps. A value
  whose exact (float64) preceding mass lies within 2 eps + 2e-6 of top_p may
  therefore fall either way. The kernel reports, per row, how many values lie
  within its fixed window (5e-5 W, W the kept mass) of the edge: the test
  checks that the window covers 2 eps + 2e-6 on every row, that every
  differing value lies in it, and that the kernel's count equals the count of
  the oracle's float64 masses (up to the values within 1e-6 W of the window's
  own edges, where the kernel's fp32-rounded masses may place them otherwise).
  Ties at the k-th value all stay.
* the reference's own filter tests (tests/test_sampler.py:34-49, 76-78).
* the fused verify sampler at the Qwen2.5 vocabulary (B = 64, gamma = 5,
  V = 151,936, T = 1) with top_k = 50, top_k = 1000 and top_p = 0.9: token ids,
  accept lengths bit-exact against the oracle; batched draft sampling with a
  filter likewise.
"""

from __future__ import annotations

import pytest
import torch

from engine import _hip
from engine import spec_scheduler as es
from oracle import sampler as S
from specdec import sampler as gs
from specdec.config import SamplingConfig

pytestmark = pytest.mark.gpu

V = 151936


def _softmax_sum_error(x, top_k):
    """|sum of torch's fp32 softmax over the sorted kept values - 1| (the
    reference's normalisation error on this row)."""
    r = S.apply_top_k(x.float(), top_k)
    s, _ = torch.sort(r, descending=True)
    return abs(float(torch.softmax(s, -1).double().sum()) - 1.0)


def _mass_before(x, top_k):
    """float64 mass before each value of a row in descending order, over what
    top-k kept (inf where top-k dropped the value)."""
    r = S.apply_top_k(x.float(), top_k).double()
    keep = torch.isfinite(r)
    w = torch.where(keep, torch.exp(r - r[keep].max()), torch.zeros_like(r))
    order = torch.argsort(r, descending=True, stable=True)
    before = torch.empty_like(w)
    before[order] = torch.cumsum(w[order], 0) - w[order]
    before = before / w.sum()
    return torch.where(keep, before, torch.full_like(before, float("inf")))


WINDOW = 5e-5  # the kernel's window around the nucleus edge, relative to the kept mass


def _compare_kept(got, want, scaled, top_k, top_p, counts=None):
    """Kept values equal where both keep; a differing kept flag only where the
    rule is decided within rounding; the kernel's window counts equal the
    oracle's. Returns (values in the window, differing)."""
    gk, wk = torch.isfinite(got), torch.isfinite(want)
    both = gk & wk
    assert torch.equal(got[both], want[both])
    amb = diff = 0
    for r in range(got.shape[0]):
        d = (gk[r] != wk[r]).nonzero().flatten()
        if not 0.0 < top_p < 1.0:
            assert d.numel() == 0, r
            if counts is not None:
                assert int(counts[r]) == 0
            continue
        rounding = 2 * _softmax_sum_error(scaled[r], top_k) + 2e-6
        assert rounding <= WINDOW, (r, rounding)
        dist = (_mass_before(scaled[r], top_k) - top_p).abs()
        near = dist < WINDOW
        amb += int(near.sum())
        diff += int(d.numel())
        assert bool(near[d].all()), (r, d.tolist()[:8])
        if counts is not None:
            edge = int(((dist - WINDOW).abs() < 1e-6).sum())
            assert abs(int(counts[r]) - int(near.sum())) <= edge, (r, int(counts[r]), int(near.sum()), edge)
    return amb, diff


@pytest.mark.parametrize("T", [1.0, 0.7])
@pytest.mark.parametrize("top_k,top_p", [(50, 1.0), (1000, 1.0), (0, 0.9), (0, 0.5), (1000, 0.9), (50, 0.5)])
def test_filter_rows_match_the_oracle(cuda, T, top_k, top_p):
    g = torch.Generator().manual_seed(top_k * 7 + int(top_p * 10) + int(T * 100))
    z = torch.randn(6, V, generator=g) * 2
    want = S.filter_logits(z, T, top_k, top_p)
    got, counts = _hip.filter_rows(z.to(cuda), T, top_k, top_p, ambiguous=True)
    got_plain = _hip.filter_rows(z.to(cuda), T, top_k, top_p)
    assert torch.equal(got, got_plain)  # the window searches change nothing kept
    amb, diff = _compare_kept(got.cpu(), want, z / T, top_k, top_p, counts.cpu())
    print("top_k {} top_p {} T {}: {} values within the window (kernel {}), {} differ".format(
        top_k, top_p, T, amb, int(counts.sum()), diff))


def test_window_count_at_a_crafted_edge(cuda):
    """Rows built so that many distinct values sit at the nucleus edge: 4,000
    logits spaced 1e-6 apart carry nearly all the mass, so each holds ~1/4000
    of W and the window (5e-5 W on each side of 0.6 W) holds at most the one
    value whose preceding mass is nearest the edge; and a row whose edge falls
    far from any value's preceding mass (count 0)."""
    z = torch.full((2, V), -30.0)
    z[0, :4000] = torch.arange(4000, dtype=torch.float32) * 1e-6
    z[1, 10] = 5.0
    z[1, 20] = 4.0
    want = S.filter_logits(z, 1.0, 0, 0.6)
    got, counts = _hip.filter_rows(z.to(cuda), 1.0, 0, 0.6, ambiguous=True)
    _compare_kept(got.cpu(), want, z, 0, 0.6, counts.cpu())
    assert int(counts[0]) <= 1
    assert int(counts[1]) == 0


def test_ties_at_the_kth_value_all_stay(cuda):
    z = torch.zeros(2, 1000)
    z[0, :10] = torch.tensor([9.0, 8.0, 7.0, 7.0, 7.0, 5.0, 4.0, 3.0, 2.0, 1.0])
    z[1, 500:505] = 6.0  # five equal maxima, top_k = 2
    want = S.filter_logits(z, 1.0, 3, 1.0)
    got = _hip.filter_rows(z.to(cuda), 1.0, 3, 1.0).cpu()
    assert torch.equal(got, want)
    assert int(torch.isfinite(got[0]).sum()) == 5 and int(torch.isfinite(got[1]).sum()) == 5


def test_reference_filter_tests_on_the_gpu(cuda):
    f = gs.apply_top_k(torch.tensor([[5.0, 4.0, 3.0, 2.0, 1.0]], device=cuda), 2).cpu()
    assert torch.isfinite(f).sum().item() == 2 and float(f[0, 0]) == 5.0
    f = gs.apply_top_p(torch.log(torch.tensor([[0.5, 0.3, 0.15, 0.05]], device=cuda)), 0.8)
    probs = torch.softmax(f, dim=-1).cpu()
    assert float(probs[0, 3]) == 0.0 and float(probs.sum()) >= 0.8 - 1e-6
    logits = torch.randn(1, 8)
    assert torch.allclose(gs.apply_top_p(logits.to(cuda), 1.0).cpu(), logits)


def test_logits_to_probs_with_filters(cuda):
    g = torch.Generator().manual_seed(3)
    z = torch.randn(4, 5000, generator=g) * 2
    cfg = SamplingConfig(temperature=0.8, top_k=100, top_p=0.9)
    got = gs.logits_to_probs(z.to(cuda), cfg).cpu()
    want = S.logits_to_probs(z, 0.8, 100, 0.9)
    assert torch.equal(got == 0, want == 0)
    assert torch.allclose(got, want, rtol=2e-6, atol=1e-9)


def _workload(seed, B=64, gamma=5):
    g = torch.Generator().manual_seed(seed)
    target = torch.randn(B, gamma + 1, V, generator=g) * 2.0
    draft = target[:, :gamma] + torch.randn(B, gamma, V, generator=g)
    u = torch.rand(B, gamma, generator=g)
    noise = torch.empty(B, V).exponential_(1, generator=g)
    return g, target, draft, u, noise


@pytest.mark.parametrize("top_k,top_p", [(50, 1.0), (1000, 1.0), (0, 0.9)])
def test_fused_sampler_with_filters(cuda, top_k, top_p):
    g, target, draft, u, noise = _workload(70 + top_k)
    q = S.logits_to_probs(draft, 1.0, top_k, top_p)
    x = torch.multinomial(q.reshape(-1, V), 1, generator=g).reshape(64, 5)
    want = S.verify_from_logits(target, draft, x, u, noise, 1.0, top_k, top_p)
    res = es.verify_sample(target.to(cuda), draft.to(cuda), x.to(cuda), u.to(cuda), noise.to(cuda), 1.0,
                           top_k=top_k, top_p=top_p)
    flags = res.flags.tolist()
    for b, (g_, w, f) in enumerate(zip(res.accepted_lists(), want, flags)):
        assert g_ == w or f, (b, g_, w)
    if top_p == 1.0:
        assert flags.count(0) >= len(flags) - 2  # top-k alone is exact; decisions rarely flagged
    print("{} of {} sequences flagged ({} with a row at the nucleus edge)".format(
        sum(1 for f in flags if f), len(flags), sum(1 for f in flags if f & _hip.FLAG_TOP_P_BAND)))


def test_draft_sample_with_filters(cuda):
    g = torch.Generator().manual_seed(5)
    z = torch.randn(16, V, generator=g) * 2
    e = torch.empty(16, V).exponential_(1, generator=g)
    for top_k, top_p in ((50, 1.0), (0, 0.9), (200, 0.5)):
        want = [S.race_argmax(S.logits_to_probs(z[b], 1.0, top_k, top_p), e[b]) for b in range(16)]
        got = es.draft_sample(z.to(cuda), 1.0, e.to(cuda), top_k=top_k, top_p=top_p)
        assert got.tolist() == want, (top_k, top_p)
