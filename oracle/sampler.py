"""CPU restatement of the reference rejection-sampling step (test infrastructure only).

Follows the reference:

* ``logits_to_probs``        -- specdec/sampler.py:19-36: greedy one-hot at
                                ``argmax`` for T <= 0, else the softmax of
                                ``logits.float() / max(T, 1e-12)`` after
                                ``apply_top_k`` then ``apply_top_p`` (no-ops at the
                                defaults top_k=0 / top_p=1.0, specdec/config.py:27-29)
* ``apply_top_k``            -- specdec/sampler.py:39-44 (values below the k-th
                                largest become -inf; ties at it stay)
* ``apply_top_p``            -- specdec/sampler.py:47-56 (descending sort, cumulative
                                softmax, the shifted mask ``cum - p >= top_p``)
* ``acceptance_probability`` -- specdec/sampler.py:86-92 (fp32 -> Python float,
                                both 1e-12 branches, ``min(1, p/q)`` in float64)
* ``residual_distribution``  -- specdec/sampler.py:72-83
* ``sample_token``           -- specdec/sampler.py:59-69 (``torch.multinomial`` on
                                the CPU)
* ``race_argmax``            -- the same draw with the randomness supplied by the
                                caller: ``argmax(probs / E)``, ``E ~ Exp(1)^V``
* ``batch_accept``           -- engine/spec_scheduler.py:41-88 with a live
                                ``torch.Generator`` (records the uniforms and the
                                exponential rows it consumed)
* ``batch_accept_noise``     -- the same rule with caller-supplied ``u[b][j]`` and
                                one ``E[b]`` row per sequence

The top-k / top-p filters are pinned by the reference's own filter tests
(tests/test_sampler.py:34-49, 76-78) and by a brute force that keeps each value
by counting larger values (top-k) or summing the mass of larger values in
float64 (top-p), on rows without ties; equal values at the nucleus boundary
are ordered by torch's (unstable) sort, so which of them stays is unpinned.

Pinned by tests/test_oracle_sampler.py: the reference's one-hot cases
(tests/test_spec_accept.py:29-73), its sampler properties (tests/test_sampler.py:
18-64), the library identity ``multinomial(p, 1, g) == argmax(p / E)`` with ``E``
drawn by ``exponential_`` from a clone of ``g`` (checked live against torch),
``batch_accept`` == ``batch_accept_noise`` on the recorded noise, and an exact
enumeration showing the accept rule reproduces the target distribution
(Leviathan et al. 2023, Thm 1) on a vocab-8 toy.
"""

from __future__ import annotations

from typing import Dict, List, Optional, Sequence, Tuple

import torch

EPS = 1e-12  # specdec/sampler.py:16


def apply_top_k(logits: torch.Tensor, top_k: int) -> torch.Tensor:
    if top_k <= 0 or top_k >= logits.shape[-1]:
        return logits
    kth_value = torch.topk(logits, top_k, dim=-1).values[..., -1, None]
    return torch.where(logits < kth_value, torch.full_like(logits, float("-inf")), logits)


def apply_top_p(logits: torch.Tensor, top_p: float) -> torch.Tensor:
    if top_p >= 1.0 or top_p <= 0.0:
        return logits
    sorted_logits, sorted_index = torch.sort(logits, descending=True, dim=-1)
    probs = torch.softmax(sorted_logits, dim=-1)
    mask = torch.cumsum(probs, dim=-1) - probs >= top_p
    sorted_logits = sorted_logits.masked_fill(mask, float("-inf"))
    return sorted_logits.scatter(-1, sorted_index, sorted_logits)


def logits_to_probs(logits: torch.Tensor, temperature: float, top_k: int = 0,
                    top_p: float = 1.0) -> torch.Tensor:
    logits = logits.float()
    if temperature <= 0.0:
        probs = torch.zeros_like(logits)
        probs.scatter_(-1, logits.argmax(dim=-1, keepdim=True), 1.0)
        return probs
    scaled = logits / max(temperature, EPS)
    return torch.softmax(apply_top_p(apply_top_k(scaled, top_k), top_p), dim=-1)


def filter_logits(logits: torch.Tensor, temperature: float, top_k: int = 0, top_p: float = 1.0) -> torch.Tensor:
    """The scaled, filtered logits whose softmax ``logits_to_probs`` returns (T > 0)."""
    return apply_top_p(apply_top_k(logits.float() / max(temperature, EPS), top_k), top_p)


def acceptance_probability(p: torch.Tensor, q: torch.Tensor, token_id: int) -> float:
    q_prob = float(q[token_id].item())
    p_prob = float(p[token_id].item())
    if q_prob <= EPS:
        return 1.0 if p_prob > EPS else 0.0
    return float(min(1.0, p_prob / q_prob))


def residual_distribution(p: torch.Tensor, q: torch.Tensor) -> torch.Tensor:
    residual = torch.clamp(p - q, min=0.0)
    total = residual.sum()
    if float(total) <= EPS:
        return p / p.sum().clamp_min(EPS)
    return residual / total


def sample_token(probs: torch.Tensor, generator: Optional[torch.Generator] = None) -> int:
    flat = probs.detach().reshape(-1).to(device="cpu", dtype=torch.float32)
    return int(torch.multinomial(flat, num_samples=1, generator=generator).item())


def draw_race_noise(vocab: int, generator: Optional[torch.Generator] = None) -> torch.Tensor:
    """The ``Exp(1)`` row one multinomial draw consumes from ``generator``."""
    return torch.empty(vocab, dtype=torch.float32).exponential_(1, generator=generator)


def race_argmax(probs: torch.Tensor, noise: torch.Tensor) -> int:
    """``argmax(probs / E)``: the multinomial draw given its exponential row."""
    flat = probs.detach().reshape(-1).to(dtype=torch.float32)
    return int(torch.argmax(flat / noise.reshape(-1).to(torch.float32)).item())


def batch_accept(p_by_sid: Dict[int, torch.Tensor], q_by_sid: Dict[int, Sequence[torch.Tensor]],
                 proposals_by_sid: Dict[int, Sequence[int]], generator: torch.Generator,
                 record: Optional[Dict[int, Tuple[List[float], torch.Tensor]]] = None
                 ) -> Dict[int, List[int]]:
    """spec_scheduler.py:46-88; ``record[sid] = (uniforms, exp row)`` if given."""
    out: Dict[int, List[int]] = {}
    for sid, p_all in p_by_sid.items():
        q_rows = q_by_sid[sid]
        props = proposals_by_sid[sid]
        accepted: List[int] = []
        us: List[float] = []
        rejected = False
        for j in range(len(props)):
            u = float(torch.rand(1, generator=generator).item())  # spec_scheduler.py:41-43
            us.append(u)
            if u < acceptance_probability(p_all[j], q_rows[j], props[j]):
                accepted.append(int(props[j]))
            else:
                resid = residual_distribution(p_all[j], q_rows[j])
                e = draw_race_noise(resid.numel(), generator)
                accepted.append(race_argmax(resid, e))
                rejected = True
                break
        if not rejected:
            e = draw_race_noise(p_all.shape[-1], generator)
            accepted.append(race_argmax(p_all[len(props)], e))
        if record is not None:
            record[sid] = (us, e)
        out[sid] = accepted
    return out


def batch_accept_noise(p: torch.Tensor, q: torch.Tensor, proposals: torch.Tensor,
                       u: torch.Tensor, noise: torch.Tensor) -> List[List[int]]:
    """Batched form: p (B, g+1, V), q (B, g, V), proposals (B, g), u (B, g), noise (B, V)."""
    B, gamma = proposals.shape
    out = []
    for b in range(B):
        accepted: List[int] = []
        rejected = False
        for j in range(gamma):
            x = int(proposals[b, j])
            if float(u[b, j]) < acceptance_probability(p[b, j], q[b, j], x):
                accepted.append(x)
            else:
                accepted.append(race_argmax(residual_distribution(p[b, j], q[b, j]), noise[b]))
                rejected = True
                break
        if not rejected:
            accepted.append(race_argmax(p[b, gamma], noise[b]))
        out.append(accepted)
    return out


def verify_from_logits(target_logits: torch.Tensor, draft_logits: torch.Tensor,
                       proposals: torch.Tensor, u: torch.Tensor, noise: torch.Tensor,
                       temperature: float, top_k: int = 0, top_p: float = 1.0) -> List[List[int]]:
    """logits_to_probs on every row (spec_scheduler.py:249, 261-263), then accept."""
    p = logits_to_probs(target_logits, temperature, top_k, top_p)
    q = logits_to_probs(draft_logits, temperature, top_k, top_p)
    return batch_accept_noise(p, q, proposals, u, noise)


def acceptance_matrix(p: torch.Tensor, q: torch.Tensor, proposals: torch.Tensor) -> torch.Tensor:
    """float64 ``a[b, j]`` = acceptance_probability(p[b, j], q[b, j], x[b, j])."""
    B, gamma = proposals.shape
    a = torch.empty((B, gamma), dtype=torch.float64)
    for b in range(B):
        for j in range(gamma):
            a[b, j] = acceptance_probability(p[b, j], q[b, j], int(proposals[b, j]))
    return a
