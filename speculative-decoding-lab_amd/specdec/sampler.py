"""Logit post-processing and the rejection-sampling primitives on the GPU.

Drop-in for the reference's specdec/sampler.py:16-99 (the part on the verify
path). Every function runs a HIP kernel of libspecverify; tensors must live on a
GPU. Randomness still comes from the caller's CPU ``torch.Generator``:
``sample_token`` draws the ``Exp(1)`` row that ``torch.multinomial`` would
consume from it (multinomial with one sample is ``argmax(p / E)`` with ``E``
from ``exponential_``), copies it to the device and races there, so the
generator state afterwards is the reference's.
"""

from __future__ import annotations

from typing import Optional

import torch

from engine import _hip
from engine._hip import call, ptr

from .config import SamplingConfig

_EPS = 1e-12  # specdec/sampler.py:16


def _rows(x: torch.Tensor) -> torch.Tensor:
    _hip.require_gpu(x.device)
    return x.detach().float().contiguous()


def logits_to_probs(logits: torch.Tensor, sampling: SamplingConfig) -> torch.Tensor:
    """Greedy one-hot (T <= 0), else ``softmax`` of ``logits / max(T, 1e-12)``
    after top-k then top-p filtering (specdec/sampler.py:19-56)."""
    top_k = int(getattr(sampling, "top_k", 0) or 0)
    top_p = float(getattr(sampling, "top_p", 1.0))
    z = _rows(logits)
    V = int(z.shape[-1])
    out = torch.empty_like(z)
    rows = z.numel() // V if V else 0
    temperature = 0.0 if sampling.is_greedy else float(sampling.temperature)
    if temperature > 0 and _hip.filtering(top_k, top_p, V):
        z = _hip.filter_rows(z, temperature, top_k, top_p)  # scaled and filtered: softmax at T = 1
        temperature = 1.0
    call("spv_logits_to_probs", ptr(z), ptr(out), rows, V, temperature, _hip.stream_of(z.device))
    return out


def apply_top_k(logits: torch.Tensor, top_k: int) -> torch.Tensor:
    """Values below the k-th largest become -inf (specdec/sampler.py:39-44)."""
    z = _rows(logits)
    return _hip.filter_rows(z, 1.0, int(top_k), 1.0).reshape(logits.shape) if _hip.filtering(top_k, 1.0, z.shape[-1]) \
        else z.reshape(logits.shape)


def apply_top_p(logits: torch.Tensor, top_p: float) -> torch.Tensor:
    """Nucleus filtering (specdec/sampler.py:47-56)."""
    z = _rows(logits)
    return _hip.filter_rows(z, 1.0, 0, float(top_p)).reshape(logits.shape) if _hip.filtering(0, top_p, z.shape[-1]) \
        else z.reshape(logits.shape)


def draw_race_noise(vocab: int, generator: Optional[torch.Generator] = None) -> torch.Tensor:
    """The ``Exp(1)`` row one ``torch.multinomial(p, 1)`` draw takes from ``generator`` (CPU)."""
    return torch.empty(int(vocab), dtype=torch.float32).exponential_(1, generator=generator)


def sample_token(probs: torch.Tensor, generator: Optional[torch.Generator] = None) -> int:
    """Draw one token id from a probability vector (specdec/sampler.py:59-69)."""
    flat = _rows(probs).reshape(-1)
    noise = draw_race_noise(flat.numel(), generator).to(flat.device, non_blocking=False)
    out = torch.empty(1, dtype=torch.int32, device=flat.device)
    call("spv_race_argmax", ptr(flat), ptr(noise), int(flat.numel()), ptr(out),
         _hip.stream_of(flat.device))
    return int(out.item())


def residual_distribution(p: torch.Tensor, q: torch.Tensor) -> torch.Tensor:
    """Normalised ``(p - q)_+``, or ``p / sum(p)`` when that is empty (specdec/sampler.py:72-83)."""
    pf, qf = _rows(p).reshape(-1), _rows(q).reshape(-1)
    if pf.numel() != qf.numel():
        raise ValueError("p and q must have the same size")
    out = torch.empty_like(pf)
    call("spv_residual", ptr(pf), ptr(qf), ptr(out), int(pf.numel()), _hip.stream_of(pf.device))
    return out.reshape(p.shape)


def acceptance_probability(p: torch.Tensor, q: torch.Tensor, token_id: int) -> float:
    """``min(1, p(x) / q(x))`` in float64 with the 1e-12 branches (specdec/sampler.py:86-92)."""
    pf, qf = _rows(p).reshape(-1), _rows(q).reshape(-1)
    token_id = int(token_id)
    if not 0 <= token_id < pf.numel():
        raise IndexError("token id {} out of range".format(token_id))
    out = torch.empty(1, dtype=torch.float64, device=pf.device)
    call("spv_accept_prob", ptr(pf), ptr(qf), token_id, ptr(out), _hip.stream_of(pf.device))
    return float(out.item())


def build_generator(seed: int, device: Optional[torch.device] = None) -> torch.Generator:
    """Deterministic CPU generator (specdec/sampler.py:95-99)."""
    generator = torch.Generator(device="cpu")
    generator.manual_seed(int(seed))
    return generator
