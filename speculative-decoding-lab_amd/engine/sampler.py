"""Seeded CPU generator for the engine (reference engine/sampler.py:20-24)."""

from __future__ import annotations

from typing import Optional

import torch

__all__ = ["build_generator"]


def build_generator(seed: int, device: Optional[torch.device] = None) -> torch.Generator:
    """Deterministic CPU generator seeded with ``seed``."""
    generator = torch.Generator(device="cpu")
    generator.manual_seed(int(seed))
    return generator
