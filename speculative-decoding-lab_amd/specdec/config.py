"""Sampling configuration used by the verify path (reference specdec/config.py:19-48)."""

from __future__ import annotations

from dataclasses import asdict, dataclass
from typing import Any, Dict


@dataclass
class SamplingConfig:
    """``temperature <= 0`` selects greedy (one-hot) decoding."""

    temperature: float = 0.0
    top_k: int = 0
    top_p: float = 1.0

    @property
    def is_greedy(self) -> bool:
        return self.temperature <= 0.0

    def describe(self) -> str:
        if self.is_greedy:
            return "greedy"
        parts = ["T={:.2f}".format(self.temperature)]
        if self.top_k > 0:
            parts.append("top_k={}".format(self.top_k))
        if self.top_p < 1.0:
            parts.append("top_p={:.2f}".format(self.top_p))
        return ", ".join(parts)

    def to_dict(self) -> Dict[str, Any]:
        payload = asdict(self)
        payload["mode"] = "greedy" if self.is_greedy else "sampling"
        return payload
