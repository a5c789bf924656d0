"""Engine configuration on the verify path (reference engine/config.py:21-62)."""

from __future__ import annotations

from dataclasses import asdict, dataclass
from typing import Any, Dict


@dataclass
class EngineConfig:
    """Model + paged KV parameters for a single serving engine."""

    model_id: str = "Qwen/Qwen2.5-1.5B"
    device: str = "auto"
    dtype: str = "auto"
    cache_dir: str = "models"
    block_size: int = 16        # tokens per physical KV block
    max_num_blocks: int = 256   # physical block capacity
    max_batch: int = 16         # soft cap on sequences per step

    def to_dict(self) -> Dict[str, Any]:
        return asdict(self)


@dataclass
class SamplingConfig:
    """Decoding temperature; ``temperature <= 0`` selects greedy decoding."""

    temperature: float = 0.0

    @property
    def is_greedy(self) -> bool:
        return self.temperature <= 0.0

    def describe(self) -> str:
        return "greedy" if self.is_greedy else "temperature={}".format(self.temperature)

    def to_dict(self) -> Dict[str, Any]:
        return {"temperature": self.temperature, "mode": "greedy" if self.is_greedy else "sampling"}
