"""KV pool sizing (reference engine/scheduler.py:351-374)."""

from __future__ import annotations

from typing import Any, Optional

import torch

from . import _hip
from .config import EngineConfig
from .kv import PagedKVCache


def bytes_per_block(num_layers: int, block_size: int, num_kv_heads: int, head_dim: int,
                    dtype: torch.dtype) -> int:
    """Bytes of one physical block across all layers, K + V (scheduler.py:351-362).

    An fp8 (e4m3) pool, which the reference does not have, also holds one fp32
    scale per (layer, block, K | V): 8 bytes per layer.
    """
    itemsize = torch.empty((), dtype=dtype).element_size()
    scales = 8 * num_layers if dtype == getattr(torch, "float8_e4m3fn", None) else 0
    return 2 * num_layers * block_size * num_kv_heads * head_dim * itemsize + scales


def build_kv(model: Any, engine_cfg: EngineConfig, device: torch.device) -> PagedKVCache:
    """A cache sized from a model's shape and the engine config (scheduler.py:365-374)."""
    return PagedKVCache(
        num_layers=model.num_layers,
        num_kv_heads=model.num_kv_heads,
        head_dim=model.head_dim,
        capacity_blocks=engine_cfg.max_num_blocks,
        block_size=engine_cfg.block_size,
        device=device,
        dtype=model.dtype,
    )


def blocks_for_hbm(num_layers: int, block_size: int, num_kv_heads: int, head_dim: int,
                   dtype: torch.dtype, device: torch.device, reserve_bytes: int = 8 << 30,
                   fraction: float = 0.9, limit_bytes: Optional[int] = None) -> int:
    """Pool capacity (blocks) that fits the GPU's free memory.

    ``fraction`` of ``free - reserve_bytes`` (optionally capped at
    ``limit_bytes``) divided by the per-block footprint of all layers.
    """
    device = _hip.require_gpu(device)
    free, _total = torch.cuda.mem_get_info(device)
    budget = max(0, int((free - reserve_bytes) * fraction))
    if limit_bytes is not None:
        budget = min(budget, int(limit_bytes))
    return budget // bytes_per_block(num_layers, block_size, num_kv_heads, head_dim, dtype)
