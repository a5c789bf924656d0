"""Pool sizing (reference engine/scheduler.py:351-374): bytes per block, the
sized cache of ``build_kv``, and the HBM-sized capacity the full-depth bench
uses."""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from engine.config import EngineConfig
from engine.scheduler import blocks_for_hbm, build_kv, bytes_per_block


@pytest.mark.parametrize("dtype,itemsize", [(torch.bfloat16, 2), (torch.float16, 2), (torch.float32, 4)])
def test_bytes_per_block_is_the_reference_formula(dtype, itemsize):
    # scheduler.py:351-362: 2 (K and V) * layers * block_size * kv_heads * head_dim * itemsize
    for layers, bs, hkv, d in [(1, 16, 2, 128), (36, 16, 2, 128), (24, 16, 2, 64), (2, 4, 2, 16)]:
        assert bytes_per_block(layers, bs, hkv, d, dtype) == 2 * layers * bs * hkv * d * itemsize


def test_bytes_per_block_at_the_full_depth_and_fp8_shapes():
    # Qwen2.5-3B-shaped pool: 36 layers, 2 kv heads, head_dim 128, bf16
    assert bytes_per_block(36, 16, 2, 128, torch.bfloat16) == 589_824
    # the same in fp8 e4m3: half the bytes plus one fp32 scale per (layer, K|V)
    assert bytes_per_block(36, 16, 2, 128, torch.float8_e4m3fn) == 294_912 + 36 * 8


def test_blocks_for_hbm_has_no_cpu_path():
    from engine._hip import HipLibraryError

    with pytest.raises(HipLibraryError):
        blocks_for_hbm(36, 16, 2, 128, torch.bfloat16, torch.device("cpu"))


@pytest.mark.gpu
def test_build_kv_sizes_the_pool_from_the_model_and_config(cuda):
    model = SimpleNamespace(num_layers=3, num_kv_heads=2, head_dim=64, dtype=torch.bfloat16)
    cfg = EngineConfig(block_size=16, max_num_blocks=96)
    kv = build_kv(model, cfg, cuda)
    assert kv.allocator.capacity == 96 and kv.block_size == 16 and kv.num_layers == 3
    assert kv.kv_memory_bytes == 96 * bytes_per_block(3, 16, 2, 64, torch.bfloat16)
    assert kv.allocator.num_allocated == 0 and kv.allocator.free_list() == list(range(96))


@pytest.mark.gpu
def test_blocks_for_hbm_fits_the_budget(cuda):
    free, _total = torch.cuda.mem_get_info(cuda)
    per = bytes_per_block(36, 16, 2, 128, torch.bfloat16)
    n = blocks_for_hbm(36, 16, 2, 128, torch.bfloat16, cuda, reserve_bytes=1 << 30, fraction=0.5)
    budget = int((free - (1 << 30)) * 0.5)
    assert n == budget // per and n * per <= budget < (n + 1) * per
    capped = blocks_for_hbm(36, 16, 2, 128, torch.bfloat16, cuda, limit_bytes=10 * per + 5)
    assert capped == 10
