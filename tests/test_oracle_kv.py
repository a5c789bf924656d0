"""CPU checks that pin the KV-pool oracle (oracle/kv_pool.py).

1. Every assertion of the reference's tests/test_kv.py:44-183 and
   tests/test_spec_accept.py:76-98, restated against the oracle.
2. The LIFO order facts the device kernels must reproduce bit for bit: first
   alloc is ``cap-1``, truncate pushes tail-first, clear pushes forward.
3. Random operation traces checked against an independent model that keeps only
   a set of owned blocks per sequence (ownership, counts and lengths), so an
   order or bookkeeping slip in the oracle shows up as a partition violation.
"""

from __future__ import annotations

import random

import pytest
import torch

from oracle.attention import gather_ctx
from oracle.kv_pool import BlockAllocator, BlockExhaustedError, PagedKVCache


def _kv(block_size=4, capacity=8):
    return PagedKVCache(num_layers=2, num_kv_heads=2, head_dim=8, capacity_blocks=capacity,
                        block_size=block_size)


def _vec(fill=1.0):
    return torch.full((2, 8), fill)


# ---------------------------------------------- reference tests/test_kv.py
def test_allocator_alloc_free_roundtrip():
    a = BlockAllocator(4)
    blocks = [a.alloc() for _ in range(4)]
    assert sorted(blocks) == [0, 1, 2, 3]
    assert a.num_allocated == 4
    a.free(blocks[0])
    a.free(blocks[1])
    assert a.num_allocated == 2
    blocks.extend([a.alloc(), a.alloc()])
    assert a.num_allocated == 4


def test_allocator_exhaustion_raises():
    a = BlockAllocator(2)
    a.alloc()
    a.alloc()
    with pytest.raises(BlockExhaustedError):
        a.alloc()
    a.free(0)
    assert a.alloc() == 0


def test_allocator_free_twice_is_idempotent():
    a = BlockAllocator(3)
    b = a.alloc()
    a.free(b)
    a.free(b)
    assert a.num_allocated == 0


def test_capacity_must_be_positive():
    with pytest.raises(ValueError):
        BlockAllocator(0)


def test_write_allocates_blocks_on_demand():
    kv = _kv()
    kv.add_sequence(0)
    kv.write(0, 0, 0, _vec(), _vec())
    assert kv.seq_lengths[0] == 1 and kv.num_allocated_blocks == 1
    kv.write(0, 0, 2, _vec(), _vec())
    assert kv.num_allocated_blocks == 1 and kv.seq_lengths[0] == 3
    kv.write(0, 0, 4, _vec(), _vec())
    assert kv.num_allocated_blocks == 2 and len(kv.block_tables[0]) == 2


def test_write_out_of_order_extends_length():
    kv = _kv()
    kv.add_sequence(0)
    kv.write(0, 0, 3, _vec(3.0), _vec(3.0))
    assert kv.seq_lengths[0] == 4 and kv.logical_tokens == 4


def test_gather_concatenates_blocks_in_order():
    kv = _kv()
    kv.add_sequence(0)
    for pos in range(9):
        kv.write(0, 0, pos, _vec(float(pos)), _vec(-float(pos)))
    keys = gather_ctx(kv, 0, 0, 9)[0]
    assert keys.shape == (9, 2, 8)
    assert torch.equal(keys[3], torch.full((2, 8), 3.0))


def test_truncate_rollback_frees_blocks():
    kv = _kv()
    kv.add_sequence(0)
    kv.add_sequence(1)
    for pos in range(10):
        kv.write(0, 0, pos, _vec(), _vec())
    before = kv.num_allocated_blocks
    assert before >= 3
    kv.truncate(0, 3)
    assert kv.seq_lengths[0] == 3 and len(kv.block_tables[0]) == 1
    assert kv.num_allocated_blocks < before
    kv.write(0, 1, 4, _vec(), _vec())
    assert kv.seq_lengths[1] == 5 and len(kv.block_tables[1]) == 2


def test_truncate_rewound_sequence_writes_identically():
    kv = _kv()
    kv.add_sequence(0)
    for pos in range(8):
        kv.write(0, 0, pos, _vec(pos + 0.5), _vec())
    kv.truncate(0, 2)
    for pos in range(2, 8):
        kv.write(0, 0, pos, _vec(pos + 0.5), _vec())
    assert torch.equal(gather_ctx(kv, 0, 0, 8)[0][5], torch.full((2, 8), 5.5))


def test_clear_frees_all_blocks():
    kv = _kv()
    kv.add_sequence(0)
    for pos in range(10):
        kv.write(0, 0, pos, _vec(), _vec())
    assert kv.num_allocated_blocks > 0
    kv.clear(0)
    assert kv.num_allocated_blocks == 0 and kv.seq_lengths[0] == 0 and kv.block_tables[0] == []


def test_reset_returns_cache_to_virgin_state():
    kv = _kv()
    kv.add_sequence(0)
    kv.add_sequence(1)
    for pos in range(6):
        kv.write(0, 0, pos, _vec(), _vec())
    kv.write(0, 1, 1, _vec(), _vec())
    assert kv.num_sequences == 2 and kv.num_allocated_blocks > 0
    kv.reset()
    assert kv.num_sequences == 0 and kv.num_allocated_blocks == 0


def test_block_utilization_metric():
    kv = _kv()
    kv.add_sequence(0)
    kv.write(0, 0, 0, _vec(), _vec())
    assert kv.block_utilization == pytest.approx(0.25)
    kv.write(0, 0, 1, _vec(), _vec())
    assert kv.block_utilization == pytest.approx(0.5)


def test_truncate_releases_physical_blocks():
    # reference tests/test_spec_accept.py:76-98
    kv = PagedKVCache(2, 2, 8, 32, 4)
    kv.add_sequence(0)
    for pos in range(10):
        kv.write(0, 0, pos, torch.randn(2, 8), torch.randn(2, 8))
    full = kv.num_allocated_blocks
    kv.truncate(0, 4)
    assert kv.seq_lengths[0] == 4
    assert full - kv.num_allocated_blocks == 2 and kv.num_allocated_blocks == 1


# ---------------------------------------------------------- LIFO order facts
def test_lifo_order_facts():
    kv = PagedKVCache(1, 1, 2, 8, 2, store=False)
    kv.add_sequence(0)
    kv.add_sequence(1)
    kv.write_block(0, [0, 1], [0, 0], None, None, chunk=5)  # 3 blocks each
    assert kv.block_tables[0] == [7, 6, 5]      # popped from the list tail
    assert kv.block_tables[1] == [4, 3, 2]
    kv.truncate(0, 1)                           # pops 5 then 6 off the table tail
    assert kv.allocator.free_list == [0, 1, 5, 6]
    kv.clear(1)                                 # frees 4, 3, 2 (forward)
    assert kv.allocator.free_list == [0, 1, 5, 6, 4, 3, 2]
    kv.write(0, 0, 2, None, None)               # next alloc pops 2
    assert kv.block_tables[0] == [7, 2]


def test_exhaustion_leaves_partial_state():
    kv = PagedKVCache(1, 1, 2, 3, 2, store=False)
    kv.add_sequence(0)
    kv.add_sequence(1)
    with pytest.raises(BlockExhaustedError):
        kv.write_block(0, [0, 1], [0, 0], None, None, chunk=4)  # needs 2 + 2 of 3
    assert kv.block_tables == [[2, 1], [0]]
    assert kv.seq_lengths == [4, 2]  # seq 1 wrote positions 0, 1 before failing at 2
    assert kv.allocator.free_list == []


# --------------------------------------------------------- random traces
def _check_partition(kv: PagedKVCache, owned):
    free = kv.allocator.free_list
    assert len(free) == len(set(free))
    tabled = [b for t in kv.block_tables for b in t]
    assert len(tabled) == len(set(tabled))
    assert set(free).isdisjoint(tabled)
    assert set(free) | set(tabled) == set(range(kv.allocator.capacity))
    assert kv.num_allocated_blocks == kv.allocator.capacity - len(free)
    for sid, blocks in owned.items():
        assert set(kv.block_tables[sid]) == blocks
        assert len(kv.block_tables[sid]) == -(-kv.seq_lengths[sid] // kv.block_size)


@pytest.mark.parametrize("seed", range(5))
def test_random_trace_keeps_pool_partitioned(seed):
    rng = random.Random(seed)
    bs, cap = 4, 48
    kv = PagedKVCache(1, 1, 2, cap, bs, store=False)
    owned = {}
    for sid in range(6):
        kv.add_sequence(sid)
        owned[sid] = set()
    for _ in range(300):
        op = rng.random()
        sid = rng.randrange(6)
        if op < 0.5:
            start = kv.seq_lengths[sid]
            chunk = rng.randint(1, 6)
            before = list(kv.block_tables[sid])
            try:
                kv.write_block(0, [sid], [start], None, None, chunk=chunk)
            except BlockExhaustedError:
                pass
            owned[sid] |= set(kv.block_tables[sid]) - set(before)
            if len(kv.block_tables[sid]) * bs < kv.seq_lengths[sid]:
                pytest.fail("length beyond allocated blocks")
        elif op < 0.85:
            new_len = rng.randint(0, kv.seq_lengths[sid])
            kv.truncate(sid, new_len)
            owned[sid] = set(kv.block_tables[sid])
        else:
            kv.clear(sid)
            owned[sid] = set()
        _check_partition(kv, owned)
