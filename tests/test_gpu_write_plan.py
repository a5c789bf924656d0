"""GPU parity of the round write plan (spv_kv_append_plan, spv_kv_write_planned)
with the plain per-layer append (spv_kv_append).

A round appends the same chunk into every layer (engine/model.py:184-187 once
per layer); only the first layer's call allocates. The plan records, at that
first call, the pool row of each chunk token; the later layers copy by it.
Two pools that take the same rounds -- one through the plan, one through
spv_kv_append with may_alloc = 0 for the later layers -- must end bit-equal:
pools (every element), tables, block counts, lengths and the free list. Cases:
the fused allocation path (small chunk), the separate allocation + write path
(a chunk too long for the fused kernel: the plan kernel), fp32 and bf16 pools,
sequences that cross block boundaries, and a pool that runs out mid-batch
(the exhausted entry and those after it write only what the reference writes).
"""

from __future__ import annotations

import random

import pytest
import torch

from engine.kv import BlockExhaustedError, PagedKVCache, WritePlan

pytestmark = pytest.mark.gpu


def _pools(cuda, L, H, d, cap, bs, dtype, nseq):
    mk = lambda: PagedKVCache(L, H, d, cap, bs, cuda, dtype, max_seqs=nseq)
    a, b = mk(), mk()
    for kv in (a, b):
        kv.k_pool.zero_()
        kv.v_pool.zero_()
        for s in range(nseq):
            kv.add_sequence(s)
    return a, b


def _equal(a: PagedKVCache, b: PagedKVCache):
    assert torch.equal(a.k_pool, b.k_pool)
    assert torch.equal(a.v_pool, b.v_pool)
    assert a.block_tables == b.block_tables
    assert a.seq_lengths == b.seq_lengths
    assert a.allocator.free_list() == b.allocator.free_list()


def _round(kv, layers, sid_t, st_t, ks, vs, plan):
    for layer in range(layers):
        kv.write_block_device(layer, sid_t, st_t, ks[layer], vs[layer], alloc=layer == 0, plan=plan)


@pytest.mark.parametrize("dtype,d,C,bs", [
    (torch.bfloat16, 128, 7, 16),    # fused allocation path (Qwen2.5-3B verify chunk)
    (torch.bfloat16, 64, 1, 16),     # draft step: one token
    (torch.float32, 64, 9, 16),      # fp32 pool
    (torch.bfloat16, 128, 40, 16),   # a long chunk: allocation kernel + plan kernel
    (torch.bfloat16, 128, 6, 4),     # small blocks: a chunk spans two or three blocks
])
def test_planned_layers_equal_plain_appends(cuda, dtype, d, C, bs):
    L, H, nseq, rounds = 4, 2, 24, 3
    rng = random.Random(d + C)
    cap = nseq * (-(-(400 + rounds * C) // bs)) + 8
    plain, planned = _pools(cuda, L, H, d, cap, bs, dtype, nseq)
    g = torch.Generator().manual_seed(C)
    lens = [rng.randint(0, 300) for _ in range(nseq)]
    for s, n in enumerate(lens):  # prompts (one call per sequence, every layer)
        if n:
            for layer in range(L):
                k = torch.randn(1, n, H, d, generator=g).to(dtype).to(cuda)
                for kv in (plain, planned):
                    kv.write_block(layer, [s], [0], k, k * 0.5)
    plan = WritePlan()
    for r in range(rounds):
        sids = rng.sample(range(nseq), 16)
        starts = [lens[s] for s in sids]
        sid_t = torch.tensor(sids, dtype=torch.int32, device=cuda)
        st_t = torch.tensor(starts, dtype=torch.int32, device=cuda)
        ks = [torch.randn(len(sids), C, H, d, generator=g).to(dtype).to(cuda) for _ in range(L)]
        vs = [torch.randn(len(sids), C, H, d, generator=g).to(dtype).to(cuda) for _ in range(L)]
        _round(plain, L, sid_t, st_t, ks, vs, None)
        _round(planned, L, sid_t, st_t, ks, vs, plan)
        assert plan.ready and (plan.B, plan.C) == (len(sids), C)
        for s in sids:
            lens[s] += C
        _equal(plain, planned)


def test_planned_layers_after_exhaustion_write_what_plain_appends_write(cuda):
    L, H, d, bs, C, nseq = 3, 2, 128, 16, 7, 12
    cap = 44  # the prompts take 40 blocks; the round needs 6 more: the 5th (entry 10) fails
    plain, planned = _pools(cuda, L, H, d, cap, bs, torch.bfloat16, nseq)
    g = torch.Generator().manual_seed(5)
    lens = [30 + 3 * s for s in range(nseq)]  # two blocks each
    for s, n in enumerate(lens):
        for layer in range(L):
            k = torch.randn(1, n, H, d, generator=g).to(torch.bfloat16).to(cuda)
            for kv in (plain, planned):
                kv.write_block(layer, [s], [0], k, k * 0.25)
    sid_t = torch.arange(nseq, dtype=torch.int32, device=cuda)
    st_t = torch.tensor(lens, dtype=torch.int32, device=cuda)
    ks = [torch.randn(nseq, C, H, d, generator=g).to(torch.bfloat16).to(cuda) for _ in range(L)]
    vs = [torch.randn(nseq, C, H, d, generator=g).to(torch.bfloat16).to(cuda) for _ in range(L)]
    plan = WritePlan()
    _round(plain, L, sid_t, st_t, ks, vs, None)
    _round(planned, L, sid_t, st_t, ks, vs, plan)
    rows = plan.rows[:nseq * C].view(nseq, C).cpu()
    assert bool((rows == -1).any()) and bool((rows >= 0).any())  # the cut lies inside the batch
    for kv in (plain, planned):
        with pytest.raises(BlockExhaustedError):
            kv.seq_lengths
    assert torch.equal(plain.k_pool, planned.k_pool)
    assert torch.equal(plain.v_pool, planned.v_pool)


def test_plan_rejects_a_different_chunk(cuda):
    plain, planned = _pools(cuda, 2, 2, 64, 64, 16, torch.bfloat16, 4)
    sid_t = torch.arange(4, dtype=torch.int32, device=cuda)
    st_t = torch.zeros(4, dtype=torch.int32, device=cuda)
    k = torch.randn(4, 5, 2, 64, device=cuda).to(torch.bfloat16)
    plan = WritePlan()
    planned.write_block_device(0, sid_t, st_t, k, k, alloc=True, plan=plan)
    with pytest.raises(ValueError, match="write plan"):
        planned.write_block_device(1, sid_t[:3], st_t[:3], k[:3], k[:3], alloc=False, plan=plan)


def test_plan_rejects_another_batch_of_the_same_shape_and_a_changed_pool(cuda):
    """A plan is tied to the tensors its recording call took and to the pool
    state after it: another batch of the same (B, C), or any later call that
    may change the tables (here a rewind), makes a planned write raise instead
    of copying into the recorded rows."""
    _, planned = _pools(cuda, 2, 2, 64, 64, 16, torch.bfloat16, 8)
    sid_t = torch.arange(4, dtype=torch.int32, device=cuda)
    st_t = torch.zeros(4, dtype=torch.int32, device=cuda)
    k = torch.randn(4, 5, 2, 64, device=cuda).to(torch.bfloat16)
    plan = WritePlan()
    planned.write_block_device(0, sid_t, st_t, k, k, alloc=True, plan=plan)
    planned.write_block_device(1, sid_t, st_t, k, k, alloc=False, plan=plan)  # the recorded chunk: fine
    other = torch.arange(4, 8, dtype=torch.int32, device=cuda)
    with pytest.raises(ValueError, match="write plan"):
        planned.write_block_device(1, other, st_t, k, k, alloc=False, plan=plan)
    planned.rewind_device(sid_t, torch.full((4,), 2, dtype=torch.int32, device=cuda),
                          torch.zeros(4, dtype=torch.int32, device=cuda))
    with pytest.raises(ValueError, match="write plan"):
        planned.write_block_device(1, sid_t, st_t, k, k, alloc=False, plan=plan)
