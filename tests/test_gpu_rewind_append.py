"""GPU parity of the one-launch commit + append (spv_kv_rewind_append).

spv_kv_rewind_append is a round's rewind (PagedKVCache.truncate / clear of the
commit loop, engine/spec_scheduler.py:296-322) followed by the next round's
first-layer append (engine/model.py:184-187) of the same batch. Three pools
take the same rounds: one through rewind_device + write_block_device, one
through rewind_append_device, and the oracle (truncate, clear, write_block in
the reference's order). Tables, lengths and the free list (bottom to top) must
equal the oracle's; the two device pools must also agree on every pool element,
the write plan and the counters. Cases: spec rounds (lengths grow by the
accepted tokens, start = the committed length) and the bench's fixed starts,
first rounds with nothing to rewind, fp32 pools, small blocks, truncations
longer than the one-launch path takes, finished sequences, a block freed while
still in a table, a pool that runs out mid-batch, a table too narrow for the
chunk, and batches past one launch's limit.
"""

from __future__ import annotations

import random

import pytest
import torch

from engine import _hip
from engine.kv import BlockExhaustedError, PagedKVCache, WritePlan
from oracle import kv_pool as ref

pytestmark = pytest.mark.gpu


def _state(kv):
    return kv.block_tables, kv.seq_lengths, kv.allocator.free_list()


def _pools(cuda, H, d, cap, bs, dtype, nseq, maxb=None):
    mk = lambda: PagedKVCache(1, H, d, cap, bs, cuda, dtype, max_seqs=nseq, max_blocks_per_seq=maxb)  # noqa: E731
    two, one = mk(), mk()
    cpu = ref.PagedKVCache(1, H, d, cap, bs, store=False)
    for kv in (two, one, cpu):
        for s in range(nseq):
            kv.add_sequence(s)
    for kv in (two, one):
        kv.k_pool.zero_()
        kv.v_pool.zero_()
    return two, one, cpu


def _load(pools, tables, lens, free):
    for kv in pools:
        kv.load_state(tables, lens, free)


def _round(cuda, pools, sids, new_lens, fin, starts, k, v):
    """One commit + append on all three pools; returns whether the oracle's
    append ran out of blocks."""
    two, one, cpu = pools
    i32 = lambda x: torch.tensor(x, dtype=torch.int32, device=cuda)  # noqa: E731
    sid_t, st_t = i32(sids), i32(starts)
    nl_t = i32(new_lens) if new_lens is not None else None
    fin_t = i32(fin) if fin is not None else None
    p_two, p_one = WritePlan(), WritePlan()
    if nl_t is not None or fin_t is not None:
        zeros = torch.zeros(len(sids), dtype=torch.int32, device=cuda)
        two.rewind_device(sid_t, nl_t if nl_t is not None else zeros - 1, fin_t if fin_t is not None else zeros)
    two.write_block_device(0, sid_t, st_t, k, v, alloc=True, plan=p_two)
    one.rewind_append_device(sid_t, nl_t, fin_t, st_t, k, v, plan=p_one)
    for i, s in enumerate(sids):
        if new_lens is not None and new_lens[i] >= 0:
            cpu.truncate(s, new_lens[i])
        if fin is not None and fin[i]:
            cpu.clear(s)
    exhausted = False
    try:
        cpu.write_block(0, sids, starts, None, None, chunk=int(k.shape[1]))
    except ref.BlockExhaustedError:
        exhausted = True
    if p_two.ready or p_one.ready:
        n = len(sids) * int(k.shape[1])
        assert torch.equal(p_two.rows[:n], p_one.rows[:n])
    return exhausted


def _check(pools, exhausted=False, overflow=False):
    two, one, cpu = pools
    ctr_two, ctr_one = two.allocator.ctr.tolist(), one.allocator.ctr.tolist()
    for w in (_hip.CTR_TOP, _hip.CTR_EXHAUSTED, _hip.CTR_PUSHED, _hip.CTR_SLOWPATH, _hip.CTR_OVERFLOW, 5):
        assert ctr_two[w] == ctr_one[w], (w, ctr_two, ctr_one)
    assert ctr_one[5] == 0  # the arrival count is back at zero
    for kv in (two, one):
        if exhausted:
            with pytest.raises(BlockExhaustedError):
                kv.seq_lengths
        elif overflow:
            with pytest.raises(IndexError):
                kv.seq_lengths
    want = cpu.snapshot()
    assert _state(two) == tuple(want)
    assert _state(one) == tuple(want)
    assert torch.equal(two.k_pool, one.k_pool)
    assert torch.equal(two.v_pool, one.v_pool)


def _qwen15(seed, B, cap, bs):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(256, 4097, (B,), generator=g).tolist()
    perm = torch.randperm(cap, generator=g).tolist()
    tables, pos = [], 0
    for L in lens:
        n = -(-L // bs)
        tables.append(perm[pos: pos + n])
        pos += n
    return lens, tables, perm[pos:]


@pytest.mark.parametrize("dtype,fixed_starts", [(torch.bfloat16, False), (torch.bfloat16, True),
                                                (torch.float32, False)])
def test_spec_rounds_match_two_calls_and_oracle(cuda, dtype, fixed_starts):
    """Batch 32, 2 kv heads, head_dim 128, blocks of 16, 6-token chunks over a
    65,536-block random-permutation pool (the Qwen2.5-1.5B verify shape)."""
    B, cap, bs, C, H, d = 32, 65536, 16, 6, 2, 128
    lens, tables, free = _qwen15(3, B, cap, bs)
    pools = _pools(cuda, H, d, cap, bs, dtype, B, maxb=300)
    _load(pools, tables, lens, free)
    rng = random.Random(7)
    g = torch.Generator(device=cuda).manual_seed(7)
    sids = list(range(B))
    L0 = list(lens)
    starts, new_lens = list(lens), None
    for r in range(5):
        k = torch.randn(B, C, H, d, generator=g, device=cuda).to(dtype)
        v = torch.randn(B, C, H, d, generator=g, device=cuda).to(dtype)
        ex = _round(cuda, pools, sids, new_lens, None, starts, k, v)
        assert not ex
        _check(pools)
        new_lens = [s + rng.randint(0, C - 1) + 1 for s in starts]
        starts = list(L0) if fixed_starts else list(new_lens)


@pytest.mark.parametrize("bs,C,cut", [(4, 6, 0), (2, 9, 0), (2, 9, 30), (16, 7, 100)])
def test_truncations_short_and_long(cuda, bs, C, cut):
    """Truncations of up to four blocks take the one-launch path; ``cut``
    tokens below the start make longer ones (the exact single-workgroup path)."""
    B, H, d = 24, 2, 64
    cap = B * (-(-(400 + 2 * C) // bs)) + 64
    pools = _pools(cuda, H, d, cap, bs, torch.bfloat16, B, maxb=-(-(400 + 2 * C) // bs) + 2)
    rng = random.Random(bs * 31 + C + cut)
    g = torch.Generator(device=cuda).manual_seed(bs + C)
    lens = [rng.randint(cut + 1, 400) for _ in range(B)]
    for s, n in enumerate(lens):
        kk = torch.randn(1, n, H, d, generator=g, device=cuda).to(torch.bfloat16)
        pools[0].write_block(0, [s], [0], kk, kk)
        pools[1].write_block(0, [s], [0], kk, kk)
        pools[2].write_block(0, [s], [0], None, None, chunk=n)
    sids = rng.sample(range(B), 16)
    new_lens = [lens[s] - rng.randint(0, cut) + rng.randint(0, C) for s in sids]
    starts = [max(0, x) for x in new_lens]
    k = torch.randn(16, C, H, d, generator=g, device=cuda).to(torch.bfloat16)
    v = torch.randn(16, C, H, d, generator=g, device=cuda).to(torch.bfloat16)
    assert not _round(cuda, pools, sids, new_lens, None, starts, k, v)
    _check(pools)


@pytest.mark.parametrize("bs,lo,every", [(16, 1, 5), (4, 600, 1)])
def test_finished_sequences_are_cleared_then_appended(cuda, bs, lo, every):
    """Some sequences finished; with blocks of 4 and every sequence finished the
    clears free ~2,700 blocks (the exact path's windowed frees)."""
    B, H, d, C = 16, 2, 128, 6
    cap = B * (-(-(700 + C) // bs)) + 64
    pools = _pools(cuda, H, d, cap, bs, torch.bfloat16, B, maxb=-(-(700 + C) // bs) + 2)
    rng = random.Random(11)
    g = torch.Generator(device=cuda).manual_seed(11)
    lens = [rng.randint(lo, 700) for _ in range(B)]
    for s, n in enumerate(lens):
        kk = torch.randn(1, n, H, d, generator=g, device=cuda).to(torch.bfloat16)
        pools[0].write_block(0, [s], [0], kk, kk)
        pools[1].write_block(0, [s], [0], kk, kk)
        pools[2].write_block(0, [s], [0], None, None, chunk=n)
    sids = list(range(B))
    new_lens = [n - rng.randint(0, 3) for n in lens]
    fin = [1 if s % every == every // 2 else 0 for s in sids]
    starts = [0 if f else n for f, n in zip(fin, new_lens)]
    k = torch.randn(B, C, H, d, generator=g, device=cuda).to(torch.bfloat16)
    assert not _round(cuda, pools, sids, new_lens, fin, starts, k, k * 0.5)
    _check(pools)


def test_block_already_free_takes_the_exact_path(cuda):
    """A block freed while still in a table: the reference's free ignores it
    (kv.py:73-74); the one launch must push it once, as the two calls do."""
    H, d, bs, C = 1, 64, 2, 3
    pools = _pools(cuda, H, d, 24, bs, torch.float32, 2)
    k6 = torch.zeros(2, 6, H, d, device=cuda)
    pools[0].write_block(0, [0, 1], [0, 0], k6, k6)
    pools[1].write_block(0, [0, 1], [0, 0], k6, k6)
    pools[2].write_block(0, [0, 1], [0, 0], None, None, chunk=6)
    victim = pools[2].block_tables[0][2]
    for kv in pools:
        kv.allocator.free(victim)
    k = torch.randn(2, C, H, d, device=cuda)
    assert not _round(cuda, pools, [0, 1], [1, 3], None, [1, 3], k, k + 1)
    pools[0]._sync_pushes()
    pools[1]._sync_pushes()
    _check(pools)


def test_exhaustion_inside_the_batch(cuda):
    """The rewind frees a few blocks, the append needs more: the allocation
    fails mid-batch exactly where the oracle's does."""
    B, H, d, bs, C = 12, 2, 128, 16, 7
    lens = [30 + 3 * s for s in range(B)]  # 40 blocks in all
    cap = 40 + 2  # the rewind frees 3, the append needs 6: entry 11 runs out
    pools = _pools(cuda, H, d, cap, bs, torch.bfloat16, B)
    g = torch.Generator(device=cuda).manual_seed(2)
    for s, n in enumerate(lens):
        kk = torch.randn(1, n, H, d, generator=g, device=cuda).to(torch.bfloat16)
        pools[0].write_block(0, [s], [0], kk, kk)
        pools[1].write_block(0, [s], [0], kk, kk)
        pools[2].write_block(0, [s], [0], None, None, chunk=n)
    sids = list(range(B))
    new_lens = [n - 16 if s % 4 == 0 else n for s, n in enumerate(lens)]  # frees three blocks
    k = torch.randn(B, C, H, d, generator=g, device=cuda).to(torch.bfloat16)
    ex = _round(cuda, pools, sids, new_lens, None, new_lens, k, k)
    assert ex
    _check(pools, exhausted=True)


def test_table_width_overflow_is_reported(cuda):
    B, H, d, bs, C, maxb = 4, 2, 64, 4, 6, 3
    pools = _pools(cuda, H, d, 64, bs, torch.bfloat16, B, maxb=maxb)
    k8 = torch.randn(B, 8, H, d, device=cuda).to(torch.bfloat16)
    pools[0].write_block(0, list(range(B)), [0] * B, k8, k8)
    pools[1].write_block(0, list(range(B)), [0] * B, k8, k8)
    pools[2].write_block(0, list(range(B)), [0] * B, None, None, chunk=8)
    k = torch.randn(B, C, H, d, device=cuda).to(torch.bfloat16)
    new_lens = [8, 7, 5, 8]
    two, one, cpu = pools
    i32 = lambda x: torch.tensor(x, dtype=torch.int32, device=cuda)  # noqa: E731
    sid_t, nl_t = i32(list(range(B))), i32(new_lens)
    two.rewind_device(sid_t, nl_t, torch.zeros(B, dtype=torch.int32, device=cuda))
    two.write_block_device(0, sid_t, nl_t, k, k)
    one.rewind_append_device(sid_t, nl_t, None, nl_t, k, k)
    for kv in (two, one):
        with pytest.raises(IndexError):
            kv.seq_lengths
    assert _state(two) == _state(one)
    assert torch.equal(two.k_pool, one.k_pool) and torch.equal(two.v_pool, one.v_pool)


def test_batch_beyond_one_launch_takes_the_two_calls(cuda):
    """1,100 entries: past the one-launch limit, the entry point enqueues the
    rewind and the append; the result is the same."""
    B, H, d, bs, C = 1100, 1, 64, 16, 2
    pools = _pools(cuda, H, d, 4 * B, bs, torch.bfloat16, B)
    g = torch.Generator(device=cuda).manual_seed(4)
    k = torch.randn(B, 20, H, d, generator=g, device=cuda).to(torch.bfloat16)
    sids = list(range(B))
    pools[0].write_block(0, sids, [0] * B, k, k)
    pools[1].write_block(0, sids, [0] * B, k, k)
    pools[2].write_block(0, sids, [0] * B, None, None, chunk=20)
    new_lens = [15 + (s % 6) for s in sids]
    kc = torch.randn(B, C, H, d, generator=g, device=cuda).to(torch.bfloat16)
    assert not _round(cuda, pools, sids, new_lens, None, new_lens, kc, kc)
    _check(pools)


def test_fp8_pool_is_refused(cuda):
    kv = PagedKVCache(1, 2, 64, 32, 16, cuda, torch.float8_e4m3fn)
    kv.add_sequence(0)
    t = torch.zeros(1, dtype=torch.int32, device=cuda)
    k = torch.zeros(1, 2, 2, 64, device=cuda)
    with pytest.raises(ValueError):
        kv.rewind_append_device(t, t, t, t, k, k)


@pytest.mark.parametrize("seed", range(6))
def test_random_rounds_match_two_calls_and_oracle(cuda, seed):
    """Seeded random rounds over a small pool: lengths shrink and grow, some
    sequences finish (and start again from 0), starts are the committed lengths
    or not, blocks of 2 to 16, chunks of 1 to 9; a round whose append runs the
    pool out is checked and the trace restarts from a fresh pool."""
    rng = random.Random(1000 + seed)
    bs = rng.choice([2, 4, 16])
    C = rng.randint(1, 9)
    H, d, B = rng.choice([1, 2]), rng.choice([64, 128]), rng.randint(1, 40)
    cap = rng.randint(B * 2, B * (-(-(300 + 2 * C) // bs)) + 8)
    dtype = rng.choice([torch.bfloat16, torch.float32])
    g = torch.Generator(device=cuda).manual_seed(seed)
    pools = _pools(cuda, H, d, cap, bs, dtype, B, maxb=-(-(300 + 4 * C) // bs) + 2)
    lens = [0] * B
    for rnd in range(8):
        sids = rng.sample(range(B), rng.randint(1, B))
        new_lens = [max(-1, lens[s] + rng.randint(-40, 2 * C)) if rng.random() < 0.8 else -1 for s in sids]
        fin = [1 if rng.random() < 0.1 else 0 for _ in sids]
        after = [0 if f else (nl if nl >= 0 else lens[s]) for s, nl, f in zip(sids, new_lens, fin)]
        starts = [a if rng.random() < 0.7 else max(0, a - rng.randint(0, C)) for a in after]
        starts = [min(x, 300) for x in starts]
        k = torch.randn(len(sids), C, H, d, generator=g, device=cuda).to(dtype)
        v = torch.randn(len(sids), C, H, d, generator=g, device=cuda).to(dtype)
        ex = _round(cuda, pools, sids, new_lens, fin, starts, k, v)
        _check(pools, exhausted=ex)
        if ex:
            return
        for s, a, st in zip(sids, after, starts):
            lens[s] = max(a, st + C)


def test_mismatched_inputs_are_refused(cuda):
    kv = PagedKVCache(1, 2, 64, 32, 16, cuda, torch.bfloat16)
    kv.add_sequence(0)
    kv.add_sequence(1)
    i32 = lambda x: torch.tensor(x, dtype=torch.int32, device=cuda)  # noqa: E731
    k = torch.zeros(2, 3, 2, 64, device=cuda, dtype=torch.bfloat16)
    with pytest.raises(ValueError):  # one start for two sequences
        kv.rewind_append_device(i32([0, 1]), None, None, i32([0]), k, k)
    with pytest.raises(ValueError):  # int64 new lengths
        kv.rewind_append_device(i32([0, 1]), torch.zeros(2, dtype=torch.int64, device=cuda), None, i32([0, 0]), k, k)
    with pytest.raises(ValueError):  # wrong head count
        kv.rewind_append_device(i32([0, 1]), None, None, i32([0, 0]), k[:, :, :1], k[:, :, :1])
    kv.rewind_append_device(i32([0, 1]), None, None, i32([0, 0]), k, k)
    assert kv.seq_lengths == [3, 3]
