"""GPU parity of the draft-cache alignment (spec_scheduler.py:296-322) and the
device metrics record (spec_scheduler.py:200-205, kv.py:186-224).

* ``align_draft``: random rounds over random draft-pool states (prompt and
  generated lengths, draft caches at ``start + gamma`` or elsewhere in
  ``[start, start + gamma + 1]``, accepted lists of every length, budget and
  eos cuts) are committed by the oracle's commit rule (oracle/spec_step.py,
  which restates the truncate / catch-up / clear loop); the device alignment
  of the same draft pool must leave identical block tables, lengths and free
  list, and report the oracle's catch-up positions and tokens for every
  sequence that keeps running. Catch-ups that pop blocks freed earlier in the
  same round (the order the reference's per-sequence loop makes) and several
  catch-ups in one batch are forced in dedicated cases; an exhausted pool
  raises ``BlockExhaustedError`` with the draft pool left as the reference
  leaves it at its exception.
* ``metrics_device``: the record equals the mirror's ``num_allocated_blocks``,
  ``logical_tokens``, ``max(seq_lengths)`` and the round's committed / finished
  counts; ``peak`` tracks the maximum over calls.
"""

from __future__ import annotations

import random

import pytest
import torch

from engine import _hip
from engine.kv import BlockExhaustedError, PagedKVCache
from engine.spec_scheduler import VerifyResult, align_draft
from oracle import kv_pool as ref
from oracle.spec_step import SeqState, commit_round

pytestmark = pytest.mark.gpu


class _Target:
    """Stands in for the target pool in commit_round where only the draft
    pool is compared."""

    def truncate(self, sid, n):
        pass

    def clear(self, sid):
        pass


def _round(rng, n_seq, gamma, bs, cap, force_all=False, budgets=None):
    """Random oracle draft pool (with a permuted free list) and one round's
    accepted lists."""
    cpu_d = ref.PagedKVCache(1, 1, 2, cap, bs, store=False)
    seqs, acc_by, chunks, starts = [], {}, [], []
    C = gamma + 1
    stray = [cpu_d.allocator.alloc() for _ in range(rng.randint(0, 12))]
    for sid in range(n_seq):
        prompt = rng.randint(1, 40)
        gen = [rng.randrange(50) for _ in range(rng.randint(1, 8))]
        L = prompt + len(gen) - 1
        d = L + gamma if force_all or rng.random() < 0.7 else rng.randint(L, L + gamma + 1)
        budget = rng.randint(len(gen), len(gen) + 3 * C) if budgets is None else budgets[sid]
        cpu_d.add_sequence(sid)
        cpu_d.write_block(0, [sid], [0], None, None, chunk=d)
        if stray and rng.random() < 0.3:
            cpu_d.allocator.free(stray.pop(rng.randrange(len(stray))))  # permute the free-list tail
        proposals = [rng.randrange(50) for _ in range(gamma)]
        n_acc = gamma if force_all else rng.randint(0, gamma)
        acc_by[sid] = proposals[:n_acc] + [rng.randrange(50)]
        chunks.append([gen[-1]] + proposals)
        starts.append(L)
        seqs.append(SeqState(sid, prompt, budget, list(gen)))
    for b in stray:
        cpu_d.allocator.free(b)
    return cpu_d, seqs, acc_by, chunks, starts


def _device_draft(cpu_d, cap, bs, cuda):
    gpu = PagedKVCache(1, 1, 2, cap, bs, cuda, torch.float32)
    tables, lens, free = cpu_d.snapshot()
    gpu.load_state(tables, lens, free)
    return gpu


def _align(gpu, ks, fin, chunks, starts, cuda, order):
    B = len(order)
    i32 = lambda x: torch.tensor(x, dtype=torch.int32, device=cuda)  # noqa: E731
    res = VerifyResult(i32([0] * B), i32([[0] * len(chunks[0])] * B), i32(ks), i32(fin), i32([0] * B))
    return align_draft(gpu, i32(order), i32(starts), res, i32(chunks))


def _check(gpu, cpu_d, cu, seqs, catchups):
    assert gpu.block_tables == cpu_d.block_tables
    assert gpu.seq_lengths == cpu_d.seq_lengths
    assert gpu.allocator.free_list() == cpu_d.allocator.free_list
    by_sid = {c.sid: c for c in catchups}
    count, pos, toks = cu.count.tolist(), cu.pos.tolist(), cu.tokens.tolist()
    for b, s in enumerate(seqs):
        c = by_sid.get(s.sid)
        if c is None or c.finished:
            assert count[b] == 0, (b, count[b])
            continue
        assert (count[b], pos[b]) == (len(c.tokens), c.pos), b
        assert toks[b][: count[b]] == c.tokens and all(t == -1 for t in toks[b][count[b]:]), b


@pytest.mark.parametrize("seed", range(8))
def test_align_matches_the_oracle(cuda, seed):
    rng = random.Random(seed)
    gamma, bs, cap = rng.choice([(3, 4, 400), (5, 16, 300), (6, 16, 300), (1, 2, 500)])
    n_seq = rng.randint(1, 24)
    cpu_d, seqs, acc_by, chunks, starts = _round(rng, n_seq, gamma, bs, cap)
    gpu = _device_draft(cpu_d, cap, bs, cuda)
    catchups = []
    ks = commit_round(seqs, acc_by, _Target(), cpu_d, eos=rng.choice([None, 7]), catchups=catchups)
    cu = _align(gpu, ks, [int(s.finished) for s in seqs], chunks, starts, cuda, [s.sid for s in seqs])
    _check(gpu, cpu_d, cu, seqs, catchups)


def test_every_sequence_catches_up_and_reuses_blocks_freed_in_the_round(cuda):
    # All proposals accepted everywhere: every running draft cache is one short;
    # with block size 2 and gamma 1 half the catch-ups open a block, and tight
    # budgets finish (and clear) sequences between them, so catch-ups pop
    # blocks that earlier sequences of the same round freed.
    rng = random.Random(11)
    gamma, bs, cap, n = 1, 2, 2400, 64
    budgets = [rng.choice([1, 2, 9]) for _ in range(n)]
    cpu_d, seqs, acc_by, chunks, starts = _round(rng, n, gamma, bs, cap, force_all=True)
    for s, b in zip(seqs, budgets):
        s.max_new_tokens = len(s.generated) + b
    gpu = _device_draft(cpu_d, cap, bs, cuda)
    catchups = []
    ks = commit_round(seqs, acc_by, _Target(), cpu_d, catchups=catchups)
    assert sum(1 for c in catchups if not c.finished) > 10
    assert any(c.finished for c in catchups) and any(s.finished for s in seqs)
    cu = _align(gpu, ks, [int(s.finished) for s in seqs], chunks, starts, cuda, [s.sid for s in seqs])
    _check(gpu, cpu_d, cu, seqs, catchups)


def test_long_clears_and_many_sequences(cuda):
    # 600 sequences; the first 100 finish with 103-block caches and no
    # catch-up, so their clears form one run of 10,300 frees (more than the
    # 8,192-block window of the parallel path); the rest mix truncations,
    # catch-ups and clears.
    rng = random.Random(3)
    gamma, bs, cap = 4, 2, 18000
    cpu_d = ref.PagedKVCache(1, 1, 2, cap, bs, store=False)
    seqs, acc_by, chunks, starts = [], {}, [], []
    for sid in range(600):
        long = sid < 100
        prompt = 200 if long else rng.choice([3, 30])
        gen = [1, 2]
        L = prompt + 1
        cpu_d.add_sequence(sid)
        cpu_d.write_block(0, [sid], [0], None, None, chunk=L + gamma)
        props = [rng.randrange(9) for _ in range(gamma)]
        acc_by[sid] = props[: 0 if long else rng.choice([0, 2, gamma])] + [5]
        chunks.append([2] + props)
        starts.append(L)
        seqs.append(SeqState(sid, prompt, 3 if long else rng.choice([3, 40]), list(gen)))
    gpu = _device_draft(cpu_d, cap, bs, cuda)
    catchups = []
    ks = commit_round(seqs, acc_by, _Target(), cpu_d, catchups=catchups)
    assert sum(s.finished for s in seqs) > 150
    cu = _align(gpu, ks, [int(s.finished) for s in seqs], chunks, starts, cuda, list(range(600)))
    _check(gpu, cpu_d, cu, seqs, catchups)


def test_exhausted_catch_up_raises_and_stops_like_the_reference(cuda):
    # A pool with no free block: the first catch-up that needs one raises; the
    # sequences before it were aligned, the ones after it untouched.
    bs = 4
    cpu_d = ref.PagedKVCache(1, 1, 2, 6, bs, store=False)
    for sid, d in enumerate([8, 5, 8]):   # two blocks each: the pool is full
        cpu_d.add_sequence(sid)
        cpu_d.write_block(0, [sid], [0], None, None, chunk=d)
    assert not cpu_d.allocator.free_list
    gpu = _device_draft(cpu_d, 6, bs, cuda)
    seqs = [SeqState(0, 5, 20, [1]), SeqState(1, 2, 20, [1]), SeqState(2, 5, 20, [1])]
    # Starts 5, 2, 5. Seq 0 commits 1: truncate 8 -> 6, both blocks kept.
    # Seq 1 commits 4: keep 6 > 5, position 5 lies in its second block (no
    # pop). Seq 2 commits 4: keep 9 > 8, position 8 needs a third block.
    acc_by = {0: [9], 1: [1, 2, 3, 4], 2: [1, 2, 3, 4]}
    chunks = [[1, 9, 9, 9], [1, 1, 2, 3], [1, 1, 2, 3]]
    catchups = []
    with pytest.raises(ref.BlockExhaustedError):
        commit_round(seqs, acc_by, _Target(), cpu_d, catchups=catchups)
    ks = [1, 4, 4]
    cu = _align(gpu, ks, [0, 0, 0], chunks, [5, 2, 5], cuda, [0, 1, 2])
    with pytest.raises(BlockExhaustedError):
        gpu.seq_lengths
    assert gpu.block_tables == cpu_d.block_tables
    assert gpu.seq_lengths == cpu_d.seq_lengths
    assert gpu.allocator.free_list() == cpu_d.allocator.free_list
    assert cu.count.tolist()[:2] == [0, 1]


def test_catch_up_behind_the_round_is_reported(cuda):
    bs = 4
    gpu = PagedKVCache(1, 1, 2, 32, bs, cuda, torch.float32)
    gpu.load_state([[31, 30], [29]], [6, 3], list(range(29)))
    i32 = lambda x: torch.tensor(x, dtype=torch.int32, device=cuda)  # noqa: E731
    res = VerifyResult(i32([0, 0]), i32([[0] * 3] * 2), i32([2, 1]), i32([0, 0]), i32([0, 0]))
    align_draft(gpu, i32([0, 1]), i32([6, 5]), res, i32([[1, 2, 3], [4, 5, 6]]))
    with pytest.raises(ValueError, match="shorter than the round's start"):
        gpu.seq_lengths
    assert gpu.seq_lengths == [8, 3]   # seq 0 caught up (6 -> 8); seq 1 (3 < start 5) left as it was


def test_metrics_record_matches_the_mirror(cuda):
    bs = 4
    gpu = PagedKVCache(1, 1, 2, 64, bs, cuda, torch.float32)
    gpu.load_state([[63, 62, 61], [], [60]], [11, 0, 2], list(range(60)))
    rec = torch.zeros((3, 6), dtype=torch.int64, device=cuda)
    peak = torch.zeros(1, dtype=torch.int64, device=cuda)
    i32 = lambda x: torch.tensor(x, dtype=torch.int32, device=cuda)  # noqa: E731
    gpu.metrics_device(rec[0], peak, i32([3, 1]), i32([0, 1]), batch=2)
    gpu.rewind([0], [4], None)
    gpu.metrics_device(rec[1], peak)
    got = rec.tolist()
    assert got[0] == [4, 13, 11, 2, 4, 1]
    assert got[1] == [2, 6, 4, 0, 0, 0]
    assert got[1][0] == gpu.num_allocated_blocks and got[1][1] == gpu.logical_tokens
    assert int(peak.item()) == 4
