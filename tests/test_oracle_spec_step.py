"""CPU checks of the commit / rewind rule oracle (oracle/spec_step.py).

Each branch of engine/spec_scheduler.py:269-322 (budget cut with Python slice
semantics, eos cut, k == 0 finish, budget finish, truncate to
``prompt + len(generated) - 1``, draft shrink-only alignment, clear) is checked
by hand-computed expectations, and ``keep == start + k`` under the cache
invariant is checked on random rounds.
"""

from __future__ import annotations

import random

from oracle.kv_pool import PagedKVCache
from oracle.spec_step import SeqState, commit_round, cut_accepted


def test_cut_accepted_branches():
    assert cut_accepted([1, 2, 3], 5, None) == ([1, 2, 3], False)
    assert cut_accepted([1, 2, 3], 2, None) == ([1, 2], False)
    assert cut_accepted([1, 2, 3], 0, None) == ([], False)
    assert cut_accepted([1, 2, 3], -1, None) == ([1, 2], False)    # Python slice acc[:-1]
    assert cut_accepted([1, 9, 3], 5, 9) == ([1], True)
    assert cut_accepted([9, 2], 5, 9) == ([], True)
    assert cut_accepted([1, 2, 9], 2, 9) == ([1, 2], False)        # eos beyond the budget cut


def _pool(n_seq, lens, bs=4, cap=64):
    kv = PagedKVCache(1, 1, 2, cap, bs, store=False)
    for s in range(n_seq):
        kv.add_sequence(s)
        if lens[s]:
            kv.write_block(0, [s], [0], None, None, chunk=lens[s])
    return kv


def test_commit_round_truncates_and_clears():
    # seq 0: prompt 5, generated [7] -> start = 5; verify wrote 4 rows -> len 9
    kv = _pool(2, [9, 9])
    seqs = [SeqState(0, 5, 10, [7]), SeqState(1, 5, 3, [7])]
    ks = commit_round(seqs, {0: [1, 2], 1: [4, 5, 6]}, kv)
    assert ks == [2, 2]                              # seq 1 cut to its budget of 2
    assert kv.seq_lengths[0] == 5 + 2                # prompt + len(generated) - 1
    assert seqs[0].generated == [7, 1, 2] and not seqs[0].finished
    assert seqs[1].finished and kv.block_tables[1] == [] and kv.seq_lengths[1] == 0


def test_commit_round_eos_first_finishes_without_truncate():
    kv = _pool(1, [9])
    seqs = [SeqState(0, 5, 10, [7])]
    assert commit_round(seqs, {0: [0, 3]}, kv, eos=0) == [0]
    assert seqs[0].finished and seqs[0].eos_hit and seqs[0].generated == [7]
    assert kv.block_tables[0] == []


def test_draft_alignment_truncates_or_catches_up():
    # prompt 5, generated [7]: start 5. Seq 0 commits 2 -> keep 7 < draft 9:
    # truncate. Seq 1 commits 4 (all 3 drafts + bonus) -> keep 9 > draft 8
    # (start + gamma): position 8 is decoded, token generated[8 - 5] = 3.
    kv = _pool(2, [9, 9])
    draft = _pool(2, [9, 8])
    seqs = [SeqState(0, 5, 10, [7]), SeqState(1, 5, 10, [7])]
    cu = []
    commit_round(seqs, {0: [1, 2], 1: [1, 2, 3, 4]}, kv, draft, catchups=cu)
    assert draft.seq_lengths == [7, 9]
    assert [(c.sid, c.pos, c.tokens, c.finished) for c in cu] == [(1, 8, [3], False)]
    # block size 4: position 8 opens block 2, popped from the free list tail,
    # which is block 61, freed a moment earlier by seq 0's truncation (the
    # draft pool handed out 63, 62, 61 to seq 0 and 60, 59 to seq 1)
    assert draft.block_tables[0] == [63, 62] and draft.block_tables[1] == [60, 59, 61]


def test_catch_up_pops_blocks_freed_earlier_in_the_round():
    # Seq 0 commits all 4 tokens and reaches its budget of 5: its catch-up
    # pops block 59 (draft blocks were 63, 62 | 61, 60), then its clear frees
    # 63, 62, 59 in forward order; seq 1's catch-up then pops 59 again: the
    # reference's per-sequence order, which the device align must replay.
    kv = _pool(2, [9, 9])
    draft = _pool(2, [8, 8])
    seqs = [SeqState(0, 5, 5, [7]), SeqState(1, 5, 10, [7])]
    cu = []
    commit_round(seqs, {0: [1, 2, 3, 4], 1: [1, 2, 3, 4]}, kv, draft, catchups=cu)
    assert seqs[0].finished and draft.block_tables[0] == []
    assert draft.block_tables[1] == [61, 60, 59]
    assert draft.allocator.free_list[-2:] == [63, 62]
    assert [(c.sid, c.pos, c.tokens, c.finished) for c in cu] == [(0, 8, [3], True), (1, 8, [3], False)]


def test_catch_up_of_several_positions():
    kv = _pool(1, [12])
    draft = _pool(1, [6])
    seqs = [SeqState(0, 5, 20, [7])]
    cu = []
    commit_round(seqs, {0: [1, 2, 3, 4, 5]}, kv, draft, catchups=cu)
    assert draft.seq_lengths == [10] and len(draft.block_tables[0]) == 3
    assert [(c.pos, c.tokens) for c in cu] == [(6, [1, 2, 3, 4])]


def test_keep_equals_start_plus_k_under_invariant():
    rng = random.Random(5)
    for _ in range(50):
        prompt = rng.randint(1, 20)
        gen = [rng.randrange(8) for _ in range(rng.randint(1, 6))]
        start = prompt + len(gen) - 1
        C = rng.randint(2, 6)
        kv = _pool(1, [start + C], cap=256)
        s = SeqState(0, prompt, 40, list(gen))
        acc = [rng.randrange(8) for _ in range(rng.randint(1, C))]
        k = commit_round([s], {0: acc}, kv)[0]
        if not s.finished:
            assert kv.seq_lengths[0] == start + k
