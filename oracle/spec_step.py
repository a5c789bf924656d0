"""CPU restatement of the per-round commit / rewind rule (test infrastructure only).

Follows engine/spec_scheduler.py:269-322 of the reference, per sequence in
``running`` order:

1. cut the accepted list to the remaining budget ``max_new - len(generated)``
   with Python slice semantics (:274-277);
2. cut at the first eos, which is not kept, and finish (:279-289);
3. ``k == 0`` finishes without a truncate (:292-295); otherwise extend
   ``generated``, finish when the budget is reached, and truncate the target
   cache to ``prompt_len + len(generated) - 1`` (:296-303);
4. align the draft cache (:305-319): truncate when it is longer than that
   length; when it is shorter, decode the missing positions ``d .. keep - 1``
   one at a time. The decode itself is model work; what it does to the pool is
   the write of each position (kv.py:125-147): blocks allocated lazily in
   logical order (kv.py:119-122) and the length raised to the position + 1.
   ``catch_up`` restates exactly that and records the positions and tokens
   (``generated[p - prompt_len]``) the draft model decodes;
5. finished -> ``clear`` both caches (:320-322).

Under the cache invariant ``seq_len == prompt_len + len(generated) - 1`` the
truncate length equals ``start + k`` with ``start`` the verify start position,
which is what the device commit computes; tests/test_oracle_spec_step.py checks
that equivalence and the rule's branches.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

from .kv_pool import PagedKVCache


@dataclass
class SeqState:
    sid: int
    prompt_len: int
    max_new_tokens: int
    generated: List[int] = field(default_factory=list)
    finished: bool = False
    eos_hit: bool = False


def cut_accepted(acc: Sequence[int], remaining: int, eos: Optional[int]) -> Tuple[List[int], bool]:
    """Budget cut then eos cut; returns (kept tokens, eos_hit)."""
    acc = list(acc)
    if len(acc) > remaining:
        acc = acc[:remaining]
    if eos is not None:
        for i, tok in enumerate(acc):
            if tok == eos:
                return acc[:i], True
    return acc, False


@dataclass
class CatchUp:
    """Draft positions ``pos .. pos + len(tokens) - 1`` decoded to align sequence ``sid``."""
    sid: int
    pos: int
    tokens: List[int]
    finished: bool = False   # the sequence finished this round (its draft cache is then cleared)


def catch_up(draft_kv: PagedKVCache, s: SeqState, keep: int) -> CatchUp:
    """The pool side of the draft catch-up loop (spec_scheduler.py:308-319):
    one write per position, in order, as the draft decode's per-layer writes
    make them (the first layer's write allocates, kv.py:119-122, and raises
    the length, kv.py:146-147)."""
    d = draft_kv.seq_lengths[s.sid]
    toks = []
    for p in range(d, keep):
        toks.append(s.generated[p - s.prompt_len])
        draft_kv._ensure_blocks_up_to(s.sid, p // draft_kv.block_size)
        if draft_kv.seq_lengths[s.sid] <= p:
            draft_kv.seq_lengths[s.sid] = p + 1
    return CatchUp(s.sid, d, toks)


def commit_round(running: Sequence[SeqState], accepted_by: Dict[int, List[int]],
                 kv: PagedKVCache, draft_kv: Optional[PagedKVCache] = None,
                 eos: Optional[int] = None, catchups: Optional[List[CatchUp]] = None) -> List[int]:
    """Apply one round's commit to ``kv`` (and ``draft_kv``); returns k per sequence.
    Draft catch-ups are appended to ``catchups`` when it is given."""
    ks = []
    for s in running:
        acc, eos_hit = cut_accepted(accepted_by[s.sid], s.max_new_tokens - len(s.generated), eos)
        if eos_hit:
            s.eos_hit = True
            s.finished = True
        k = len(acc)
        ks.append(k)
        if k == 0:
            s.finished = True
        else:
            s.generated.extend(acc)
            if len(s.generated) >= s.max_new_tokens:
                s.finished = True
            keep = s.prompt_len + len(s.generated) - 1
            kv.truncate(s.sid, keep)
            if draft_kv is not None:
                d_len = draft_kv.seq_lengths[s.sid]
                if d_len > keep:
                    draft_kv.truncate(s.sid, keep)
                elif d_len < keep:
                    c = catch_up(draft_kv, s, keep)
                    c.finished = s.finished
                    if catchups is not None:
                        catchups.append(c)
        if s.finished:
            kv.clear(s.sid)
            if draft_kv is not None:
                draft_kv.clear(s.sid)
    return ks
