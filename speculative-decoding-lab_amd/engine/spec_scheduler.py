"""Rejection sampling and commit of a speculative round on the GPU.

Drop-in for the verify part of the reference's engine/spec_scheduler.py:

* ``batch_accept``  -- spec_scheduler.py:46-88 with the reference's live CPU
  ``torch.Generator``. The acceptance probabilities of every position come
  from the device in one launch; the host then draws the uniforms and the one
  ``Exp(1)`` race row per sequence in exactly the reference's order (a uniform
  per examined position, then the multinomial's exponential row), and a second
  launch makes the decisions and races on the device.
* ``verify_sample`` -- the fused form with caller-supplied randomness
  (``u[B, gamma]``, ``E[B, V]``): softmax/greedy rows from logits, decisions,
  residual/bonus race and the commit cut of spec_scheduler.py:274-303, all on
  the device, outputs left on the device.
* ``VerifyStep``    -- one verify round of a continuous batch: per layer
  ``write_block`` + ``verify_attention``, then ``verify_sample`` on the
  round's logits and ``rewind_device`` of the KV pool with the device-computed
  lengths and finished flags (spec_scheduler.py:255-322 minus the model).
* ``draft_sample``  -- one draft step's proposals (spec_scheduler.py:243-252:
  ``logits_to_probs`` + ``sample_token`` per row) for the whole batch in one
  launch, with caller-supplied ``Exp(1)`` rows; ``draft_sample_with_generator``
  draws those rows from the reference's generator in its order.
* ``DraftLoop``     -- the paged part of the gamma draft decode steps (per layer
  one-token append + decode attention, engine/model.py:123-153) and each step's
  sampling, with device-resident positions so the loop captures as one graph.
* ``align_draft``   -- the draft cache's side of the commit
  (spec_scheduler.py:296-322: truncate, catch-up allocation, clear) in one
  launch on the device, reporting the catch-up tokens the draft model decodes.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence

import torch

from . import _hip
from ._hip import call, ptr
from .attention import VerifyPlan, verify_attention
from .kv import PagedKVCache, WritePlan

_workspace = _hip.Workspace()
_draft_workspace = _hip.Workspace()


def _draw_uniform(generator: torch.Generator) -> float:
    """The accept coin of one position (spec_scheduler.py:41-43)."""
    return float(torch.rand(1, generator=generator).item())


@dataclass
class VerifyResult:
    """Device int32 outputs of one verify-sampling launch.

    ``flags[b]`` is 0 when sequence b's accepted list is the reference's for
    the same logits, uniforms and noise. Given logits, p and q are this
    library's fp32 softmax, a few 1e-6 from torch's; a nonzero word marks a
    result the reference may have decided otherwise (``_hip.FLAG_*`` bits: a
    uniform inside the error band of ``min(1, p/q)``, a drawn token within the
    keys' error of another, a filtered row whose nucleus edge lies within
    rounding)."""

    accept_len: torch.Tensor   # (B,) drafts accepted
    out_tokens: torch.Tensor   # (B, gamma+1) accepted drafts then the drawn token, -1 padded
    n_commit: torch.Tensor     # (B,) tokens kept after the budget / eos cut
    finished: torch.Tensor     # (B,) 1 = sequence finished this round
    new_len: torch.Tensor      # (B,) cache length to rewind to, -1 = no truncate
    flags: Optional[torch.Tensor] = None  # (B,) flag word, 0 = certain

    def accepted_lists(self) -> List[List[int]]:
        lens = self.accept_len.tolist()
        toks = self.out_tokens.tolist()
        return [row[: n + 1] for row, n in zip(toks, lens)]

    def flagged(self) -> List[int]:
        """Batch positions whose result the reference may have decided otherwise."""
        return [] if self.flags is None else [b for b, f in enumerate(self.flags.tolist()) if f]


def _launch_sample(target: torch.Tensor, draft: torch.Tensor, proposals: torch.Tensor,
                   u: torch.Tensor, noise: Optional[torch.Tensor], temperature: float,
                   is_probs: bool, start_pos: Optional[torch.Tensor], remaining: Optional[torch.Tensor],
                   eos_id: Optional[int], decide_only: bool, accept_prob: Optional[torch.Tensor],
                   result: Optional[VerifyResult], draft_stats: Optional[torch.Tensor] = None,
                   flags: Optional[torch.Tensor] = None) -> None:
    B, C, V = (int(x) for x in target.shape)
    gamma = C - 1
    dev = target.device
    ws_bytes = _hip.lib().spv_verify_sample_workspace_bytes(B, gamma, V)
    if ws_bytes == 0:
        raise ValueError("unsupported verify-sampling shape B={} gamma={} V={}".format(B, gamma, V))
    ws = _workspace.get(ws_bytes, dev)
    r = result
    if flags is None and r is not None:
        flags = r.flags
    call("spv_verify_sample", ptr(target), ptr(draft), 1 if is_probs else 0, float(temperature),
         ptr(proposals), ptr(u), ptr(noise), ptr(draft_stats), ptr(start_pos), ptr(remaining),
         -1 if eos_id is None else int(eos_id), B, gamma, V,
         ptr(r.accept_len) if r else None, ptr(r.out_tokens) if r else None,
         ptr(r.n_commit) if r else None, ptr(r.finished) if r else None,
         ptr(r.new_len) if r else None, ptr(accept_prob), ptr(flags), 1 if decide_only else 0,
         ptr(ws), int(ws_bytes), _hip.stream_of(dev))


@dataclass
class DraftCatchUp:
    """Device int32 outputs of a draft alignment: sequence b's draft model
    decodes ``tokens[b, :count[b]]`` at positions ``pos[b], pos[b] + 1, ...``
    (blocks and length are already in place; ``tokens`` is -1 padded)."""

    count: torch.Tensor    # (B,)
    pos: torch.Tensor      # (B,)
    tokens: torch.Tensor   # (B, gamma+1)


def align_draft(draft_kv: PagedKVCache, seq_ids: torch.Tensor, start_pos: torch.Tensor, result: VerifyResult,
                chunk_tokens: torch.Tensor, out: Optional[DraftCatchUp] = None) -> DraftCatchUp:
    """Align the draft cache with a verify round's commit (spec_scheduler.py:296-322).

    ``seq_ids``/``start_pos`` (B,) int32 device: the round's sequences and their
    start positions; ``result``: the round's ``VerifyResult`` (``n_commit``,
    ``finished``); ``chunk_tokens`` (B, gamma+1) int32 device: the verify
    chunk's tokens (the pending token, then the proposals). Per sequence, in
    batch order: the draft cache is truncated to ``start + n_commit`` when
    longer; when shorter, the missing positions get their blocks (in the
    reference's allocation order) and the returned catch-up names the tokens
    to decode there; finished sequences are cleared. No host synchronisation.
    """
    dev = draft_kv.device
    B = int(seq_ids.numel())
    C = int(chunk_tokens.shape[1]) if chunk_tokens.dim() == 2 else 0
    if chunk_tokens.shape[0] != B or chunk_tokens.dtype != torch.int32 or not chunk_tokens.is_contiguous():
        raise ValueError("chunk_tokens must be a contiguous (B, gamma+1) int32 tensor")
    if out is None:
        out = DraftCatchUp(torch.empty(B, dtype=torch.int32, device=dev), torch.empty(B, dtype=torch.int32, device=dev),
                           torch.empty((B, C), dtype=torch.int32, device=dev))
    draft_kv.align_device(seq_ids, start_pos, result.n_commit, result.finished, chunk_tokens,
                          out.count, out.pos, out.tokens)
    return out


def _new_result(B: int, gamma: int, dev: torch.device) -> VerifyResult:
    z = lambda *s: torch.empty(s, dtype=torch.int32, device=dev)  # noqa: E731
    return VerifyResult(z(B), z(B, gamma + 1), z(B), z(B), z(B), z(B))


def verify_sample(target: torch.Tensor, draft: torch.Tensor, proposals: torch.Tensor,
                  u: torch.Tensor, noise: Optional[torch.Tensor], temperature: float,
                  start_pos: Optional[torch.Tensor] = None, remaining: Optional[torch.Tensor] = None,
                  eos_id: Optional[int] = None, is_probs: bool = False,
                  result: Optional[VerifyResult] = None, validate: bool = True,
                  top_k: int = 0, top_p: float = 1.0,
                  draft_stats: Optional[torch.Tensor] = None) -> VerifyResult:
    """Fused accept / resample / bonus / commit cut of one round (device in, device out).

    ``target`` (B, gamma+1, V) and ``draft`` (B, gamma, V) are fp32 logits (or
    probabilities with ``is_probs``); ``proposals`` (B, gamma); ``u`` (B, gamma)
    uniforms; ``noise`` (B, V) ``Exp(1)`` rows (unused for greedy logits).
    ``top_k``/``top_p`` filter both sides' logits first (logits_to_probs,
    specdec/sampler.py:19-56; sampling mode only): every row is scaled and
    filtered in one launch, then sampled at temperature 1; with top_p a
    sequence whose rows have values within rounding of the nucleus edge gets
    ``FLAG_TOP_P_BAND``. ``draft_stats`` (B, gamma, 2) float32: the draft
    rows' statistics as ``draft_sample`` / ``DraftLoop`` wrote them when they
    drew the proposals at this temperature (the draft loop's q,
    spec_scheduler.py:243-252), so only the target rows are read for their
    normalisers (not used with filters, which this call applies itself).
    ``validate=False`` skips the proposal-range check (a host synchronisation).
    """
    dev = _hip.require_gpu(target.device)
    B, C, V = target.shape
    gamma = C - 1
    if tuple(draft.shape) != (B, gamma, V) or tuple(proposals.shape) != (B, gamma) or \
            tuple(u.shape) != (B, gamma):
        raise ValueError("inconsistent verify-sampling shapes")
    greedy = not is_probs and not temperature > 0
    if noise is not None and tuple(noise.shape) != (B, V):
        raise ValueError("noise must be (B, V)")
    if noise is None and not greedy:
        raise ValueError("sampling needs the Exp(1) noise rows")
    t = target.float().contiguous()
    d = draft.float().contiguous()
    amb = None
    if not greedy and not is_probs and _hip.filtering(top_k, top_p, V):
        t, amb_t = _hip.filter_rows(t, temperature, top_k, top_p, ambiguous=True)
        d, amb_d = _hip.filter_rows(d, temperature, top_k, top_p, ambiguous=True)
        amb = amb_t.sum(1) + amb_d.sum(1)
        temperature = 1.0
        draft_stats = None
    if draft_stats is not None:
        if is_probs or tuple(draft_stats.shape) != (B, gamma, 2) or draft_stats.dtype != torch.float32 \
                or not draft_stats.is_contiguous() or draft_stats.device != dev:
            raise ValueError("draft_stats must be a contiguous (B, gamma, 2) float32 device tensor of logits rows")
    x = _hip.i32(proposals, dev)
    if validate and (int(x.min().item()) < 0 or int(x.max().item()) >= V):
        raise IndexError("proposal token ids must lie in [0, V)")
    uf = u.to(device=dev, dtype=torch.float32).contiguous()
    nz = None if noise is None else noise.to(device=dev, dtype=torch.float32).contiguous()
    sp = None if start_pos is None else _hip.i32(start_pos, dev)
    rem = None if remaining is None else _hip.i32(remaining, dev)
    if result is None:
        result = _new_result(int(B), int(gamma), dev)
    _launch_sample(t, d, x, uf, nz, temperature, is_probs, sp, rem, eos_id, False, None, result,
                   draft_stats=draft_stats)
    if amb is not None:
        result.flags.bitwise_or_((amb > 0).to(torch.int32) * _hip.FLAG_TOP_P_BAND)
    return result


def acceptance_probabilities(target: torch.Tensor, draft: torch.Tensor, proposals: torch.Tensor,
                             temperature: float = 1.0, is_probs: bool = True) -> torch.Tensor:
    """float64 (B, gamma) acceptance probabilities of every position (one launch)."""
    dev = _hip.require_gpu(target.device)
    B, C, V = target.shape
    t = target.float().contiguous()
    d = draft.float().contiguous()
    x = _hip.i32(proposals, dev)
    a = torch.empty((B, C - 1), dtype=torch.float64, device=dev)
    u = torch.zeros((B, C - 1), dtype=torch.float32, device=dev)
    _launch_sample(t, d, x, u, None, temperature, is_probs, None, None, None, True, a, None)
    return a


def batch_accept(p_by_sid: Dict[int, torch.Tensor], q_by_sid: Dict[int, Sequence[torch.Tensor]],
                 proposals_by_sid: Dict[int, Sequence[int]], generator: torch.Generator
                 ) -> Dict[int, List[int]]:
    """Accept/reject each sequence's draft block (spec_scheduler.py:46-88).

    ``p_by_sid[sid]`` is the ``(gamma+1, V)`` target distribution block,
    ``q_by_sid[sid]`` the ``gamma`` draft rows, ``proposals_by_sid[sid]`` the
    proposed ids; returns the committed token list (length 1..gamma+1) per
    sequence, consuming ``generator`` exactly as the reference does.
    """
    sids = list(p_by_sid.keys())
    if not sids:
        return {}
    gammas = {len(proposals_by_sid[s]) for s in sids}
    if len(gammas) != 1:
        # Mixed draft lengths: sequences are independent, keep dict order.
        out: Dict[int, List[int]] = {}
        for s in sids:
            out.update(batch_accept({s: p_by_sid[s]}, {s: q_by_sid[s]}, {s: proposals_by_sid[s]},
                                    generator))
        return out
    gamma = gammas.pop()
    dev = _hip.require_gpu(p_by_sid[sids[0]].device)
    p = torch.stack([p_by_sid[s].float() for s in sids]).contiguous()
    q = torch.stack([torch.stack([r.float() for r in q_by_sid[s]]) for s in sids]).contiguous()
    B, C, V = p.shape
    if C != gamma + 1 or tuple(q.shape) != (B, gamma, V):
        raise ValueError("p rows must be gamma+1 and q rows gamma per sequence")
    x = torch.tensor([list(proposals_by_sid[s]) for s in sids], dtype=torch.int32, device=dev)
    a = acceptance_probabilities(p, q, x, is_probs=True).tolist()
    # Host draws, in the reference's order.
    u = torch.full((B, gamma), 2.0, dtype=torch.float32)
    noise = torch.empty((B, V), dtype=torch.float32)
    for b in range(B):
        for j in range(gamma):
            uj = _draw_uniform(generator)
            u[b, j] = uj
            if not uj < a[b][j]:
                break
        noise[b] = torch.empty(V, dtype=torch.float32).exponential_(1, generator=generator)
    res = verify_sample(p, q, x, u.to(dev), noise.to(dev), 1.0, is_probs=True)
    lists = res.accepted_lists()
    return {s: lists[i] for i, s in enumerate(sids)}


class VerifyStep:
    """One verify round over a continuous batch on one GPU.

    The caller supplies, per round: the batch's sequence ids and start
    positions (``kv.seq_lengths`` at round start), per-layer ``(q, k, v)`` of the
    ``gamma+1`` verify tokens, the target/draft logits of the round, the draft
    proposals, and the randomness. The round writes the K/V of every layer,
    runs verify attention per layer (the layers share one ``VerifyPlan``, made
    after the first layer's append allocated the round's blocks), samples, and
    rewinds the pool on the device with the sampled lengths. Nothing
    synchronises with the host.

    ``sample_and_commit(..., apply=False)`` holds the round's commit instead:
    the next ``attend_layers`` over the same sequence ids (same order) applies
    it together with its first layer's append in one launch
    (``rewind_append_device``: the two calls' exact result). Any other batch, or
    ``flush()``, applies it on its own first. Until then the pool still holds
    the round's uncommitted tail, so a caller that reads or changes the pool
    between rounds (admission, metrics) calls ``flush()`` first.
    """

    def __init__(self, kv: PagedKVCache, gamma: int, temperature: float, eos_id: Optional[int] = None):
        self.kv = kv
        self.gamma = int(gamma)
        self.temperature = float(temperature)
        self.eos_id = eos_id
        self._write_plan = WritePlan()  # the round's rows, recorded by its first layer's append
        self._pending = None  # (sequence ids, their VerifyResult): a commit not yet applied

    def flush(self) -> None:
        """Apply a held commit (``sample_and_commit(..., apply=False)``)."""
        if self._pending is not None:
            sids, res = self._pending
            self._pending = None
            self.kv.rewind_device(_hip.i32(sids, self.kv.device), res.new_len, res.finished)

    def attend_layers(self, seq_ids: Sequence[int], start_positions: Sequence[int],
                      q_layers: Sequence[torch.Tensor], k_layers: Sequence[torch.Tensor],
                      v_layers: Sequence[torch.Tensor],
                      outs: Optional[Sequence[torch.Tensor]] = None,
                      events: Optional[list] = None) -> List[torch.Tensor]:
        """Append and attend, layer by layer. With ``events`` (a list), timing
        events are recorded on the current stream and appended to it: before
        each layer's append, before its attention, and after the last attention
        (``2 * layers + 1`` events)."""
        chunk = self.gamma + 1
        max_ctx = max(int(s) for s in start_positions) + chunk
        sid_t = _hip.i32(seq_ids, self.kv.device)
        st_t = _hip.i32(start_positions, self.kv.device)
        results = []
        self.kv._grow_width(-(-max_ctx // self.kv.block_size))

        def mark():
            if events is not None:
                e = torch.cuda.Event(enable_timing=True)
                e.record()
                events.append(e)

        pending = None
        if self._pending is not None:
            if list(self._pending[0]) == [int(s) for s in seq_ids] and not self.kv.fp8:
                pending = self._pending[1]
                self._pending = None
            else:
                self.flush()
        plan = None
        for layer in range(len(q_layers)):
            mark()
            kl = k_layers[layer].to(self.kv.dtype).contiguous()
            vl = v_layers[layer].to(self.kv.dtype).contiguous()
            if layer == 0 and pending is not None:
                # the previous round's commit, then this round's allocating append: one launch
                self.kv.rewind_append_device(sid_t, pending.new_len, pending.finished, st_t, kl, vl,
                                             layer=0, plan=self._write_plan)
            else:
                # the first layer's call allocates the chunk's blocks for every layer
                # (and records where its tokens went: the later layers copy by that plan)
                self.kv.write_block_device(layer, sid_t, st_t, kl, vl, alloc=layer == 0, plan=self._write_plan)
            if plan is None:  # the round's attention plan, once its blocks exist
                plan = VerifyPlan(self.kv, sid_t, st_t, chunk, int(q_layers[layer].shape[2]), max_ctx)
            mark()
            results.append(verify_attention(q_layers[layer], self.kv, layer, sid_t, st_t, max_ctx,
                                            out=None if outs is None else outs[layer], plan=plan))
        mark()
        return results

    def sample_and_commit(self, seq_ids: Sequence[int], start_positions: Sequence[int],
                          target_logits: torch.Tensor, draft_logits: torch.Tensor,
                          proposals: torch.Tensor, u: torch.Tensor, noise: Optional[torch.Tensor],
                          remaining: Optional[Sequence[int]] = None, apply: bool = True,
                          draft_stats: Optional[torch.Tensor] = None) -> VerifyResult:
        """Fused accept / resample / bonus and the commit cut; then the pool's
        rewind, or (``apply=False``) the commit held for the next round.
        ``draft_stats``: the draft rows' statistics from the draft loop
        (``verify_sample``)."""
        self.flush()
        dev = self.kv.device
        sid_t = _hip.i32(seq_ids, dev)
        st_t = _hip.i32(start_positions, dev)
        rem_t = None if remaining is None else _hip.i32(remaining, dev)
        res = verify_sample(target_logits, draft_logits, proposals, u, noise, self.temperature,
                            start_pos=st_t, remaining=rem_t, eos_id=self.eos_id, validate=False,
                            draft_stats=draft_stats)
        if apply:
            self.kv.rewind_device(sid_t, res.new_len, res.finished)
        else:
            self._pending = ([int(s) for s in seq_ids], res)
        return res


def draft_sample(logits: torch.Tensor, temperature: float, noise: Optional[torch.Tensor] = None,
                 out: Optional[torch.Tensor] = None, top_k: int = 0, top_p: float = 1.0,
                 stats: Optional[torch.Tensor] = None, flags: Optional[torch.Tensor] = None) -> torch.Tensor:
    """One draft step's proposals for every row in one launch (spec_scheduler.py:243-252).

    ``logits`` (B, V) fp32 draft logits (rows may be strided, elements
    contiguous); row b's token is ``sample_token(logits_to_probs(logits[b]))``
    drawn as ``argmax(q / noise[b])`` with the caller's ``Exp(1)`` rows
    ``noise`` (B, V), or the first-index argmax when ``temperature <= 0``
    (``noise`` unused). ``out``: an int32 device view of B entries to write
    (e.g. column s of the (B, gamma) proposals), else a new tensor. ``top_k``
    / ``top_p`` filter the rows first (sampling mode). ``stats``: a float32
    (B, 2) view (e.g. ``draft_stats[:, s]``) for each row's softmax statistics,
    what ``verify_sample`` takes as ``draft_stats``; ``flags``: an int32 view
    of B entries for each draw's flag word (``_hip.FLAG_DRAW_BAND`` when the
    token's key lies within rounding of another's). No host synchronisation.
    """
    dev = _hip.require_gpu(logits.device)
    if logits.dim() != 2 or logits.stride(1) != 1 or logits.dtype != torch.float32:
        raise ValueError("logits must be a (B, V) float32 tensor with contiguous rows")
    B, V = (int(x) for x in logits.shape)
    greedy = not temperature > 0
    if not greedy and _hip.filtering(top_k, top_p, V):
        logits = _hip.filter_rows(logits, temperature, top_k, top_p)
        temperature = 1.0
    if not greedy:
        if noise is None or tuple(noise.shape) != (B, V) or noise.dtype != torch.float32 or not noise.is_contiguous():
            raise ValueError("sampling needs contiguous float32 Exp(1) rows of shape (B, V)")
    if out is None:
        out = torch.empty(B, dtype=torch.int32, device=dev)
    if out.dtype != torch.int32 or out.dim() != 1 or out.numel() != B or out.device != dev:
        raise ValueError("out must be an int32 device vector of B entries")
    stride = int(out.stride(0))
    # the statistics and flags share the tokens' row stride (in their own units)
    if stats is not None and (stats.dtype != torch.float32 or tuple(stats.shape) != (B, 2) or stats.stride(1) != 1
                              or stats.stride(0) != 2 * stride or stats.device != dev):
        raise ValueError("stats must be a float32 (B, 2) device view with row stride 2 x out's stride")
    if flags is not None and (flags.dtype != torch.int32 or flags.dim() != 1 or flags.numel() != B
                              or flags.stride(0) != stride or flags.device != dev):
        raise ValueError("flags must be an int32 device view of B entries with out's stride")
    ws_bytes = _hip.lib().spv_draft_sample_workspace_bytes(max(B, 1), V)
    if ws_bytes == 0:
        raise ValueError("unsupported draft-sampling shape B={} V={}".format(B, V))
    ws = _draft_workspace.get(ws_bytes, dev)
    call("spv_draft_sample", ptr(logits), int(logits.stride(0)), float(temperature),
         None if greedy else ptr(noise), B, V, ptr(out), stride, ptr(stats), ptr(flags), ptr(ws), int(ws_bytes),
         _hip.stream_of(dev))
    return out


def draft_sample_with_generator(q_logits: torch.Tensor, sampling, generator: torch.Generator) -> List[int]:
    """The reference's per-row loop of one draft step (spec_scheduler.py:246-251:
    ``logits_to_probs`` then ``sample_token`` drawing from ``generator``) as one
    launch: the B ``Exp(1)`` rows the B multinomial draws consume are drawn from
    ``generator`` on the host in batch order (also when greedy, where the
    reference's draw from a one-hot row still consumes them), then raced on the
    device. Returns the B token ids; the generator ends where the reference's does."""
    top_k = int(getattr(sampling, "top_k", 0) or 0)
    top_p = float(getattr(sampling, "top_p", 1.0))
    z = q_logits.detach().float().contiguous()
    B, V = (int(x) for x in z.shape)
    noise = torch.stack([torch.empty(V, dtype=torch.float32).exponential_(1, generator=generator)
                         for _ in range(B)]) if B else torch.empty(0, V)
    temperature = 0.0 if sampling.is_greedy else float(sampling.temperature)
    return draft_sample(z, temperature, noise.to(z.device), top_k=top_k, top_p=top_p).tolist()


class DraftLoop:
    """The paged part of the gamma draft decode steps and their sampling.

    Per step s (positions ``ctx + s``, device-resident) and draft layer l: the
    new token's K/V are written at ``ctx + s`` (allocating at layer 0, the
    write-then-attend order of engine/model.py:123-153), then decode attention
    of the step's query over positions ``0 .. ctx + s``; after the last layer
    the step's proposals are drawn from its draft logits into column s of the
    (B, gamma) proposals (spec_scheduler.py:243-252). Every launch goes to the
    current stream and nothing synchronises with the host, so ``run`` can be
    captured in a HIP graph; the draft model between the steps is the caller's.
    """

    def __init__(self, kv: PagedKVCache, gamma: int, temperature: float):
        self.kv = kv
        self.gamma = int(gamma)
        self.temperature = float(temperature)
        self._write_plan = WritePlan()  # a step's rows, recorded by its first layer's append

    def run(self, seq_ids: torch.Tensor, ctx: torch.Tensor, max_ctx: int,
            q_steps: Sequence[Sequence[torch.Tensor]], k_steps: Sequence[Sequence[torch.Tensor]],
            v_steps: Sequence[Sequence[torch.Tensor]], logits_steps: Sequence[torch.Tensor],
            noise_steps: Optional[Sequence[torch.Tensor]] = None,
            proposals: Optional[torch.Tensor] = None,
            attn_out: Optional[Sequence[Sequence[torch.Tensor]]] = None,
            stats: Optional[torch.Tensor] = None, flags: Optional[torch.Tensor] = None):
        """``seq_ids``/``ctx`` (B,) int32 device: the sequences and their draft
        cache lengths before the loop; ``max_ctx`` >= max(ctx) (host int).
        ``q_steps[s][l]`` (B, 1, Hq, d), ``k_steps``/``v_steps[s][l]`` (B, 1,
        Hkv, d), ``logits_steps[s]`` (B, V) fp32, ``noise_steps[s]`` (B, V)
        Exp(1) rows (None when greedy). ``stats`` (B, gamma, 2) float32 and
        ``flags`` (B, gamma) int32, optional: each step's draft-row statistics
        (``VerifyStep.sample_and_commit(draft_stats=...)``) and draw flags.
        Returns (proposals (B, gamma) int32, attention outputs [s][l])."""
        kv = self.kv
        dev = kv.device
        B = int(seq_ids.numel())
        if proposals is None:
            proposals = torch.empty((B, self.gamma), dtype=torch.int32, device=dev)
        outs = []
        for s in range(self.gamma):
            pos = ctx + s
            outs_s = []
            plan = None
            for layer in range(len(q_steps[s])):
                kv.write_block_device(layer, seq_ids, pos, k_steps[s][layer], v_steps[s][layer], alloc=layer == 0,
                                      plan=self._write_plan)
                if plan is None:  # the step's attention plan, once its blocks exist
                    plan = VerifyPlan(kv, seq_ids, pos, 1, int(q_steps[s][layer].shape[2]), max_ctx + s + 1)
                o = None if attn_out is None else attn_out[s][layer]
                outs_s.append(verify_attention(q_steps[s][layer], kv, layer, seq_ids, pos, max_ctx + s + 1, out=o,
                                               plan=plan))
            outs.append(outs_s)
            draft_sample(logits_steps[s], self.temperature, None if noise_steps is None else noise_steps[s],
                         out=proposals[:, s], stats=None if stats is None else stats[:, s],
                         flags=None if flags is None else flags[:, s])
        return proposals, outs
