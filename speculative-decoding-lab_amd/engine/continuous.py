"""One-GPU continuous batching of speculative verify rounds.

The round loop of the reference's speculative engine
(engine/spec_scheduler.py:166-222, ``run_spec_continuous``) applied to the
device verify path:

* requests arrive at integer steps and are admitted in arrival order when the
  batch has room and the pool can hold the request's whole lifetime (prompt,
  budget and one verify chunk) next to what the running sequences may still
  claim. The reference admits every due request and fails when the pool runs
  out; reserving lifetimes makes exhaustion impossible instead;
* every running sequence then takes one round. With a draft pool, the draft
  side first proposes gamma tokens per sequence (``DraftLoop``: per step and
  draft layer a one-token append and decode attention, then batched sampling;
  spec_scheduler.py:243-252); otherwise the proposals are given. The K/V of the
  gamma+1 verify tokens of every layer are appended, verify attention runs per
  layer, the round is sampled (accept / residual / bonus) and the pool is
  rewound on the device to the committed length (``VerifyStep``). The draft
  pool is then aligned on the device (``align_draft``: truncate, catch-up
  allocation, clear; spec_scheduler.py:305-322) and the catch-up tokens are
  decoded into it;
* sequences that reach their budget (or eos) leave; their blocks went back to
  the free stacks in the same launches;
* after the round's admissions the scheduler metrics of the reference
  (spec_scheduler.py:200-205: batch size, block utilisation, peak blocks of
  both pools) are recorded on the device and read back once at the end.

The target and draft models are outside this path, so a ``SyntheticVerifyModel``
stands in for them: seeded device tensors of the shapes one round consumes
(queries, keys and values per layer, target and draft logits, proposals drawn
from the draft distribution, uniforms and ``Exp(1)`` rows; with a draft pool
also the draft layers' queries, keys and values per step and the draft
sampling's ``Exp(1)`` rows). With target logits ``N(0, 2^2)`` and draft logits
``target + N(0, sigma^2)`` over a 151,936-entry vocabulary, sigma = 1.05
accepts a proposal with probability about 0.6.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Callable, List, Optional, Sequence

import torch

from . import _hip
from .attention import VerifyPlan, verify_attention
from .kv import PagedKVCache
from .spec_scheduler import DraftCatchUp, DraftLoop, VerifyResult, VerifyStep, align_draft, draft_sample


@dataclass
class Request:
    """One generation request (the reference's WorkloadRequest: arrival step,
    prompt length, token budget)."""

    sid: int
    arrive_step: int
    prompt_len: int
    max_new_tokens: int


@dataclass
class SeqState:
    """A running sequence. As in the reference, the cache holds the prompt and
    every generated token but the last (``length == prompt_len + generated - 1``):
    the prefill's token is the first generated one and the pending input of the
    first verify round."""

    sid: int
    length: int            # tokens in the cache (the next verify round's start)
    max_new_tokens: int
    lifetime_blocks: int   # blocks the sequence may hold at most
    generated: int = 1
    finished: bool = False


@dataclass
class RoundInfo:
    """What one verify round saw and produced (handed to ``on_round``)."""

    step: int
    sids: List[int]
    starts: List[int]
    result: VerifyResult
    inputs: dict
    outputs: List[torch.Tensor]
    seconds: float
    gpu_ms: Optional[dict] = None   # {"append", "attend", "sample"} when timed with events
    draft_outputs: Optional[List[List[torch.Tensor]]] = None   # [step][draft layer] decode attention
    catch_up: Optional[DraftCatchUp] = None                    # the draft alignment's catch-up
    catch_up_outputs: Optional[List[torch.Tensor]] = None      # [draft layer] catch-up decode attention
    catch_up_rows: Optional[List[int]] = None                  # batch rows decoded in the catch-up


@dataclass
class DriverResult:
    """Counters of one run, named as in the reference's SchedulerResult
    (engine/scheduler.py:60-80): ``tokens_per_round`` holds the committed count
    ``k`` of every sequence in every round, ``batch_hist`` the batch size of
    every round."""

    gamma: int
    steps: int = 0
    rounds: int = 0
    round_seconds: List[float] = field(default_factory=list)
    gpu_ms: List[dict] = field(default_factory=list)
    batch_hist: List[int] = field(default_factory=list)
    block_util_hist: List[float] = field(default_factory=list)
    tokens_per_round: List[int] = field(default_factory=list)
    kv_peak_blocks: int = 0
    draft_kv_peak_blocks: int = 0
    draft_forward_calls: int = 0
    admitted: int = 0
    finished: int = 0
    # sequence-rounds whose verify result, and draft draws, carry a flag: a
    # result the reference's own fp32 softmax may have decided otherwise
    flagged_rounds: int = 0
    flagged_draws: int = 0

    @property
    def mean_tokens_per_round(self) -> float:
        return sum(self.tokens_per_round) / len(self.tokens_per_round) if self.tokens_per_round else 0.0

    @property
    def mean_acceptance(self) -> float:
        """Mean committed tokens per sequence and round over ``gamma + 1``
        (engine/spec_scheduler.py:214-217)."""
        return self.mean_tokens_per_round / (self.gamma + 1)


class SyntheticVerifyModel:
    """Seeded device stand-ins for the per-round model outputs.

    Per layer one set of queries / keys / values for ``max_batch`` sequences is
    drawn once and its first ``B`` rows serve every round; ``n_sets`` sets of
    logits (with proposals, uniforms and noise) alternate between rounds. Prompt
    K/V come from one bank of ``prompt_cap`` token rows. Without a draft side
    the proposals are given, and so are the draft rows' softmax statistics at
    ``temperature`` (as the draft sampler keeps them when it draws).
    """

    def __init__(self, num_layers: int, num_q_heads: int, num_kv_heads: int, head_dim: int, vocab: int,
                 gamma: int, max_batch: int, device: torch.device, dtype: torch.dtype = torch.bfloat16,
                 seed: int = 0, draft_sigma: float = 1.05, prompt_cap: int = 8192, n_sets: int = 2,
                 temperature: float = 1.0, draft_layers: int = 0, draft_heads: tuple = (0, 0, 0)) -> None:
        g = torch.Generator(device=device).manual_seed(seed)
        C = gamma + 1
        self.num_layers, self.gamma, self.vocab = num_layers, gamma, vocab
        self.draft_layers = draft_layers
        self.temperature = float(temperature)
        self.q = [torch.randn(max_batch, C, num_q_heads, head_dim, device=device, generator=g).to(dtype)
                  for _ in range(num_layers)]
        self.k = [torch.randn(max_batch, C, num_kv_heads, head_dim, device=device, generator=g).to(dtype)
                  for _ in range(num_layers)]
        self.v = [torch.randn(max_batch, C, num_kv_heads, head_dim, device=device, generator=g).to(dtype)
                  for _ in range(num_layers)]
        self.bank_k = torch.randn(1, prompt_cap, num_kv_heads, head_dim, device=device, generator=g).to(dtype)
        self.bank_v = torch.randn(1, prompt_cap, num_kv_heads, head_dim, device=device, generator=g).to(dtype)
        self.sets = []
        for _ in range(n_sets):
            target = torch.randn(max_batch, C, vocab, device=device, generator=g) * 2.0
            draft = target[:, :gamma] + torch.randn(max_batch, gamma, vocab, device=device, generator=g) * draft_sigma
            probs = torch.softmax(draft.reshape(-1, vocab) / max(temperature, 1e-12), dim=-1)
            proposals = torch.multinomial(probs, 1, generator=g).reshape(max_batch, gamma).to(torch.int32)
            u = torch.rand(max_batch, gamma, device=device, generator=g)
            noise = torch.empty(max_batch, vocab, device=device).exponential_(1, generator=g)
            draft = draft.contiguous()
            # the draft rows' statistics as the draft sampler writes them (its
            # tokens are not used: the proposals above are the round's)
            dstats = torch.empty(max_batch, gamma, 2, dtype=torch.float32, device=device)
            scratch = torch.empty(max_batch, gamma, dtype=torch.int32, device=device)
            for j in range(gamma):
                draft_sample(draft[:, j], temperature, noise, out=scratch[:, j], stats=dstats[:, j])
            self.sets.append((target.contiguous(), draft, proposals, u, noise, dstats))
            del probs, scratch
        if draft_layers:
            # draft side: per step and draft layer one token's q / k / v (the
            # catch-up decode uses step 0's), a prompt bank, and per set the
            # draft sampling's Exp(1) rows of every step
            dhq, dhkv, dd = draft_heads
            rnd = lambda *shape: torch.randn(*shape, device=device, generator=g).to(dtype)  # noqa: E731
            self.dq = [[rnd(max_batch, 1, dhq, dd) for _ in range(draft_layers)] for _ in range(gamma)]
            self.dk = [[rnd(max_batch, 1, dhkv, dd) for _ in range(draft_layers)] for _ in range(gamma)]
            self.dv = [[rnd(max_batch, 1, dhkv, dd) for _ in range(draft_layers)] for _ in range(gamma)]
            self.dbank_k = rnd(1, prompt_cap, dhkv, dd)
            self.dbank_v = rnd(1, prompt_cap, dhkv, dd)
            self.draft_noise = [torch.empty(gamma, max_batch, vocab, device=device).exponential_(1, generator=g)
                                for _ in range(n_sets)]

    def prompt_kv(self, n: int):
        if n > self.bank_k.shape[1]:
            raise ValueError("prompt longer than the synthetic bank")
        return self.bank_k[:, :n], self.bank_v[:, :n]

    def draft_prompt_kv(self, n: int):
        return self.dbank_k[:, :n], self.dbank_v[:, :n]

    def round_inputs(self, round_idx: int, B: int) -> dict:
        i = round_idx % len(self.sets)
        target, draft, proposals, u, noise, dstats = self.sets[i]
        inp = {
            "q": [x[:B] for x in self.q], "k": [x[:B] for x in self.k], "v": [x[:B] for x in self.v],
            "target": target[:B], "draft": draft[:B], "proposals": proposals[:B], "u": u[:B], "noise": noise[:B],
            "draft_stats": dstats[:B],
        }
        if self.draft_layers:
            inp["dq"] = [[x[:B] for x in st] for st in self.dq]
            inp["dk"] = [[x[:B] for x in st] for st in self.dk]
            inp["dv"] = [[x[:B] for x in st] for st in self.dv]
            inp["draft_noise"] = [self.draft_noise[i][s, :B] for s in range(self.gamma)]
        return inp


class SpecContinuousDriver:
    """Continuous batching of speculative rounds over one device pool (and,
    when ``draft_kv`` is given, the draft model's pool beside it)."""

    def __init__(self, kv: PagedKVCache, model: SyntheticVerifyModel, gamma: int, max_batch: int,
                 temperature: float = 1.0, eos_id: Optional[int] = None,
                 draft_kv: Optional[PagedKVCache] = None) -> None:
        self.kv = kv
        self.model = model
        self.gamma = int(gamma)
        self.max_batch = int(max_batch)
        self.temperature = float(temperature)
        self.step_fn = VerifyStep(kv, gamma, temperature, eos_id)
        self.draft_kv = draft_kv
        self.draft_loop = DraftLoop(draft_kv, gamma, temperature) if draft_kv is not None else None
        if draft_kv is not None and not getattr(model, "draft_layers", 0):
            raise ValueError("a draft pool needs a model with draft layers")
        self.running: List[SeqState] = []
        # the pending (last committed) token per sequence id, on the device
        self._pending = torch.zeros(0, dtype=torch.int32, device=kv.device)
        # metrics records (spec_scheduler.py:200-205), one row per step, on the device
        self._rec = self._drec = None
        self._peak = torch.zeros(1, dtype=torch.int64, device=kv.device)
        self._dpeak = torch.zeros(1, dtype=torch.int64, device=kv.device)
        self._nrec = 0

    # ------------------------------------------------------------ admission
    def _blocks_for(self, tokens: int, kv: Optional[PagedKVCache] = None) -> int:
        return -(-tokens // (kv or self.kv).block_size)

    def lifetime_blocks(self, prompt_len: int, max_new_tokens: int, kv: Optional[PagedKVCache] = None) -> int:
        """Most blocks a request can hold: while it runs the cache holds at most
        ``prompt_len + max_new_tokens - 2`` tokens and a round appends
        ``gamma + 1`` more (the draft cache: gamma proposals, then at most one
        catch-up position)."""
        return self._blocks_for(prompt_len + max(max_new_tokens, 1) + self.gamma - 1, kv)

    def _pools(self) -> List[PagedKVCache]:
        return [self.kv] if self.draft_kv is None else [self.kv, self.draft_kv]

    def _flush_arrivals(self, due: List[Request], result: DriverResult) -> List[Request]:
        """Admit due requests in arrival order while the batch and the pools have
        room (first come, first served: a request that does not fit holds back
        the ones behind it); returns the ones left waiting."""
        waiting = []
        pools = self._pools()
        free = [kv.allocator.num_free for kv in pools]
        reserved = [sum(s.lifetime_blocks if kv is self.kv else
                        self.lifetime_blocks(s.length - s.generated + 1, s.max_new_tokens, kv)
                        for s in self.running) -
                    sum(self._blocks_for(s.length, kv) for s in self.running) for kv in pools]
        for i, r in enumerate(due):
            need = [self.lifetime_blocks(r.prompt_len, r.max_new_tokens, kv) for kv in pools]
            for kv, n in zip(pools, need):
                if n > kv.allocator.capacity:
                    raise ValueError("request {} needs {} blocks, more than the pool's {}".format(
                        r.sid, n, kv.allocator.capacity))
            if len(self.running) >= self.max_batch or any(f - rs < n for f, rs, n in zip(free, reserved, need)):
                waiting.extend(due[i:])
                break
            self.kv.add_sequence(r.sid)
            k, v = self.model.prompt_kv(r.prompt_len)
            for layer in range(self.model.num_layers):  # prefill's K/V write (model.py:369-399)
                self.kv.write_block(layer, [r.sid], [0], k, v)
            if self.draft_kv is not None:  # the draft sees the same prompt (spec_scheduler.py:158-160)
                self.draft_kv.add_sequence(r.sid)
                dk, dv = self.model.draft_prompt_kv(r.prompt_len)
                for layer in range(self.model.draft_layers):
                    self.draft_kv.write_block(layer, [r.sid], [0], dk, dv)
                if r.sid >= self._pending.numel():
                    grown = torch.zeros(max(r.sid + 1, 2 * self._pending.numel()), dtype=torch.int32,
                                        device=self.kv.device)
                    grown[: self._pending.numel()] = self._pending
                    self._pending = grown
                self._pending[r.sid] = 0  # the prefill's token (synthetic)
            for j, kv in enumerate(pools):
                free[j] -= self._blocks_for(r.prompt_len, kv)
                reserved[j] += need[j] - self._blocks_for(r.prompt_len, kv)
            self.running.append(SeqState(r.sid, r.prompt_len, r.max_new_tokens, need[0]))
            result.admitted += 1
        return waiting

    # ---------------------------------------------------------------- round
    def _round(self, step: int, result: DriverResult, on_round: Optional[Callable[[RoundInfo], None]],
               sync_timing: bool, gpu_timing) -> None:
        running = self.running
        sids = [s.sid for s in running]
        starts = [s.length for s in running]
        remaining = [s.max_new_tokens - s.generated for s in running]
        B = len(running)
        dev = self.kv.device
        inp = self.model.round_inputs(result.rounds, B)
        if sync_timing:
            torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        per_layer = gpu_timing is True or gpu_timing == "layers"
        evs = [] if per_layer else None
        round_evs = None
        if gpu_timing == "round":  # the round's span only: no event between its kernels
            round_evs = [torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)]
            round_evs[0].record()
        sid_t = _hip.i32(sids, dev)
        st_t = _hip.i32(starts, dev)
        d_outs = cu = d_stats = d_flags = None
        if self.draft_kv is not None:
            # gamma draft steps from the draft cache's length (== start); the
            # draws keep each draft row's softmax statistics for the decisions
            max_ctx = max(starts)
            self.draft_kv._grow_width(self._blocks_for(max_ctx + self.gamma + 1, self.draft_kv))
            greedy = not self.temperature > 0
            d_stats = torch.empty((B, self.gamma, 2), dtype=torch.float32, device=dev)
            d_flags = torch.empty((B, self.gamma), dtype=torch.int32, device=dev)
            props, d_outs = self.draft_loop.run(
                sid_t, st_t, max_ctx, inp["dq"], inp["dk"], inp["dv"],
                [inp["draft"][:, j] for j in range(self.gamma)], None if greedy else inp["draft_noise"],
                stats=d_stats, flags=d_flags)
            inp["proposals"] = props
            result.draft_forward_calls += self.gamma
        outs = self.step_fn.attend_layers(sids, starts, inp["q"], inp["k"], inp["v"], events=evs)
        if d_stats is None and self.model.temperature == self.temperature:
            d_stats = inp["draft_stats"]  # the given proposals' draft statistics
        res = self.step_fn.sample_and_commit(sids, starts, inp["target"], inp["draft"], inp["proposals"],
                                             inp["u"], inp["noise"], remaining, draft_stats=d_stats)
        if self.draft_kv is not None:
            sid_l = sid_t.long()
            pending = self._pending[sid_l]
            chunk = torch.cat((pending.unsqueeze(1), inp["proposals"]), 1).contiguous()
            cu = align_draft(self.draft_kv, sid_t, st_t, res, chunk)
            last = res.out_tokens.gather(1, (res.n_commit.long() - 1).clamp(min=0).unsqueeze(1)).squeeze(1)
            self._pending[sid_l] = torch.where(res.n_commit > 0, last, pending)
        if per_layer:
            evs.append(torch.cuda.Event(enable_timing=True))
            evs[-1].record()
        # the round's one host synchronisation
        counts = [res.n_commit, res.finished, res.flags] + (
            [cu.count, (d_flags != 0).any(1).to(torch.int32), cu.pos] if cu is not None else [])
        host = torch.stack(counts).tolist()
        n_commit, finished = host[0], host[1]
        result.flagged_rounds += sum(1 for f in host[2] if f)
        if cu is not None:
            result.flagged_draws += sum(host[4])
        cu_outs = cu_rows = None
        if cu is not None and any(host[3]):
            cu_outs, cu_rows = self._catch_up(host[3], host[5], sids, inp, result)
        if round_evs is not None:
            round_evs[1].record()
        if sync_timing:
            torch.cuda.synchronize(dev)  # the catch-up's launches are the round's too
        dt = time.perf_counter() - t0
        gms = None
        if round_evs is not None:
            torch.cuda.synchronize(dev)
            gms = {"round": round_evs[0].elapsed_time(round_evs[1])}
            result.gpu_ms.append(gms)
        elif per_layer:
            torch.cuda.synchronize(dev)
            nl = len(inp["q"])
            gms = {"append": sum(evs[2 * i].elapsed_time(evs[2 * i + 1]) for i in range(nl)),
                   "attend": sum(evs[2 * i + 1].elapsed_time(evs[2 * i + 2]) for i in range(nl)),
                   "sample": evs[2 * nl].elapsed_time(evs[2 * nl + 1]),
                   "round": evs[0].elapsed_time(evs[-1])}
            result.gpu_ms.append(gms)
        result.round_seconds.append(dt)
        result.tokens_per_round.extend(n_commit)
        if on_round is not None:
            on_round(RoundInfo(step, sids, starts, res, inp, outs, dt, gms, d_outs, cu, cu_outs, cu_rows))
        keep = []
        for s, n, f in zip(running, n_commit, finished):
            s.generated += n
            s.length += n
            if f:
                s.finished = True
                result.finished += 1
            else:
                keep.append(s)
        self.running = keep
        result.rounds += 1

    def _catch_up(self, counts: List[int], pos: List[int], sids: List[int], inp: dict, result: DriverResult):
        """Decode the catch-up positions the alignment reported (``counts`` and
        first positions ``pos`` per batch row, read with the round's host
        synchronisation; their blocks and lengths are in place): per draft layer
        a one-token write and decode attention for the sequences concerned
        (spec_scheduler.py:308-319, here batched over the sequences). Per
        catch-up position one pinned upload of the rows' ids and positions, then
        only device-argument calls: no host synchronisation. Returns the
        attention outputs of the last catch-up position per layer and the batch
        rows decoded."""
        dev = self.kv.device
        rows_all = [b for b, c in enumerate(counts) if c > 0]
        outs = None
        for j in range(max(counts)):
            rows = [b for b in rows_all if counts[b] > j]
            ps = [pos[b] + j for b in rows]
            meta = torch.tensor([[sids[b] for b in rows], ps, rows], dtype=torch.int32, pin_memory=True)
            meta = meta.to(dev, non_blocking=True)
            rs_t, ps_t, idx = meta[0], meta[1], meta[2].long()
            max_ctx = max(ps) + 1
            plan = None
            outs = []
            for layer in range(self.model.draft_layers):
                q = inp["dq"][0][layer][idx]
                # the alignment allocated these positions' blocks: no allocation here
                self.draft_kv.write_block_device(layer, rs_t, ps_t, inp["dk"][0][layer][idx],
                                                 inp["dv"][0][layer][idx], alloc=False)
                if plan is None:
                    plan = VerifyPlan(self.draft_kv, rs_t, ps_t, 1, int(q.shape[2]), max_ctx)
                outs.append(verify_attention(q, self.draft_kv, layer, rs_t, ps_t, max_ctx, plan=plan))
            result.draft_forward_calls += 1
        return outs, rows_all

    # -------------------------------------------------------------- metrics
    def _record(self, result: DriverResult) -> None:
        """The reference's per-step record (spec_scheduler.py:200-205), on the device."""
        n = self._nrec
        if self._rec is None or n >= self._rec.shape[0]:
            rows = max(256, 2 * n)
            for name in ("_rec", "_drec"):
                t = torch.zeros((rows, 6), dtype=torch.int64, device=self.kv.device)
                old = getattr(self, name)
                if old is not None:
                    t[: old.shape[0]] = old
                setattr(self, name, t)
        self.kv.metrics_device(self._rec[n], self._peak)
        if self.draft_kv is not None:
            self.draft_kv.metrics_device(self._drec[n], self._dpeak)
        self._nrec += 1
        result.batch_hist.append(len(self.running))

    def _collect(self, result: DriverResult) -> None:
        n = self._nrec
        if n == 0:
            return
        rec = self._rec[:n].tolist()
        bs = self.kv.block_size
        result.block_util_hist = [r[1] / (r[0] * bs) if r[0] else 0.0 for r in rec]
        result.kv_peak_blocks = int(self._peak.item())
        if self.draft_kv is not None:
            result.draft_kv_peak_blocks = int(self._dpeak.item())

    def run(self, requests: Sequence[Request], max_steps: Optional[int] = None,
            on_round: Optional[Callable[[RoundInfo], None]] = None, sync_timing: bool = False,
            gpu_timing=False) -> DriverResult:
        """Steps until every request has finished (or ``max_steps``), in the
        reference's order (spec_scheduler.py:181-208): admit the requests due at
        step 0; then per step run a round over the running sequences, advance
        the step, admit the requests due by then, and record the metrics.

        ``sync_timing`` drains the device before each round so that
        ``round_seconds`` holds the round alone; ``gpu_timing`` True (or
        "layers") records events around every layer's append and attention and
        around the sampling (``gpu_ms`` per round, in ms; the events add their
        own gaps between the kernels), "round" only around the round. A
        callable gives the mode per step."""
        result = DriverResult(self.gamma)
        self._nrec = 0
        self._peak.zero_()
        self._dpeak.zero_()
        pending = sorted(requests, key=lambda r: (r.arrive_step, r.sid))
        step = 0
        due = [r for r in pending if r.arrive_step <= step]
        pending = [r for r in pending if r.arrive_step > step]
        waiting = self._flush_arrivals(due, result) if due else []
        while self.running or pending or waiting:
            if self.running:
                self._round(step, result, on_round, sync_timing,
                            gpu_timing(step) if callable(gpu_timing) else gpu_timing)
            step += 1
            due = waiting + [r for r in pending if r.arrive_step <= step]
            pending = [r for r in pending if r.arrive_step > step]
            waiting = self._flush_arrivals(due, result) if due else []
            self._record(result)
            if max_steps is not None and step >= max_steps:
                break
        result.steps = step
        self._collect(result)
        return result


def poisson_requests(n: int, rate: float, prompt_lo: int, prompt_hi: int, new_lo: int, new_hi: int,
                     seed: int = 0, first_sid: int = 0, log_uniform: bool = True) -> List[Request]:
    """``n`` requests with Poisson arrivals (``rate`` per step), prompt lengths
    uniform or log-uniform in ``[prompt_lo, prompt_hi]`` and budgets uniform in
    ``[new_lo, new_hi]``."""
    import math

    g = torch.Generator().manual_seed(seed)
    out, t = [], 0.0
    for i in range(n):
        t += float(torch.empty(1).exponential_(rate, generator=g)) if rate > 0 else 0.0
        u = float(torch.rand(1, generator=g))
        if log_uniform:
            L = int(math.exp(math.log(prompt_lo) + (math.log(prompt_hi) - math.log(prompt_lo)) * u))
        else:
            L = int(prompt_lo + (prompt_hi - prompt_lo) * u)
        budget = int(torch.randint(new_lo, new_hi + 1, (1,), generator=g))
        out.append(Request(first_sid + i, int(t), L, budget))
    return out
