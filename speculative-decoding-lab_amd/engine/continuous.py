"""One-GPU continuous batching of speculative verify rounds.

The round loop of the reference's speculative engine
(engine/spec_scheduler.py:166-222, ``run_spec_continuous``) applied to the
device verify path:

* requests arrive at integer steps and are admitted in arrival order when the
  batch has room and the pool can hold the request's whole lifetime (prompt,
  budget and one verify chunk) next to what the running sequences may still
  claim. The reference admits every due request and fails when the pool runs
  out; reserving lifetimes makes exhaustion impossible instead;
* every running sequence then takes one verify round: the K/V of the gamma+1
  verify tokens of every layer are appended, verify attention runs per layer,
  the round is sampled (accept / residual / bonus) and the pool is rewound on
  the device to the committed length (``VerifyStep``);
* sequences that reach their budget (or eos) leave; their blocks went back to
  the free stack in the same rewind.

The target and draft models are outside this path, so a ``SyntheticVerifyModel``
stands in for them: seeded device tensors of the shapes one round consumes
(queries, keys and values per layer, target and draft logits, proposals drawn
from the draft distribution, uniforms and ``Exp(1)`` rows). With target logits
``N(0, 2^2)`` and draft logits ``target + N(0, sigma^2)`` over a 151,936-entry
vocabulary, sigma = 1.05 accepts a proposal with probability about 0.6.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Callable, List, Optional, Sequence

import torch

from .kv import PagedKVCache
from .spec_scheduler import VerifyResult, VerifyStep


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
    tokens_per_round: List[int] = field(default_factory=list)
    kv_peak_blocks: int = 0
    admitted: int = 0
    finished: int = 0

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
    K/V come from one bank of ``prompt_cap`` token rows.
    """

    def __init__(self, num_layers: int, num_q_heads: int, num_kv_heads: int, head_dim: int, vocab: int,
                 gamma: int, max_batch: int, device: torch.device, dtype: torch.dtype = torch.bfloat16,
                 seed: int = 0, draft_sigma: float = 1.05, prompt_cap: int = 8192, n_sets: int = 2,
                 temperature: float = 1.0) -> None:
        g = torch.Generator(device=device).manual_seed(seed)
        C = gamma + 1
        self.num_layers, self.gamma, self.vocab = num_layers, gamma, vocab
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
            self.sets.append((target.contiguous(), draft.contiguous(), proposals, u, noise))
            del probs

    def prompt_kv(self, n: int):
        if n > self.bank_k.shape[1]:
            raise ValueError("prompt longer than the synthetic bank")
        return self.bank_k[:, :n], self.bank_v[:, :n]

    def round_inputs(self, round_idx: int, B: int) -> dict:
        target, draft, proposals, u, noise = self.sets[round_idx % len(self.sets)]
        return {
            "q": [x[:B] for x in self.q], "k": [x[:B] for x in self.k], "v": [x[:B] for x in self.v],
            "target": target[:B], "draft": draft[:B], "proposals": proposals[:B], "u": u[:B], "noise": noise[:B],
        }


class SpecContinuousDriver:
    """Continuous batching of verify rounds over one device pool."""

    def __init__(self, kv: PagedKVCache, model: SyntheticVerifyModel, gamma: int, max_batch: int,
                 temperature: float = 1.0, eos_id: Optional[int] = None) -> None:
        self.kv = kv
        self.model = model
        self.gamma = int(gamma)
        self.max_batch = int(max_batch)
        self.step_fn = VerifyStep(kv, gamma, temperature, eos_id)
        self.running: List[SeqState] = []

    # ------------------------------------------------------------ admission
    def _blocks_for(self, tokens: int) -> int:
        return -(-tokens // self.kv.block_size)

    def lifetime_blocks(self, prompt_len: int, max_new_tokens: int) -> int:
        """Most blocks a request can hold: while it runs the cache holds at most
        ``prompt_len + max_new_tokens - 2`` tokens and a round appends
        ``gamma + 1`` more."""
        return self._blocks_for(prompt_len + max(max_new_tokens, 1) + self.gamma - 1)

    def _flush_arrivals(self, due: List[Request], result: DriverResult) -> List[Request]:
        """Admit due requests in arrival order while the batch and the pool have
        room (first come, first served: a request that does not fit holds back
        the ones behind it); returns the ones left waiting."""
        waiting = []
        free = self.kv.allocator.num_free
        reserved = sum(s.lifetime_blocks - self._blocks_for(s.length) for s in self.running)
        for i, r in enumerate(due):
            need = self.lifetime_blocks(r.prompt_len, r.max_new_tokens)
            if need > self.kv.allocator.capacity:
                raise ValueError("request {} needs {} blocks, more than the pool's {}".format(
                    r.sid, need, self.kv.allocator.capacity))
            if len(self.running) >= self.max_batch or free - reserved < need:
                waiting.extend(due[i:])
                break
            self.kv.add_sequence(r.sid)
            k, v = self.model.prompt_kv(r.prompt_len)
            for layer in range(self.model.num_layers):  # prefill's K/V write (model.py:369-399)
                self.kv.write_block(layer, [r.sid], [0], k, v)
            free -= self._blocks_for(r.prompt_len)
            reserved += need - self._blocks_for(r.prompt_len)
            self.running.append(SeqState(r.sid, r.prompt_len, r.max_new_tokens, need))
            result.admitted += 1
        return waiting

    # ---------------------------------------------------------------- round
    def _round(self, step: int, result: DriverResult, on_round: Optional[Callable[[RoundInfo], None]],
               sync_timing: bool, gpu_timing: bool) -> None:
        running = self.running
        sids = [s.sid for s in running]
        starts = [s.length for s in running]
        remaining = [s.max_new_tokens - s.generated for s in running]
        B = len(running)
        inp = self.model.round_inputs(result.rounds, B)
        if sync_timing:
            torch.cuda.synchronize(self.kv.device)
        t0 = time.perf_counter()
        evs = [] if gpu_timing else None
        outs = self.step_fn.attend_layers(sids, starts, inp["q"], inp["k"], inp["v"], events=evs)
        res = self.step_fn.sample_and_commit(sids, starts, inp["target"], inp["draft"], inp["proposals"],
                                             inp["u"], inp["noise"], remaining)
        if gpu_timing:
            evs.append(torch.cuda.Event(enable_timing=True))
            evs[-1].record()
        n_commit = res.n_commit.tolist()  # the round's one host synchronisation
        finished = res.finished.tolist()
        dt = time.perf_counter() - t0
        gms = None
        if gpu_timing:
            torch.cuda.synchronize(self.kv.device)
            nl = len(inp["q"])
            gms = {"append": sum(evs[2 * i].elapsed_time(evs[2 * i + 1]) for i in range(nl)),
                   "attend": sum(evs[2 * i + 1].elapsed_time(evs[2 * i + 2]) for i in range(nl)),
                   "sample": evs[2 * nl].elapsed_time(evs[2 * nl + 1]),
                   "round": evs[0].elapsed_time(evs[-1])}
            result.gpu_ms.append(gms)
        result.round_seconds.append(dt)
        result.batch_hist.append(B)
        result.tokens_per_round.extend(n_commit)
        if on_round is not None:
            on_round(RoundInfo(step, sids, starts, res, inp, outs, dt, gms))
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

    def run(self, requests: Sequence[Request], max_steps: Optional[int] = None,
            on_round: Optional[Callable[[RoundInfo], None]] = None, sync_timing: bool = False,
            gpu_timing: bool = False) -> DriverResult:
        """Steps until every request has finished (or ``max_steps``).

        ``sync_timing`` drains the device before each round so that
        ``round_seconds`` holds the round alone; ``gpu_timing`` records events
        around every layer's append and attention and around the sampling
        (``gpu_ms`` per round, in ms)."""
        result = DriverResult(self.gamma)
        pending = sorted(requests, key=lambda r: (r.arrive_step, r.sid))
        step = 0
        waiting: List[Request] = []
        while True:
            due = waiting + [r for r in pending if r.arrive_step <= step]
            pending = [r for r in pending if r.arrive_step > step]
            waiting = self._flush_arrivals(due, result) if due else []
            if self.running:
                self._round(step, result, on_round, sync_timing, gpu_timing)
                used = self.kv.allocator.capacity - self.kv.allocator.num_free
                result.kv_peak_blocks = max(result.kv_peak_blocks, used)
            step += 1
            if max_steps is not None and step >= max_steps:
                break
            if not self.running and not pending and not waiting:
                break
        result.steps = step
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
