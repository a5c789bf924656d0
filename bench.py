#!/usr/bin/env python3
"""Benchmark of the paged-KV speculative verify step on one MI355X.

Workload (Qwen2.5-1.5B-shaped single-layer verify, gamma = 5): batch 32, 12 q /
2 kv heads, head_dim 128, block 16, bf16 KV; context lengths U[256, 4096]; block
tables are a random permutation of a 65,536-block pool; the rest of the pool is
the free list. One step =

  1. the commit of the replica's previous round (rewind of the pool to start +
     n_commit with the lengths that round sampled) and the append of this
     round's 6 verify tokens of every sequence (device allocation + copy), in
     one launch (``rewind_append_device``: the two calls' exact result),
  2. the round's attention plan (``VerifyPlan``: the split of the batch over
     the workgroups and their first block ids, made once per round and shared
     by the round's layers),
  3. verify attention of the 6 rows x 12 heads over the paged context,
  4. fused rejection sampling of the round over a 151,936-entry vocabulary
     (target logits N(0, 2^2), draft = target + N(0, 1), T = 1, caller noise),
     whose committed lengths the replica's next step rewinds to.

``parts_us.append_rewind`` times that one launch; ``append_rewind_separate``
the same work as the two calls (``write_block_device``, ``rewind_device``).

All inputs are resident in HBM before timing. The batch exists in 8 replicas on
disjoint random pages of the pool, each with its own draw of the context
lengths (seeds seed .. seed + 7, so the headline is not one draw's luck), and
the logits in 2 sets; consecutive steps use different replicas, so none finds
its K/V in the 256 MB last-level cache -- each call reads HBM as one layer of
a deep model would.

The timed region is exactly ``--steps`` steps, launched back to back on the
current stream behind a bounded device-side delay (so the host has queued
them all before the GPU reaches the first), with HIP events around the whole
region and around every attention call. The headline ``value`` is the
verify-attention HBM bandwidth: algorithmic bytes of the timed calls / (their
summed kernel durations + each call's share of its round's plan, the plan's
time over the 28 layers of Qwen2.5-1.5B that share it); ``roofline`` rates
the attention kernel alone. ``spec_step_us_per_seq`` is the whole step
per sequence over the same region; ``graph_ms_per_step`` is the same step as a
captured graph replay (outside the timed region). ``cpu_baseline`` times the
CPU oracle's whole step (per-token write loop, gather + repeat_interleave +
masked SDPA per sequence, batch_accept with a live generator, tail-first
truncate with the free-list scan) on the host, with all host threads and with
one.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "speculative-decoding-lab_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
METRIC = "verify-attn HBM GB/s (% of peak) + spec-step us/seq, gamma=5, 1 GPU"

B, HQ, HKV, D, BS, GAMMA, CAP, VOCAB = 32, 12, 2, 128, 16, 5, 65536, 151936
C = GAMMA + 1
# Timed calls cycle over REPLICAS copies of the batch on disjoint pages of the
# pool (~700 MB of K/V in all) and over two sets of logits, so that no call
# finds its data in the 256 MB last-level cache left by the previous one:
# every call reads HBM, as one layer of a deep model does.
REPLICAS, LOGIT_SETS = 8, 2
# Layers of Qwen2.5-1.5B: the attention calls of one verify round that share its plan.
LAYERS_PER_ROUND = 28


def attention_bytes(lens, chunk=C, hq=HQ, hkv=HKV, d=D, bs=BS):
    """Algorithmic HBM bytes of one verify-attention call (one layer, bf16):
    per sequence of context ``L`` the K and V rows of the ``L + chunk``
    attended keys, the query read and output write, the block-table entries and
    the start / id words."""
    total = 0
    for L in lens:
        n = L + chunk
        total += n * 2 * hkv * d * 2
        total += 2 * chunk * hq * d * 2
        total += 4 * math.ceil(n / bs) + 8
    return total


def sample_bytes(batch, draft_stats=True):
    """Algorithmic bytes of one fused sampling call (T > 0): per sequence the
    target rows, the noise row and the raced draft row (a rejection), the
    uniforms, proposals and the draft entries at them, and the start / outputs.
    Without the draft rows' statistics (kept by the draft sampler that drew
    the proposals) every draft row is read in full as well."""
    if not draft_stats:
        return batch * ((C + GAMMA) * VOCAB * 4 + VOCAB * 4 + GAMMA * 8 + 12)
    # target rows, noise row, raced draft row; per position u, proposal, q[x], (max, sum)
    return batch * ((C + 2) * VOCAB * 4 + GAMMA * 20 + 12)


def workload_lens(seed=0):
    """Context lengths of the batch, U[256, 4096]; the generator continues into
    the block-table permutation."""
    import torch

    g = torch.Generator().manual_seed(seed)
    return torch.randint(256, 4097, (B,), generator=g).tolist(), g


def replica_lens(seed=0):
    """Context lengths of each replica: replica r is the draw of seed + r."""
    return [workload_lens(seed + r)[0] for r in range(REPLICAS)]


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "verify_attn_qwen15_b32_traffic.md")


def attn_source_hash():
    """Identifies the verify-attention source revision a profile was taken on."""
    import hashlib

    h = hashlib.sha256()
    for f in ("verify_attn.hip", "spv_common.h"):
        with open(os.path.join(PKG, "csrc", f), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


def measured_traffic():
    """HBM bytes per verify-attention call from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (scaled by the copy-kernel factor), or None
    when the summary was taken on a different verify-attention source."""
    try:
        text = open(TRAFFIC_PROFILE).read()
        src_hash = attn_source_hash()
    except OSError:
        return None
    fields = {}
    for line in text.splitlines():
        if ":" in line:
            k, v = line.split(":", 1)
            fields[k.strip()] = v.strip().strip("`")
    if fields.get("verify-attention source hash") != src_hash:
        return None
    try:
        return int(float(fields["traffic_bytes_per_call"]))
    except (KeyError, ValueError):
        return None


def build_workload(dev, seed=0):
    import torch

    from engine.kv import PagedKVCache

    rlens = replica_lens(seed)
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(CAP, generator=g).tolist()
    tables, pos = [], 0
    for lens in rlens:
        for L in lens:
            n = -(-L // BS)
            tables.append(perm[pos: pos + n])
            pos += n
    free = perm[pos:]
    kv = PagedKVCache(1, HKV, D, CAP, BS, dev, torch.bfloat16, max_seqs=B * REPLICAS,
                      max_blocks_per_seq=-(-(4096 + C) // BS) + 1)
    kv.load_state(tables, [L for lens in rlens for L in lens], free)
    gd = torch.Generator(device=dev).manual_seed(seed)
    keys, values = [], []
    for r, lens in enumerate(rlens):
        for s, L in enumerate(lens):
            k = torch.randn(1, L, HKV, D, generator=gd, device=dev).to(torch.bfloat16)
            v = torch.randn(1, L, HKV, D, generator=gd, device=dev).to(torch.bfloat16)
            kv.write_block(0, [r * B + s], [0], k, v)
            if r == 0:
                keys.append(k[0])
                values.append(v[0])
    w = {
        "lens": rlens[0],
        "rlens": rlens,
        "tables0": tables[:B],
        "free": free,
        "kv": kv,
        "keys": keys,
        "values": values,
        "q": torch.randn(B, C, HQ, D, generator=gd, device=dev).to(torch.bfloat16),
        "k_new": torch.randn(B, C, HKV, D, generator=gd, device=dev).to(torch.bfloat16),
        "v_new": torch.randn(B, C, HKV, D, generator=gd, device=dev).to(torch.bfloat16),
        "sids": [torch.arange(r * B, (r + 1) * B, dtype=torch.int32, device=dev) for r in range(REPLICAS)],
        "start": [torch.tensor(lens, dtype=torch.int32, device=dev) for lens in rlens],
        "max_ctx": [max(lens) + C for lens in rlens],
        "logits": [],
    }
    from engine.spec_scheduler import draft_sample

    for _ in range(LOGIT_SETS):
        target = torch.randn(B, C, VOCAB, generator=gd, device=dev) * 2.0
        draft = (target[:, :GAMMA] + torch.randn(B, GAMMA, VOCAB, generator=gd, device=dev)).contiguous()
        # the draft side: each draft step draws the batch's proposals from its
        # logits and keeps the rows' softmax statistics (spec_scheduler.py:243-252)
        proposals = torch.empty(B, GAMMA, dtype=torch.int32, device=dev)
        dstats = torch.empty(B, GAMMA, 2, dtype=torch.float32, device=dev)
        for j in range(GAMMA):
            dn = torch.empty(B, VOCAB, device=dev).exponential_(1, generator=gd)
            draft_sample(draft[:, j], 1.0, dn, out=proposals[:, j], stats=dstats[:, j])
            del dn
        w["logits"].append((target.contiguous(), draft, proposals, dstats))
    w["u"] = torch.rand(B, GAMMA, generator=gd, device=dev)
    w["noise"] = torch.empty(B, VOCAB, device=dev).exponential_(1, generator=gd)
    w["attn_out"] = torch.empty_like(w["q"])
    return w


def make_step(w):
    """Closures of one verify step for replica r / logits set t: append the
    verify tokens, attention, fused sampling, rewind."""
    from engine.attention import VerifyPlan, verify_attention
    from engine.spec_scheduler import _new_result, verify_sample

    kv = w["kv"]
    # one result per replica: a rewind applies the lengths sampled against its
    # own replica's start positions
    results = [_new_result(B, GAMMA, kv.device) for _ in range(REPLICAS)]
    for res in results:  # nothing to commit before a replica's first round
        res.new_len.fill_(-1)
        res.finished.zero_()
    plans = [VerifyPlan(kv, w["sids"][r], w["start"][r], C, HQ, w["max_ctx"][r]) for r in range(REPLICAS)]

    def append(r):
        kv.write_block_device(0, w["sids"][r], w["start"][r], w["k_new"], w["v_new"])

    def plan(r):  # once the round's blocks exist (after its first append); into the replica's buffer
        plans[r] = VerifyPlan(kv, w["sids"][r], w["start"][r], C, HQ, w["max_ctx"][r], buf=plans[r].buf)

    def attend(r):
        verify_attention(w["q"], kv, 0, w["sids"][r], w["start"][r], w["max_ctx"][r], out=w["attn_out"],
                         plan=plans[r])

    def sample(t, r=0, own_stats=False):
        target, draft, proposals, dstats = w["logits"][t]
        verify_sample(target, draft, proposals, w["u"], w["noise"], 1.0,
                      start_pos=w["start"][r], result=results[r], validate=False,
                      draft_stats=None if own_stats else dstats)

    def rewind(r):
        kv.rewind_device(w["sids"][r], results[r].new_len, results[r].finished)

    def rewind_append(r):  # the replica's last commit, then this round's append: one launch
        kv.rewind_append_device(w["sids"][r], results[r].new_len, results[r].finished, w["start"][r],
                                w["k_new"], w["v_new"])

    def step(i, events=None):
        r, t = i % REPLICAS, i % LOGIT_SETS
        rewind_append(r)
        plan(r)
        if events is not None:
            events.arm()
        attend(r)
        sample(t, r)

    return step, {"append": append, "plan": plan, "attend": attend, "sample": sample, "rewind": rewind,
                  "rewind_append": rewind_append}, \
        results[0]


def graph_of(fn, reps, torch):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    torch.cuda.synchronize()
    return g


def time_graph(g, iters, torch):
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(iters):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / iters  # ms per replay


def copy_bandwidth(dev, nbytes=1 << 30):
    """GB/s of a plain device copy (read + write) of ``nbytes`` -- the box's
    achievable HBM rate, also the normaliser for the FETCH/WRITE counters."""
    import torch

    src = torch.empty(nbytes // 4, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    g = graph_of(lambda: dst.copy_(src), 5, torch)
    ms = time_graph(g, 4, torch) / 5
    return 2 * nbytes / (ms * 1e-3) / 1e9


def sleep_cycles_per_ms(torch):
    """Rate of ``torch.cuda._sleep`` (a bounded spin on the device clock), for
    the delay queued ahead of the timed region."""
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record()
    torch.cuda._sleep(2_000_000)
    b.record()
    torch.cuda.synchronize()
    return 2_000_000 / max(a.elapsed_time(b), 1e-3)


class KernelEvents:
    """A start / stop hipEvent pair for one attention call, armed through the
    library's timing hook (spv_time_next_attention): the HIP runtime records
    the kernel's own start and end timestamps into them, on the stream the
    kernel runs on -- the interval rocprofv3 reports for the kernel."""

    def __init__(self):
        import ctypes

        from engine import _hip

        self.lib = _hip.lib()  # resolves the HIP runtime already in the process
        self.lib.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.lib.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.ev = [ctypes.c_void_p(), ctypes.c_void_p()]
        for e in self.ev:
            if self.lib.hipEventCreate(ctypes.byref(e)) != 0:
                raise RuntimeError("hipEventCreate failed")

    def arm(self):
        self.lib.spv_time_next_attention(self.ev[0], self.ev[1])

    def elapsed_ms(self):
        import ctypes

        ms = ctypes.c_float()
        if self.lib.hipEventElapsedTime(ctypes.byref(ms), self.ev[0], self.ev[1]) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value

    def close(self):
        for e in self.ev:
            self.lib.hipEventDestroy(e)


def timed_steps(step, steps, torch, host_us_per_step=400.0):
    """Exactly ``steps`` steps on the current stream, queued behind a bounded
    device-side delay long enough for the host to enqueue all of them, so the
    GPU never waits on a launch. torch events bracket the region; every
    attention call's kernel records its own start / end into a HIP event pair.
    Returns (ms per step, per-call attention kernel ms list)."""
    rate = sleep_cycles_per_ms(torch)
    delay_ms = min(400.0, 5.0 + steps * host_us_per_step / 1000.0)
    ev = [KernelEvents() for _ in range(steps)]
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    torch.cuda._sleep(int(rate * delay_ms))
    start.record()
    for i in range(steps):
        step(i, ev[i])
    end.record()
    queued_ms = (time.perf_counter() - t0) * 1e3
    torch.cuda.synchronize()
    if queued_ms > delay_ms:
        print("bench: warning: the host took {:.1f} ms to queue the timed steps, more than the {:.1f} ms "
              "delay ahead of them".format(queued_ms, delay_ms), file=sys.stderr, flush=True)
    attn_ms = [e.elapsed_ms() for e in ev]
    for e in ev:
        e.close()
    return start.elapsed_time(end) / steps, attn_ms


def cpu_baseline(w, dev, budget_s=12.0):
    """The CPU oracle's whole verify step on the host, timed with all host
    threads and with one: the per-token write loop with lazy allocation from the
    LIFO free list (the workload's own, ~30k entries), the per-block gather +
    repeat_interleave + masked SDPA per sequence, logits_to_probs of every row
    and batch_accept with a live generator, and the commit's tail-first
    truncate with the free list's membership scan. Replica 0 of the workload,
    bf16 K/V and queries as on the GPU (and once with fp32 K/V on all threads).
    ``value`` is the attention part in GB/s of the same algorithmic bytes as the
    GPU headline."""
    import torch

    from oracle import attention as ref_attn
    from oracle import kv_pool as ref
    from oracle import sampler as S

    lens = w["lens"]
    target, draft, proposals, _ = (x.cpu() for x in w["logits"][0])
    props = proposals.tolist()
    sids = list(range(B))
    nbytes = attention_bytes(lens)
    gen = torch.Generator().manual_seed(1234)

    def pool(dtype):
        """The oracle's pool of replica 0 in ``dtype`` (the GPU pool's bf16 values, exact in fp32)."""
        cpu = ref.PagedKVCache(1, HKV, D, CAP, BS, dtype=dtype)
        cpu.load_state(w["tables0"], lens, w["free"])
        for s, L in enumerate(lens):
            k, v = w["keys"][s].to(dtype).cpu(), w["values"][s].to(dtype).cpu()
            for bi, phys in enumerate(w["tables0"][s]):
                n = min(BS, L - bi * BS)
                cpu.k[0, phys, :n] = k[bi * BS: bi * BS + n]
                cpu.v[0, phys, :n] = v[bi * BS: bi * BS + n]
        return cpu, w["k_new"].to(dtype).cpu(), w["v_new"].to(dtype).cpu(), w["q"].to(dtype).cpu()

    def one_step(cpu, k_new, v_new, q):
        t = [time.perf_counter()]
        cpu.write_block(0, sids, lens, k_new, v_new)
        t.append(time.perf_counter())
        ref_attn.paged_attention_extend(q, cpu, 0, sids, lens, HQ)
        t.append(time.perf_counter())
        p = S.logits_to_probs(target, 1.0)
        qd = S.logits_to_probs(draft, 1.0)
        acc = S.batch_accept({s: p[s] for s in sids}, {s: list(qd[s]) for s in sids},
                             {s: props[s] for s in sids}, gen)
        t.append(time.perf_counter())
        for s in sids:
            cpu.truncate(s, lens[s] + len(acc[s]))
        t.append(time.perf_counter())
        return [b - a for a, b in zip(t, t[1:])]

    def run(args_, threads, budget):
        torch.set_num_threads(threads)
        one_step(*args_)  # warm-up
        rows, t_end = [], time.perf_counter() + budget
        while (time.perf_counter() < t_end or len(rows) < 3) and len(rows) < 200:
            rows.append(one_step(*args_))
        med = [sorted(r[i] for r in rows)[len(rows) // 2] for i in range(4)]
        step_s = sorted(sum(r) for r in rows)[len(rows) // 2]
        return {
            "attn_gbs": round(nbytes / med[1] / 1e9, 3),
            "spec_step_us_per_seq": round(step_s * 1e6 / B, 1),
            "parts_ms": {k: round(v * 1e3, 2) for k, v in zip(("append", "attend", "sample", "rewind"), med)},
            "runs": len(rows),
        }

    threads = os.cpu_count() or 1
    bf16 = pool(torch.bfloat16)
    allc = run(bf16, threads, budget_s * 0.45)
    one = run(bf16, 1, budget_s * 0.25)
    del bf16
    f32 = run(pool(torch.float32), threads, budget_s * 0.3)
    torch.set_num_threads(threads)
    return {
        "value": allc["attn_gbs"],
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": "the oracle's whole verify step on replica 0 of the workload (32 sequences, 1 layer, bf16 K/V and "
                  "queries as on the GPU): per-token write loop, per-block gather + repeat_interleave + masked SDPA "
                  "per sequence, softmax of all 352 logits rows + batch_accept with a live generator, tail-first "
                  "truncate with the free-list scan over ~30k free blocks; medians of {} runs on {} threads and {} "
                  "runs on 1 thread (and {} runs with fp32 K/V on {} threads). value = the attention part in "
                  "GB/s of bf16 bytes".format(allc["runs"], threads, one["runs"], f32["runs"], threads),
        "spec_step_us_per_seq": allc["spec_step_us_per_seq"],
        "parts_ms": allc["parts_ms"],
        "one_thread": {"value": one["attn_gbs"], "spec_step_us_per_seq": one["spec_step_us_per_seq"],
                       "parts_ms": one["parts_ms"]},
        "fp32_kv": {"value": f32["attn_gbs"], "spec_step_us_per_seq": f32["spec_step_us_per_seq"],
                    "parts_ms": f32["parts_ms"]},
    }


# Full-depth continuous batching: Qwen2.5-3B-shaped model, gamma 6.
FD_LAYERS, FD_HQ, FD_HKV, FD_D, FD_BS, FD_GAMMA, FD_BATCH = 36, 16, 2, 128, 16, 6, 128
FD_CTX = (512, 8192)          # prompt lengths, log-uniform
FD_BUDGET = (32, 160)         # new tokens per request, uniform
FD_RATE = 4.0                 # Poisson arrivals per step once the first batch is in
FD_SIGMA = 1.05               # draft = target + N(0, sigma^2): acceptance ~0.6 per draft
FD_BREAKDOWN_ROUNDS = 3       # rounds with events around every layer's append and attention
# The draft model of the whole-round variant: Qwen2.5-0.5B-shaped layers.
DD_LAYERS, DD_HQ, DD_HKV, DD_D = 24, 14, 2, 64


def fp16_verify(dev, seed=0, dtype=None):
    """The headline verify attention over an fp16 pool with fp16 queries (the
    reference's GPU dtype): the same replicas, context lengths and page
    scatter, each sequence's keys written through position L + chunk, planned
    calls cycling over the replicas as one captured graph. ``dtype``: the
    pool's and the queries' type (fp16 unless given)."""
    import torch

    from engine.attention import VerifyPlan, verify_attention
    from engine.kv import PagedKVCache

    rlens = replica_lens(seed)
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(CAP, generator=g).tolist()
    tables, pos = [], 0
    for lens in rlens:
        for L in lens:
            n = -(-(L + C) // BS)
            tables.append(perm[pos: pos + n])
            pos += n
    dtype = dtype or torch.float16
    kv = PagedKVCache(1, HKV, D, CAP, BS, dev, dtype, max_seqs=B * REPLICAS,
                      max_blocks_per_seq=-(-(4096 + C) // BS) + 1)
    kv.load_state(tables, [0] * len(tables), perm[pos:])
    gd = torch.Generator(device=dev).manual_seed(seed + 1000)
    for r, lens in enumerate(rlens):
        for s, L in enumerate(lens):
            k = torch.randn(1, L + C, HKV, D, generator=gd, device=dev).to(dtype)
            v = torch.randn(1, L + C, HKV, D, generator=gd, device=dev).to(dtype)
            kv.write_block(0, [r * B + s], [0], k, v)
    q = torch.randn(B, C, HQ, D, generator=gd, device=dev).to(dtype)
    out = torch.empty_like(q)
    sids = [torch.arange(r * B, (r + 1) * B, dtype=torch.int32, device=dev) for r in range(REPLICAS)]
    starts = [torch.tensor(lens, dtype=torch.int32, device=dev) for lens in rlens]
    max_ctx = [max(lens) + C for lens in rlens]
    plans = [VerifyPlan(kv, sids[r], starts[r], C, HQ, max_ctx[r]) for r in range(REPLICAS)]

    def call(r):
        verify_attention(q, kv, 0, sids[r], starts[r], max_ctx[r], out=out, plan=plans[r])

    for r in range(REPLICAS):
        call(r)
    torch.cuda.synchronize()
    reps = 3 * REPLICAS
    ga = graph_of(lambda: [call(i % REPLICAS) for i in range(reps)], 1, torch)
    us = time_graph(ga, 5, torch) * 1000.0 / reps
    nbytes = sum(attention_bytes(rlens[i % REPLICAS]) for i in range(reps)) / reps
    del ga, kv
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return {"workload": "the verify attention above over an fp16 pool with fp16 queries (planned calls, "
                        "captured graph)",
            "attn_us": round(us, 2), "attn_gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
            "attn_bytes_per_call": round(nbytes)}


def pool_partition_ok(kv, cap):
    """The pool invariant after a run: the free list and the block tables
    together hold every block of the pool exactly once."""
    owned = [blk for tab in kv.block_tables for blk in tab]
    free = kv.allocator.free_list()
    return len(owned) + len(free) == cap and sorted(owned + free) == list(range(cap))


def full_depth(dev, rounds, warmup, seed=0, pool_frac=0.75, draft=False):
    """Continuous batching at full depth on one GPU.

    A pool sized to most of the device's free HBM (its free list shuffled, as
    after a long run), 128 requests at step 0 and a Poisson stream behind them
    keep the batch at its cap of 128 sequences; every round appends the 7 verify
    tokens in each of 36 layers, runs 36 verify attentions, the fused sampling
    and the rewind (``engine.continuous``). Rounds are timed on the host
    (device drained before each, one synchronisation at its end) and on the
    device with events around the round only; FD_BREAKDOWN_ROUNDS further
    rounds record events around every layer's append and attention for the
    per-layer figures (those events add their own gaps between the kernels:
    about 330 us per round of 36 layers, so they are kept out of the round
    times). With ``draft`` the rounds are whole speculative rounds: a
    Qwen2.5-0.5B-shaped draft model's pool beside the target's (24 layers,
    14q/2kv heads, head_dim 64), gamma draft steps per round (per draft layer
    the token's append and decode attention, then the batch's draws, which
    keep the draft rows' statistics for the verify decisions), the verify
    layers, sampling and commit, and the draft cache's alignment. At the end
    the pools must be partitioned by their free lists and tables.
    """
    import statistics

    import torch

    from engine.continuous import SpecContinuousDriver, SyntheticVerifyModel, poisson_requests
    from engine.kv import PagedKVCache, WritePlan
    from engine.scheduler import blocks_for_hbm, bytes_per_block

    chunk = FD_GAMMA + 1
    model = SyntheticVerifyModel(FD_LAYERS, FD_HQ, FD_HKV, FD_D, VOCAB, FD_GAMMA, FD_BATCH, dev,
                                 torch.bfloat16, seed=seed, draft_sigma=FD_SIGMA, prompt_cap=FD_CTX[1],
                                 draft_layers=DD_LAYERS if draft else 0, draft_heads=(DD_HQ, DD_HKV, DD_D))
    # The pool: pool_frac of the free HBM, in blocks of all 36 layers' K and V
    # (engine.scheduler's sizing of the reference's build_kv); with the draft
    # model, its pool takes a share in proportion to its bytes per block.
    block_bytes = bytes_per_block(FD_LAYERS, FD_BS, FD_HKV, FD_D, torch.bfloat16)
    dblock_bytes = bytes_per_block(DD_LAYERS, FD_BS, DD_HKV, DD_D, torch.bfloat16)
    _free, total = torch.cuda.mem_get_info(dev)
    tshare = block_bytes / (block_bytes + dblock_bytes) if draft else 1.0
    cap = blocks_for_hbm(FD_LAYERS, FD_BS, FD_HKV, FD_D, torch.bfloat16, dev, reserve_bytes=0,
                         fraction=pool_frac * tshare)
    maxb = -(-(FD_CTX[1] + FD_BUDGET[1] + chunk) // FD_BS) + 1
    n_req = FD_BATCH + int(FD_RATE * (rounds + warmup + FD_BREAKDOWN_ROUNDS)) + 16
    kv = PagedKVCache(FD_LAYERS, FD_HKV, FD_D, cap, FD_BS, dev, torch.bfloat16, max_seqs=n_req,
                      max_blocks_per_seq=maxb)
    g = torch.Generator().manual_seed(seed + 1)
    kv.allocator.load_free_list(torch.randperm(cap, generator=g).to(torch.int32))
    dkv, dcap = None, 0
    if draft:
        dcap = blocks_for_hbm(DD_LAYERS, FD_BS, DD_HKV, DD_D, torch.bfloat16, dev, reserve_bytes=0,
                              fraction=pool_frac * (1.0 - tshare) / (1.0 - pool_frac * tshare))
        dkv = PagedKVCache(DD_LAYERS, DD_HKV, DD_D, dcap, FD_BS, dev, torch.bfloat16, max_seqs=n_req,
                           max_blocks_per_seq=maxb + 1)
        dkv.allocator.load_free_list(torch.randperm(dcap, generator=g).to(torch.int32))
    first = poisson_requests(FD_BATCH, 0.0, FD_CTX[0], FD_CTX[1], *FD_BUDGET, seed=seed + 2)
    stream = poisson_requests(n_req - FD_BATCH, FD_RATE, FD_CTX[0], FD_CTX[1], *FD_BUDGET, seed=seed + 3,
                              first_sid=FD_BATCH)
    drv = SpecContinuousDriver(kv, model, FD_GAMMA, FD_BATCH, temperature=1.0, draft_kv=dkv)
    per_round = []

    def on_round(info):
        n = len(info.sids)
        per_round.append({"batch": n, "host_s": info.seconds, "gpu": info.gpu_ms,
                          "attn_bytes": attention_bytes(info.starts, chunk, FD_HQ, FD_HKV, FD_D, FD_BS),
                          "ctx": sum(info.starts) / n, "k": info.result.n_commit.tolist()})

    res = drv.run(first + stream, max_steps=rounds + warmup + FD_BREAKDOWN_ROUNDS, on_round=on_round,
                  sync_timing=True, gpu_timing=lambda step: "round" if step < warmup + rounds else "layers")
    torch.cuda.synchronize()
    # the pools after the run: every block exactly once, in a table or free
    if not pool_partition_ok(kv, cap) or (dkv is not None and not pool_partition_ok(dkv, dcap)):
        raise AssertionError("full depth: a pool is not partitioned by its free list and tables")
    timed = per_round[warmup:warmup + rounds]
    brk = per_round[warmup + rounds:]
    med = statistics.median
    host_us = med(r["host_s"] for r in timed) * 1e6
    gpu_us = med(r["gpu"]["round"] for r in timed) * 1e3
    attend_ms = sum(r["gpu"]["attend"] for r in brk)
    attn_gbs = sum(r["attn_bytes"] for r in brk) * FD_LAYERS / (attend_ms * 1e-3) / 1e9
    ks = [k for r in timed for k in r["k"]]
    batch = sum(r["batch"] for r in timed) / len(timed)
    # A later layer's append alone: the write plan recorded by a first layer's
    # append of the running sequences' next chunk, then the 35 later layers'
    # planned copies replayed as a graph (no event between them).
    sid_t = torch.tensor([q.sid for q in drv.running], dtype=torch.int32, device=dev)
    st_t = torch.tensor([q.length for q in drv.running], dtype=torch.int32, device=dev)
    kn = torch.randn(len(drv.running), chunk, FD_HKV, FD_D, device=dev).to(torch.bfloat16)
    wplan = WritePlan()
    kv.write_block_device(0, sid_t, st_t, kn, kn, alloc=True, plan=wplan)
    gw = graph_of(lambda: [kv.write_block_device(layer, sid_t, st_t, kn, kn, alloc=False, plan=wplan)
                           for layer in range(1, FD_LAYERS)], 1, torch)
    planned_us = time_graph(gw, 5, torch) * 1e3 / (FD_LAYERS - 1)
    out = {
        "workload": "Qwen2.5-3B-shaped continuous batching: {} layers, {}q/{}kv heads, head_dim {}, "
                    "block {}, bf16 KV, gamma {}, batch cap {}, prompts log-U[{},{}], budgets U[{},{}], "
                    "Poisson arrivals {}/step, draft = target + N(0,{}^2) over V={}, T=1; pool of {} blocks "
                    "({:.1f} GB of {:.1f} GB HBM) with a shuffled free list".format(
                        FD_LAYERS, FD_HQ, FD_HKV, FD_D, FD_BS, FD_GAMMA, FD_BATCH, FD_CTX[0], FD_CTX[1],
                        FD_BUDGET[0], FD_BUDGET[1], FD_RATE, FD_SIGMA, VOCAB, cap, cap * block_bytes / 1e9,
                        total / 1e9),
        "rounds": len(timed),
        "mean_batch": round(batch, 1),
        "mean_ctx": round(sum(r["ctx"] for r in timed) / len(timed), 1),
        "us_per_round": round(host_us, 1),
        "us_per_seq": round(host_us / batch, 3),
        "gpu_us_per_round": round(gpu_us, 1),
        "gpu_us_per_seq": round(gpu_us / batch, 3),
        "breakdown_rounds": len(brk),
        "attend_us_per_layer": round(med(r["gpu"]["attend"] for r in brk) * 1e3 / FD_LAYERS, 2),
        "append_us_per_layer": round(med(r["gpu"]["append"] for r in brk) * 1e3 / FD_LAYERS, 2),
        "sample_rewind_us": round(med(r["gpu"]["sample"] for r in brk) * 1e3, 1),
        "append_planned_us": round(planned_us, 2),
        "attn_gbs": round(attn_gbs, 1),
        "mean_commit_per_seq_round": round(sum(ks) / len(ks), 3),
        "mean_acceptance": round(sum(ks) / len(ks) / chunk, 4),
        "admitted": res.admitted,
        "finished": res.finished,
        "pool_blocks": cap,
        "peak_blocks": res.kv_peak_blocks,
        "pool_partitioned": True,
    }
    if draft:
        out["workload"] += "; with the draft side: a Qwen2.5-0.5B-shaped draft model ({} layers, {}q/{}kv heads, " \
            "head_dim {}) over its own pool of {} blocks: gamma draft steps, verify, commit and the draft " \
            "cache's alignment per round".format(DD_LAYERS, DD_HQ, DD_HKV, DD_D, dcap)
        out["draft_pool_blocks"] = dcap
        out["draft_peak_blocks"] = res.draft_kv_peak_blocks
        out["draft_forward_calls_per_round"] = round(res.draft_forward_calls / max(res.rounds, 1), 2)
        out["flagged_draws"] = res.flagged_draws
    out["flagged_rounds"] = res.flagged_rounds
    del kv, dkv, model, drv
    torch.cuda.empty_cache()
    return out


# Long context: Qwen2.5-0.5B-shaped heads, fp8 (e4m3) KV with per-block scales.
LC_B, LC_HQ, LC_HKV, LC_D, LC_GAMMA, LC_CTX, LC_REPLICAS = 16, 14, 2, 64, 8, 32768, 4


def long_context(dev, seed=0):
    """Verify attention over 32768-token contexts (16 sequences, 14q/2kv heads,
    head_dim 64, gamma 8 -> 9 rows) on an fp8 pool and on a bf16 pool of the
    same contexts, and the fp8 append of the 9 verify tokens. Four layers of
    K/V (N(0,1), quantised by the fp8 append) serve as replicas that the timed
    calls cycle over, so no call finds its pages in the last-level cache."""
    import torch

    from engine.attention import VerifyPlan, verify_attention
    from engine.kv import PagedKVCache

    chunk = LC_GAMMA + 1
    lens = [LC_CTX] * LC_B
    blocks = LC_B * (-(-(LC_CTX + chunk) // BS))
    g = torch.Generator(device=dev).manual_seed(seed)
    out = {"workload": "Qwen2.5-0.5B-shaped long-context verify: batch {}, ctx {}, gamma {} ({} rows), "
                       "{}q/{}kv heads, head_dim {}, block {}; fp8 e4m3 KV with one fp32 scale per (layer, "
                       "block, K|V), and the same contexts in bf16; calls cycle over {} layers".format(
                           LC_B, LC_CTX, LC_GAMMA, chunk, LC_HQ, LC_HKV, LC_D, BS, LC_REPLICAS)}
    q = torch.randn(LC_B, chunk, LC_HQ, LC_D, generator=g, device=dev).to(torch.bfloat16)
    kn = torch.randn(LC_B, chunk, LC_HKV, LC_D, generator=g, device=dev).to(torch.bfloat16)
    vn = torch.randn(LC_B, chunk, LC_HKV, LC_D, generator=g, device=dev).to(torch.bfloat16)
    sid = torch.arange(LC_B, dtype=torch.int32, device=dev)
    st = torch.tensor(lens, dtype=torch.int32, device=dev)
    reps = 3 * LC_REPLICAS
    for name, dtype in (("fp8", torch.float8_e4m3fn), ("bf16", torch.bfloat16)):
        kv = PagedKVCache(LC_REPLICAS, LC_HKV, LC_D, blocks + LC_B, BS, dev, dtype, max_seqs=LC_B,
                          max_blocks_per_seq=-(-(LC_CTX + chunk) // BS) + 1)
        for s in range(LC_B):
            kv.add_sequence(s)
        for layer in range(LC_REPLICAS):
            for s in range(LC_B):
                k = torch.randn(1, LC_CTX, LC_HKV, LC_D, generator=g, device=dev).to(torch.bfloat16)
                v = torch.randn(1, LC_CTX, LC_HKV, LC_D, generator=g, device=dev).to(torch.bfloat16)
                kv.write_block(layer, [s], [0], k, v)
        for layer in range(LC_REPLICAS):  # the verify chunk, written before it is attended
            kv.write_block(layer, list(range(LC_B)), lens, kn, vn)
        o = torch.empty_like(q)
        # every layer of the round reads the same tables: one plan serves all calls
        pl = VerifyPlan(kv, sid, st, chunk, LC_HQ, LC_CTX + chunk)
        attend = lambda i: verify_attention(q, kv, i % LC_REPLICAS, sid, st, LC_CTX + chunk, out=o, plan=pl)
        for i in range(LC_REPLICAS):
            attend(i)
        torch.cuda.synchronize()
        gr = graph_of(lambda: [attend(i) for i in range(reps)], 1, torch)
        us = time_graph(gr, 5, torch) * 1000.0 / reps
        kv_bytes = 1 if name == "fp8" else 2
        nbytes = sum((L + chunk) * 2 * LC_HKV * LC_D * kv_bytes + 2 * chunk * LC_HQ * LC_D * 2
                     + (4 + (8 if name == "fp8" else 0)) * math.ceil((L + chunk) / BS) + 8 for L in lens)
        out[name + "_attn_us"] = round(us, 2)
        out[name + "_attn_gbs"] = round(nbytes / (us * 1e-6) / 1e9, 1)
        out[name + "_attn_bytes_per_call"] = nbytes
        if name == "fp8":
            # append of the verify chunk into the fp8 pool (blocks exist: quantise only)
            ap = lambda i: kv.write_block_device(i % LC_REPLICAS, sid, st, kn, vn, alloc=False)
            ga = graph_of(lambda: [ap(i) for i in range(reps)], 1, torch)
            out["fp8_append_us"] = round(time_graph(ga, 5, torch) * 1000.0 / reps, 2)
        del kv, gr
        torch.cuda.empty_cache()
    return out


def draft_decode(dev, seed=0):
    """One draft decode step's paged work per layer at a Qwen2.5-0.5B-shaped
    draft (14q/2kv heads, head_dim 64, bf16): append the one new token of
    each sequence, then decode attention (one query row) over its context.
    Batch 32 with the verify workload's context lengths; calls cycle over 8
    replicas on disjoint pages."""
    import torch

    from engine.attention import VerifyPlan, verify_attention
    from engine.kv import PagedKVCache, WritePlan

    hq, hkv, d, reps = 14, 2, 64, 8
    lens, g = workload_lens(seed)
    need = [-(-(L + 1) // BS) for L in lens]
    cap = sum(need) * reps + 64
    kv = PagedKVCache(1, hkv, d, cap, BS, dev, torch.bfloat16, max_seqs=B * reps,
                      max_blocks_per_seq=max(need) + 1)
    ids = torch.randperm(cap, generator=g).tolist()
    tables, pos = [], 0
    for _ in range(reps):
        for n, L in zip(need, lens):
            tables.append(ids[pos: pos + -(-L // BS)])
            pos += n
    free = ids[pos:]
    kv.load_state(tables, lens * reps, free)
    kv.k_pool.normal_()
    kv.v_pool.normal_()
    gd = torch.Generator(device=dev).manual_seed(seed + 5)
    q = torch.randn(B, 1, hq, d, generator=gd, device=dev).to(torch.bfloat16)
    kn = torch.randn(B, 1, hkv, d, generator=gd, device=dev).to(torch.bfloat16)
    vn = torch.randn(B, 1, hkv, d, generator=gd, device=dev).to(torch.bfloat16)
    sids = [torch.arange(r * B, (r + 1) * B, dtype=torch.int32, device=dev) for r in range(reps)]
    st = torch.tensor(lens, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    max_ctx = max(lens) + 1
    for r in range(reps):  # the new token's blocks exist from here on
        kv.write_block_device(0, sids[r], st, kn, vn)
    # one plan per replica (a draft step's layers share their step's plan)
    plans = [VerifyPlan(kv, sids[r], st, 1, hq, max_ctx) for r in range(reps)]
    attend = lambda i: verify_attention(q, kv, 0, sids[i % reps], st, max_ctx, out=out, plan=plans[i % reps])
    append = lambda i: kv.write_block_device(0, sids[i % reps], st, kn, vn, alloc=False)
    # each replica's write plan (its blocks exist: the allocating append only records it)
    wplans = [WritePlan() for _ in range(reps)]
    for r in range(reps):
        kv.write_block_device(0, sids[r], st, kn, vn, alloc=True, plan=wplans[r])
    append_planned = lambda i: kv.write_block_device(0, sids[i % reps], st, kn, vn, alloc=False,
                                                     plan=wplans[i % reps])
    n = 3 * reps
    for i in range(reps):
        attend(i)
    torch.cuda.synchronize()
    ga = graph_of(lambda: [attend(i) for i in range(n)], 1, torch)
    attn_us = time_graph(ga, 5, torch) * 1000.0 / n
    gw = graph_of(lambda: [append(i) for i in range(n)], 1, torch)
    app_us = time_graph(gw, 5, torch) * 1000.0 / n
    gwp = graph_of(lambda: [append_planned(i) for i in range(n)], 1, torch)
    app_planned_us = time_graph(gwp, 5, torch) * 1000.0 / n
    nbytes = attention_bytes(lens, 1, hq, hkv, d, BS)
    # Batched draft sampling of one step (B rows of V draft logits, T = 1) and
    # one whole draft step at the draft model's depth as a captured graph:
    # per layer the one-token append and decode attention (layers cycle over
    # the replicas' pages, so each reads HBM), then the step's sampling.
    from engine.spec_scheduler import draft_sample

    logits = [torch.randn(B, VOCAB, generator=gd, device=dev) * 2.0 for _ in range(2)]
    noise = [torch.empty(B, VOCAB, device=dev).exponential_(1, generator=gd) for _ in range(2)]
    toks = torch.empty(B, dtype=torch.int32, device=dev)
    samp = lambda i: draft_sample(logits[i % 2], 1.0, noise[i % 2], out=toks)
    gs = graph_of(lambda: [samp(i) for i in range(n)], 1, torch)
    samp_us = time_graph(gs, 5, torch) * 1000.0 / n
    depth = 24

    def draft_step(i):
        for layer in range(depth):
            r = (i * depth + layer) % reps
            # the first layer's append allocates (and records the step's write
            # plan); the later layers copy by the plan, as DraftLoop does
            kv.write_block_device(0, sids[r], st, kn, vn, alloc=layer == 0, plan=wplans[r])
            if layer == 0:  # the step's plan, made once its blocks exist
                plans[r] = VerifyPlan(kv, sids[r], st, 1, hq, max_ctx, buf=plans[r].buf)
            verify_attention(q, kv, 0, sids[r], st, max_ctx, out=out, plan=plans[r])
        samp(i)

    gstep = graph_of(lambda: [draft_step(i) for i in range(2)], 1, torch)
    step_us = time_graph(gstep, 5, torch) * 1000.0 / 2
    res = {"workload": "Qwen2.5-0.5B-shaped draft decode: batch 32, one query row, 14q/2kv heads, head_dim 64, "
                       "block 16, bf16 KV, the verify workload's contexts (U[256,4096], seed 0); 8 replicas; "
                       "draft sampling of 32 rows over V=151936 at T=1; a draft step = the step's attention plan, 24 layers "
                       "of append + decode attention, then the sampling, as one captured graph",
           "attn_us": round(attn_us, 2), "attn_gbs": round(nbytes / (attn_us * 1e-6) / 1e9, 1),
           "attn_bytes_per_call": nbytes, "append_us": round(app_us, 2),
           "append_planned_us": round(app_planned_us, 2),
           "sample_us": round(samp_us, 2),
           "sample_gbs": round(2 * B * VOCAB * 4 / (samp_us * 1e-6) / 1e9, 1),
           "step_24_layers_us": round(step_us, 1)}
    del kv, ga, gw, gs, gstep
    torch.cuda.empty_cache()
    return res


# Prefill: Qwen2.5-3B-shaped prompts (16 q / 2 kv heads, head_dim 128, bf16).
PF_B, PF_HQ, PF_HKV, PF_D = 4, 16, 2, 128
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16


def prefill_flops(lengths, hq=PF_HQ, d=PF_D):
    """Algorithmic FLOPs of causal prefill: per row of L positions, query i
    meets i + 1 keys in q.k and in p.v (2 flops per multiply-add)."""
    return sum(hq * 4 * d * L * (L + 1) // 2 for L in lengths)


def prefill(dev, seed=0):
    """Causal chunk prefill attention at the Qwen2.5-3B shape: 4 prompts with
    lengths log-uniform in [512, 8192] (seeded) in one padded chunk, timed as
    a captured graph of back-to-back calls; TFLOP/s of the algorithmic causal
    FLOPs against MI355X's dense bf16 peak."""
    import torch

    from engine.attention import prefill_attention

    g = torch.Generator().manual_seed(seed + 17)
    lengths = [int(math.exp(math.log(512) + (math.log(8192) - math.log(512)) * float(u)))
               for u in torch.rand(PF_B, generator=g)]
    Lc = max(lengths)
    gd = torch.Generator(device=dev).manual_seed(seed + 17)
    q = torch.randn(PF_B, Lc, PF_HQ, PF_D, generator=gd, device=dev).to(torch.bfloat16)
    k = torch.randn(PF_B, Lc, PF_HKV, PF_D, generator=gd, device=dev).to(torch.bfloat16)
    v = torch.randn(PF_B, Lc, PF_HKV, PF_D, generator=gd, device=dev).to(torch.bfloat16)
    lens = torch.tensor(lengths, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    call = lambda: prefill_attention(q, k, v, lens, out=out)
    call()
    torch.cuda.synchronize()
    n = 4
    gr = graph_of(lambda: [call() for _ in range(n)], 1, torch)
    us = time_graph(gr, 5, torch) * 1000.0 / n
    flops = prefill_flops(lengths)
    tf = flops / (us * 1e-6) / 1e12
    del gr, q, k, v, out
    torch.cuda.empty_cache()
    return {"workload": "Qwen2.5-3B-shaped causal prefill chunk: {} prompts of {} tokens in one chunk of {}, "
                        "16q/2kv heads, head_dim 128, bf16".format(PF_B, lengths, Lc),
            "us": round(us, 1), "tflops": round(tf, 1), "flops_per_call": flops,
            "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": MFMA_BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4)},
            "us_per_token": round(us / sum(lengths), 4)}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--full-depth-rounds", type=int, default=24,
                    help="rounds of the 36-layer continuous-batching measurement (0 skips it)")
    ap.add_argument("--no-long-context", action="store_true",
                    help="skip the side measurements: fp16 verify attention, draft decode, prefill and the 32768-token fp8 / bf16 verify attention")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: the library has no multi-GPU path "
              "(--gpus {} requested)".format(args.gpus), file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    print("bench: building workload", file=sys.stderr, flush=True)
    w = build_workload(dev, args.seed)
    step, parts, res = make_step(w)
    for i in range(max(1, args.warmup) * REPLICAS):
        step(i)
    torch.cuda.synchronize()
    print("bench: warm-up done, timing {} steps".format(args.steps), file=sys.stderr, flush=True)

    # Timed region: exactly --steps steps, events around each attention call.
    ms_per_step, attn_ms = timed_steps(step, args.steps, torch)
    rl = w["rlens"]
    attn_bytes_timed = sum(attention_bytes(rl[i % REPLICAS]) for i in range(args.steps))
    attn_us = 1000.0 * sum(attn_ms) / len(attn_ms)
    kernel_gbs = attn_bytes_timed / (sum(attn_ms) * 1e-3) / 1e9

    # Outside the timed region: the step as a captured graph (one replay runs
    # REPLICAS steps), and per-part graphs of back-to-back calls cycling over
    # the replicas / logits sets.
    g_step = graph_of(lambda: [step(i) for i in range(REPLICAS)], 1, torch)
    for _ in range(2):
        g_step.replay()
    graph_ms_per_step = time_graph(g_step, 4, torch) / REPLICAS
    reps = 3 * REPLICAS
    part_us = {}
    g_att = graph_of(lambda: [parts["attend"](i % REPLICAS) for i in range(reps)], 1, torch)
    part_us["attend"] = time_graph(g_att, 5, torch) * 1000.0 / reps
    g_plan = graph_of(lambda: [parts["plan"](i % REPLICAS) for i in range(reps)], 1, torch)
    part_us["plan"] = time_graph(g_plan, 5, torch) * 1000.0 / reps
    del g_plan
    g_smp = graph_of(lambda: [parts["sample"](i % LOGIT_SETS, i % REPLICAS) for i in range(reps)], 1, torch)
    part_us["sample"] = time_graph(g_smp, 5, torch) * 1000.0 / reps
    g_own = graph_of(lambda: [parts["sample"](i % LOGIT_SETS, i % REPLICAS, True) for i in range(reps)], 1, torch)
    part_us["sample_own_draft_stats"] = time_graph(g_own, 5, torch) * 1000.0 / reps
    del g_own
    g_ra = graph_of(lambda: [parts["rewind_append"](i % REPLICAS) for i in range(reps)], 1, torch)
    part_us["append_rewind"] = time_graph(g_ra, 5, torch) * 1000.0 / reps
    del g_ra
    g_ar = graph_of(lambda: [(parts["append"](i % REPLICAS), parts["rewind"](i % REPLICAS)) for i in range(reps)],
                    1, torch)
    part_us["append_rewind_separate"] = time_graph(g_ar, 5, torch) * 1000.0 / reps
    del g_ar
    # the same sampling with top-k / top-p filtering of both sides' logits
    from engine.spec_scheduler import _new_result, verify_sample

    fres = _new_result(B, GAMMA, dev)
    for name, tk, tp in (("sample_top_k50", 50, 1.0), ("sample_top_p0.9", 0, 0.9)):
        def filtered(i, tk=tk, tp=tp):
            target, draft, proposals, _ = w["logits"][i % LOGIT_SETS]
            verify_sample(target, draft, proposals, w["u"], w["noise"], 1.0, start_pos=w["start"][0], result=fres,
                          validate=False, top_k=tk, top_p=tp)
        g_f = graph_of(lambda: [filtered(i) for i in range(4)], 1, torch)
        part_us[name] = time_graph(g_f, 3, torch) * 1000.0 / 4
        del g_f
    torch.cuda.synchronize()
    print("bench: timings done", file=sys.stderr, flush=True)

    # each call's share of its round's plan (LAYERS_PER_ROUND calls share one)
    plan_share_us = part_us["plan"] / LAYERS_PER_ROUND
    attn_gbs = attn_bytes_timed / ((sum(attn_ms) + args.steps * plan_share_us * 1e-3) * 1e-3) / 1e9
    copy_gbs = copy_bandwidth(dev)
    lens = w["lens"]
    all_lens = [L for r in rl for L in r]
    samp_gbs = sample_bytes(B) / (part_us["sample"] * 1e-6) / 1e9
    samp_own_gbs = sample_bytes(B, False) / (part_us["sample_own_draft_stats"] * 1e-6) / 1e9
    accept = res.accept_len.float().mean().item()

    line = {
        "metric": METRIC,
        "value": round(attn_gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "Qwen2.5-1.5B-shaped paged verify step: batch 32, gamma 5 (6 rows), "
                        "12q/2kv heads, head_dim 128, block 16, ctx U[256,4096], 65536-block pool, "
                        "1 layer; fused sampling over V=151936 fp32 at T=1; 8 replicas of the batch on "
                        "disjoint pages, each its own context draw (seeds {}..{}), cycled so no call "
                        "reuses the last-level cache".format(args.seed, args.seed + REPLICAS - 1),
            "global_batch": B,
            "seq_len": int(sum(all_lens) / len(all_lens)),
            "parallelism": "single-gpu",
        },
        "pct_of_peak": round(100.0 * attn_gbs / HBM_PEAK_GBS, 2),
        "copy_gbs": round(copy_gbs, 1),
        "attn_us": round(attn_us, 2),
        "plan_us": round(part_us["plan"], 2),
        "layers_per_round": LAYERS_PER_ROUND,
        "attn_us_with_plan_share": round(attn_us + plan_share_us, 2),
        "attn_kernel_gbs": round(kernel_gbs, 1),
        "attn_bytes_per_call": round(attn_bytes_timed / args.steps),
        "spec_step_us_per_seq": round(ms_per_step * 1000.0 / B, 3),
        "graph_ms_per_step": round(graph_ms_per_step, 4),
        "graph_spec_step_us_per_seq": round(graph_ms_per_step * 1000.0 / B, 3),
        "parts_us": {k: round(v, 2) for k, v in part_us.items()},
        "sample_gbs": round(samp_gbs, 1),
        "sample_bytes": sample_bytes(B),
        "sample_own_draft_stats_gbs": round(samp_own_gbs, 1),
        "mean_ctx": round(sum(all_lens) / len(all_lens), 1),
        "mean_accepted_drafts": round(accept, 3),
        "roofline": {
            "bound": "hbm",
            "achieved": round(kernel_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(kernel_gbs / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(),
        },
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        print("bench: cpu baseline", file=sys.stderr, flush=True)
        line["cpu_baseline"] = cpu_baseline(w, dev)
    if not args.no_long_context:
        print("bench: fp16 verify attention", file=sys.stderr, flush=True)
        line["fp16_verify"] = fp16_verify(dev, args.seed)
        print("bench: draft decode", file=sys.stderr, flush=True)
        line["draft_decode"] = draft_decode(dev, args.seed)
        print("bench: prefill", file=sys.stderr, flush=True)
        line["prefill"] = prefill(dev, args.seed)
    if args.full_depth_rounds > 0:
        del g_step, g_att, g_smp, step, parts, res, w
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        print("bench: full-depth continuous batching", file=sys.stderr, flush=True)
        line["full_depth"] = full_depth(dev, args.full_depth_rounds, 4, args.seed)
        print("bench: full-depth continuous batching with the draft side", file=sys.stderr, flush=True)
        line["full_depth_draft"] = full_depth(dev, args.full_depth_rounds, 4, args.seed, draft=True)
    if not args.no_long_context:
        if args.full_depth_rounds <= 0:
            del g_step, g_att, g_smp, step, parts, res, w
            torch.cuda.synchronize()
            torch.cuda.empty_cache()
        print("bench: long-context fp8 / bf16 attention", file=sys.stderr, flush=True)
        line["long_context"] = long_context(dev, args.seed)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
