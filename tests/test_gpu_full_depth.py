"""Continuous batching at the full Qwen2.5-3B shape, replayed by the oracle.

36 layers, 16 q / 2 kv heads, head_dim 128, block 16, bf16 K/V, gamma 6,
batch cap 128 with prompts log-uniform in [512, 8192] (the first 128 requests
at step 0, a Poisson stream behind them), V = 151,936 at T = 1, over a pool
sized by ``engine.scheduler.blocks_for_hbm`` to 3/4 of the free HBM (about
230 GB on an MI355X) whose free list is shuffled, as after a long run.

After each of four rounds the oracle replays it: admissions (the prompt's
allocation, layer 0: only the first layer allocates), the verify chunk's
allocation, and the commit (engine/spec_scheduler.py:269-322) with the
device's accepted lists, which must equal the oracle's ``verify_from_logits``
on the same logits and randomness for every unflagged sequence. Block tables,
lengths and the free list (bottom to top) must be identical to the oracle's
(``oracle.kv_pool.PagedKVCache(store=False)``, metadata only), and the pool
must be partitioned by the free list and the tables. One layer per round
(0, 17, 35, 8) is checked: its stored chunk rows bit for bit against the
round's K/V inputs, and its attention output against
``oracle.attention.extend_attention_dense`` over the K/V gathered from the
pool, in fp32 at the bf16 bar (per sequence relative L2 <= 2e-3, every
element within one bf16 ulp plus 2e-3 max |ref|).
"""

from __future__ import annotations

import pytest
import torch

from engine.attention import gather_ctx
from engine.continuous import SpecContinuousDriver, SyntheticVerifyModel, poisson_requests
from engine.kv import PagedKVCache
from engine.scheduler import blocks_for_hbm
from oracle import attention as ref_attn
from oracle import kv_pool as ref
from oracle import sampler as S
from oracle.spec_step import SeqState, commit_round

pytestmark = pytest.mark.gpu

L_, HQ, HKV, D, BS, V, GAMMA, BATCH = 36, 16, 2, 128, 16, 151936, 6, 128
CHECK_LAYERS = (0, 17, 35, 8)


def _bf16_check(out, want):
    out = out.float().cpu()
    want = want.float()
    for b in range(out.shape[0]):
        scale = float(want[b].abs().max())
        err = (out[b] - want[b]).abs()
        rel = float(err.norm() / want[b].norm())
        assert rel <= 2e-3, (b, rel)
        assert bool((err <= 2.0 ** -7 * want[b].abs() + 2e-3 * scale).all()), (b, float(err.max()), scale)


def test_full_depth_rounds_match_the_oracle(cuda):
    C = GAMMA + 1
    torch.cuda.empty_cache()
    model = SyntheticVerifyModel(L_, HQ, HKV, D, V, GAMMA, BATCH, cuda, torch.bfloat16, seed=11,
                                 draft_sigma=1.05, prompt_cap=8192)
    cap = blocks_for_hbm(L_, BS, HKV, D, torch.bfloat16, cuda, reserve_bytes=0, fraction=0.75)
    reqs = poisson_requests(BATCH, 0.0, 512, 8192, 32, 160, seed=12) + \
        poisson_requests(24, 4.0, 512, 8192, 32, 160, seed=13, first_sid=BATCH)
    maxb = -(-(8192 + 160 + C) // BS) + 1
    kv = PagedKVCache(L_, HKV, D, cap, BS, cuda, torch.bfloat16, max_seqs=len(reqs), max_blocks_per_seq=maxb)
    perm = torch.randperm(cap, generator=torch.Generator().manual_seed(14)).to(torch.int32)
    kv.allocator.load_free_list(perm)
    cpu = ref.PagedKVCache(L_, HKV, D, cap, BS, store=False)
    cpu.allocator.free_list = perm.tolist()
    assert kv.allocator.free_list() == cpu.allocator.free_list
    print("pool: {} blocks ({:.1f} GB)".format(cap, kv.kv_memory_bytes / 1e9), flush=True)

    by_sid = {r.sid: r for r in reqs}
    mirror = {}
    host_logits = {}
    seen = {"rounds": 0, "flagged": 0, "admitted": 0}

    def on_round(info):
        for sid in info.sids:
            if sid not in mirror:  # admitted before this round, in arrival order
                r = by_sid[sid]
                cpu.add_sequence(sid)
                cpu.write_block(0, [sid], [0], None, None, chunk=r.prompt_len)
                mirror[sid] = SeqState(sid, r.prompt_len, r.max_new_tokens, [-1])
                seen["admitted"] += 1
        running = [mirror[s] for s in info.sids]
        assert info.starts == [cpu.seq_lengths[s] for s in info.sids]
        inp = info.inputs
        B = len(info.sids)
        # the round's verify chunk: layer 0 allocates
        cpu.write_block(0, info.sids, info.starts, None, None, chunk=C)
        # one layer: the committed chunk rows as stored, and the attention over
        # the pool (the round has been committed: the pool holds start + k rows,
        # the chunk's other rows are the round's inputs the kernel attended)
        layer = CHECK_LAYERS[seen["rounds"] % len(CHECK_LAYERS)]
        n_commit = info.result.n_commit.tolist()
        assert min(n_commit) > 0  # budgets of 32+ tokens: nothing finishes in four rounds
        keys, values = [], []
        for b, sid in enumerate(info.sids):
            st, n = info.starts[b], n_commit[b]
            ctx = gather_ctx(kv, layer, sid, st + n).cpu()
            kb, vb = inp["k"][layer][b].cpu(), inp["v"][layer][b].cpu()
            assert torch.equal(ctx[0, st:], kb[:n]) and torch.equal(ctx[1, st:], vb[:n])
            keys.append(torch.cat((ctx[0, :st], kb)))
            values.append(torch.cat((ctx[1, :st], vb)))
        want = ref_attn.extend_attention_dense(inp["q"][layer].cpu(), keys, values, info.starts, HQ)
        _bf16_check(info.outputs[layer], want)
        # the sampling against the oracle, the commit with the device's lists
        key = (inp["target"].data_ptr(), B)
        if key not in host_logits:
            host_logits[key] = tuple(x.cpu() for x in (inp["target"], inp["draft"], inp["proposals"], inp["u"],
                                                       inp["noise"]))
        t, dr, pr, u, nz = host_logits[key]
        want_acc = S.verify_from_logits(t[:B], dr[:B], pr[:B], u[:B], nz[:B], 1.0)
        got_acc = info.result.accepted_lists()
        flags = info.result.flags.tolist()
        for b in range(B):
            assert got_acc[b] == want_acc[b] or flags[b], (b, got_acc[b], want_acc[b])
        seen["flagged"] += sum(1 for f in flags if f)
        ks = commit_round(running, dict(zip(info.sids, got_acc)), cpu)
        assert info.result.n_commit.tolist() == ks
        assert kv.block_tables == cpu.block_tables
        assert kv.seq_lengths == cpu.seq_lengths
        free = kv.allocator.free_list()
        assert free == cpu.allocator.free_list
        owned = [blk for tab in kv.block_tables for blk in tab]
        assert len(set(owned)) == len(owned) and not set(owned) & set(free)
        assert len(owned) + len(free) == cap
        seen["rounds"] += 1
        print("round {}: batch {}, mean start {:.0f}, layer {} checked, {} committed, {} blocks held".format(
            seen["rounds"], B, sum(info.starts) / B, layer, sum(ks), len(owned)), flush=True)

    drv = SpecContinuousDriver(kv, model, GAMMA, BATCH, temperature=1.0)
    res = drv.run(reqs, max_steps=4, on_round=on_round)
    assert seen["rounds"] == res.rounds == 4
    assert seen["admitted"] >= BATCH
    assert seen["flagged"] <= 4, seen
    print("flagged sequence-rounds: {}".format(seen["flagged"]))
    del kv, model, drv
    torch.cuda.empty_cache()
