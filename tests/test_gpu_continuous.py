"""GPU parity of continuous batching (``engine.continuous``) with the oracle.

Requests arrive in a Poisson stream faster than the batch cap and the small
pool admit them, so admission has to wait. After every round the oracle replays the round on the
CPU in the same order: it admits the new sequences (prompt K/V write), writes
the verify K/V of every layer, runs the reference's per-sequence attention, the
rejection rule on the same logits and randomness, and the reference's commit
rule. Attention must agree within the fp32 tolerance; accepted tokens,
committed counts, finished flags, block tables, lengths and the free list must
be identical.
"""

from __future__ import annotations

import pytest
import torch

from engine.continuous import SpecContinuousDriver, SyntheticVerifyModel, poisson_requests
from engine.kv import PagedKVCache
from oracle import attention as ref_attn
from oracle import kv_pool as ref
from oracle import sampler as S
from oracle.spec_step import SeqState, commit_round

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("eos", [None, 5])
def test_continuous_batching_matches_oracle(cuda, eos):
    L, Hq, Hkv, d, bs, V, gamma, max_batch, cap = 2, 4, 2, 16, 4, 24, 3, 5, 32
    model = SyntheticVerifyModel(L, Hq, Hkv, d, V, gamma, max_batch, cuda, torch.float32, seed=3,
                                 draft_sigma=1.0, prompt_cap=48, n_sets=3)
    gpu = PagedKVCache(L, Hkv, d, cap, bs, cuda, torch.float32)
    cpu = ref.PagedKVCache(L, Hkv, d, cap, bs)
    reqs = poisson_requests(14, 2.5, 3, 40, 2, 16, seed=5)
    by_sid = {r.sid: r for r in reqs}
    drv = SpecContinuousDriver(gpu, model, gamma, max_batch, temperature=1.0, eos_id=eos)
    mirror = {}
    seen = {"rounds": 0, "waits": 0, "max_batch": 0}

    def on_round(info):
        for sid in info.sids:
            if sid not in mirror:  # admitted before this round, in arrival order
                r = by_sid[sid]
                cpu.add_sequence(sid)
                k, v = model.prompt_kv(r.prompt_len)
                for layer in range(L):
                    cpu.write_block(layer, [sid], [0], k.cpu(), v.cpu())
                mirror[sid] = SeqState(sid, r.prompt_len, r.max_new_tokens, [-1])
                if r.arrive_step < info.step:
                    seen["waits"] += 1
        running = [mirror[s] for s in info.sids]
        assert info.starts == [cpu.seq_lengths[s] for s in info.sids]
        inp = info.inputs
        for layer in range(L):
            cpu.write_block(layer, info.sids, info.starts, inp["k"][layer].cpu(), inp["v"][layer].cpu())
            want = ref_attn.paged_attention_extend(inp["q"][layer].cpu(), cpu, layer, info.sids, info.starts, Hq)
            torch.testing.assert_close(info.outputs[layer].cpu(), want, atol=1e-5, rtol=1e-5)
        acc = S.verify_from_logits(inp["target"].cpu(), inp["draft"].cpu(), inp["proposals"].cpu(),
                                   inp["u"].cpu(), inp["noise"].cpu(), 1.0)
        assert info.result.accepted_lists() == acc
        ks = commit_round(running, dict(zip(info.sids, acc)), cpu, eos=eos)
        assert info.result.n_commit.tolist() == ks
        assert [bool(f) for f in info.result.finished.tolist()] == [s.finished for s in running]
        assert gpu.block_tables == cpu.block_tables
        assert gpu.seq_lengths == cpu.seq_lengths
        assert gpu.allocator.free_list() == cpu.allocator.free_list
        seen["rounds"] += 1
        seen["max_batch"] = max(seen["max_batch"], len(info.sids))

    res = drv.run(reqs, max_steps=400, on_round=on_round)
    assert res.admitted == res.finished == len(reqs)
    assert seen["rounds"] == res.rounds and res.rounds > 5
    assert seen["waits"] > 0, "admission never had to wait"
    assert seen["max_batch"] > 1
    assert all(m.finished for m in mirror.values())
    assert gpu.allocator.num_free == cap and len(cpu.allocator.free_list) == cap
    assert sum(res.tokens_per_round) == sum(len(m.generated) - 1 for m in mirror.values())
    assert res.kv_peak_blocks <= cap


def test_admission_reserves_lifetimes(cuda):
    """No round can exhaust the pool: every admitted request's whole lifetime fits."""
    L, Hq, Hkv, d, bs, V, gamma = 1, 2, 1, 16, 4, 16, 5
    model = SyntheticVerifyModel(L, Hq, Hkv, d, V, gamma, 8, cuda, torch.float32, seed=1,
                                 draft_sigma=0.1, prompt_cap=64, n_sets=2)
    cap = 24
    gpu = PagedKVCache(L, Hkv, d, cap, bs, cuda, torch.float32)
    drv = SpecContinuousDriver(gpu, model, gamma, 8)
    reqs = poisson_requests(20, 0.0, 10, 60, 10, 30, seed=2)  # all arrive at step 0
    peak = []

    def on_round(info):
        assert sum(s.lifetime_blocks for s in drv.running) <= cap
        peak.append(cap - gpu.allocator.num_free)

    res = drv.run(reqs, max_steps=2000, on_round=on_round)
    assert res.finished == len(reqs)
    assert max(peak) <= cap and gpu.allocator.num_free == cap
