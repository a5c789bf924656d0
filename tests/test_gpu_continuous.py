"""GPU parity of continuous batching (``engine.continuous``) with the oracle.

Requests arrive in a Poisson stream faster than the batch cap and the small
pool admit them, so admission has to wait. After every round the oracle replays the round on the
CPU in the same order: it admits the new sequences (prompt K/V write), writes
the verify K/V of every layer, runs the reference's per-sequence attention, the
rejection rule on the same logits and randomness, and the reference's commit
rule. Attention must agree within the fp32 tolerance (one case runs fp16
pools and queries at Qwen2.5-1.5B heads, on the MFMA attention, at the fp16
bar: per sequence relative L2 <= 1e-3, elements within 2^-10 relative +
1e-3 max|ref|); accepted tokens,
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

from test_gpu_attention import _f16_check

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("eos,dtype", [(None, torch.float32), (5, torch.float32), (5, torch.float16)])
def test_continuous_batching_matches_oracle(cuda, eos, dtype):
    # fp16: the reference's GPU dtype, at Qwen2.5-1.5B heads (the MFMA attention)
    if dtype == torch.float16:
        L, Hq, Hkv, d, bs, V, gamma, max_batch, cap = 2, 12, 2, 128, 16, 24, 3, 5, 32
    else:
        L, Hq, Hkv, d, bs, V, gamma, max_batch, cap = 2, 4, 2, 16, 4, 24, 3, 5, 32
    model = SyntheticVerifyModel(L, Hq, Hkv, d, V, gamma, max_batch, cuda, dtype, seed=3,
                                 draft_sigma=1.0, prompt_cap=48, n_sets=3)
    gpu = PagedKVCache(L, Hkv, d, cap, bs, cuda, dtype)
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
                    cpu.write_block(layer, [sid], [0], k.float().cpu(), v.float().cpu())
                mirror[sid] = SeqState(sid, r.prompt_len, r.max_new_tokens, [-1])
                if r.arrive_step < info.step:
                    seen["waits"] += 1
        running = [mirror[s] for s in info.sids]
        assert info.starts == [cpu.seq_lengths[s] for s in info.sids]
        inp = info.inputs
        for layer in range(L):
            cpu.write_block(layer, info.sids, info.starts, inp["k"][layer].float().cpu(),
                            inp["v"][layer].float().cpu())
            want = ref_attn.paged_attention_extend(inp["q"][layer].float().cpu(), cpu, layer, info.sids,
                                                   info.starts, Hq)
            if dtype == torch.float16:
                _f16_check(info.outputs[layer], want)
            else:
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


@pytest.mark.parametrize("temperature,eos", [(1.0, None), (1.0, 5), (0.0, None)])
def test_continuous_with_draft_side_matches_oracle(cuda, temperature, eos):
    """The whole round with a draft pool: gamma draft steps (append + decode
    attention per draft layer, batched sampling), verify, commit, the device
    draft alignment and its catch-up decode, replayed by the oracle; both pools
    identical after every round, and the device metrics equal to the mirror's
    counts at every record point."""
    L, Hq, Hkv, d, bs, V, gamma, max_batch, cap = 2, 4, 2, 16, 4, 24, 3, 5, 40
    DL, dHq, dHkv, dd = 2, 2, 1, 16
    model = SyntheticVerifyModel(L, Hq, Hkv, d, V, gamma, max_batch, cuda, torch.float32, seed=7,
                                 draft_sigma=0.3, prompt_cap=48, n_sets=3, temperature=max(temperature, 1e-3),
                                 draft_layers=DL, draft_heads=(dHq, dHkv, dd))
    gpu = PagedKVCache(L, Hkv, d, cap, bs, cuda, torch.float32)
    gpu_d = PagedKVCache(DL, dHkv, dd, cap, bs, cuda, torch.float32)
    cpu = ref.PagedKVCache(L, Hkv, d, cap, bs)
    cpu_d = ref.PagedKVCache(DL, dHkv, dd, cap, bs)
    reqs = poisson_requests(12, 2.0, 3, 30, 2, 14, seed=9)
    by_sid = {r.sid: r for r in reqs}
    drv = SpecContinuousDriver(gpu, model, gamma, max_batch, temperature=temperature, eos_id=eos, draft_kv=gpu_d)
    mirror = {}
    seen = {"rounds": 0, "catch_ups": 0, "catch_up_rounds": 0, "records": []}

    record = drv._record

    def checked_record(result):
        record(result)
        seen["records"].append((gpu.num_allocated_blocks, gpu.logical_tokens, gpu_d.num_allocated_blocks))

    drv._record = checked_record

    def on_round(info):
        for sid in info.sids:
            if sid not in mirror:
                r = by_sid[sid]
                cpu.add_sequence(sid)
                cpu_d.add_sequence(sid)
                k, v = model.prompt_kv(r.prompt_len)
                for layer in range(L):
                    cpu.write_block(layer, [sid], [0], k.cpu(), v.cpu())
                dk, dv = model.draft_prompt_kv(r.prompt_len)
                for layer in range(DL):
                    cpu_d.write_block(layer, [sid], [0], dk.cpu(), dv.cpu())
                mirror[sid] = SeqState(sid, r.prompt_len, r.max_new_tokens, [0])
        running = [mirror[s] for s in info.sids]
        inp = info.inputs
        assert info.starts == [cpu_d.seq_lengths[s] for s in info.sids]
        # the gamma draft steps
        props = inp["proposals"].cpu()
        for j in range(gamma):
            pos = [st + j for st in info.starts]
            for layer in range(DL):
                cpu_d.write_block(layer, info.sids, pos, inp["dk"][j][layer].cpu(), inp["dv"][j][layer].cpu())
                want = ref_attn.paged_attention_extend(inp["dq"][j][layer].cpu(), cpu_d, layer, info.sids, pos, dHq)
                torch.testing.assert_close(info.draft_outputs[j][layer].cpu(), want, atol=1e-5, rtol=1e-5)
            for b in range(len(info.sids)):
                q = S.logits_to_probs(inp["draft"][b, j].cpu(), temperature)
                tok = S.race_argmax(q, inp["draft_noise"][j][b].cpu()) if temperature > 0 else int(q.argmax())
                assert int(props[b, j]) == tok, (b, j)
        # verify
        for layer in range(L):
            cpu.write_block(layer, info.sids, info.starts, inp["k"][layer].cpu(), inp["v"][layer].cpu())
            want = ref_attn.paged_attention_extend(inp["q"][layer].cpu(), cpu, layer, info.sids, info.starts, Hq)
            torch.testing.assert_close(info.outputs[layer].cpu(), want, atol=1e-5, rtol=1e-5)
        acc = S.verify_from_logits(inp["target"].cpu(), inp["draft"].cpu(), props, inp["u"].cpu(),
                                   inp["noise"].cpu(), temperature)
        assert info.result.accepted_lists() == acc
        catchups = []
        ks = commit_round(running, dict(zip(info.sids, acc)), cpu, cpu_d, eos=eos, catchups=catchups)
        assert info.result.n_commit.tolist() == ks
        # the catch-up: positions, tokens and its decode
        count, cpos, ctok = (x.tolist() for x in (info.catch_up.count, info.catch_up.pos, info.catch_up.tokens))
        live = {c.sid: c for c in catchups if not c.finished}
        for b, sid in enumerate(info.sids):
            c = live.get(sid)
            assert count[b] == (len(c.tokens) if c else 0), b
            if c:
                assert cpos[b] == c.pos and ctok[b][: count[b]] == c.tokens
        rows = info.catch_up_rows or []
        assert rows == [b for b in range(len(info.sids)) if count[b]]
        for layer in range(DL):
            for b in rows:
                cpu_d.write(layer, info.sids[b], cpos[b], inp["dk"][0][layer][b, 0].cpu(), inp["dv"][0][layer][b, 0].cpu())
            if rows:
                sids_r = [info.sids[b] for b in rows]
                want = ref_attn.paged_attention_extend(inp["dq"][0][layer][rows].cpu(), cpu_d, layer, sids_r,
                                                       [cpos[b] for b in rows], dHq)
                torch.testing.assert_close(info.catch_up_outputs[layer].cpu(), want, atol=1e-5, rtol=1e-5)
        seen["catch_ups"] += len(rows)
        seen["catch_up_rounds"] += 1 if rows else 0
        for g, c in ((gpu, cpu), (gpu_d, cpu_d)):
            assert g.block_tables == c.block_tables
            assert g.seq_lengths == c.seq_lengths
            assert g.allocator.free_list() == c.allocator.free_list
        seen["rounds"] += 1

    res = drv.run(reqs, max_steps=400, on_round=on_round)
    assert res.admitted == res.finished == len(reqs)
    assert seen["rounds"] == res.rounds > 5
    assert seen["catch_ups"] > 0, "no round accepted every proposal"
    assert res.draft_forward_calls == gamma * res.rounds + seen["catch_up_rounds"]
    assert gpu.allocator.num_free == cap and gpu_d.allocator.num_free == cap
    # device metrics == the mirror's counts at every record point
    assert len(res.block_util_hist) == len(res.batch_hist) == len(seen["records"]) == res.steps
    for u, (alloc, tok, _) in zip(res.block_util_hist, seen["records"]):
        assert u == (tok / (alloc * bs) if alloc else 0.0)
    assert res.kv_peak_blocks == max(r[0] for r in seen["records"])
    assert res.draft_kv_peak_blocks == max(r[2] for r in seen["records"])


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
