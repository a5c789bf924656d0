"""GPU parity of whole verify rounds (append -> attention -> sample -> rewind).

A small continuous batch runs several rounds through ``engine.spec_scheduler.
VerifyStep`` and, in lockstep, through the oracle (per-token writes, masked SDPA
per sequence, batch_accept on the same noise, the reference's commit rule).
After every round the pool state (tables, lengths, free list) must be identical
and the attention outputs within the fp32 tolerance of the reference's tests.
With the commit held (``apply=False``) each round's commit goes with the next
round's first append (one launch, or on its own once the batch changes): the
pool must then equal the oracle's after every append, and after the last flush.
The same rounds over an fp16 pool with fp16 queries at Qwen2.5-1.5B heads run
the MFMA attention (fp16 tolerance) and leave the pool equal to the oracle's.
"""

from __future__ import annotations

import pytest
import torch

from engine.kv import PagedKVCache
from engine.spec_scheduler import VerifyStep
from oracle import attention as ref_attn
from oracle import kv_pool as ref
from oracle import sampler as S
from oracle.spec_step import SeqState, commit_round

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("defer", [False, True])
def test_verify_rounds_match_oracle(cuda, defer):
    torch.manual_seed(0)
    B, gamma, Hq, Hkv, d, bs, V, cap = 5, 3, 4, 2, 16, 4, 32, 96
    C = gamma + 1
    gpu = PagedKVCache(1, Hkv, d, cap, bs, cuda, torch.float32)
    cpu = ref.PagedKVCache(1, Hkv, d, cap, bs)
    g = torch.Generator().manual_seed(1)
    seqs = []
    for s in range(B):
        gpu.add_sequence(s)
        cpu.add_sequence(s)
        prompt = 3 + 4 * s
        k = torch.randn(1, prompt, Hkv, d, generator=g)
        v = torch.randn(1, prompt, Hkv, d, generator=g)
        gpu.write_block(0, [s], [0], k.to(cuda), v.to(cuda))
        cpu.write_block(0, [s], [0], k, v)
        seqs.append(SeqState(s, prompt, 12 + s, [int(torch.randint(V, (1,), generator=g))]))
    step = VerifyStep(gpu, gamma, temperature=1.0)
    for rnd in range(6):
        running = [s for s in seqs if not s.finished]
        if not running:
            break
        sids = [s.sid for s in running]
        starts = [cpu.seq_lengths[s] for s in sids]
        n = len(sids)
        q = torch.randn(n, C, Hq, d, generator=g)
        k = torch.randn(n, C, Hkv, d, generator=g)
        v = torch.randn(n, C, Hkv, d, generator=g)
        out = step.attend_layers(sids, starts, [q.to(cuda)], [k.to(cuda)], [v.to(cuda)])[0]
        cpu.write_block(0, sids, starts, k, v)
        if defer:  # the previous commit and this append are applied now
            assert gpu.block_tables == cpu.block_tables
            assert gpu.seq_lengths == cpu.seq_lengths
            assert gpu.allocator.free_list() == cpu.allocator.free_list
        want = ref_attn.paged_attention_extend(q, cpu, 0, sids, starts, Hq)
        assert torch.allclose(out.cpu(), want, atol=1e-5, rtol=1e-5)
        target = torch.randn(n, C, V, generator=g) * 2
        draft = target[:, :gamma] + torch.randn(n, gamma, V, generator=g)
        x = torch.multinomial(S.logits_to_probs(draft, 1.0).reshape(-1, V), 1, generator=g).reshape(n, gamma)
        u = torch.rand(n, gamma, generator=g)
        noise = torch.empty(n, V).exponential_(1, generator=g)
        remaining = [s.max_new_tokens - len(s.generated) for s in running]
        res = step.sample_and_commit(sids, starts, target.to(cuda), draft.to(cuda), x.to(cuda),
                                     u.to(cuda), noise.to(cuda), remaining, apply=not defer)
        acc = S.verify_from_logits(target, draft, x, u, noise, 1.0)
        assert res.accepted_lists() == acc
        ks = commit_round(running, {s: a for s, a in zip(sids, acc)}, cpu)
        assert res.n_commit.tolist() == ks
        if defer:
            continue
        assert gpu.block_tables == cpu.block_tables
        assert gpu.seq_lengths == cpu.seq_lengths
        assert gpu.allocator.free_list() == cpu.allocator.free_list
    step.flush()
    assert gpu.block_tables == cpu.block_tables
    assert gpu.seq_lengths == cpu.seq_lengths
    assert gpu.allocator.free_list() == cpu.allocator.free_list


@pytest.mark.parametrize("defer", [False, True])
def test_fp16_verify_rounds_on_the_mfma_path(cuda, defer):
    """Whole rounds over an fp16 pool with fp16 queries (the reference's GPU
    dtype) at Qwen2.5-1.5B heads (12/2, head_dim 128, block 16): the MFMA
    attention, the append and the commit. Pool state equals the oracle's; the
    attention is held to the fp16 bar (per sequence relative L2 <= 1e-3, every
    element within 2^-10 relative + 1e-3 max|ref|) against the oracle in fp32
    on the same fp16 values."""
    from test_gpu_attention import _f16_check

    B, gamma, Hq, Hkv, d, bs, V, cap = 6, 5, 12, 2, 128, 16, 64, 512
    C = gamma + 1
    gpu = PagedKVCache(1, Hkv, d, cap, bs, cuda, torch.float16)
    cpu = ref.PagedKVCache(1, Hkv, d, cap, bs)
    g = torch.Generator().manual_seed(7)
    h = lambda t: t.half()
    seqs = []
    for s in range(B):
        gpu.add_sequence(s)
        cpu.add_sequence(s)
        prompt = 1 + 97 * s
        k = h(torch.randn(1, prompt, Hkv, d, generator=g))
        v = h(torch.randn(1, prompt, Hkv, d, generator=g))
        gpu.write_block(0, [s], [0], k.to(cuda), v.to(cuda))
        cpu.write_block(0, [s], [0], k.float(), v.float())
        seqs.append(SeqState(s, prompt, 20 + 3 * s, [int(torch.randint(V, (1,), generator=g))]))
    step = VerifyStep(gpu, gamma, temperature=1.0)
    for rnd in range(5):
        running = [s for s in seqs if not s.finished]
        if not running:
            break
        sids = [s.sid for s in running]
        starts = [cpu.seq_lengths[s] for s in sids]
        n = len(sids)
        q = h(torch.randn(n, C, Hq, d, generator=g))
        k = h(torch.randn(n, C, Hkv, d, generator=g))
        v = h(torch.randn(n, C, Hkv, d, generator=g))
        out = step.attend_layers(sids, starts, [q.to(cuda)], [k.to(cuda)], [v.to(cuda)])[0]
        cpu.write_block(0, sids, starts, k.float(), v.float())
        _f16_check(out, ref_attn.paged_attention_extend(q.float(), cpu, 0, sids, starts, Hq))
        target = torch.randn(n, C, V, generator=g) * 2
        draft = target[:, :gamma] + torch.randn(n, gamma, V, generator=g)
        x = torch.multinomial(S.logits_to_probs(draft, 1.0).reshape(-1, V), 1, generator=g).reshape(n, gamma)
        u = torch.rand(n, gamma, generator=g)
        noise = torch.empty(n, V).exponential_(1, generator=g)
        remaining = [s.max_new_tokens - len(s.generated) for s in running]
        res = step.sample_and_commit(sids, starts, target.to(cuda), draft.to(cuda), x.to(cuda),
                                     u.to(cuda), noise.to(cuda), remaining, apply=not defer)
        acc = S.verify_from_logits(target, draft, x, u, noise, 1.0)
        assert res.accepted_lists() == acc
        ks = commit_round(running, {s: a for s, a in zip(sids, acc)}, cpu)
        assert res.n_commit.tolist() == ks
        if not defer:
            assert gpu.block_tables == cpu.block_tables
            assert gpu.seq_lengths == cpu.seq_lengths
            assert gpu.allocator.free_list() == cpu.allocator.free_list
    step.flush()
    assert gpu.block_tables == cpu.block_tables
    assert gpu.seq_lengths == cpu.seq_lengths
    assert gpu.allocator.free_list() == cpu.allocator.free_list
    # the pool holds the oracle's fp16 values bit for bit
    from engine.attention import gather_ctx
    for s in range(B):
        L = cpu.seq_lengths[s]
        got = gather_ctx(gpu, 0, s, L)
        assert got.dtype == torch.float16
        assert torch.equal(got.float().cpu(), ref_attn.gather_ctx(cpu, 0, s, L).float())
