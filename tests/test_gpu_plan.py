"""GPU parity of planned verify attention (``VerifyPlan``, spv_verify_attn_plan /
spv_verify_attn_planned) with the unplanned call and the oracle.

A plan only moves the split of the batch over the workgroups and each
workgroup's first block ids out of the call; the arithmetic is the same, so
planned outputs must equal unplanned ones bit for bit. Cases: the
Qwen2.5-1.5B verify shape (equal pieces), a batch whose segments outnumber the
workgroups (the cost-balanced split, several pieces per workgroup), head_dim 64
with four query tiles, one-row draft decode, pieces longer than the 512-entry
block-id window, fp8 pages, fp16 pages with fp16
queries, and one plan serving several layers. (The
head_dim-128 kernels with four query tiles do not use a plan; their case checks
that a planned call of that shape still runs and matches.) The plan's
once-per-round length check raises the reference's IndexError like the
unplanned call's does.
"""

from __future__ import annotations

import pytest
import torch

from engine.attention import VerifyPlan, verify_attention
from engine.kv import PagedKVCache
from oracle import attention as ref_attn

from test_gpu_attention import _bf16_check, _dense_pool

pytestmark = pytest.mark.gpu


def _lens(n, lo, hi, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(lo, hi + 1, (n,), generator=g).tolist()


@pytest.mark.parametrize("B,Hq,Hkv,d,C,lo,hi", [
    (32, 12, 2, 128, 6, 256, 4096),    # Qwen2.5-1.5B verify: equal pieces
    (160, 12, 2, 128, 6, 16, 3000),    # segments outnumber the workgroups: cost-balanced split
    (160, 16, 2, 128, 7, 16, 3000),    # four query tiles at head_dim 128: the plan is not used
    (16, 14, 2, 64, 9, 100, 12000),    # head_dim 64, four query tiles
    (128, 2, 2, 128, 2, 12000, 13000),  # cost-balanced pieces of more than 512 pages (restaged ids)
    (48, 14, 2, 64, 1, 1, 3000),       # draft decode: one row
    (3, 32, 4, 128, 5, 1, 40),         # tiny contexts, more workgroups than pages
])
def test_planned_equals_unplanned_and_the_oracle(cuda, B, Hq, Hkv, d, C, lo, hi):
    lens = _lens(B, lo, hi, seed=B + d)
    gpu, keys, values = _dense_pool(cuda, lens, C, Hkv, d, 16, torch.bfloat16, seed=B)
    g = torch.Generator().manual_seed(B * 3 + C)
    q = torch.randn(B, C, Hq, d, generator=g).to(torch.bfloat16).to(cuda)
    sids = list(range(B))
    max_ctx = max(lens) + C
    plain = verify_attention(q, gpu, 0, sids, lens, max_ctx)
    plan = VerifyPlan(gpu, sids, lens, C, Hq, max_ctx)
    planned = verify_attention(q, gpu, 0, sids, lens, max_ctx, plan=plan)
    planned2 = verify_attention(q, gpu, 0, sids, lens, max_ctx, plan=plan)  # the plan is reusable
    assert torch.equal(planned, plain)
    assert torch.equal(planned2, plain)
    assert gpu.seq_lengths == [L + C for L in lens]  # no bad read flagged
    rows = list(range(0, B, max(1, B // 6)))
    want = ref_attn.extend_attention_dense(q[rows].float().cpu(), [keys[r] for r in rows],
                                           [values[r] for r in rows], [lens[r] for r in rows], Hq)
    _bf16_check(planned[rows], want)


def test_one_plan_serves_every_layer(cuda):
    B, Hq, Hkv, d, C, layers = 24, 12, 2, 128, 6, 3
    lens = _lens(B, 100, 2500, seed=4)
    cap = sum(-(-(L + C) // 16) for L in lens) + 8
    gpu = PagedKVCache(layers, Hkv, d, cap, 16, cuda, torch.bfloat16, max_seqs=B)
    g = torch.Generator().manual_seed(8)
    for s in range(B):
        gpu.add_sequence(s)
    for layer in range(layers):
        for s, L in enumerate(lens):
            k = torch.randn(1, L, Hkv, d, generator=g).to(torch.bfloat16).to(cuda)
            gpu.write_block(layer, [s], [0], k, torch.randn_like(k))
    sid_t = torch.arange(B, dtype=torch.int32, device=cuda)
    st_t = torch.tensor(lens, dtype=torch.int32, device=cuda)
    kn = [torch.randn(B, C, Hkv, d, generator=g).to(torch.bfloat16).to(cuda) for _ in range(layers)]
    q = [torch.randn(B, C, Hq, d, generator=g).to(torch.bfloat16).to(cuda) for _ in range(layers)]
    max_ctx = max(lens) + C
    plan = None
    for layer in range(layers):
        gpu.write_block_device(layer, sid_t, st_t, kn[layer], kn[layer] * 0.5, alloc=layer == 0)
        if layer == 0:
            plan = VerifyPlan(gpu, sid_t, st_t, C, Hq, max_ctx)  # after the round's allocation
        got = verify_attention(q[layer], gpu, layer, sid_t, st_t, max_ctx, plan=plan)
        assert torch.equal(got, verify_attention(q[layer], gpu, layer, sid_t, st_t, max_ctx)), layer


def test_planned_fp8_pages(cuda):
    from test_gpu_fp8 import _fp8_pool_with

    lens = [2000, 37, 700, 1, 129, 1500, 5000, 64]
    Hq, H, d, C = 14, 2, 64, 9
    gpu, cpu, g = _fp8_pool_with(cuda, lens, H, d, 16, C, 9)
    q = torch.randn(len(lens), C, Hq, d, generator=g).to(torch.bfloat16).to(cuda)
    sids = list(range(len(lens)))
    max_ctx = max(lens) + C
    plan = VerifyPlan(gpu, sids, lens, C, Hq, max_ctx)
    assert torch.equal(verify_attention(q, gpu, 0, sids, lens, max_ctx, plan=plan),
                       verify_attention(q, gpu, 0, sids, lens, max_ctx))


@pytest.mark.parametrize("d,C,Hq", [(128, 6, 12), (64, 9, 14)])
def test_planned_fp16_pages(cuda, d, C, Hq):
    # fp16 pools take fp16 queries on the MFMA path; their plan is made for them
    from test_gpu_attention import _f16_check

    lens = _lens(24, 1, 3000, seed=d)
    gpu, keys, values = _dense_pool(cuda, lens, C, 2, d, 16, torch.float16, seed=d + 3)
    q = torch.randn(len(lens), C, Hq, d, generator=torch.Generator().manual_seed(d)).to(torch.float16)
    qd = q.to(cuda)
    sids = list(range(len(lens)))
    max_ctx = max(lens) + C
    plan = VerifyPlan(gpu, sids, lens, C, Hq, max_ctx)
    planned = verify_attention(qd, gpu, 0, sids, lens, max_ctx, plan=plan)
    assert torch.equal(planned, verify_attention(qd, gpu, 0, sids, lens, max_ctx))
    rows = list(range(0, len(lens), 4))
    _f16_check(planned[rows], ref_attn.extend_attention_dense(q[rows], [keys[r] for r in rows],
                                                              [values[r] for r in rows], [lens[r] for r in rows], Hq))


def test_plan_reports_unwritten_keys(cuda):
    lens, C, Hq, Hkv, d = [300, 500], 6, 12, 2, 128
    gpu, _, _ = _dense_pool(cuda, lens, C, Hkv, d, 16, torch.bfloat16, seed=1)
    assert gpu.seq_lengths == [306, 506]
    # a chunk starting one past the written keys reads a position never written
    with pytest.raises(IndexError, match="never written"):
        VerifyPlan(gpu, [0, 1], [301, 500], C, Hq, 600)
        gpu.seq_lengths
    plan = VerifyPlan(gpu, [0, 1], lens, C, Hq, 600)
    q = torch.randn(2, C, Hq, d, device=cuda).to(torch.bfloat16)
    verify_attention(q, gpu, 0, [0, 1], lens, 600, plan=plan)
    assert gpu.seq_lengths == [306, 506]
    with pytest.raises(ValueError, match="does not match its plan"):
        verify_attention(q, gpu, 0, [0, 1], lens, 700, plan=plan)
