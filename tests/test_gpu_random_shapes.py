"""GPU parity of verify attention over a seeded sweep of shapes.

Each case draws head_dim (64 / 128), kv heads (1, 2, 4), the GQA ratio
(1 .. 8), the chunk (1 .. 9 rows), the batch and the start positions (zeros,
block boundaries and random lengths mixed), then checks:

* bf16 pools: the unplanned call against the oracle's dense extend attention
  at the bf16 bar of test_gpu_attention (per sequence relative L2 <= 2e-3 and
  every element within one bf16 ulp + 2e-3 max |ref|), and the planned call
  bit for bit against the unplanned one;
* fp16 pools with fp16 queries: the same two checks at the fp16 bar (per
  sequence relative L2 <= 1e-3, every element within 2^-10 relative + 1e-3
  max |ref|), 8 cases of their own draws;
* fp8 pools: the call against the oracle on the dequantised pool, same bar;
* fp32 pools (the VALU path): against the oracle at atol = rtol = 1e-5.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from engine.attention import VerifyPlan, verify_attention
from oracle import attention as ref_attn
from test_gpu_attention import _bf16_check, _dense_pool, _f16_check
from test_gpu_fp8 import _fp8_pool_with

pytestmark = pytest.mark.gpu

N_CASES = 16


def _draw(seed):
    rng = np.random.default_rng(1000 + seed)
    d = int(rng.choice([64, 128]))
    hkv = int(rng.choice([1, 2, 4]))
    ratio = int(rng.choice([1, 2, 3, 4, 6, 7, 8]))
    C = int(rng.integers(1, 10))
    B = int(rng.choice([1, 3, 17, 40, 130, 260]))
    hi = 3000 if B <= 40 else 300  # keeps the oracle's work small
    lens = rng.integers(0, hi + 1, size=B)
    special = rng.random(B)
    lens = np.where(special < 0.1, 0, lens)
    lens = np.where((special >= 0.1) & (special < 0.2), (lens // 16) * 16, lens)
    lens = np.where((special >= 0.2) & (special < 0.25), 1, lens)
    return d, hkv, hkv * ratio, C, [int(x) for x in lens]


def _planned_and_oracle(cuda, seed, dtype, check):
    d, hkv, hq, C, lens = _draw(seed)
    B = len(lens)
    gpu, keys, values = _dense_pool(cuda, lens, C, hkv, d, 16, dtype, seed=seed)
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, C, hq, d, generator=g).to(dtype).to(cuda)
    sids = list(range(B))
    max_ctx = max(lens) + C
    plain = verify_attention(q, gpu, 0, sids, lens, max_ctx)
    plan = VerifyPlan(gpu, sids, lens, C, hq, max_ctx)
    planned = verify_attention(q, gpu, 0, sids, lens, max_ctx, plan=plan)
    assert torch.equal(planned, plain), (d, hkv, hq, C, B)
    assert gpu.seq_lengths == [L + C for L in lens]  # no bad read flagged
    rows = list(range(0, B, max(1, B // 8)))
    want = ref_attn.extend_attention_dense(q[rows].float().cpu(), [keys[r] for r in rows],
                                           [values[r] for r in rows], [lens[r] for r in rows], hq)
    check(plain[rows], want)


@pytest.mark.parametrize("seed", range(N_CASES))
def test_bf16_random_shape(cuda, seed):
    _planned_and_oracle(cuda, seed, torch.bfloat16, _bf16_check)


@pytest.mark.parametrize("seed", range(100, 100 + N_CASES, 2))
def test_fp16_random_shape(cuda, seed):
    # fp16 pools with fp16 queries (the MFMA path), other draws than the bf16 cases
    _planned_and_oracle(cuda, seed, torch.float16, _f16_check)


@pytest.mark.parametrize("seed", range(0, N_CASES, 2))
def test_fp8_random_shape(cuda, seed):
    d, hkv, hq, C, lens = _draw(seed)
    lens = [max(L, 1) for L in lens][:40]  # an fp8 sequence starts with a written prefix
    gpu, cpu, g = _fp8_pool_with(cuda, lens, hkv, d, 16, C, seed)
    q = torch.randn(len(lens), C, hq, d, generator=g).to(torch.bfloat16)
    sids = list(range(len(lens)))
    out = verify_attention(q.to(cuda), gpu, 0, sids, lens, max(lens) + C).float().cpu()
    want = ref_attn.paged_attention_extend(q.float(), cpu.dequantized(), 0, sids, lens, hq)
    _bf16_check(out, want)


@pytest.mark.parametrize("seed", range(1, N_CASES, 4))
def test_fp32_random_shape_valu_path(cuda, seed):
    d, hkv, hq, C, lens = _draw(seed)
    lens = lens[:17]
    gpu, keys, values = _dense_pool(cuda, lens, C, hkv, d, 16, torch.float32, seed=seed)
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(len(lens), C, hq, d, generator=g)
    out = verify_attention(q.to(cuda), gpu, 0, list(range(len(lens))), lens, max(lens) + C).cpu()
    want = ref_attn.extend_attention_dense(q, keys, values, lens, hq)
    torch.testing.assert_close(out, want, atol=1e-5, rtol=1e-5)
