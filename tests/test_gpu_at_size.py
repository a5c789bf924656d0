"""Verify attention at the full sizes of the two deep workloads, against the oracle.

* Qwen2.5-3B-shaped full-depth step: batch 128, 16 q / 2 kv heads, head_dim
  128, block 16, bf16, contexts log-uniform in [512, 8192], gamma 6 (7 rows).
  The pool has 36 layers and the test attends layer 35, so every K/V offset the
  kernel forms is beyond 2^31 elements (and 2^32 bytes); the tables come from a
  shuffled free list. The batch of 128 sequences x 2 kv heads fills every
  workgroup with segments, so the cost-balanced split runs (four query tiles).
* Qwen2.5-0.5B-shaped long context: batch 16, 32,768 keys, 14 q / 2 kv heads,
  head_dim 64, gamma 8 (9 rows), fp8 e4m3 pool with per-(layer, block, K|V)
  scales. The reference side runs on K/V decoded on the host from the pool's
  raw codes and scales (the codes themselves are pinned bit-exact against the
  oracle's quantiser in test_gpu_fp8.py).

Both compare with ``oracle.attention.extend_attention_dense`` in fp32 at the
bf16 bar (per sequence relative L2 <= 2e-3, and every element within one bf16
ulp plus 2e-3 * max |ref|).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from engine.attention import verify_attention
from engine.kv import PagedKVCache
from oracle import attention as ref_attn
from oracle.kv_fp8 import e4m3_decode

pytestmark = pytest.mark.gpu


def _bf16_check(out, want):
    out = out.float().cpu()
    want = want.float()
    for b in range(out.shape[0]):
        scale = float(want[b].abs().max())
        err = (out[b] - want[b]).abs()
        rel = float(err.norm() / want[b].norm())
        assert rel <= 2e-3, (b, rel)
        assert bool((err <= 2.0 ** -7 * want[b].abs() + 2e-3 * scale).all()), (b, float(err.max()), scale)


def test_full_depth_shape_at_layer_35_of_36(cuda):
    L_, B, C, Hq, Hkv, d, bs, layer = 36, 128, 7, 16, 2, 128, 16, 35
    g = torch.Generator().manual_seed(4)
    lens = [int(math.exp(math.log(512) + (math.log(8192) - math.log(512)) * float(u)))
            for u in torch.rand(B, generator=g)]
    need = sum(-(-(L + C) // bs) for L in lens)
    cap = need + 1024
    assert (layer * cap) * Hkv * bs * d > 2 ** 31  # every page offset of layer 35 is past 2^31 elements
    kv = PagedKVCache(L_, Hkv, d, cap, bs, cuda, torch.bfloat16, max_seqs=B,
                      max_blocks_per_seq=-(-(8192 + C) // bs) + 1)
    kv.allocator.load_free_list(torch.randperm(cap, generator=g).to(torch.int32))
    keys, values = [], []
    for s, L in enumerate(lens):
        kv.add_sequence(s)
        k = torch.randn(L + C, Hkv, d, generator=g).to(torch.bfloat16)
        v = torch.randn(L + C, Hkv, d, generator=g).to(torch.bfloat16)
        kv.write_block(layer, [s], [0], k[:L].unsqueeze(0).to(cuda), v[:L].unsqueeze(0).to(cuda))
        keys.append(k)
        values.append(v)
    kc = torch.stack([k[L:] for k, L in zip(keys, lens)]).to(cuda)
    vc = torch.stack([v[L:] for v, L in zip(values, lens)]).to(cuda)
    kv.write_block(layer, list(range(B)), lens, kc, vc)  # the verify chunk of the whole batch
    assert kv.seq_lengths == [L + C for L in lens]
    q = torch.randn(B, C, Hq, d, generator=g).to(torch.bfloat16)
    out = verify_attention(q.to(cuda), kv, layer, list(range(B)), lens, max(lens) + C)
    assert kv.seq_lengths == [L + C for L in lens]  # no forbidden read was flagged
    _bf16_check(out, ref_attn.extend_attention_dense(q, keys, values, lens, Hq))


def _decoded_context(kv, layer, sid, n):
    """K and V of positions 0..n-1 decoded on the host from the pool's raw
    e4m3 codes and the blocks' fp32 scales: (n, Hkv, d) each."""
    bs = kv.block_size
    table = kv.block_tables[sid][: -(-n // bs)]
    idx = torch.tensor(table, dtype=torch.long)
    kc = kv.k_pool.view(torch.uint8)[layer, idx.to(kv.device)].cpu().numpy()   # (nb, H, bs, d)
    vc = kv.v_pool.view(torch.uint8)[layer, idx.to(kv.device)].cpu().numpy()   # (nb, H, d, bs)
    sc = kv.scales[layer, idx.to(kv.device)].cpu().numpy()                      # (nb, 2)
    k = e4m3_decode(kc) * sc[:, 0, None, None, None]
    v = e4m3_decode(vc) * sc[:, 1, None, None, None]
    k = np.transpose(k, (0, 2, 1, 3)).reshape(-1, kv.num_kv_heads, kv.head_dim)[:n]
    v = np.transpose(v, (0, 3, 1, 2)).reshape(-1, kv.num_kv_heads, kv.head_dim)[:n]
    return torch.from_numpy(k.astype(np.float32)), torch.from_numpy(v.astype(np.float32))


def test_long_context_fp8_at_32768_keys(cuda):
    B, ctx, C, Hq, Hkv, d, bs = 16, 32768, 9, 14, 2, 64, 16
    g = torch.Generator(device=cuda).manual_seed(5)
    cap = B * (-(-(ctx + C) // bs)) + 16
    kv = PagedKVCache(1, Hkv, d, cap, bs, cuda, torch.float8_e4m3fn, max_seqs=B,
                      max_blocks_per_seq=-(-(ctx + C) // bs) + 1)
    for s in range(B):
        kv.add_sequence(s)
        k = torch.randn(1, ctx, Hkv, d, generator=g, device=cuda).to(torch.bfloat16)
        v = torch.randn(1, ctx, Hkv, d, generator=g, device=cuda).to(torch.bfloat16)
        kv.write_block(0, [s], [0], k, v)
    kn = torch.randn(B, C, Hkv, d, generator=g, device=cuda).to(torch.bfloat16)
    vn = torch.randn(B, C, Hkv, d, generator=g, device=cuda).to(torch.bfloat16)
    kv.write_block(0, list(range(B)), [ctx] * B, kn, vn)
    q = torch.randn(B, C, Hq, d, generator=g, device=cuda).to(torch.bfloat16)
    out = verify_attention(q, kv, 0, list(range(B)), [ctx] * B, ctx + C)
    keys, values = zip(*[_decoded_context(kv, 0, s, ctx + C) for s in range(B)])
    want = ref_attn.extend_attention_dense(q.cpu(), list(keys), list(values), [ctx] * B, Hq)
    _bf16_check(out, want)
