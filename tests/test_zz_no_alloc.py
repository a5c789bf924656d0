"""spv_verify_attn_static -- verify attention with no allocation -- against spv_verify_attn.

The allocation-free entry point runs the same kernels with their counters and
partials in the library's static device array. Its outputs must equal the
workspace entry point's bit for bit (the merges add partials in a fixed order),
on two calls in a row where the second is smaller (fewer sequences, shorter
contexts: the array keeps the first call's partials and its counters must be
back at zero), on the MFMA path (bf16) and the VALU path (fp32, split
contexts). A call whose workspace exceeds the array is rejected before
anything is enqueued.
"""

from __future__ import annotations

import math

import pytest
import torch

from engine import _hip
from engine.attention import verify_attention
from engine.kv import PagedKVCache

pytestmark = pytest.mark.gpu


def _static_fn():
    return _hip.lib().spv_verify_attn_static  # typed by engine._hip.SIGNATURES


def _pool(cuda, lens, C, Hkv, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    bs = 16
    cap = sum(-(-(L + C) // bs) for L in lens) + 8
    kv = PagedKVCache(1, Hkv, d, cap, bs, cuda, dtype, max_seqs=len(lens))
    kv.allocator.load_free_list(torch.randperm(cap, generator=g).to(torch.int32))
    for s, L in enumerate(lens):
        kv.add_sequence(s)
        kv.write_block(0, [s], [0], torch.randn(1, L + C, Hkv, d, generator=g).to(dtype).to(cuda),
                       torch.randn(1, L + C, Hkv, d, generator=g).to(dtype).to(cuda))
    return kv, g


def _static_attention(q, kv, lens, max_ctx):
    B, C, Hq, d = q.shape
    out = torch.full_like(q, float("nan"))
    sid = torch.arange(B, dtype=torch.int32, device=q.device)
    st = torch.tensor(lens, dtype=torch.int32, device=q.device)
    rc = _static_fn()(out.data_ptr(), q.data_ptr(), _hip.dtype_code(q.dtype), kv.k_pool.data_ptr(),
                      kv.v_pool.data_ptr(), kv._dt, None, kv.tables_dev.data_ptr(), kv.max_blocks_per_seq,
                      sid.data_ptr(), st.data_ptr(), kv.lens_dev.data_ptr(), kv.allocator.ctr.data_ptr(), B, C,
                      Hq, kv.num_kv_heads, d, kv.block_size, 0, kv.allocator.capacity, max_ctx,
                      1.0 / math.sqrt(d), None)
    return rc, out


@pytest.mark.parametrize("dtype,d,Hq,first,second", [
    # MFMA path: the Qwen2.5-1.5B-shaped verify batch, then a smaller one
    (torch.bfloat16, 128, 12, (32, 256, 4096), (8, 16, 900)),
    # MFMA path over an fp16 pool with fp16 queries, head_dim 64
    (torch.float16, 64, 14, (40, 256, 3000), (5, 16, 700)),
    # VALU path (fp32 pool), contexts split across workgroups
    (torch.float32, 64, 4, (6, 100, 1500), (3, 1, 300)),
])
def test_static_matches_workspace_entry_point_twice(cuda, dtype, d, Hq, first, second):
    C, Hkv = 6, 2
    for n, lo, hi in (first, second):
        g = torch.Generator().manual_seed(n + hi)
        lens = torch.randint(lo, hi + 1, (n,), generator=g).tolist()
        kv, g = _pool(cuda, lens, C, Hkv, d, dtype, seed=n)
        q = torch.randn(n, C, Hq, d, generator=g).to(dtype).to(cuda)
        want = verify_attention(q, kv, 0, list(range(n)), lens, max(lens) + C)
        rc, got = _static_attention(q, kv, lens, max(lens) + C)
        torch.cuda.synchronize()
        assert rc == _hip.SPV_OK
        assert torch.equal(got, want)
        assert kv.seq_lengths == [L + C for L in lens]  # nothing flagged


def test_static_rejects_a_workspace_beyond_its_array(cuda):
    # fp32 queries (VALU path) over 64 sequences of up to 65,536 keys need
    # ~1 GB of split partials, far beyond the static array.
    # every sequence holds its chunk, so the inputs are valid even if launched
    kv, g = _pool(cuda, [0] * 64, 6, 2, 128, torch.float32, seed=1)
    max_ctx = 65536
    assert _hip.lib().spv_verify_attn_workspace_bytes(64, 6, 12, 2, 128, 16, max_ctx) > \
        _hip.lib().spv_verify_attn_static_max_bytes()
    kv._grow_width(-(-max_ctx // 16))
    q = torch.zeros(64, 6, 12, 128, device=cuda)
    rc, out = _static_attention(q, kv, [0] * 64, max_ctx)
    torch.cuda.synchronize()
    assert rc == _hip.SPV_ERR_WORKSPACE
    assert bool(torch.isnan(out).all())  # nothing was enqueued
