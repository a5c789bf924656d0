"""GPU parity of the fp8 (e4m3) KV pool with the oracle.

Appends into an fp8 pool must leave exactly the oracle's codes (K pages and
transposed V pages) and per-(layer, block, K | V) scales, and the same tables,
lengths and free list, over random traces with overwrites, growth of a
block's scale, rewinds and reuse of freed blocks. Verify attention and
gather_ctx on the fp8 pool are compared with the oracle run on the dequantised
K/V (the reference path on ``decode(code) * scale``): within 1e-5 for fp32
queries, and for bf16 within the bf16 bar of the attention tests (relative L2
error per sequence <= 2e-3, every element within one bf16 ulp + 2e-3 * max).
"""

from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from engine.attention import gather_ctx, verify_attention
from engine.kv import BlockExhaustedError, PagedKVCache
from oracle import attention as ref_attn
from oracle.kv_fp8 import Fp8PagedKVCache, e4m3_decode
from oracle.kv_pool import BlockExhaustedError as RefExhausted
from test_gpu_attention import _bf16_check

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn


def _codes(gpu: PagedKVCache):
    k = gpu.k_pool.view(torch.uint8).permute(0, 1, 3, 2, 4).cpu()   # (L, cap, bs, H, d)
    v = gpu.v_pool.view(torch.uint8).permute(0, 1, 4, 2, 3).cpu()   # (L, cap, bs, H, d)
    return k, v


def _same(gpu: PagedKVCache, cpu: Fp8PagedKVCache):
    assert gpu.block_tables == cpu.block_tables
    assert gpu.seq_lengths == cpu.seq_lengths
    assert gpu.allocator.free_list() == cpu.allocator.free_list
    k, v = _codes(gpu)
    assert torch.equal(k, cpu.k) and torch.equal(v, cpu.v)
    assert np.array_equal(gpu.scales.cpu().numpy().view(np.uint32), cpu.scales.view(np.uint32))


def test_append_encodes_like_torch(cuda):
    """A block whose largest element is 448 has scale 1: its codes are the
    e4m3 encodings of the inputs (ties, subnormals, the saturation edge)."""
    vals = e4m3_decode(np.arange(0, 0x7F, dtype=np.uint8)).astype(np.float64)
    mids = ((vals[:-1] + vals[1:]) / 2).astype(np.float32)
    rng = np.random.default_rng(0)
    H, d, bs = 2, 64, 16
    n = bs * H * d
    x = np.concatenate([mids, -mids, rng.uniform(-448, 448, n).astype(np.float32),
                        rng.uniform(-0.03, 0.03, n).astype(np.float32)])[:n - 1]
    x = np.concatenate([np.array([448.0], dtype=np.float32), x]).reshape(1, bs, H, d)
    gpu = PagedKVCache(1, H, d, 4, bs, cuda, FP8)
    cpu = Fp8PagedKVCache(1, H, d, 4, bs)
    for kv in (gpu, cpu):
        kv.add_sequence(0)
    t = torch.from_numpy(x)
    gpu.write_block(0, [0], [0], t.to(cuda), (-t).to(cuda))
    cpu.write_block(0, [0], [0], t, -t)
    assert float(gpu.scales[0, gpu.block_tables[0][0], 0]) == 1.0
    want = torch.from_numpy(x).to(FP8).view(torch.uint8)[0]   # torch's own conversion
    k, _ = _codes(gpu)
    assert torch.equal(k[0, gpu.block_tables[0][0]], want)
    _same(gpu, cpu)


def _trace(cuda, seed, dtype=torch.float32, n_ops=80, H=2, d=16, bs=4, cap=24, layers=2, n_seq=5):
    rng = random.Random(seed)
    g = torch.Generator().manual_seed(seed)
    gpu = PagedKVCache(layers, H, d, cap, bs, cuda, FP8)
    cpu = Fp8PagedKVCache(layers, H, d, cap, bs)
    for s in range(n_seq):
        gpu.add_sequence(s)
        cpu.add_sequence(s)
    for _ in range(n_ops):
        op = rng.random()
        if op < 0.55:
            sids = rng.sample(range(n_seq), rng.randint(1, 3))
            chunk = rng.randint(1, 7)
            starts = [max(0, cpu.seq_lengths[s] - rng.randint(0, 3)) for s in sids]
            layer = rng.randrange(layers)
            scale = 10.0 ** rng.uniform(-3, 2)
            kn = (torch.randn(len(sids), chunk, H, d, generator=g) * scale).to(dtype)
            vn = (torch.randn(len(sids), chunk, H, d, generator=g) * scale).to(dtype)
            err_g = err_c = False
            try:
                gpu.write_block(layer, sids, starts, kn.to(cuda), vn.to(cuda))
            except BlockExhaustedError:
                err_g = True
            try:
                cpu.write_block(layer, sids, starts, kn, vn)
            except RefExhausted:
                err_c = True
            assert err_g == err_c
        elif op < 0.85:
            s = rng.randrange(n_seq)
            n = rng.randint(0, cpu.seq_lengths[s])
            gpu.truncate(s, n)
            cpu.truncate(s, n)
        else:
            s = rng.randrange(n_seq)
            gpu.clear(s)
            cpu.clear(s)
        _same(gpu, cpu)
    return gpu, cpu


@pytest.mark.parametrize("seed", range(3))
def test_fp8_trace_matches_oracle(cuda, seed):
    _trace(cuda, seed)


def test_fp8_trace_bf16_inputs_and_wide_heads(cuda):
    _trace(cuda, 11, dtype=torch.bfloat16, n_ops=40, H=2, d=64, bs=16, cap=12)


def test_fp8_layers_of_one_round_allocate_once(cuda):
    """write_block_device: the first layer allocates (and zeroes the scales of
    the new blocks in every layer), the others quantise into the same blocks."""
    H, d, bs, layers = 2, 64, 16, 3
    gpu = PagedKVCache(layers, H, d, 32, bs, cuda, FP8)
    cpu = Fp8PagedKVCache(layers, H, d, 32, bs)
    g = torch.Generator().manual_seed(2)
    for kv in (gpu, cpu):
        for s in range(3):
            kv.add_sequence(s)
    for layer in range(layers):
        p = torch.randn(3, 20, H, d, generator=g)
        gpu.write_block(layer, [0, 1, 2], [0, 0, 0], p.to(cuda), (p * 3).to(cuda))
        cpu.write_block(layer, [0, 1, 2], [0, 0, 0], p, p * 3)
    sids, starts = [2, 0, 1], [20, 20, 20]
    sid_t = torch.tensor(sids, dtype=torch.int32, device=cuda)
    st_t = torch.tensor(starts, dtype=torch.int32, device=cuda)
    for layer in range(layers):
        kn = torch.randn(3, 9, H, d, generator=g) * (layer + 1)
        vn = torch.randn(3, 9, H, d, generator=g)
        gpu.write_block_device(layer, sid_t, st_t, kn.to(cuda), vn.to(cuda), alloc=layer == 0)
        cpu.write_block(layer, sids, starts, kn, vn)
    _same(gpu, cpu)


@pytest.mark.parametrize("qdtype", [torch.float32, torch.bfloat16])
def test_fp8_attention_matches_oracle_on_dequantized_kv(cuda, qdtype):
    Hq, H, d, bs, C = 14, 2, 64, 16, 9
    lens = [37, 300, 1, 129]
    gpu = PagedKVCache(1, H, d, 96, bs, cuda, FP8)
    cpu = Fp8PagedKVCache(1, H, d, 96, bs)
    g = torch.Generator().manual_seed(4)
    for s, L in enumerate(lens):
        gpu.add_sequence(s)
        cpu.add_sequence(s)
        k = torch.randn(1, L, H, d, generator=g)
        v = torch.randn(1, L, H, d, generator=g)
        gpu.write_block(0, [s], [0], k.to(cuda), v.to(cuda))
        cpu.write_block(0, [s], [0], k, v)
    kn = torch.randn(4, C, H, d, generator=g)
    vn = torch.randn(4, C, H, d, generator=g)
    sids = [0, 1, 2, 3]
    gpu.write_block(0, sids, lens, kn.to(cuda), vn.to(cuda))
    cpu.write_block(0, sids, lens, kn, vn)
    _same(gpu, cpu)
    q = torch.randn(4, C, Hq, d, generator=g).to(qdtype)
    out = verify_attention(q.to(cuda), gpu, 0, sids, lens, max(lens) + C).float().cpu()
    want = ref_attn.paged_attention_extend(q.float(), cpu.dequantized(), 0, sids, lens, Hq)
    if qdtype == torch.float32:
        torch.testing.assert_close(out, want, atol=1e-5, rtol=1e-5)
    else:
        _bf16_check(out, want)
    # gather_ctx returns the dequantised context
    for s, L in enumerate(lens):
        got = gather_ctx(gpu, 0, s, L + C).cpu()
        want_ctx = ref_attn.gather_ctx(cpu.dequantized(), 0, s, L + C)
        assert torch.equal(got, want_ctx)


def _fp8_pool_with(cuda, lens, H, d, bs, C, seed):
    cap = sum(-(-(L + C) // bs) for L in lens) + 4
    gpu = PagedKVCache(1, H, d, cap, bs, cuda, FP8, max_seqs=len(lens))
    cpu = Fp8PagedKVCache(1, H, d, cap, bs)
    g = torch.Generator().manual_seed(seed)
    for s, L in enumerate(lens):
        gpu.add_sequence(s)
        cpu.add_sequence(s)
        k = torch.randn(1, L, H, d, generator=g).to(torch.bfloat16)
        v = torch.randn(1, L, H, d, generator=g).to(torch.bfloat16)
        gpu.write_block(0, [s], [0], k.to(cuda), v.to(cuda))
        cpu.write_block(0, [s], [0], k, v)
    sids = list(range(len(lens)))
    kn = torch.randn(len(lens), C, H, d, generator=g).to(torch.bfloat16)
    vn = torch.randn(len(lens), C, H, d, generator=g).to(torch.bfloat16)
    gpu.write_block(0, sids, lens, kn.to(cuda), vn.to(cuda))
    cpu.write_block(0, sids, lens, kn, vn)
    return gpu, cpu, g


@pytest.mark.parametrize("Hq,H,d,C,lens", [
    (14, 2, 64, 9, [2000, 37, 700, 1, 129, 1500]),     # head_dim 64, pieces split across workgroups
    (12, 2, 128, 6, [3000, 256, 1, 999, 4000, 17]),    # head_dim 128
    (12, 2, 128, 6, [(i * 37) % 211 + 1 for i in range(140)]),  # segments outnumber workgroups
    (14, 2, 64, 1, [(i * 997) % 3001 + 1 for i in range(32)]),  # draft decode: one row, G = 7
])
def test_fp8_mfma_attention_matches_oracle(cuda, Hq, H, d, C, lens):
    """bf16 queries over an fp8 pool take the MFMA path: codes converted to
    bf16 in registers, the K scale on the scores and the V scale on P."""
    gpu, cpu, g = _fp8_pool_with(cuda, lens, H, d, 16, C, 9)
    q = torch.randn(len(lens), C, Hq, d, generator=g).to(torch.bfloat16)
    sids = list(range(len(lens)))
    out = verify_attention(q.to(cuda), gpu, 0, sids, lens, max(lens) + C).float().cpu()
    want = ref_attn.paged_attention_extend(q.float(), cpu.dequantized(), 0, sids, lens, Hq)
    _bf16_check(out, want)


def _fp8_pool_scaled(cuda, lens, H, d, C, v_mag, seed):
    """An fp8 pool whose V rows of sequence s are N(0, 1) times v_mag(s, pos):
    the block scales (amax / 448) then cover zero, tiny and huge values."""
    cap = sum(-(-(L + C) // 16) for L in lens) + 4
    gpu = PagedKVCache(1, H, d, cap, 16, cuda, FP8, max_seqs=len(lens))
    cpu = Fp8PagedKVCache(1, H, d, cap, 16)
    g = torch.Generator().manual_seed(seed)
    for s, L in enumerate(lens):
        gpu.add_sequence(s)
        cpu.add_sequence(s)
        k = torch.randn(1, L + C, H, d, generator=g)
        mag = torch.tensor([v_mag(s, p) for p in range(L + C)], dtype=torch.float32).view(1, L + C, 1, 1)
        v = torch.randn(1, L + C, H, d, generator=g) * mag
        k, v = k.to(torch.bfloat16), v.to(torch.bfloat16)
        gpu.write_block(0, [s], [0], k.to(cuda), v.to(cuda))
        cpu.write_block(0, [s], [0], k, v)
    return gpu, cpu, g


@pytest.mark.parametrize("d,Hq,C", [(64, 14, 9), (128, 12, 6), (64, 14, 1), (128, 16, 7)])
def test_fp8_attention_over_extreme_v_scales(cuda, d, Hq, C):
    """V block scales of every class the fp16 P V path distinguishes: tiny
    (below 2^-15: V amax ~1e-4 and ~1e-7), zero (all-zero V blocks), ordinary,
    huge (2^8 and above: V amax ~1e6 and ~3e9, where O is rescaled around the
    page), and all of them mixed block by block within one sequence. Compared
    with the oracle on the dequantised K/V at the bf16 bar."""
    mags = [1e-4, 0.0, 1.0, 1e6, 3e9, 1e-7]

    def v_mag(s, p):
        if s < len(mags):
            return mags[s]
        return mags[(p // 16 + s) % len(mags)]  # mixed: the class changes every block

    lens = [700, 333, 1500, 64, 900, 2100, 1234, 3000]
    gpu, cpu, g = _fp8_pool_scaled(cuda, lens, 2, d, C, v_mag, seed=d + C)
    scales_v = gpu.scales[0, :, 1].cpu()
    assert float(scales_v.max()) >= 2.0 ** 8 and float(scales_v[scales_v > 0].min()) < 2.0 ** -15
    assert bool((scales_v == 0).any())
    q = torch.randn(len(lens), C, Hq, d, generator=g).to(torch.bfloat16)
    sids = list(range(len(lens)))
    out = verify_attention(q.to(cuda), gpu, 0, sids, [L for L in lens], max(lens) + C).float().cpu()
    want = ref_attn.paged_attention_extend(q.float(), cpu.dequantized(), 0, sids, lens, Hq)
    assert torch.isfinite(out).all()
    for b in range(len(lens)):
        if float(want[b].abs().max()) == 0.0:  # all-zero V: the output is exactly zero
            assert float(out[b].abs().max()) == 0.0, b
        else:
            _bf16_check(out[b:b + 1], want[b:b + 1])
