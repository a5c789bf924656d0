"""GPU parity of the device KV pool against the oracle (bit-exact).

The reference's own KV tests (tests/test_kv.py:44-183, tests/test_spec_accept.py:
76-98) run unchanged against ``engine.kv`` on the GPU; then block tables, sequence
lengths, the free list (bottom -> top) and stored K/V are compared with the
oracle after scripted and random operation traces, including pool exhaustion,
the already-free slow path, and the Qwen2.5-1.5B-shaped workload at its full
65,536-block pool (random-permutation tables, append 6 tokens, rewind to L+i).
"""

from __future__ import annotations

import random

import pytest
import torch

from engine.attention import gather_ctx
from engine.kv import BlockAllocator, BlockExhaustedError, PagedKVCache
from oracle import kv_pool as ref

pytestmark = pytest.mark.gpu


def _kv(dev, block_size=4, capacity=8):
    return PagedKVCache(2, 2, 8, capacity, block_size, dev, torch.float32)


def _vec(dev, fill=1.0):
    return torch.full((2, 8), fill, dtype=torch.float32, device=dev)


def _same_state(gpu: PagedKVCache, cpu: ref.PagedKVCache):
    assert gpu.block_tables == cpu.block_tables
    assert gpu.seq_lengths == cpu.seq_lengths
    assert gpu.allocator.free_list() == cpu.allocator.free_list
    assert gpu.num_allocated_blocks == cpu.num_allocated_blocks


# ------------------------------------------------- reference tests, on the GPU
def test_allocator_alloc_free_roundtrip(cuda):
    a = BlockAllocator(4, cuda, torch.float32)
    blocks = [a.alloc() for _ in range(4)]
    assert sorted(blocks) == [0, 1, 2, 3] and blocks[0] == 3
    assert a.num_allocated == 4
    a.free(blocks[0])
    a.free(blocks[1])
    assert a.num_allocated == 2
    blocks.extend([a.alloc(), a.alloc()])
    assert a.num_allocated == 4


def test_allocator_exhaustion_raises(cuda):
    a = BlockAllocator(2, cuda, torch.float32)
    a.alloc()
    a.alloc()
    with pytest.raises(BlockExhaustedError):
        a.alloc()
    a.free(0)
    assert a.alloc() == 0


def test_allocator_free_twice_is_idempotent(cuda):
    a = BlockAllocator(3, cuda, torch.float32)
    b = a.alloc()
    a.free(b)
    a.free(b)
    assert a.num_allocated == 0
    assert a.free_list() == [0, 1, 2]


def test_write_allocates_blocks_on_demand(cuda):
    kv = _kv(cuda)
    kv.add_sequence(0)
    kv.write(0, 0, 0, _vec(cuda), _vec(cuda))
    assert kv.seq_lengths[0] == 1 and kv.num_allocated_blocks == 1
    kv.write(0, 0, 2, _vec(cuda), _vec(cuda))
    assert kv.num_allocated_blocks == 1 and kv.seq_lengths[0] == 3
    kv.write(0, 0, 4, _vec(cuda), _vec(cuda))
    assert kv.num_allocated_blocks == 2 and len(kv.block_tables[0]) == 2


def test_write_out_of_order_extends_length(cuda):
    kv = _kv(cuda)
    kv.add_sequence(0)
    kv.write(0, 0, 3, _vec(cuda, 3.0), _vec(cuda, 3.0))
    assert kv.seq_lengths[0] == 4 and kv.logical_tokens == 4


def test_gather_concatenates_blocks_in_order(cuda):
    kv = _kv(cuda)
    kv.add_sequence(0)
    for pos in range(9):
        kv.write(0, 0, pos, _vec(cuda, float(pos)), _vec(cuda, -float(pos)))
    stacked = gather_ctx(kv, 0, 0, 9)
    assert stacked.shape == (2, 9, 2, 8)
    assert torch.equal(stacked[0][3], torch.full((2, 8), 3.0, device=cuda))
    assert torch.equal(stacked[1][8], torch.full((2, 8), -8.0, device=cuda))


def test_truncate_rollback_frees_blocks(cuda):
    kv = _kv(cuda)
    kv.add_sequence(0)
    kv.add_sequence(1)
    for pos in range(10):
        kv.write(0, 0, pos, _vec(cuda), _vec(cuda))
    before = kv.num_allocated_blocks
    assert before >= 3
    kv.truncate(0, 3)
    assert kv.seq_lengths[0] == 3 and len(kv.block_tables[0]) == 1
    assert kv.num_allocated_blocks < before
    kv.write(0, 1, 4, _vec(cuda), _vec(cuda))
    assert kv.seq_lengths[1] == 5 and len(kv.block_tables[1]) == 2


def test_truncate_rewound_sequence_writes_identically(cuda):
    kv = _kv(cuda)
    kv.add_sequence(0)
    for pos in range(8):
        kv.write(0, 0, pos, _vec(cuda, pos + 0.5), _vec(cuda))
    kv.truncate(0, 2)
    for pos in range(2, 8):
        kv.write(0, 0, pos, _vec(cuda, pos + 0.5), _vec(cuda))
    assert torch.equal(gather_ctx(kv, 0, 0, 8)[0][5], torch.full((2, 8), 5.5, device=cuda))


def test_clear_frees_all_blocks(cuda):
    kv = _kv(cuda)
    kv.add_sequence(0)
    for pos in range(10):
        kv.write(0, 0, pos, _vec(cuda), _vec(cuda))
    kv.clear(0)
    assert kv.num_allocated_blocks == 0 and kv.seq_lengths[0] == 0 and kv.block_tables[0] == []


def test_reset_returns_cache_to_virgin_state(cuda):
    kv = _kv(cuda)
    kv.add_sequence(0)
    kv.add_sequence(1)
    for pos in range(6):
        kv.write(0, 0, pos, _vec(cuda), _vec(cuda))
    kv.write(0, 1, 1, _vec(cuda), _vec(cuda))
    assert kv.num_sequences == 2 and kv.num_allocated_blocks > 0
    k_before = kv.k_pool
    kv.reset()
    assert kv.num_sequences == 0 and kv.num_allocated_blocks == 0
    assert kv.k_pool is k_before


def test_block_utilization_metric(cuda):
    kv = _kv(cuda)
    kv.add_sequence(0)
    kv.write(0, 0, 0, _vec(cuda), _vec(cuda))
    assert kv.block_utilization == pytest.approx(0.25)
    kv.write(0, 0, 1, _vec(cuda), _vec(cuda))
    assert kv.block_utilization == pytest.approx(0.5)


def test_truncate_releases_physical_blocks(cuda):
    kv = PagedKVCache(2, 2, 8, 32, 4, cuda, torch.float32)
    kv.add_sequence(0)
    for pos in range(10):
        kv.write(0, 0, pos, torch.randn(2, 8, device=cuda), torch.randn(2, 8, device=cuda))
    full = kv.num_allocated_blocks
    kv.truncate(0, 4)
    assert kv.seq_lengths[0] == 4
    assert full - kv.num_allocated_blocks == 2 and kv.num_allocated_blocks == 1


def test_cpu_device_is_refused():
    with pytest.raises(RuntimeError):
        PagedKVCache(1, 1, 8, 4, 4, torch.device("cpu"), torch.float32)


# ----------------------------------------------------- oracle parity traces
def test_lifo_order_and_exhaustion_match_oracle(cuda):
    gpu = PagedKVCache(1, 1, 2, 8, 2, cuda, torch.float32)
    cpu = ref.PagedKVCache(1, 1, 2, 8, 2, store=False)
    for kv in (gpu, cpu):
        kv.add_sequence(0)
        kv.add_sequence(1)
    k = torch.zeros(2, 5, 1, 2, device=cuda)
    gpu.write_block(0, [0, 1], [0, 0], k, k)
    cpu.write_block(0, [0, 1], [0, 0], None, None, chunk=5)
    _same_state(gpu, cpu)
    assert gpu.block_tables == [[7, 6, 5], [4, 3, 2]]
    gpu.truncate(0, 1)
    cpu.truncate(0, 1)
    gpu.clear(1)
    cpu.clear(1)
    _same_state(gpu, cpu)
    # exhaustion mid-batch: seq 0 needs 4 more blocks, seq 1 needs 5, 7 are free
    assert gpu.allocator.num_free == 7
    k = torch.zeros(2, 9, 1, 2, device=cuda)
    with pytest.raises(BlockExhaustedError):
        gpu.write_block(0, [0, 1], [1, 0], k, k)
    with pytest.raises(ref.BlockExhaustedError):
        cpu.write_block(0, [0, 1], [1, 0], None, None, chunk=9)
    _same_state(gpu, cpu)
    assert gpu.seq_lengths == [10, 6] and len(gpu.block_tables[1]) == 3


def _random_trace(cuda, seed, n_ops=120, bs=4, cap=40, n_seq=6, dtype=torch.float32):
    rng = random.Random(seed)
    H, d = 2, 8
    gpu = PagedKVCache(2, H, d, cap, bs, cuda, dtype)
    cpu = ref.PagedKVCache(2, H, d, cap, bs, dtype=dtype)
    for s in range(n_seq):
        gpu.add_sequence(s)
        cpu.add_sequence(s)
    g = torch.Generator().manual_seed(seed)
    for _ in range(n_ops):
        op = rng.random()
        if op < 0.45:
            sids = rng.sample(range(n_seq), rng.randint(1, 3))
            chunk = rng.randint(1, 6)
            starts = [max(0, cpu.seq_lengths[s] - rng.randint(0, 2)) for s in sids]
            layer = rng.randrange(2)
            kn = torch.randn(len(sids), chunk, H, d, generator=g).to(dtype)
            vn = torch.randn(len(sids), chunk, H, d, generator=g).to(dtype)
            err_g = err_c = False
            try:
                gpu.write_block(layer, sids, starts, kn.to(cuda), vn.to(cuda))
            except BlockExhaustedError:
                err_g = True
            try:
                cpu.write_block(layer, sids, starts, kn, vn)
            except ref.BlockExhaustedError:
                err_c = True
            assert err_g == err_c
        elif op < 0.8:
            sids = rng.sample(range(n_seq), rng.randint(1, 4))
            new = [rng.randint(0, cpu.seq_lengths[s]) if rng.random() < 0.8 else -1 for s in sids]
            fin = [1 if rng.random() < 0.2 else 0 for _ in sids]
            gpu.rewind(sids, new, fin)
            for s, n, f in zip(sids, new, fin):
                if n >= 0:
                    cpu.truncate(s, n)
                if f:
                    cpu.clear(s)
        elif op < 0.9:
            s = rng.randrange(n_seq)
            n = rng.randint(0, cpu.seq_lengths[s])
            gpu.truncate(s, n)
            cpu.truncate(s, n)
        else:
            s = rng.randrange(n_seq)
            gpu.clear(s)
            cpu.clear(s)
        _same_state(gpu, cpu)
    return gpu, cpu


@pytest.mark.parametrize("seed", range(4))
def test_random_trace_matches_oracle(cuda, seed):
    gpu, cpu = _random_trace(cuda, seed)
    # stored K/V of every live position, through gather_ctx and key/value_map
    for layer in range(2):
        for s in range(cpu.num_sequences):
            n = cpu.seq_lengths[s]
            if n == 0:
                continue
            got = gather_ctx(gpu, layer, s, n).cpu()
            want = torch.stack([torch.cat([cpu.k[layer, b] for b in cpu.block_tables[s]])[:n],
                                torch.cat([cpu.v[layer, b] for b in cpu.block_tables[s]])[:n]])
            assert torch.equal(got, want)
        phys = list(range(cpu.allocator.capacity))
        assert torch.equal(gpu.key_map(layer, phys).cpu(), cpu.key_map(layer, phys))
        assert torch.equal(gpu.value_map(layer, phys).cpu(), cpu.value_map(layer, phys))


def test_bf16_trace_matches_oracle(cuda):
    gpu, cpu = _random_trace(cuda, 99, n_ops=60, dtype=torch.bfloat16)
    phys = list(range(cpu.allocator.capacity))
    assert torch.equal(gpu.key_map(1, phys).cpu(), cpu.key_map(1, phys))
    assert torch.equal(gpu.value_map(1, phys).cpu(), cpu.value_map(1, phys))


def test_already_free_block_takes_exact_slow_path(cuda):
    gpu = PagedKVCache(1, 1, 2, 12, 2, cuda, torch.float32)
    cpu = ref.PagedKVCache(1, 1, 2, 12, 2, store=False)
    for kv in (gpu, cpu):
        kv.add_sequence(0)
        kv.add_sequence(1)
    k = torch.zeros(2, 6, 1, 2, device=cuda)
    gpu.write_block(0, [0, 1], [0, 0], k, k)
    cpu.write_block(0, [0, 1], [0, 0], None, None, chunk=6)
    victim = cpu.block_tables[0][2]
    gpu.allocator.free(victim)      # freed while still listed in a table
    cpu.allocator.free(victim)
    gpu.rewind([0, 1], [1, 3], [0, 1])
    cpu.truncate(0, 1)
    cpu.truncate(1, 3)
    cpu.clear(1)
    gpu._sync_pushes()
    _same_state(gpu, cpu)
    assert int(gpu.allocator.ctr[2].item()) == 1  # one call took the sequential path


def test_already_free_block_in_a_short_truncation_takes_exact_slow_path(cuda):
    # truncations only, a few blocks each: the path that frees the tail blocks
    # loaded with the block counts must detect the already-free one too
    gpu = PagedKVCache(1, 1, 2, 12, 2, cuda, torch.float32)
    cpu = ref.PagedKVCache(1, 1, 2, 12, 2, store=False)
    for kv in (gpu, cpu):
        kv.add_sequence(0)
        kv.add_sequence(1)
    k = torch.zeros(2, 6, 1, 2, device=cuda)
    gpu.write_block(0, [0, 1], [0, 0], k, k)
    cpu.write_block(0, [0, 1], [0, 0], None, None, chunk=6)
    victim = cpu.block_tables[0][2]
    gpu.allocator.free(victim)
    cpu.allocator.free(victim)
    gpu.rewind([0, 1], [1, 3], [0, 0])
    cpu.truncate(0, 1)
    cpu.truncate(1, 3)
    gpu._sync_pushes()
    _same_state(gpu, cpu)
    assert int(gpu.allocator.ctr[2].item()) == 1
    # and without the victim the same rewind takes the fast path
    gpu.rewind([0, 1], [0, 1], [0, 0])
    cpu.truncate(0, 0)
    cpu.truncate(1, 1)
    gpu._sync_pushes()
    _same_state(gpu, cpu)
    assert int(gpu.allocator.ctr[2].item()) == 1


def _qwen15_pool(seed=0, B=32, cap=65536, bs=16, C=6):
    """Random-permutation tables over a 64k-block pool, lengths U[256, 4096]."""
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(256, 4097, (B,), generator=g).tolist()
    perm = torch.randperm(cap, generator=g).tolist()
    tables, pos = [], 0
    for L in lens:
        n = -(-L // bs)
        tables.append(perm[pos: pos + n])
        pos += n
    free = perm[pos:]
    return lens, tables, free


def test_qwen15_shaped_append_and_rewind_match_oracle(cuda):
    B, cap, bs, C = 32, 65536, 16, 6
    lens, tables, free = _qwen15_pool()
    gpu = PagedKVCache(1, 2, 128, cap, bs, cuda, torch.bfloat16, max_seqs=B)
    cpu = ref.PagedKVCache(1, 2, 128, cap, bs, store=False)
    gpu.load_state(tables, lens, free)
    cpu.load_state(tables, lens, free)
    _same_state(gpu, cpu)
    k = torch.randn(B, C, 2, 128, device=cuda, dtype=torch.bfloat16)
    gpu.write_block(0, list(range(B)), lens, k, k)
    cpu.write_block(0, list(range(B)), lens, None, None, chunk=C)
    _same_state(gpu, cpu)
    g = torch.Generator().manual_seed(1)
    acc = torch.randint(0, C, (B,), generator=g).tolist()  # i accepted drafts
    new_lens = [L + i + 1 for L, i in zip(lens, acc)]
    fin = [1 if b % 7 == 3 else 0 for b in range(B)]
    gpu.rewind(list(range(B)), new_lens, fin)
    for b in range(B):
        cpu.truncate(b, new_lens[b])
        if fin[b]:
            cpu.clear(b)
    _same_state(gpu, cpu)


def test_rewind_device_inputs_refresh_mirrors(cuda):
    gpu = PagedKVCache(1, 1, 2, 32, 4, cuda, torch.float32)
    cpu = ref.PagedKVCache(1, 1, 2, 32, 4, store=False)
    for kv in (gpu, cpu):
        for s in range(3):
            kv.add_sequence(s)
    k = torch.zeros(3, 9, 1, 2, device=cuda)
    gpu.write_block(0, [0, 1, 2], [0, 0, 0], k, k)
    cpu.write_block(0, [0, 1, 2], [0, 0, 0], None, None, chunk=9)
    sid = torch.tensor([2, 0, 1], dtype=torch.int32, device=cuda)
    nl = torch.tensor([3, -1, 5], dtype=torch.int32, device=cuda)
    fin = torch.tensor([0, 1, 1], dtype=torch.int32, device=cuda)
    gpu.rewind_device(sid, nl, fin)
    cpu.truncate(2, 3)
    cpu.clear(0)
    cpu.truncate(1, 5)
    cpu.clear(1)
    _same_state(gpu, cpu)


@pytest.mark.parametrize("dtype,chunk", [(torch.bfloat16, 6), (torch.bfloat16, 20), (torch.float32, 7)])
def test_append_into_filled_pool_touches_only_the_chunk(cuda, dtype, chunk):
    """Block 16, d 128: V rows are rebuilt whole (old keys read back); every
    pool element outside the appended positions must be left as it was."""
    B, cap, bs, H, d = 12, 256, 16, 2, 128
    g = torch.Generator().manual_seed(11)
    lens = torch.randint(0, 70, (B,), generator=g).tolist()
    perm = torch.randperm(cap, generator=g).tolist()
    tables, pos = [], 0
    for L in lens:
        n = -(-L // bs)
        tables.append(perm[pos: pos + n])
        pos += n
    gpu = PagedKVCache(2, H, d, cap, bs, cuda, dtype, max_seqs=B)
    gpu.load_state(tables, lens, perm[pos:])
    cpu = ref.PagedKVCache(2, H, d, cap, bs, store=False)
    cpu.load_state(tables, lens, perm[pos:])
    # Every element of both layers holds a distinct-looking value beforehand.
    gpu.k_pool.copy_(torch.randn(gpu.k_pool.shape, generator=g).to(dtype))
    gpu.v_pool.copy_(torch.randn(gpu.v_pool.shape, generator=g).to(dtype))
    k0, v0 = gpu.k_pool.cpu().clone(), gpu.v_pool.cpu().clone()
    kn = torch.randn(B, chunk, H, d, generator=g).to(dtype)
    vn = torch.randn(B, chunk, H, d, generator=g).to(dtype)
    gpu.write_block(1, list(range(B)), lens, kn.to(cuda), vn.to(cuda))
    cpu.write_block(1, list(range(B)), lens, None, None, chunk=chunk)
    _same_state(gpu, cpu)
    # Expected pools: the initial contents with the chunk placed (V transposed per block).
    for b, L in enumerate(lens):
        for j in range(chunk):
            p = L + j
            blk = cpu.block_tables[b][p // bs]
            k0[1, blk, :, p % bs, :] = kn[b, j]
            v0[1, blk, :, :, p % bs] = vn[b, j]
    assert torch.equal(gpu.k_pool.cpu(), k0)
    assert torch.equal(gpu.v_pool.cpu(), v0)


@pytest.mark.parametrize("n_seq,blocks,truncate_to", [(40, 300, None), (1100, 2, 17), (24, 90, 33)])
def test_large_rewinds_match_oracle(cuda, n_seq, blocks, truncate_to):
    """Rewinds beyond the flattened path's limits (more than 8192 freed blocks,
    more than 1024 entries) and long clears mixed with truncates inside them."""
    bs = 16
    cap = n_seq * blocks + 64
    g = torch.Generator().manual_seed(n_seq)
    perm = torch.randperm(cap, generator=g).tolist()
    tables = [perm[i * blocks:(i + 1) * blocks] for i in range(n_seq)]
    lens = [blocks * bs - int(torch.randint(0, bs, (1,), generator=g)) for _ in range(n_seq)]
    free = perm[n_seq * blocks:]
    gpu = PagedKVCache(1, 1, 8, cap, bs, cuda, torch.float32, max_seqs=n_seq, max_blocks_per_seq=blocks)
    cpu = ref.PagedKVCache(1, 1, 8, cap, bs, store=False)
    gpu.load_state(tables, lens, free)
    cpu.load_state(tables, lens, free)
    sids = list(range(n_seq))
    if truncate_to is None:
        new, fin = [-1] * n_seq, [1] * n_seq
    else:
        new = [truncate_to + (s % 5) for s in sids]
        fin = [1 if s % 3 == 0 else 0 for s in sids]
    gpu.rewind(sids, new, fin)
    for s, nl, f in zip(sids, new, fin):
        if nl >= 0:
            cpu.truncate(s, nl)
        if f:
            cpu.clear(s)
    _same_state(gpu, cpu)


@pytest.mark.parametrize("exhaust", [False, True])
def test_later_layers_write_without_allocating(cuda, exhaust):
    """A verify round writes every layer of one chunk; only the first call
    allocates. Later layers (alloc=False) must store exactly what per-layer
    host-checked writes store, and after an exhaustion at the first layer they
    keep its verdict: the same sequences and positions are cut off."""
    H, d, bs = 2, 8, 2
    cap = 7 if exhaust else 16
    gpu = PagedKVCache(2, H, d, cap, bs, cuda, torch.float32)
    cpu = ref.PagedKVCache(2, H, d, cap, bs)
    for kv in (gpu, cpu):
        for s in range(3):
            kv.add_sequence(s)
    g = torch.Generator().manual_seed(4)
    k0 = torch.randn(3, 3, H, d, generator=g)
    gpu.write_block(0, [0, 1, 2], [0, 0, 0], k0.to(cuda), k0.to(cuda))
    cpu.write_block(0, [0, 1, 2], [0, 0, 0], k0, k0)
    gpu.write_block(1, [0, 1, 2], [0, 0, 0], k0.to(cuda), k0.to(cuda))
    cpu.write_block(1, [0, 1, 2], [0, 0, 0], k0, k0)
    sids, starts = [2, 0, 1], [3, 3, 1]
    kn = [torch.randn(3, 5, H, d, generator=g) for _ in range(2)]
    vn = [torch.randn(3, 5, H, d, generator=g) for _ in range(2)]
    sid_t = torch.tensor(sids, dtype=torch.int32, device=cuda)
    st_t = torch.tensor(starts, dtype=torch.int32, device=cuda)
    for layer in range(2):
        gpu.write_block_device(layer, sid_t, st_t, kn[layer].to(cuda), vn[layer].to(cuda), alloc=layer == 0)
    raised = False
    for layer in range(2):
        try:
            cpu.write_block(layer, sids, starts, kn[layer], vn[layer])
        except ref.BlockExhaustedError:
            raised = True  # the reference stops at the raise
            break
    assert raised == exhaust
    if exhaust:
        with pytest.raises(BlockExhaustedError):
            gpu.seq_lengths
    _same_state(gpu, cpu)
    if exhaust:
        # Sequence 2 (batch index 0) fails: 1 free block for 2 missing ones.
        # It writes positions 3..5; sequences 0 and 1 come after it and write
        # nothing. Layer 1 (written without allocating) holds its own data in
        # exactly the positions layer 0 wrote.
        assert cpu.seq_lengths == [3, 3, 6]
        for s in range(3):
            n = cpu.seq_lengths[s]
            got0 = gather_ctx(gpu, 0, s, n).cpu()
            want0 = torch.stack([torch.cat([cpu.k[0, b] for b in cpu.block_tables[s]])[:n],
                                 torch.cat([cpu.v[0, b] for b in cpu.block_tables[s]])[:n]])
            assert torch.equal(got0, want0)
            got1 = gather_ctx(gpu, 1, s, n).cpu()
            if s == 2:
                want1 = torch.stack([torch.cat([k0[2], kn[1][0, :3]]), torch.cat([k0[2], vn[1][0, :3]])])
            else:
                want1 = torch.stack([k0[s], k0[s]])
            assert torch.equal(got1, want1)
    else:
        for layer in range(2):
            for s in range(3):
                n = cpu.seq_lengths[s]
                got = gather_ctx(gpu, layer, s, n).cpu()
                want = torch.stack([torch.cat([cpu.k[layer, b] for b in cpu.block_tables[s]])[:n],
                                    torch.cat([cpu.v[layer, b] for b in cpu.block_tables[s]])[:n]])
                assert torch.equal(got, want)


@pytest.mark.parametrize("chunk,maxb", [(6, 3), (40, 12)])
def test_table_width_caps_a_device_append_and_reports_it(cuda, chunk, maxb):
    """A device-side append whose chunk needs more blocks than a table holds
    gets the blocks that fit, writes only the tokens inside them, and the next
    metadata query raises IndexError; the state equals the oracle's after the
    same writes cut at max_blocks_per_seq * block_size. chunk 6 runs the
    one-launch append, chunk 40 (11 blocks) the allocation + copy kernels."""
    bs, cap, H, d = 4, 32, 2, 8
    gpu = PagedKVCache(1, H, d, cap, bs, cuda, torch.float32, max_seqs=2, max_blocks_per_seq=maxb)
    cpu = ref.PagedKVCache(1, H, d, cap, bs)
    for s in (0, 1):
        gpu.add_sequence(s)
        cpu.add_sequence(s)
    g = torch.Generator().manual_seed(chunk)
    k = torch.randn(2, chunk, H, d, generator=g)
    v = torch.randn(2, chunk, H, d, generator=g)
    starts = [10, 0]  # sequence 0 overflows its table, sequence 1 fits
    fit = maxb * bs - starts[0]
    assert 0 < fit < chunk and starts[1] + chunk <= maxb * bs
    gpu.write_block_device(0, torch.tensor([0, 1], dtype=torch.int32, device=cuda),
                           torch.tensor(starts, dtype=torch.int32, device=cuda), k.to(cuda), v.to(cuda))
    with pytest.raises(IndexError):
        gpu.seq_lengths
    cpu.write_block(0, [0], [starts[0]], k[:1, :fit], v[:1, :fit])
    cpu.write_block(0, [1], [starts[1]], k[1:], v[1:])
    _same_state(gpu, cpu)
    assert gpu.seq_lengths == [maxb * bs, chunk]
    for s in (0, 1):
        n = gpu.seq_lengths[s]
        got = gather_ctx(gpu, 0, s, n).cpu()
        want = torch.stack((torch.cat([cpu.key_map(0, [p])[0] for p in cpu.block_tables[s]])[:n],
                            torch.cat([cpu.value_map(0, [p])[0] for p in cpu.block_tables[s]])[:n]))
        assert torch.equal(got[:, starts[s]:], want[:, starts[s]:])
