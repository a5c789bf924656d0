"""GPU parity of paged verify attention against the oracle.

* fp32 pools (VALU path): the reference's extend test structure and the CPU
  check workload (4 sequences, L = 37/64/100/129, 4/2 heads, d = 64, C = 5) at
  atol = rtol = 1e-5, like the reference's own tests;
* bf16 pools: the Qwen2.5-1.5B-shaped workload (B = 32, 12/2 heads, d = 128,
  block 16, L ~ U[256, 4096], C = 6, random-permutation tables over 65,536
  blocks) on the MFMA path against the oracle run in fp32 on the same bf16
  values. Tolerance (bf16 output): per sequence ||out - ref|| / ||ref|| <= 2e-3,
  plus every element within 1 bf16 ulp (2^-7 relative) + 2e-3 * max |ref| --
  the output itself is rounded to bf16 (up to 2^-9 relative);
* fp16 pools and queries (the reference's GPU default) on the MFMA path: the
  same shapes, the cost-balanced split, and fp16 V at the top of its range and
  in its subnormals. Tolerance: per sequence relative L2 error <= 1e-3 and
  every element within 2^-10 relative + 1e-3 * max |ref|;
* size-independent properties: key positions beyond L full of NaN never reach
  the output; one context split and many splits agree.
"""

from __future__ import annotations

import math

import pytest
import torch

from engine.attention import (_expand_to_q_heads, gather_ctx, paged_attention_decode,
                              paged_attention_extend, verify_attention)
from engine.kv import PagedKVCache
from oracle import attention as ref_attn
from oracle import kv_pool as ref

pytestmark = pytest.mark.gpu


def test_expand_to_q_heads_repeats_kv(cuda):
    kv = torch.randn(5, 2, 8, device=cuda)
    e = _expand_to_q_heads(kv, 4)
    assert torch.equal(e[:, 1], kv[:, 0]) and torch.equal(e[:, 2], kv[:, 1])


def _write_both(gpu, cpu, layer, sid, keys, values):
    n = keys.shape[0]
    gpu.write_block(layer, [sid], [0], keys.unsqueeze(0).to(gpu.device), values.unsqueeze(0).to(gpu.device))
    cpu.write_block(layer, [sid], [0], keys.unsqueeze(0), values.unsqueeze(0))
    assert gpu.seq_lengths[sid] == n


def test_extend_matches_oracle_reference_test_shape(cuda):
    # reference tests/test_paged_attention_extend.py:56-77: 7-token prompt, chunk 5, bs 4
    torch.manual_seed(1)
    Hq, Hkv, d, bs = 4, 2, 16, 4
    gpu = PagedKVCache(2, Hkv, d, 64, bs, cuda, torch.float32)
    cpu = ref.PagedKVCache(2, Hkv, d, 64, bs)
    gpu.add_sequence(0)
    cpu.add_sequence(0)
    _write_both(gpu, cpu, 0, 0, torch.randn(7, Hkv, d), torch.randn(7, Hkv, d))
    start, chunk = 7, 5
    ck, cv, q = torch.randn(1, chunk, Hkv, d), torch.randn(1, chunk, Hkv, d), torch.randn(1, chunk, Hq, d)
    gpu.write_block(0, [0], [start], ck.to(cuda), cv.to(cuda))
    cpu.write_block(0, [0], [start], ck, cv)
    out = paged_attention_extend(q.to(cuda), gpu, 0, [0], [start], Hq)
    assert out.shape == (1, chunk, Hq, d)
    want = ref_attn.paged_attention_extend(q, cpu, 0, [0], [start], Hq)
    assert torch.allclose(out.cpu(), want, atol=1e-5, rtol=1e-5)
    for j in range(chunk):  # row j == full attention over the prefix 0..start+j
        pair = ref_attn.gather_ctx(cpu, 0, 0, start + j + 1)
        row = ref_attn.full_attention(q[0, j], pair[0], pair[1], Hq)
        assert torch.allclose(out[0, j].cpu(), row, atol=1e-5, rtol=1e-5)


def test_decode_matches_oracle(cuda):
    torch.manual_seed(2)
    Hq, Hkv, d, bs = 4, 2, 8, 4
    gpu = PagedKVCache(2, Hkv, d, 64, bs, cuda, torch.float32)
    cpu = ref.PagedKVCache(2, Hkv, d, 64, bs)
    lens = [1, 4, 7]
    for s, n in enumerate(lens):
        gpu.add_sequence(s)
        cpu.add_sequence(s)
        _write_both(gpu, cpu, 0, s, torch.randn(n, Hkv, d), torch.randn(n, Hkv, d))
    q = torch.randn(3, Hq, d)
    out = paged_attention_decode(q.to(cuda), gpu, 0, [0, 1, 2], lens, Hq).cpu()
    for s, n in enumerate(lens):
        pair = ref_attn.gather_ctx(cpu, 0, s, n)
        assert torch.allclose(out[s], ref_attn.full_attention(q[s], pair[0], pair[1], Hq),
                              atol=1e-5, rtol=1e-5)


def _dense_pool(cuda, lens, C, Hkv, d, bs, dtype, seed, cap=None, nan_fill=False, perm=True, vmul=None):
    """Pool holding K/V for positions 0..L+C-1 of each sequence, written through
    write_block, with tables scattered over the pool. ``vmul(n)``: factors
    (n, 1, 1) of the n positions' values (before rounding to ``dtype``)."""
    g = torch.Generator().manual_seed(seed)
    need = [-(-(L + C) // bs) for L in lens]
    cap = cap or sum(need) + 8
    gpu = PagedKVCache(1, Hkv, d, cap, bs, cuda, dtype, max_seqs=len(lens))
    if nan_fill:
        gpu.k_pool.fill_(float("nan"))
        gpu.v_pool.fill_(float("nan"))
    ids = torch.randperm(cap, generator=g).tolist() if perm else list(range(cap))
    tables, pos = [], 0
    for n in need:
        tables.append(ids[pos: pos + n])
        pos += n
    gpu.load_state(tables, [0] * len(lens), ids[pos:])
    keys = [torch.randn(L + C, Hkv, d, generator=g).to(dtype) for L in lens]
    values = [torch.randn(L + C, Hkv, d, generator=g) for L in lens]
    values = [(v if vmul is None else v.clamp(-4, 4) * vmul(v.shape[0])).to(dtype) for v in values]
    for s, L in enumerate(lens):
        if L:
            gpu.write_block(0, [s], [0], keys[s][:L].unsqueeze(0).to(cuda),
                            values[s][:L].unsqueeze(0).to(cuda))
    # the verify chunk is appended for the whole batch in one call
    kc = torch.stack([k[L:] for k, L in zip(keys, lens)]).to(cuda)
    vc = torch.stack([v[L:] for v, L in zip(values, lens)]).to(cuda)
    gpu.write_block(0, list(range(len(lens))), lens, kc, vc)
    return gpu, keys, values


def test_cpu_check_workload_fp32(cuda):
    lens, C, Hq, Hkv, d, bs = [37, 64, 100, 129], 5, 4, 2, 64, 16
    gpu, keys, values = _dense_pool(cuda, lens, C, Hkv, d, bs, torch.float32, seed=0)
    q = torch.randn(len(lens), C, Hq, d, generator=torch.Generator().manual_seed(5))
    out = paged_attention_extend(q.to(cuda), gpu, 0, list(range(4)), lens, Hq).cpu()
    want = ref_attn.extend_attention_dense(q, keys, values, lens, Hq)
    assert torch.allclose(out, want, atol=1e-5, rtol=1e-5)


def _bf16_check(out, want):
    """bf16 tolerance: per sequence, relative L2 error ||out - ref|| / ||ref|| <= 2e-3,
    and every element within one bf16 ulp (2^-7 relative) plus 2e-3 * max|ref|.
    (Rounding the output to bf16 alone costs up to half an ulp, 2^-9 relative,
    so an element-wise 2e-3 relative bound is below the output's own precision.)"""
    out = out.float().cpu()
    want = want.float()
    for b in range(out.shape[0]):
        scale = float(want[b].abs().max())
        err = (out[b] - want[b]).abs()
        rel = float(err.norm() / want[b].norm())
        assert rel <= 2e-3, (b, rel)
        assert bool((err <= 2.0 ** -7 * want[b].abs() + 2e-3 * scale).all()), (b, float(err.max()), scale)


@pytest.mark.parametrize("seed", [0, 1])
def test_qwen15_shaped_bf16_mfma(cuda, seed):
    g = torch.Generator().manual_seed(100 + seed)
    B, C, Hq, Hkv, d, bs = 32, 6, 12, 2, 128, 16
    lens = torch.randint(256, 4097, (B,), generator=g).tolist()
    gpu, keys, values = _dense_pool(cuda, lens, C, Hkv, d, bs, torch.bfloat16, seed=seed, cap=65536)
    q = torch.randn(B, C, Hq, d, generator=g).to(torch.bfloat16)
    out = paged_attention_extend(q.to(cuda), gpu, 0, list(range(B)), lens, Hq)
    want = ref_attn.extend_attention_dense(q, keys, values, lens, Hq)
    _bf16_check(out, want)


@pytest.mark.parametrize("shape", [
    # (C, Hq, Hkv, d): G = C * Hq/Hkv
    (7, 16, 2, 128),   # 3B-shaped: G = 56, four 16-row tiles
    (9, 14, 2, 64),    # 0.5B-shaped heads: G = 63, d = 64
    (2, 16, 2, 128),   # G = 16, one tile
    (3, 12, 2, 128),   # G = 18, two tiles with padding
    (1, 4, 2, 128),    # decode G = 2: one padded tile
    (1, 14, 2, 64),    # 0.5B-shaped draft decode: G = 7
    (1, 12, 2, 128),   # 1.5B-shaped decode: G = 6
    (1, 2, 2, 128),    # G = 1
    (2, 14, 2, 64),    # G = 14
])
def test_bf16_shapes(cuda, shape):
    C, Hq, Hkv, d = shape
    g = torch.Generator().manual_seed(sum(shape))
    lens = [0, 1, 15, 16, 17, 255, 300, 1000]
    gpu, keys, values = _dense_pool(cuda, lens, C, Hkv, d, 16, torch.bfloat16, seed=7)
    q = torch.randn(len(lens), C, Hq, d, generator=g).to(torch.bfloat16)
    out = paged_attention_extend(q.to(cuda), gpu, 0, list(range(len(lens))), lens, Hq)
    want = ref_attn.extend_attention_dense(q, keys, values, lens, Hq)
    _bf16_check(out, want)


def _f16_check(out, want):
    """fp16 tolerance: per sequence, relative L2 error <= 1e-3, and every element
    within 2^-10 relative (two fp16 ulps) plus 1e-3 * max|ref|. The output is
    rounded to fp16 (up to 2^-12 relative) and P enters P V as fp16."""
    assert out.dtype == torch.float16
    out = out.double().cpu()
    want = want.double()
    for b in range(out.shape[0]):
        scale = float(want[b].abs().max())
        err = (out[b] - want[b]).abs()
        rel = float(err.norm() / want[b].norm())
        assert rel <= 1e-3, (b, rel)
        assert bool((err <= 2.0 ** -10 * want[b].abs() + 1e-3 * scale).all()), (b, float(err.max()), scale)


@pytest.mark.parametrize("shape", [
    # (B, C, Hq, Hkv, d): fp16 pools and queries (the reference's GPU default) on the MFMA path
    (32, 6, 12, 2, 128),  # Qwen2.5-1.5B verify
    (8, 7, 16, 2, 128),   # 3B-shaped: four query tiles
    (8, 9, 14, 2, 64),    # 0.5B-shaped heads: four tiles at d = 64
    (8, 3, 12, 2, 128),   # G = 18, two tiles with padding
    (8, 1, 14, 2, 64),    # 0.5B-shaped draft decode: G = 7
    (160, 6, 12, 2, 128),  # segments outnumber the workgroups: the cost-balanced split
    (160, 7, 16, 2, 128),  # the same with four query tiles (the full-depth 3B kernel)
    (160, 9, 14, 2, 64),   # and at head_dim 64
])
def test_fp16_mfma_shapes(cuda, shape):
    B, C, Hq, Hkv, d = shape
    g = torch.Generator().manual_seed(sum(shape) + 5)
    lens = ([0, 1, 15, 16, 17, 255, 300, 1000] if B == 8 else
            torch.randint(16, 4097 if B == 32 else 1500, (B,), generator=g).tolist())
    gpu, keys, values = _dense_pool(cuda, lens, C, Hkv, d, 16, torch.float16, seed=B + C, cap=65536)
    q = torch.randn(B, C, Hq, d, generator=g).to(torch.float16)
    out = paged_attention_extend(q.to(cuda), gpu, 0, list(range(B)), lens, Hq)
    rows = list(range(B)) if B <= 32 else list(range(0, B, 9))
    want = ref_attn.extend_attention_dense(q[rows], [keys[r] for r in rows], [values[r] for r in rows],
                                           [lens[r] for r in rows], Hq)
    _f16_check(out[rows], want)


@pytest.mark.parametrize("case", ["large", "subnormal", "mixed"])
def test_fp16_value_magnitudes(cuda, case):
    """fp16 V near the top of fp16's range (|V| up to 6e4), in its subnormals
    (|V| below 1e-5), and both within one sequence. Element-wise bound: two fp16
    ulps relative, 1e-3 of the sequence's largest output, and two subnormal
    spacings (2^-23) absolute, where the output itself is subnormal."""
    def vmul(n):
        pos = torch.arange(n, dtype=torch.float32)[:, None, None]
        if case == "large":
            return torch.full_like(pos, 1.5e4)
        if case == "subnormal":
            return torch.full_like(pos, 2e-6)
        return torch.where(pos % 5 == 0, 2e-6, 1.5e4)
    lens, C, Hq, Hkv, d = [400, 190, 3000], 6, 12, 2, 128
    gpu, keys, values = _dense_pool(cuda, lens, C, Hkv, d, 16, torch.float16, seed=17, vmul=vmul)
    q = torch.randn(len(lens), C, Hq, d, generator=torch.Generator().manual_seed(18)).to(torch.float16)
    out = paged_attention_extend(q.to(cuda), gpu, 0, list(range(len(lens))), lens, Hq)
    assert bool(torch.isfinite(out).all())
    want = ref_attn.extend_attention_dense(q, keys, values, lens, Hq).double()
    out = out.double().cpu()
    for b in range(len(lens)):
        err = (out[b] - want[b]).abs()
        scale = float(want[b].abs().max())
        # the output's own fp16 rounding, with the subnormals' absolute spacing 2^-24
        assert bool((err <= 2.0 ** -10 * want[b].abs() + 1e-3 * scale + 2.0 ** -23).all()), \
            (b, case, float(err.max()), scale)


def test_bf16_draft_decode_batch(cuda):
    """paged_attention_decode at a draft model's shape (one row, 14/2 heads,
    head_dim 64) over ragged contexts: the padded single-tile MFMA path."""
    g = torch.Generator().manual_seed(31)
    B, Hq, Hkv, d = 48, 14, 2, 64
    lens = torch.randint(1, 3000, (B,), generator=g).tolist()
    gpu, keys, values = _dense_pool(cuda, [L - 1 for L in lens], 1, Hkv, d, 16, torch.bfloat16, seed=31)
    q = torch.randn(B, Hq, d, generator=g).to(torch.bfloat16)
    out = paged_attention_decode(q.to(cuda), gpu, 0, list(range(B)), lens, Hq)
    want = ref_attn.extend_attention_dense(q.unsqueeze(1), keys, values, [L - 1 for L in lens], Hq).squeeze(1)
    _bf16_check(out.unsqueeze(1), want.unsqueeze(1))


def test_stale_nan_beyond_context_never_leaks(cuda):
    lens, C, Hq, Hkv, d = [5, 40, 77], 6, 12, 2, 128
    gpu, keys, values = _dense_pool(cuda, lens, C, Hkv, d, 16, torch.bfloat16, seed=3, nan_fill=True)
    q = torch.randn(3, C, Hq, d).to(torch.bfloat16)
    out = paged_attention_extend(q.to(cuda), gpu, 0, [0, 1, 2], lens, Hq)
    assert bool(torch.isfinite(out.float()).all())
    _bf16_check(out, ref_attn.extend_attention_dense(q, keys, values, lens, Hq))
    gpu32, k32, v32 = _dense_pool(cuda, lens, C, Hkv, 64, 16, torch.float32, seed=3, nan_fill=True)
    q32 = torch.randn(3, C, 4, 64)
    out32 = paged_attention_extend(q32.to(cuda), gpu32, 0, [0, 1, 2], lens, 4).cpu()
    assert torch.allclose(out32, ref_attn.extend_attention_dense(q32, k32, v32, lens, 4), atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("C,Hq", [(6, 12), (3, 12), (7, 16)])
def test_output_writes_stay_inside_the_batch(cuda, C, Hq):
    # G = 36 / 18 rows leave padded query tiles; the output buffer sits between
    # guard regions that must come back untouched, and every row is written.
    lens, Hkv, d = [300, 17, 1000, 0, 129], 2, 128
    gpu, keys, values = _dense_pool(cuda, lens, C, Hkv, d, 16, torch.bfloat16, seed=12)
    B = len(lens)
    q = torch.randn(B, C, Hq, d, generator=torch.Generator().manual_seed(13)).to(torch.bfloat16)
    n, guard = B * C * Hq * d, 4096
    buf = torch.full((n + 2 * guard,), 3.0, dtype=torch.bfloat16, device=cuda)
    buf[guard:guard + n] = float("nan")
    out = buf[guard:guard + n].view(B, C, Hq, d)
    verify_attention(q.to(cuda), gpu, 0, list(range(B)), lens, max(lens) + C, out=out)
    host = buf.float().cpu()
    assert bool((host[:guard] == 3.0).all()) and bool((host[guard + n:] == 3.0).all())
    assert bool(torch.isfinite(host[guard:guard + n]).all())
    _bf16_check(out, ref_attn.extend_attention_dense(q, keys, values, lens, Hq))


def test_repeated_calls_are_identical_and_leave_counters_zero(cuda):
    # Sequences cut between workgroups are merged by the last one to arrive;
    # its arrival counters live at the head of the workspace and must be zero
    # again after every call, and the fixed-order merges make reruns bitwise equal.
    import engine.attention as A

    g = torch.Generator().manual_seed(21)
    lens = torch.randint(256, 4097, (32,), generator=g).tolist()
    gpu, keys, values = _dense_pool(cuda, lens, 6, 2, 128, 16, torch.bfloat16, seed=21, cap=20000)
    q = torch.randn(32, 6, 12, 128, generator=g).to(torch.bfloat16).to(cuda)
    outs = [verify_attention(q, gpu, 0, list(range(32)), lens, max(lens) + 6).clone() for _ in range(3)]
    torch.cuda.synchronize()
    assert all(torch.equal(outs[0], o) for o in outs[1:])
    counters = A._workspace.current(cuda)[: 1 << 18]
    assert int(counters.count_nonzero()) == 0
    _bf16_check(outs[0], ref_attn.extend_attention_dense(q.cpu(), keys, values, lens, 12))


def test_split_count_does_not_change_result(cuda):
    # The same batch with max_ctx raised (more, partly empty splits) gives the same output.
    lens, C, Hq, Hkv, d = [700, 33], 6, 12, 2, 128
    gpu, keys, values = _dense_pool(cuda, lens, C, Hkv, d, 16, torch.bfloat16, seed=4)
    q = torch.randn(2, C, Hq, d).to(torch.bfloat16).to(cuda)
    a = verify_attention(q, gpu, 0, [0, 1], lens, max(lens) + C)
    b = verify_attention(q, gpu, 0, [0, 1], lens, 4096)
    assert torch.equal(a, b)


def test_gather_ctx_matches_written_values(cuda):
    lens, C = [20, 3], 2
    gpu, keys, values = _dense_pool(cuda, lens, C, 2, 16, 4, torch.float32, seed=9)
    for s, L in enumerate(lens):
        got = gather_ctx(gpu, 0, s, L + C).cpu()
        assert torch.equal(got[0], keys[s]) and torch.equal(got[1], values[s])


@pytest.mark.parametrize("B,C,Hq", [(160, 7, 16), (130, 6, 12)])
def test_page_balanced_split_when_segments_outnumber_workgroups(cuda, B, C, Hq):
    # With at least as many (sequence, kv head) segments as workgroups the
    # pages are split evenly across workgroups: long segments are cut over
    # several of them (partials merged by the last to arrive), short ones are
    # whole inside one. Log-uniform lengths make both happen.
    import math

    import engine.attention as A

    Hkv, d = 2, 128
    g = torch.Generator().manual_seed(B + C)
    lens = [int(math.exp(math.log(16) + (math.log(3000) - math.log(16)) * float(u)))
            for u in torch.rand(B, generator=g)]
    gpu, keys, values = _dense_pool(cuda, lens, C, Hkv, d, 16, torch.bfloat16, seed=B)
    q = torch.randn(B, C, Hq, d, generator=g).to(torch.bfloat16).to(cuda)
    outs = [verify_attention(q, gpu, 0, list(range(B)), lens, max(lens) + C).clone() for _ in range(2)]
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    assert int(torch.count_nonzero(A._workspace.current(cuda)[: 1 << 18])) == 0
    _bf16_check(outs[0], ref_attn.extend_attention_dense(q.cpu(), keys, values, lens, Hq))


@pytest.mark.parametrize("n_short,n_long,d", [(280, 24, 128), (300, 6, 64), (257, 0, 128)])
def test_balanced_split_with_piece_costs(cuda, n_short, n_long, d):
    """Cost-balanced split with many one- and two-page segments beside long
    ones: workgroups hold several whole segments, ranges end among a segment's
    overhead units (that segment starts in the next workgroup), and long
    segments are cut over several workgroups."""
    import engine.attention as A

    Hq, Hkv, C = 12, 2, 6
    g = torch.Generator().manual_seed(n_short + n_long)
    lens = [int(x) for x in torch.randint(1, 27, (n_short,), generator=g)]
    lens += [int(x) for x in torch.randint(600, 3000, (n_long,), generator=g)]
    order = torch.randperm(len(lens), generator=g).tolist()
    lens = [lens[i] for i in order]
    B = len(lens)
    gpu, keys, values = _dense_pool(cuda, lens, C, Hkv, d, 16, torch.bfloat16, seed=B + d)
    q = torch.randn(B, C, Hq, d, generator=g).to(torch.bfloat16).to(cuda)
    outs = [verify_attention(q, gpu, 0, list(range(B)), lens, max(lens) + C).clone() for _ in range(2)]
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    assert int(torch.count_nonzero(A._workspace.current(cuda)[: 1 << 18])) == 0
    _bf16_check(outs[0], ref_attn.extend_attention_dense(q.cpu(), keys, values, lens, Hq))


def _balanced_pieces(pages, hkv, cost, nw):
    """Pieces of the cost-balanced split, as the host sees them: every
    (sequence, kv head) segment is `cost` overhead units followed by its
    pages, laid end to end; workgroup w takes units [w T / nw, (w + 1) T / nw).
    Returns the page count of every non-empty (workgroup, segment) piece."""
    seg = [n for n in pages for _ in range(hkv)]
    total = sum(n + cost for n in seg)
    starts, s0 = [], 0
    for n in seg:
        starts.append(s0)
        s0 += n + cost
    pieces = []
    for w in range(nw):
        a, b = w * total // nw, (w + 1) * total // nw
        for st, n in zip(starts, seg):
            lo, hi = max(a, st + cost), min(b, st + cost + n)
            if hi > lo:
                pieces.append(hi - lo)
    return pieces


@pytest.mark.parametrize("d", [64, 128])
def test_pieces_longer_than_the_block_id_window(cuda, d):
    """Cost-balanced split with pieces of more than 512 pages: a workgroup
    stages a piece's block ids in windows of 512 and restages them mid-walk.
    128 sequences of 12,000-13,000 keys over 2 kv heads (256 segments)."""
    Hq, Hkv, C, B = 2, 2, 2, 128
    g = torch.Generator().manual_seed(d)
    lens = [int(x) for x in torch.randint(12000, 13000, (B,), generator=g)]
    pages = [-(-(L + C) // 16) for L in lens]
    nw = torch.cuda.get_device_properties(0).multi_processor_count
    cost = 32 * 8192 // (16 * d * 2 * 2)  # the kernel's piece cost, bf16 pages
    pieces = _balanced_pieces(pages, Hkv, cost, nw)
    assert B * Hkv >= nw and max(pieces) > 512, (nw, max(pieces))
    gpu, keys, values = _dense_pool(cuda, lens, C, Hkv, d, 16, torch.bfloat16, seed=d + 1)
    q = torch.randn(B, C, Hq, d, generator=g).to(torch.bfloat16)
    out = verify_attention(q.to(cuda), gpu, 0, list(range(B)), lens, max(lens) + C)
    _bf16_check(out, ref_attn.extend_attention_dense(q, keys, values, lens, Hq))


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 128), (torch.float32, 64)])
def test_reading_unwritten_keys_is_reported(cuda, dtype, d):
    """verify_attention over a chunk that was never appended (start + chunk
    beyond the sequence's length, here also beyond its blocks, so a table slot
    is unset) reads block 0 instead of faulting and raises IndexError at the
    next metadata query; the flag is cleared by raising it. The MFMA path
    (bf16) and the VALU path (fp32)."""
    lens, C, Hq = [40, 20], 6, 4
    gpu, keys, values = _dense_pool(cuda, lens, C, 2, d, 16, dtype, seed=5)
    q = torch.randn(2, C, Hq, d).to(dtype).to(cuda)
    ok = verify_attention(q, gpu, 0, [0, 1], lens, max(lens) + C)
    assert gpu.seq_lengths == [L + C for L in lens]  # a correct call raises nothing
    verify_attention(q, gpu, 0, [0, 1], [40, 40], 46)  # sequence 1 holds 26 keys in 2 blocks
    torch.cuda.synchronize()
    with pytest.raises(IndexError):
        gpu.seq_lengths
    assert gpu.seq_lengths == [L + C for L in lens]
    again = verify_attention(q, gpu, 0, [0, 1], lens, max(lens) + C)
    assert torch.equal(ok, again)


def test_timing_hook_records_the_kernel_and_changes_nothing(cuda):
    """spv_time_next_attention: the next attention call records its kernels'
    start and end into the caller's HIP events (a positive interval below the
    whole call's wall time) and computes exactly what an untimed call does; the
    arming serves one call only."""
    import ctypes

    from engine import _hip

    lib = _hip.lib()
    lib.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
    lib.hipEventDestroy.argtypes = [ctypes.c_void_p]
    lens, C, Hq = [300, 2000, 17], 6, 12
    for dtype, d in ((torch.bfloat16, 128), (torch.float32, 64)):  # one kernel; two (split + merge)
        gpu, keys, values = _dense_pool(cuda, lens, C, 2, d, 16, dtype, seed=8)
        q = torch.randn(3, C, Hq, d).to(dtype).to(cuda)
        plain = verify_attention(q, gpu, 0, [0, 1, 2], lens, max(lens) + C)
        ev = [ctypes.c_void_p(), ctypes.c_void_p()]
        for e in ev:
            assert lib.hipEventCreate(ctypes.byref(e)) == 0
        assert lib.spv_time_next_attention(ev[0], ev[1]) == 0
        timed = verify_attention(q, gpu, 0, [0, 1, 2], lens, max(lens) + C)
        after = verify_attention(q, gpu, 0, [0, 1, 2], lens, max(lens) + C)  # not armed any more
        torch.cuda.synchronize()
        ms = ctypes.c_float()
        assert lib.hipEventElapsedTime(ctypes.byref(ms), ev[0], ev[1]) == 0
        assert 0.0 < ms.value < 50.0
        assert torch.equal(plain, timed) and torch.equal(plain, after)
        for e in ev:
            lib.hipEventDestroy(e)
