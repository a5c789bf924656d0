"""CPU checks that pin the attention oracle (oracle/attention.py).

* the reference's GQA mapping test (tests/test_attention.py:73-81);
* the reference's extend test shape (tests/test_paged_attention_extend.py:56-77):
  a prefilled prompt plus an appended chunk, extend row j == full attention over
  the prefix ``0..start+j``, at atol = rtol = 1e-5;
* an independent float64 brute force written with explicit loops (softmax of
  q.k/sqrt(d) over keys ``<= start + j`` of kv head ``h // (Hq/Hkv)``), at the
  CPU check workload's shapes -- a wrong head mapping, mask bound or scale fails it.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle.attention import (expand_to_q_heads, extend_attention_dense, full_attention,
                              gather_ctx, paged_attention_extend)
from oracle.kv_pool import PagedKVCache


def brute_force_extend(q, keys, values, starts, num_q_heads):
    """float64 loops: q (B, C, Hq, d); keys[b]/values[b] (ctx, Hkv, d)."""
    B, C, Hq, d = q.shape
    ratio = num_q_heads // keys[0].shape[1]
    out = torch.zeros((B, C, Hq, d), dtype=torch.float64)
    for b in range(B):
        k = keys[b].double()
        v = values[b].double()
        for j in range(C):
            n = int(starts[b]) + j + 1
            for h in range(Hq):
                kh = h // ratio
                qv = q[b, j, h].double()
                scores = [float(torch.dot(qv, k[t, kh])) / math.sqrt(d) for t in range(n)]
                m = max(scores)
                w = [math.exp(s - m) for s in scores]
                tot = sum(w)
                acc = torch.zeros(d, dtype=torch.float64)
                for t in range(n):
                    acc += (w[t] / tot) * v[t, kh]
                out[b, j, h] = acc
    return out


def test_expand_to_q_heads_repeats_kv():
    kv = torch.randn(5, 2, 8)
    e = expand_to_q_heads(kv, 4)
    assert e.shape == (5, 4, 8)
    assert torch.equal(e[:, 0], kv[:, 0]) and torch.equal(e[:, 1], kv[:, 0])
    assert torch.equal(e[:, 2], kv[:, 1]) and torch.equal(e[:, 3], kv[:, 1])


def test_extend_matches_prefix_full_attention():
    torch.manual_seed(1)
    Hq, Hkv, d, bs = 4, 2, 16, 4
    kv = PagedKVCache(1, Hkv, d, 64, bs)
    kv.add_sequence(0)
    prompt_k, prompt_v = torch.randn(7, Hkv, d), torch.randn(7, Hkv, d)
    for p in range(7):
        kv.write(0, 0, p, prompt_k[p], prompt_v[p])
    start, chunk = 7, 5
    q = torch.randn(1, chunk, Hq, d)
    ck, cv = torch.randn(chunk, Hkv, d), torch.randn(chunk, Hkv, d)
    for j in range(chunk):
        kv.write(0, 0, start + j, ck[j], cv[j])
    out = paged_attention_extend(q, kv, 0, [0], [start], Hq)
    assert out.shape == (1, chunk, Hq, d)
    for j in range(chunk):
        pair = gather_ctx(kv, 0, 0, start + j + 1)
        ref = full_attention(q[0, j], pair[0], pair[1], Hq)
        assert torch.allclose(out[0, j], ref, atol=1e-5, rtol=1e-5)


def test_extend_matches_float64_brute_force_cpu_check_shapes():
    # CPU check workload: Hq=4, Hkv=2, d=64, bs=16, C=5, L = 37/64/100/129, fp32, seed 0.
    g = torch.Generator().manual_seed(0)
    Hq, Hkv, d, bs, C = 4, 2, 64, 16, 5
    lens = [37, 64, 100, 129]
    keys = [torch.randn(L + C, Hkv, d, generator=g) for L in lens]
    values = [torch.randn(L + C, Hkv, d, generator=g) for L in lens]
    q = torch.randn(len(lens), C, Hq, d, generator=g)
    got = extend_attention_dense(q, keys, values, lens, Hq)
    ref = brute_force_extend(q, keys, values, lens, Hq)
    assert torch.allclose(got.double(), ref, atol=1e-5, rtol=1e-5)
    # and the paged form over a scattered pool gives the same numbers
    kv = PagedKVCache(1, Hkv, d, 64, bs)
    for b, L in enumerate(lens):
        kv.add_sequence(b)
    for b, L in enumerate(lens):
        for p in range(L + C):
            kv.write(0, b, p, keys[b][p], values[b][p])
    paged = paged_attention_extend(q, kv, 0, list(range(4)), lens, Hq)
    assert torch.allclose(paged, got, atol=1e-6, rtol=1e-6)


def test_brute_force_catches_wrong_head_mapping():
    # The brute force distinguishes h // ratio from h % Hkv (a plausible slip).
    g = torch.Generator().manual_seed(3)
    keys = [torch.randn(9, 2, 8, generator=g)]
    values = [torch.randn(9, 2, 8, generator=g)]
    q = torch.randn(1, 2, 4, 8, generator=g)
    good = brute_force_extend(q, keys, values, [7], 4)
    swapped = [k[:, [0, 1]] for k in keys]  # same tensor; build h % Hkv mapping by reordering q heads
    q_mod = q[:, :, [0, 2, 1, 3]]
    bad = brute_force_extend(q_mod, swapped, values, [7], 4)[:, :, [0, 2, 1, 3]]
    assert not torch.allclose(good, bad, atol=1e-3)


# ------------------------------------------------------------ prefill chunk
from oracle.attention import paged_attention_prefill_chunk  # noqa: E402


def brute_force_prefill(q, k, v, lengths, num_q_heads):
    """float64 loops: position j < L_b attends keys 0..j; zeros beyond L_b."""
    B, C, Hq, d = q.shape
    ratio = num_q_heads // k.shape[2]
    out = torch.zeros((B, C, Hq, d), dtype=torch.float64)
    for b in range(B):
        for j in range(int(lengths[b])):
            for h in range(Hq):
                kh = h // ratio
                qv = q[b, j, h].double()
                scores = [float(torch.dot(qv, k[b, t, kh].double())) / math.sqrt(d) for t in range(j + 1)]
                m = max(scores)
                w = [math.exp(s - m) for s in scores]
                tot = sum(w)
                acc = torch.zeros(d, dtype=torch.float64)
                for t in range(j + 1):
                    acc += (w[t] / tot) * v[b, t, kh].double()
                out[b, j, h] = acc
    return out


def test_prefill_matches_causal_sdpa_on_the_reference_test_shape():
    # reference tests/test_attention.py:144-164: q = k = v, lengths [4, 6], chunk 6
    torch.manual_seed(0)
    Hq, d = 4, 8
    query = torch.randn(2, 6, Hq, d)
    out = paged_attention_prefill_chunk(query, query, query, Hq, [4, 6])
    for index, length in enumerate([4, 6]):
        block = query[index][:length].transpose(0, 1)[None]
        want = torch.nn.functional.scaled_dot_product_attention(block, block, block, is_causal=True)[0]
        assert torch.allclose(out[index][:length], want.transpose(0, 1), atol=1e-5, rtol=1e-5)
        assert torch.equal(out[index][length:], torch.zeros_like(out[index][length:]))


def test_prefill_padding_is_exactly_zero_and_finite():
    # reference tests/test_attention.py:167-175
    torch.manual_seed(1)
    query = torch.randn(2, 5, 4, 8)
    out = paged_attention_prefill_chunk(query, query, query, 4, [2, 5])
    assert torch.equal(out[0][2:], torch.zeros_like(out[0][2:]))
    assert bool(torch.isfinite(out).all())


@pytest.mark.parametrize("Hq,Hkv", [(4, 2), (6, 2), (2, 2)])
def test_prefill_matches_float64_brute_force(Hq, Hkv):
    g = torch.Generator().manual_seed(Hq * 10 + Hkv)
    B, C, d = 3, 7, 16
    q = torch.randn(B, C, Hq, d, generator=g)
    k = torch.randn(B, C, Hkv, d, generator=g)
    v = torch.randn(B, C, Hkv, d, generator=g)
    lengths = [7, 1, 4]
    out = paged_attention_prefill_chunk(q, k, v, Hq, lengths)
    want = brute_force_prefill(q, k, v, lengths, Hq)
    assert torch.allclose(out.double(), want, atol=1e-5, rtol=1e-5)


def test_brute_force_prefill_catches_a_shifted_causal_bound():
    # a mask one key too wide (j + 2 instead of j + 1) must fail the comparison
    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(1, 5, 2, 8, generator=g) for _ in range(3))
    out = paged_attention_prefill_chunk(q, k, v, 2, [5])
    wrong = torch.zeros_like(out)
    for j in range(5):
        n = min(j + 2, 5)
        s = torch.einsum("hd,thd->ht", q[0, j], k[0, :n]) / math.sqrt(8)
        wrong[0, j] = torch.einsum("ht,thd->hd", torch.softmax(s, -1), v[0, :n])
    assert not torch.allclose(out, wrong, atol=1e-3)


def test_prefill_equals_extend_from_position_zero():
    # the chunk attends itself causally: the same as extend with start 0 over
    # a pool holding the chunk's keys
    g = torch.Generator().manual_seed(9)
    Hq, Hkv, d, bs, n = 4, 2, 16, 4, 11
    q = torch.randn(1, n, Hq, d, generator=g)
    k = torch.randn(1, n, Hkv, d, generator=g)
    v = torch.randn(1, n, Hkv, d, generator=g)
    kv = PagedKVCache(1, Hkv, d, 8, bs)
    kv.add_sequence(0)
    kv.write_block(0, [0], [0], k, v)
    ext = paged_attention_extend(q, kv, 0, [0], [0], Hq)
    pre = paged_attention_prefill_chunk(q, k, v, Hq, [n])
    assert torch.allclose(ext, pre, atol=1e-6, rtol=1e-5)
