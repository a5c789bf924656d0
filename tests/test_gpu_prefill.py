"""GPU parity of chunked prefill attention (paged_attention_prefill_chunk,
engine/attention.py:121-167) against the oracle.

* the reference's own prefill tests (tests/test_attention.py:144-175) on the
  GPU: fp32, q = k = v, lengths [4, 6] and [2, 5], atol = rtol = 1e-5 against
  causal SDPA, the padded tail exactly zero, every output finite;
* bf16 (MFMA path) at the Qwen2.5-3B prompt shapes (16 q / 2 kv heads,
  head_dim 128, prompt lengths 512 .. 8192 in one padded chunk), at the
  Qwen2.5-0.5B heads (14 / 2, head_dim 64) and at GQA ratios 1, 6, 8 and 16,
  against the oracle in fp32 on the same bf16 values at the bf16 bar (per row
  relative L2 <= 2e-3, every element within one bf16 ulp + 2e-3 max |ref|);
  the padding is filled with NaN and must not reach any output;
* V of any magnitude on the MFMA path, which stages V in fp16 times a power of
  two taken from the first key tile: tiles 10^6 apart (the later tile past
  fp16 at the first tile's scale, so the block runs again with the power of
  two of its whole key range), values near 1e30 and near 1e-30, a first tile
  of zeros;
* the workgroup orders: equal prompts (XCD-affine), unequal prompts (longest
  processing time first, ties, empty prompts, 64 prompts) and more than 64
  prompts (slice order), every block computed exactly once;
* fp16 inputs on the MFMA path (Qwen2.5-3B and 0.5B heads, GQA ratios 1-7, V
  near the top of fp16's range and in its subnormals), fp16 and fp32 inputs on
  the VALU path (other head dims);
* the same keys attended by prefill and by paged verify attention from
  position 0 agree.
"""

from __future__ import annotations

import pytest
import torch

from engine.attention import paged_attention_prefill_chunk, prefill_attention, verify_attention
from engine.kv import PagedKVCache
from oracle import attention as ref_attn

pytestmark = pytest.mark.gpu


def _bf16_check(out, want, lengths):
    out = out.double().cpu()  # float64: the norms of outputs near 1e30 stay finite
    want = want.double()
    for b, n in enumerate(lengths):
        if n == 0:
            continue
        o, w = out[b, :n], want[b, :n]
        scale = float(w.abs().max())
        err = (o - w).abs()
        rel = float(err.norm() / w.norm())
        assert rel <= 2e-3, (b, rel)
        assert bool((err <= 2.0 ** -7 * w.abs() + 2e-3 * scale).all()), (b, float(err.max()), scale)


def test_reference_prefill_tests_on_the_gpu(cuda):
    torch.manual_seed(0)
    Hq, d = 4, 8
    query = torch.randn(2, 6, Hq, d)
    out = paged_attention_prefill_chunk(query.to(cuda), query.to(cuda), query.to(cuda), Hq, [4, 6]).cpu()
    for index, length in enumerate([4, 6]):
        block = query[index][:length].transpose(0, 1)[None]
        want = torch.nn.functional.scaled_dot_product_attention(block, block, block, is_causal=True)[0]
        assert torch.allclose(out[index][:length], want.transpose(0, 1), atol=1e-5, rtol=1e-5)
        assert torch.equal(out[index][length:], torch.zeros_like(out[index][length:]))
    query = torch.randn(2, 5, Hq, d)
    out = paged_attention_prefill_chunk(query.to(cuda), query.to(cuda), query.to(cuda), Hq, [2, 5]).cpu()
    assert torch.equal(out[0][2:], torch.zeros_like(out[0][2:]))
    assert bool(torch.isfinite(out).all())
    want = ref_attn.paged_attention_prefill_chunk(query, query, query, Hq, [2, 5])
    assert torch.allclose(out, want, atol=1e-5, rtol=1e-5)


def _chunk(B, Lc, Hq, Hkv, d, lengths, seed, dtype=torch.bfloat16, nan_pad=True):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Lc, Hq, d, generator=g).to(dtype)
    k = torch.randn(B, Lc, Hkv, d, generator=g).to(dtype)
    v = torch.randn(B, Lc, Hkv, d, generator=g).to(dtype)
    if nan_pad:
        for b, n in enumerate(lengths):
            for t in (q, k, v):
                t[b, n:] = float("nan")
    return q, k, v


def _check_padding(out, lengths):
    host = out.float().cpu()
    for b, n in enumerate(lengths):
        assert bool((host[b, n:] == 0).all()), b
    assert bool(torch.isfinite(host).all())


@pytest.mark.parametrize("lengths", [[512, 2999, 8192], [8192]])
def test_qwen3b_prompt_shapes_bf16(cuda, lengths):
    Hq, Hkv, d = 16, 2, 128
    B, Lc = len(lengths), max(lengths)
    q, k, v = _chunk(B, Lc, Hq, Hkv, d, lengths, seed=Lc + B)
    out = paged_attention_prefill_chunk(q.to(cuda), k.to(cuda), v.to(cuda), Hq, lengths)
    _check_padding(out, lengths)
    want = ref_attn.paged_attention_prefill_chunk(q.float(), k.float(), v.float(), Hq, lengths)
    _bf16_check(out, want, lengths)


@pytest.mark.parametrize("Hq,Hkv,d,lengths", [
    (14, 2, 64, [1, 100, 1000, 2047]),   # Qwen2.5-0.5B heads, ratio 7: 36 positions per workgroup
    (12, 2, 128, [300, 64, 65, 1]),      # ratio 6 (Qwen2.5-1.5B heads)
    (4, 4, 128, [257, 31]),              # ratio 1: 256 positions per workgroup
    (32, 2, 128, [200, 17]),             # ratio 16: 16 positions per workgroup
    (8, 1, 64, [129, 0]),                # ratio 8, an empty row
])
def test_bf16_head_ratios(cuda, Hq, Hkv, d, lengths):
    B, Lc = len(lengths), max(lengths) + 5
    q, k, v = _chunk(B, Lc, Hq, Hkv, d, lengths, seed=Hq * 100 + d)
    out = paged_attention_prefill_chunk(q.to(cuda), k.to(cuda), v.to(cuda), Hq, lengths)
    _check_padding(out, lengths)
    want = ref_attn.paged_attention_prefill_chunk(q.float(), k.float(), v.float(), Hq, lengths)
    _bf16_check(out, want, lengths)


@pytest.mark.parametrize("B,Hq,Hkv,d,L,Lc", [
    (4, 16, 2, 128, 700, 1000),   # 8 slices: one per XCD
    (8, 16, 2, 128, 300, 300),    # 16 slices: two per XCD, no padding block
    (2, 16, 2, 128, 1500, 1600),  # 4 slices: every second block of one on each XCD
    (1, 14, 2, 64, 999, 1203),    # 2 slices: every fourth block
    (3, 16, 2, 128, 640, 700),    # 6 slices: the default order
])
def test_equal_prompt_dispatch(cuda, B, Hq, Hkv, d, L, Lc):
    # Equal lengths select the XCD-affine dispatch when the slices divide or
    # are divided by 8; every (sequence, kv head, block) must be computed once,
    # the padding blocks past L included.
    lengths = [L] * B
    q, k, v = _chunk(B, Lc, Hq, Hkv, d, lengths, seed=B * 1000 + L)
    out = paged_attention_prefill_chunk(q.to(cuda), k.to(cuda), v.to(cuda), Hq, lengths)
    _check_padding(out, lengths)
    want = ref_attn.paged_attention_prefill_chunk(q.float(), k.float(), v.float(), Hq, lengths)
    _bf16_check(out, want, lengths)


@pytest.mark.parametrize("Hq,Hkv,d,lengths,Lc", [
    (16, 2, 128, [0, 1200, 64, 1200, 333], 1300),  # equal longest prompts (ties), an empty one
    (12, 2, 128, [901, 17, 450, 1, 1023, 640, 77, 2, 300], 1024),  # ratio 6: 42 positions per block
    (24, 8, 64, [513, 100, 1999], 2000),  # ratio 3: 85 positions per block
    (8, 2, 128, [(37 * i) % 101 for i in range(64)], 100),  # 64 prompts (the most ordered by length)
    (4, 1, 64, [(13 * i) % 41 for i in range(70)], 40),  # 70 prompts: slice order
])
def test_unequal_prompt_dispatch(cuda, Hq, Hkv, d, lengths, Lc):
    # Unequal lengths (up to 64 prompts) take the longest-processing-time
    # order computed in every workgroup; every (sequence, kv head, block) must
    # be computed exactly once, the blocks without rows included.
    B = len(lengths)
    q, k, v = _chunk(B, Lc, Hq, Hkv, d, lengths, seed=B * 7 + Lc)
    out = paged_attention_prefill_chunk(q.to(cuda), k.to(cuda), v.to(cuda), Hq, lengths)
    _check_padding(out, lengths)
    want = ref_attn.paged_attention_prefill_chunk(q.float(), k.float(), v.float(), Hq, lengths)
    _bf16_check(out, want, lengths)


@pytest.mark.parametrize("case", ["rising", "falling", "huge", "tiny", "zero_first"])
@pytest.mark.parametrize("d", [128, 64])
def test_bf16_value_magnitudes(cuda, case, d):
    Hq, Hkv, lengths = 8, 2, [400, 190]
    B, Lc = len(lengths), max(lengths)
    q, k, v = _chunk(B, Lc, Hq, Hkv, d, lengths, seed=7 + d, nan_pad=False)
    pos = torch.arange(Lc, dtype=torch.float32)[None, :, None, None]
    if case == "rising":  # keys 0..63 small, later ones 10^6 larger: a rescale after the first tile
        f = torch.where(pos < 64, 1e-3, 1e3)
    elif case == "falling":
        f = torch.where(pos < 64, 1e3, 1e-3)
    elif case == "huge":
        f = torch.full_like(pos, 1e30)
    elif case == "tiny":
        f = torch.full_like(pos, 1e-30)
    else:  # the first tile all zero: its scale is 1, the next tile sets none smaller unless it must
        f = torch.where(pos < 64, 0.0, 3e4)
    v = (v.float() * f).to(torch.bfloat16)
    out = paged_attention_prefill_chunk(q.to(cuda), k.to(cuda), v.to(cuda), Hq, lengths)
    want = ref_attn.paged_attention_prefill_chunk(q.float(), k.float(), v.float(), Hq, lengths)
    _bf16_check(out, want, lengths)


@pytest.mark.parametrize("dtype,d", [(torch.float32, 128), (torch.float16, 40), (torch.float32, 40)])
def test_valu_path_matches_oracle(cuda, dtype, d):
    Hq, Hkv, lengths = 6, 2, [150, 1, 77]
    B, Lc = len(lengths), 160
    q, k, v = _chunk(B, Lc, Hq, Hkv, d, lengths, seed=d, dtype=dtype)
    out = paged_attention_prefill_chunk(q.to(cuda), k.to(cuda), v.to(cuda), Hq, lengths)
    _check_padding(out, lengths)
    want = ref_attn.paged_attention_prefill_chunk(q.float(), k.float(), v.float(), Hq, lengths)
    tol = 1e-5 if dtype == torch.float32 else 2e-3
    for b, n in enumerate(lengths):
        assert torch.allclose(out[b, :n].float().cpu(), want[b, :n], atol=tol, rtol=tol), b


def _f16_check(out, want, lengths):
    out = out.double().cpu()
    want = want.double()
    for b, n in enumerate(lengths):
        if n == 0:
            continue
        o, w = out[b, :n], want[b, :n]
        scale = float(w.abs().max())
        err = (o - w).abs()
        rel = float(err.norm() / w.norm())
        assert rel <= 1e-3, (b, rel)
        assert bool((err <= 2.0 ** -10 * w.abs() + 1e-3 * scale).all()), (b, float(err.max()), scale)


@pytest.mark.parametrize("Hq,Hkv,d,lengths", [
    (16, 2, 128, [512, 2999, 1200, 0]),  # Qwen2.5-3B heads (the reference runs fp16 on the GPU)
    (14, 2, 64, [1, 100, 1000, 777]),    # Qwen2.5-0.5B heads, ratio 7
    (12, 2, 128, [300, 64, 65, 1]),      # ratio 6
    (4, 4, 128, [257, 31]),              # ratio 1
])
def test_fp16_mfma_path(cuda, Hq, Hkv, d, lengths):
    # fp16 inputs take the MFMA kernel: S^T with the f16 MFMA, V staged as it is
    B, Lc = len(lengths), max(lengths) + 3
    q, k, v = _chunk(B, Lc, Hq, Hkv, d, lengths, seed=Hq * 10 + d + 1, dtype=torch.float16)
    out = paged_attention_prefill_chunk(q.to(cuda), k.to(cuda), v.to(cuda), Hq, lengths)
    assert out.dtype == torch.float16
    _check_padding(out, lengths)
    want = ref_attn.paged_attention_prefill_chunk(q.float(), k.float(), v.float(), Hq, lengths)
    _f16_check(out, want, lengths)


@pytest.mark.parametrize("case", ["large", "subnormal", "mixed"])
def test_fp16_value_magnitudes(cuda, case):
    # fp16 V near the top of the range, in the subnormals, and both within one prompt
    Hq, Hkv, d, lengths = 8, 2, 128, [400, 190]
    B, Lc = len(lengths), max(lengths)
    q, k, v = _chunk(B, Lc, Hq, Hkv, d, lengths, seed=11, dtype=torch.float16, nan_pad=False)
    pos = torch.arange(Lc, dtype=torch.float32)[None, :, None, None]
    if case == "large":
        f = torch.full_like(pos, 1.5e4)
    elif case == "subnormal":
        f = torch.full_like(pos, 2e-6)
    else:
        f = torch.where(pos < 64, 2e-6, 1.5e4)
    v = (v.float().clamp(-4, 4) * f).to(torch.float16)
    out = paged_attention_prefill_chunk(q.to(cuda), k.to(cuda), v.to(cuda), Hq, lengths)
    want = ref_attn.paged_attention_prefill_chunk(q.float(), k.float(), v.float(), Hq, lengths)
    out = out.double().cpu()
    for b, n in enumerate(lengths):
        o, w = out[b, :n], want[b, :n].double()
        scale = float(w.abs().max())
        # the output's own fp16 rounding, with the subnormals' absolute spacing 2^-24
        assert bool(((o - w).abs() <= 2.0 ** -10 * w.abs() + 1e-3 * scale + 2.0 ** -23).all()), (b, case)


def test_device_lengths_are_clamped_to_the_chunk(cuda):
    # a length beyond the chunk reads nothing beyond it: it acts as the chunk length
    Hq, Hkv, d, Lc = 16, 2, 128, 100
    q, k, v = _chunk(2, Lc, Hq, Hkv, d, [Lc, Lc], seed=3, nan_pad=False)
    lens = torch.tensor([Lc + 500, 40], dtype=torch.int32, device=cuda)
    out = prefill_attention(q.to(cuda), k.to(cuda), v.to(cuda), lens)
    want = ref_attn.paged_attention_prefill_chunk(q.float(), k.float(), v.float(), Hq, [Lc, 40])
    _bf16_check(out, want, [Lc, 40])
    _check_padding(out, [Lc, 40])


def test_prefill_agrees_with_verify_attention_from_position_zero(cuda):
    # the chunk's keys written to a paged pool and attended from start 0 by the
    # verify kernel give the prefill kernel's result
    Hq, Hkv, d, n = 12, 2, 128, 700
    q, k, v = _chunk(1, n, Hq, Hkv, d, [n], seed=11, nan_pad=False)
    kv = PagedKVCache(1, Hkv, d, 64, 16, cuda, torch.bfloat16)
    kv.add_sequence(0)
    kv.write_block(0, [0], [0], k.to(cuda), v.to(cuda))
    ext = verify_attention(q.to(cuda), kv, 0, [0], [0], n).float().cpu()
    pre = prefill_attention(q.to(cuda), k.to(cuda), v.to(cuda), [n]).float().cpu()
    want = ref_attn.paged_attention_prefill_chunk(q.float(), k.float(), v.float(), Hq, [n])
    _bf16_check(pre, want, [n])
    _bf16_check(ext, want, [n])
    assert float((ext - pre).abs().max()) <= 2.0 ** -6 * float(want.abs().max())
