"""The fp8 (e4m3) restatement pinned against torch and the mathematics.

``encode`` / ``decode`` are checked bit-exactly against torch's
``float8_e4m3fn`` conversions (round to nearest even; torch turns values above
464 into NaN where this format saturates, so the comparison stops there). The
pool's quantisation rule is checked by bounds that a dropped term or a wrong
order would break: every stored row within half an e4m3 step (times the
block's scale) of its input, the block's largest element at exactly
``+-448 * scale`` up to the rounding of the scale, rows re-encoded when a later
chunk raises the scale, and allocation starting every block at scale 0.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.kv_fp8 import Fp8PagedKVCache, e4m3_decode, e4m3_encode
from oracle.kv_pool import BlockExhaustedError


def _torch_codes(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.asarray(x, dtype=np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_decode_matches_torch_for_every_code():
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    got = e4m3_decode(codes)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan) and nan.sum() == 2
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_encode_is_the_inverse_of_decode_on_codes():
    codes = np.array([c for c in range(256) if c & 0x7F != 0x7F], dtype=np.uint8)
    assert np.array_equal(e4m3_encode(e4m3_decode(codes)), codes)


def test_encode_matches_torch_on_dense_grids():
    rng = np.random.default_rng(0)
    vals = e4m3_decode(np.arange(0, 0x7F, dtype=np.uint8)).astype(np.float64)
    mids = (vals[:-1] + vals[1:]) / 2  # exact ties between neighbours
    grids = [
        rng.uniform(-464, 464, 200_000),
        rng.uniform(-2.0 ** -5, 2.0 ** -5, 50_000),     # subnormals and the first normals
        np.concatenate([mids, -mids]),
        np.concatenate([np.nextafter(mids, 0), np.nextafter(mids, 1e9)]),
        np.array([0.0, -0.0, 448.0, -448.0, 463.99, 464.0, -464.0, 2.0 ** -6, 2.0 ** -9, 2.0 ** -10]),
    ]
    for x in grids:
        x = x.astype(np.float32)
        assert np.array_equal(e4m3_encode(x), _torch_codes(x))


def test_encode_saturates_above_464():
    assert e4m3_encode(np.array([465.0, 1e30, np.inf], dtype=np.float32)).tolist() == [0x7E] * 3
    assert e4m3_encode(np.array([-1e30, -np.inf], dtype=np.float32)).tolist() == [0xFE] * 2


def _pool(cap=8, bs=4, H=2, d=4, layers=2):
    kv = Fp8PagedKVCache(layers, H, d, cap, bs)
    for s in range(3):
        kv.add_sequence(s)
    return kv


def _deq_rows(kv, layer, sid, kind):
    pool = kv.k if kind == 0 else kv.v
    out = []
    for blk, phys in enumerate(kv.block_tables[sid]):
        out.append(e4m3_decode(pool[layer, phys].numpy()) * kv.scales[layer, phys, kind])
    return np.concatenate(out, 0)[: kv.seq_lengths[sid]]


def test_stored_rows_within_half_a_step_and_peak_at_448():
    kv = _pool()
    g = torch.Generator().manual_seed(1)
    x = torch.randn(1, 7, 2, 4, generator=g) * 3
    y = torch.randn(1, 7, 2, 4, generator=g)
    kv.write_block(0, [0], [0], x, y)
    for kind, src in ((0, x), (1, y)):
        got = _deq_rows(kv, 0, 0, kind)
        ref = src[0].numpy()
        for blk, phys in enumerate(kv.block_tables[0]):
            sc = kv.scales[0, phys, kind]
            rows = slice(blk * 4, min(7, blk * 4 + 4))
            a = np.abs(ref[rows]).max()
            assert sc == np.float32(np.float32(a) / np.float32(448))
            # half an e4m3 step: 2^-4 relative for normals, 2^-10 * scale below 2^-6
            err = np.abs(got[rows] - ref[rows])
            bound = np.maximum(np.abs(ref[rows]) * 2.0 ** -4, 2.0 ** -10 * sc) * (1 + 1e-6)
            assert np.all(err <= bound)
            peak = np.abs(got[rows]).max()
            assert abs(peak - a) <= a * 2.0 ** -22


def test_growth_reencodes_the_other_rows_and_scale_never_shrinks():
    kv = _pool()
    small = torch.full((1, 2, 2, 4), 0.5)
    big = torch.full((1, 1, 2, 4), 8.0)
    kv.write_block(0, [0], [0], small, small)
    phys = kv.block_tables[0][0]
    sc0 = kv.scales[0, phys, 0]
    codes0 = kv.k[0, phys, :2].numpy().copy()
    kv.write_block(0, [0], [2], big, big)
    sc1 = kv.scales[0, phys, 0]
    assert sc1 == np.float32(np.float32(8.0) / np.float32(448)) and sc1 > sc0
    want = e4m3_encode((e4m3_decode(codes0) * sc0) / sc1)
    assert np.array_equal(kv.k[0, phys, :2].numpy(), want)
    assert np.allclose(_deq_rows(kv, 0, 0, 0)[:2], 0.5, rtol=2.0 ** -4)
    # a smaller chunk afterwards keeps the scale and leaves the other rows alone
    before = kv.k[0, phys].numpy().copy()
    kv.write_block(0, [0], [3], small[:, :1], small[:, :1])
    assert kv.scales[0, phys, 0] == sc1
    assert np.array_equal(kv.k[0, phys, :3].numpy(), before[:3])


def test_allocation_resets_scales_in_every_layer():
    kv = _pool(cap=2, bs=4, layers=3)
    x = torch.full((1, 4, 2, 4), 100.0)
    for layer in range(3):
        kv.write_block(layer, [0], [0], x, x)
    phys = kv.block_tables[0][0]
    assert np.all(kv.scales[:, phys, :] > 0)
    kv.clear(0)
    kv.write_block(0, [1], [0], x[:, :1] * 0.01, x[:, :1] * 0.01)
    assert kv.block_tables[1][0] == phys
    assert kv.scales[0, phys, 0] == np.float32(np.float32(1.0) / np.float32(448))
    assert np.all(kv.scales[1:, phys, :] == 0)


def test_exhaustion_writes_the_tokens_before_the_failing_one():
    kv = _pool(cap=2, bs=4)
    x = torch.randn(2, 6, 2, 4, generator=torch.Generator().manual_seed(3))
    with pytest.raises(BlockExhaustedError):
        kv.write_block(0, [0, 1], [0, 0], x, x)
    assert kv.seq_lengths[:2] == [6, 0] and len(kv.block_tables[0]) == 2
    kv2 = _pool(cap=3, bs=4)
    with pytest.raises(BlockExhaustedError):
        kv2.write_block(0, [0, 1], [0, 0], x, x)
    assert kv2.seq_lengths[:2] == [6, 4]
    assert np.allclose(_deq_rows(kv2, 0, 1, 0), x[1, :4].numpy(), rtol=2.0 ** -4, atol=1e-3)


def test_dequantized_view_shares_tables_and_values():
    kv = _pool()
    x = torch.randn(2, 5, 2, 4, generator=torch.Generator().manual_seed(5))
    kv.write_block(1, [0, 2], [0, 0], x, x * 2)
    dq = kv.dequantized()
    assert dq.block_tables == kv.block_tables and dq.seq_lengths == kv.seq_lengths
    phys = kv.block_tables[2][1]
    want = e4m3_decode(kv.v[1, phys].numpy()) * kv.scales[1, phys, 1]
    assert np.array_equal(dq.v[1, phys].numpy(), want)
