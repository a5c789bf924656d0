"""CPU restatement of the fp8 (OCP e4m3) KV pool (test infrastructure only).

The reference pool stores K/V in the model dtype (engine/kv.py:99-101); an fp8
pool with one fp32 scale per (layer, block, K | V) is the library's own storage
format for long contexts. Its rule, restated here from the device kernels:

* a stored code q means ``decode(q) * scale`` (fp32 product);
* a block handed out by the allocator gets scale 0 in every layer;
* writing a chunk's rows into a block (per layer, separately for K and V):
  ``a = max |x|`` over those rows (all heads and dims), ``scale' = max(scale,
  a / 448)``; if ``scale' > scale`` every other row of the block is re-encoded
  as ``encode((decode(q) * scale) / scale')``; the chunk's rows are stored as
  ``encode(x / scale')`` (code 0 when ``scale'`` is 0). Every product and
  quotient is a correctly rounded float32 operation, in that order;
* ``encode`` is OCP e4m3 with round-to-nearest-even, saturating at +-448
  (the sign of the input, zero included, is kept).

Allocation, exhaustion and lengths follow ``oracle.kv_pool.PagedKVCache`` (the
reference's per-token write loop, engine/kv.py:119-147): on exhaustion the
tokens before the failing one are written (and quantised) and the error is
raised.

Pinned by tests/test_oracle_fp8.py: ``encode`` and ``decode`` bit-exact
against torch's ``float8_e4m3fn`` conversion over every code and over dense
value grids (ties, subnormals, the saturation boundary); the quantisation rule
by error bounds (every stored row within half an e4m3 step of its input), by
the block's largest element decoding to ``+-448 * scale``, by the growth rule
(re-encoded rows), and by allocation resetting scales.
"""

from __future__ import annotations

from typing import Optional, Sequence

import numpy as np
import torch

from .kv_pool import BlockExhaustedError, PagedKVCache

E4M3_MAX = np.float32(448.0)
_MIN_NORMAL = np.float32(2.0 ** -6)


def e4m3_encode(x) -> np.ndarray:
    """float32 -> uint8 e4m3 codes: nearest even, saturating at +-448."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32)
    sign = ((u >> np.uint32(24)) & np.uint32(0x80)).astype(np.uint32)
    a = np.minimum(np.abs(x), E4M3_MAX)
    a = np.where(np.isnan(a), np.float32(0.0), a).astype(np.float32)
    sub = a < _MIN_NORMAL
    m_sub = np.rint(a * np.float32(512.0)).astype(np.uint32)  # m * 2^-9, m in 0..8
    ua = a.view(np.uint32)
    r = ua + np.uint32(0x7FFFF) + ((ua >> np.uint32(20)) & np.uint32(1))
    with np.errstate(over="ignore"):
        normal = (((r >> np.uint32(23)) - np.uint32(120)) << np.uint32(3)) | ((r >> np.uint32(20)) & np.uint32(7))
    code = np.where(sub, m_sub, normal) & np.uint32(0x7F)
    return (sign | code).astype(np.uint8)


def _decode_table() -> np.ndarray:
    t = np.zeros(256, dtype=np.float32)
    for c in range(256):
        s, e, m = c >> 7, (c >> 3) & 15, c & 7
        if e == 15 and m == 7:
            v = np.float32(np.nan)
        elif e == 0:
            v = np.float32(m) * np.float32(2.0 ** -9)
        else:
            v = np.float32((1.0 + m / 8.0) * 2.0 ** (e - 7))
        t[c] = -v if s else v
    return t


_DECODE = _decode_table()


def e4m3_decode(codes) -> np.ndarray:
    """uint8 e4m3 codes -> float32 (exact)."""
    return _DECODE[np.asarray(codes, dtype=np.uint8)]


class Fp8PagedKVCache(PagedKVCache):
    """``oracle.kv_pool.PagedKVCache`` with e4m3 codes and per-(layer, block,
    K | V) scales. ``k`` / ``v`` hold uint8 codes in the reference layout
    ``(layers, cap, block_size, kv_heads, d)``; ``scales`` is
    ``(layers, cap, 2)`` float32 (K, V)."""

    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int,
                 capacity_blocks: int, block_size: int) -> None:
        super().__init__(num_layers, num_kv_heads, head_dim, capacity_blocks, block_size,
                         dtype=torch.uint8)
        self.scales = np.zeros((num_layers, capacity_blocks, 2), dtype=np.float32)

    # allocation: kv.py:119-122, plus the scale reset of a block handed out
    def _ensure_blocks_up_to(self, seq_id: int, max_block_index: int) -> None:
        table = self.block_tables[seq_id]
        while len(table) <= max_block_index:
            blk = self.allocator.alloc()
            self.scales[:, blk, :] = 0.0
            table.append(blk)

    def write(self, layer: int, seq_id: int, token_pos: int, kvec, vvec) -> None:
        self.write_block(layer, [seq_id], [token_pos], kvec.reshape(1, 1, *kvec.shape[-2:]),
                         vvec.reshape(1, 1, *vvec.shape[-2:]))

    def write_block(self, layer: int, seq_ids: Sequence[int], start_positions: Sequence[int],
                    k_new: Optional[torch.Tensor], v_new: Optional[torch.Tensor],
                    chunk: Optional[int] = None) -> None:
        C = int(k_new.shape[1]) if chunk is None else int(chunk)
        bs = self.block_size
        for b, sid in enumerate(seq_ids):
            s0 = int(start_positions[b])
            n, failed = 0, None
            for j in range(C):
                try:
                    self._ensure_blocks_up_to(sid, (s0 + j) // bs)
                except BlockExhaustedError as e:
                    failed = e
                    break
                n += 1
            if n and k_new is not None:
                kx = k_new[b].detach().to(torch.float32).numpy()
                vx = v_new[b].detach().to(torch.float32).numpy()
                for blk in range(s0 // bs, (s0 + n - 1) // bs + 1):
                    lo = max(s0, blk * bs) - blk * bs
                    hi = min(s0 + n, (blk + 1) * bs) - blk * bs
                    j0 = blk * bs + lo - s0
                    phys = self.block_tables[sid][blk]
                    self._quantize(self.k, 0, layer, phys, lo, hi, kx[j0: j0 + hi - lo])
                    self._quantize(self.v, 1, layer, phys, lo, hi, vx[j0: j0 + hi - lo])
            if n and self.seq_lengths[sid] < s0 + n:
                self.seq_lengths[sid] = s0 + n
            if failed is not None:
                raise failed

    def _quantize(self, pool: torch.Tensor, kind: int, layer: int, phys: int, lo: int, hi: int,
                  x: np.ndarray) -> None:
        codes = pool[layer, phys].numpy()  # (bs, Hkv, d), a view
        a = np.float32(np.max(np.abs(x))) if x.size else np.float32(0.0)
        old = np.float32(self.scales[layer, phys, kind])
        sc = np.float32(max(old, np.float32(a / E4M3_MAX)))
        if sc > old:
            others = [r for r in range(self.block_size) if not lo <= r < hi]
            vals = (e4m3_decode(codes[others]) * old) / sc
            codes[others] = e4m3_encode(vals.astype(np.float32))
        if sc > 0:
            codes[lo:hi] = e4m3_encode((x / sc).astype(np.float32))
        else:
            codes[lo:hi] = 0
        self.scales[layer, phys, kind] = sc

    def dequantized(self) -> PagedKVCache:
        """A float32 ``oracle.kv_pool.PagedKVCache`` with the same tables,
        lengths and free list whose K/V are ``decode(code) * scale``."""
        out = PagedKVCache(self.num_layers, self.num_kv_heads, self.head_dim, self.allocator.capacity,
                           self.block_size, dtype=torch.float32)
        out.load_state(self.block_tables, self.seq_lengths, self.allocator.free_list)
        ks = self.scales[:, :, 0][:, :, None, None, None]
        vs = self.scales[:, :, 1][:, :, None, None, None]
        out.k = torch.from_numpy((e4m3_decode(self.k.numpy()) * ks).astype(np.float32))
        out.v = torch.from_numpy((e4m3_decode(self.v.numpy()) * vs).astype(np.float32))
        return out
