"""CPU restatement of the reference paged extend attention (test infrastructure only).

Follows engine/attention.py of the reference:

* ``expand_to_q_heads``      -- attention.py:32-38 (``repeat_interleave``: q head h
                                reads kv head ``h // (Hq/Hkv)``)
* ``gather_ctx``             -- attention.py:41-63 (blocks concatenated in logical
                                order, only ``length`` cells taken)
* ``full_attention``         -- attention.py:66-93 (unmasked SDPA)
* ``paged_attention_extend`` -- attention.py:170-216 (boolean causal mask
                                ``mask[j, i] = i <= start + j``, one SDPA per sequence)
* ``paged_attention_prefill_chunk`` -- attention.py:121-167 (causal SDPA over each
                                row's first ``chunk_query_lengths[b]`` positions of
                                the dense chunk, zeros for the padded tail)

``extend_attention_dense`` runs the same per-sequence mask + SDPA on dense
per-sequence K/V (what ``gather_ctx`` would return), so large synthetic
workloads need not be materialised in the reference pool layout first.

Pinned by tests/test_oracle_attention.py: the reference's GQA mapping test
(tests/test_attention.py:73-81), extend == per-row prefix ``full_attention``
(tests/test_paged_attention_extend.py:56-77, 1e-5), and an independent float64
brute-force softmax(QK^T/sqrt(d))V written with explicit loops; the prefill
chunk by the reference's prefill tests (tests/test_attention.py:144-175: the
symmetric q = k = v case against causal SDPA at 1e-5, an exactly zero padded
tail, finite outputs), the same float64 brute force with a causal mask, and
its agreement with ``paged_attention_extend`` at start 0 over the same keys.
"""

from __future__ import annotations

from typing import List, Sequence

import torch
import torch.nn.functional as F

from .kv_pool import PagedKVCache


def expand_to_q_heads(kv: torch.Tensor, num_q_heads: int) -> torch.Tensor:
    ratio = num_q_heads // kv.shape[-2]
    return kv if ratio == 1 else kv.repeat_interleave(ratio, dim=-2)


def gather_ctx(kv: PagedKVCache, layer: int, seq_id: int, length: int) -> torch.Tensor:
    """``(2, length, kv_heads, d)``: row 0 = K, row 1 = V."""
    if length <= 0:
        return torch.zeros((2, 0, kv.num_kv_heads, kv.head_dim), dtype=kv.dtype)
    table = kv.block_tables[seq_id]
    bs = kv.block_size
    ks, vs = [], []
    for bi in range(-(-length // bs)):
        take = min(bs, length - bi * bs)
        ks.append(kv.k[layer, table[bi], :take])
        vs.append(kv.v[layer, table[bi], :take])
    return torch.stack((torch.cat(ks, 0), torch.cat(vs, 0)), 0)


def full_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                   num_q_heads: int) -> torch.Tensor:
    """query (Hq, d); key/value (ctx, Hkv, d) -> (Hq, d)."""
    k4 = expand_to_q_heads(key, num_q_heads).transpose(0, 1).unsqueeze(0)
    v4 = expand_to_q_heads(value, num_q_heads).transpose(0, 1).unsqueeze(0)
    q4 = query.unsqueeze(0).unsqueeze(2)
    return F.scaled_dot_product_attention(q4, k4, v4).squeeze(0).squeeze(1)


def _extend_one(q: torch.Tensor, key: torch.Tensor, value: torch.Tensor, start: int,
                num_q_heads: int) -> torch.Tensor:
    """q (chunk, Hq, d); key/value (start+chunk, Hkv, d) -> (chunk, Hq, d)."""
    chunk = q.shape[0]
    length = start + chunk
    key = expand_to_q_heads(key, num_q_heads)
    value = expand_to_q_heads(value, num_q_heads)
    mask = torch.zeros((chunk, length), dtype=torch.bool)
    for j in range(chunk):
        mask[j, : start + j + 1] = True
    q4 = q.transpose(0, 1).unsqueeze(0)
    k4 = key.transpose(0, 1).unsqueeze(0)
    v4 = value.transpose(0, 1).unsqueeze(0)
    out = F.scaled_dot_product_attention(q4, k4, v4, attn_mask=mask.unsqueeze(0))
    return out[0].transpose(0, 1)


def paged_attention_extend(query_3d: torch.Tensor, kv: PagedKVCache, layer: int,
                           seq_ids: Sequence[int], start_positions: Sequence[int],
                           num_q_heads: int) -> torch.Tensor:
    """``(B, chunk, Hq, d)``; keys include the chunk's own rows (write-then-attend)."""
    B, chunk = query_3d.shape[:2]
    outs: List[torch.Tensor] = []
    for b in range(B):
        start = int(start_positions[b])
        ctx = gather_ctx(kv, layer, seq_ids[b], start + chunk)
        outs.append(_extend_one(query_3d[b], ctx[0], ctx[1], start, num_q_heads))
    return torch.stack(outs, 0)


def extend_attention_dense(query_3d: torch.Tensor, keys: Sequence[torch.Tensor],
                           values: Sequence[torch.Tensor],
                           start_positions: Sequence[int], num_q_heads: int,
                           compute_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Same math as ``paged_attention_extend`` over dense per-sequence context.

    ``keys[b]``/``values[b]`` hold at least ``start_positions[b] + chunk`` rows
    ``(ctx, Hkv, d)``. Inputs are upcast to ``compute_dtype`` (exact for bf16 ->
    fp32) and the result is returned in ``compute_dtype``.
    """
    B, chunk = query_3d.shape[:2]
    outs = []
    for b in range(B):
        start = int(start_positions[b])
        n = start + chunk
        outs.append(_extend_one(query_3d[b].to(compute_dtype),
                                keys[b][:n].to(compute_dtype),
                                values[b][:n].to(compute_dtype), start, num_q_heads))
    return torch.stack(outs, 0)


def paged_attention_prefill_chunk(query_3d: torch.Tensor, key_3d: torch.Tensor, value_3d: torch.Tensor,
                                  num_q_heads: int, chunk_query_lengths: Sequence[int]) -> torch.Tensor:
    """``(B, chunk, Hq, d)``: row ``b`` position ``j < L_b`` attends ``0 .. j`` of
    its own chunk (GQA expanded), positions ``>= L_b`` are zeros."""
    B, chunk = query_3d.shape[:2]
    outs = []
    for b in range(B):
        n = int(chunk_query_lengths[b])
        q4 = query_3d[b][:n].transpose(0, 1).unsqueeze(0)
        k4 = expand_to_q_heads(key_3d[b][:n], num_q_heads).transpose(0, 1).unsqueeze(0)
        v4 = expand_to_q_heads(value_3d[b][:n], num_q_heads).transpose(0, 1).unsqueeze(0)
        out = F.scaled_dot_product_attention(q4, k4, v4, is_causal=True)[0].transpose(0, 1)
        if chunk > n:
            out = torch.cat((out, torch.zeros((chunk - n,) + tuple(out.shape[1:]), dtype=out.dtype)), 0)
        outs.append(out)
    return torch.stack(outs, 0)
