"""Paged attention entry points backed by the gfx950 HIP kernels.

Drop-in for the reference's engine/attention.py on the verify path:

* ``gather_ctx``             -- attention.py:41-63, one gather kernel
* ``paged_attention_extend`` -- attention.py:170-216, one verify-attention launch
                                (plus a merge launch when contexts are split)
* ``paged_attention_decode`` -- attention.py:96-118 as the one-row case of extend
                                (``start = length - 1``, chunk 1)
* ``paged_attention_prefill_chunk`` -- attention.py:121-167, one causal prefill
                                launch over the dense chunk (``prefill_attention``
                                takes the lengths as a device tensor)
* ``_expand_to_q_heads``     -- attention.py:32-38 (kept for API parity; the
                                kernels never materialise the expansion: kv head
                                ``h // (Hq/Hkv)`` is indexed directly)

``paged_attention_extend`` reads the block tables and lengths from the device
metadata of :class:`engine.kv.PagedKVCache`; the K/V of the query chunk must
already be written (write-then-attend, engine/model.py:182-190).

A round calls the attention once per layer with the same sequences and start
positions. ``VerifyPlan`` computes what those calls share (the split of the
batch over the workgroups and each workgroup's first pages) once; calls given
the plan start their page walk one round trip after launch.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence, Union

import torch

from . import _hip
from ._hip import call, ptr
from .kv import PagedKVCache

_workspace = _hip.Workspace()


def _expand_to_q_heads(kv: torch.Tensor, num_q_heads: int) -> torch.Tensor:
    """Broadcast ``(.., kv_heads, d)`` to ``(.., num_q_heads, d)`` (attention.py:32-38)."""
    ratio = num_q_heads // kv.shape[-2]
    return kv if ratio == 1 else kv.repeat_interleave(ratio, dim=-2)


def gather_ctx(kv: PagedKVCache, layer: int, seq_id: int, length: int) -> torch.Tensor:
    """The stored K/V prefix of one sequence, ``(2, length, kv_heads, d)`` (K row 0, V row 1);
    an fp8 pool's is dequantised to float32 (code * scale of its block)."""
    length = int(length)
    out_dtype = torch.float32 if kv.fp8 else kv.dtype
    out = torch.empty((2, max(length, 0), kv.num_kv_heads, kv.head_dim), dtype=out_dtype,
                      device=kv.device)
    if length <= 0:
        return out
    seq_id = kv._check_sid(seq_id)
    kv._refresh()
    if -(-length // kv.block_size) > kv._nb[seq_id]:
        raise IndexError("length {} exceeds the blocks of sequence {}".format(length, seq_id))
    call("spv_kv_gather", ptr(kv.k_pool), ptr(kv.v_pool), kv._dt, ptr(kv.scales), ptr(kv.tables_dev),
         kv.max_blocks_per_seq, seq_id, length, int(layer), kv.allocator.capacity, kv.block_size,
         kv.num_kv_heads, kv.head_dim, ptr(out), _hip.stream_of(kv.device))
    return out


class VerifyPlan:
    """The shared part of one round's attention calls, computed on the device.

    Made once the round's blocks are allocated (after the first layer's
    append) for the round's sequences, start positions (int32 device tensors
    or lists), chunk length, query heads and ``max_ctx``; every layer's
    ``verify_attention`` given it must use exactly those. It also checks, once,
    that every sequence's written length covers its chunk (the per-call check
    of unplanned calls). Valid while the round's start positions and block
    tables stand.
    """

    def __init__(self, kv: PagedKVCache, seq_ids: Union[Sequence[int], torch.Tensor],
                 start_positions: Union[Sequence[int], torch.Tensor], chunk: int, num_q_heads: int,
                 max_ctx: int, buf: Optional[torch.Tensor] = None) -> None:
        self.kv = kv
        self.seq_ids = _hip.i32(seq_ids, kv.device)
        self.start = _hip.i32(start_positions, kv.device)
        self.B = int(self.seq_ids.numel())
        self.chunk, self.num_q_heads, self.max_ctx = int(chunk), int(num_q_heads), int(max_ctx)
        self.ws_bytes: Optional[int] = None  # the calls' workspace size, asked by the first
        if self.max_ctx > kv.max_blocks_per_seq * kv.block_size:
            kv._grow_width(-(-self.max_ctx // kv.block_size))
        nbytes = int(_hip.lib().spv_verify_attn_plan_bytes(max(self.B, 1)))
        if buf is not None and nbytes and (buf.numel() * buf.element_size() < nbytes or buf.device != kv.device):
            raise ValueError("plan buffer too small or on another device")
        # ``buf``: a buffer of an earlier plan to write this one into (no allocation)
        self.buf = (buf if buf is not None else torch.empty(nbytes, dtype=torch.uint8, device=kv.device)) \
            if nbytes else None
        if self.B and self.buf is not None:
            call("spv_verify_attn_plan", ptr(kv.tables_dev), kv.max_blocks_per_seq, ptr(self.seq_ids),
                 ptr(self.start), ptr(kv.lens_dev), ptr(kv.allocator.ctr), self.B, self.chunk, self.num_q_heads,
                 kv.num_kv_heads, kv.head_dim, kv.block_size, kv._dt, kv.allocator.capacity, self.max_ctx,
                 ptr(self.buf), int(self.buf.numel() * self.buf.element_size()), _hip.stream_of(kv.device))
            kv._stale = True

    def check(self, kv: PagedKVCache, B: int, chunk: int, num_q_heads: int, max_ctx: int) -> None:
        if kv is not self.kv or (B, chunk, num_q_heads, max_ctx) != (self.B, self.chunk, self.num_q_heads,
                                                                      self.max_ctx):
            raise ValueError("the attention call does not match its plan")


def verify_attention(query_3d: torch.Tensor, kv: PagedKVCache, layer: int,
                     seq_ids: Union[Sequence[int], torch.Tensor],
                     start_positions: Union[Sequence[int], torch.Tensor], max_ctx: int,
                     scale: Optional[float] = None, out: Optional[torch.Tensor] = None,
                     plan: Optional[VerifyPlan] = None) -> torch.Tensor:
    """Device-argument form of ``paged_attention_extend``.

    ``seq_ids``/``start_positions`` may be int32 device tensors (no host sync);
    ``max_ctx`` must bound ``start + chunk`` for every row. ``plan``: the
    round's ``VerifyPlan`` (same sequences, starts, chunk, heads, max_ctx).
    """
    B, chunk, hq, d = query_3d.shape
    if d != kv.head_dim or hq % kv.num_kv_heads:
        raise ValueError("query heads/dim do not match the cache")
    if query_3d.device != kv.device:
        raise ValueError("query must live on {}".format(kv.device))
    q = query_3d.contiguous()
    if out is None:
        out = torch.empty_like(q)
    if B == 0:
        return out
    if plan is not None:
        plan.check(kv, B, chunk, hq, int(max_ctx))
        sid_t, start_t = plan.seq_ids, plan.start
    else:
        sid_t = _hip.i32(seq_ids, kv.device)
        start_t = _hip.i32(start_positions, kv.device)
    if max_ctx > kv.max_blocks_per_seq * kv.block_size:
        kv._grow_width(-(-max_ctx // kv.block_size))
    scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
    if plan is not None:  # a round's calls share their shapes: the size is asked once
        if plan.ws_bytes is None:
            plan.ws_bytes = int(_hip.lib().spv_verify_attn_workspace_bytes(B, chunk, hq, kv.num_kv_heads, d,
                                                                         kv.block_size, int(max_ctx)))
        ws_bytes = plan.ws_bytes
    else:
        ws_bytes = _hip.lib().spv_verify_attn_workspace_bytes(B, chunk, hq, kv.num_kv_heads, d,
                                                              kv.block_size, int(max_ctx))
    stream = _hip.stream_of(kv.device)
    ws = _workspace.get(ws_bytes, kv.device, stream) if ws_bytes else None
    args = (ptr(out), ptr(q), _hip.dtype_code(q.dtype), ptr(kv.k_pool), ptr(kv.v_pool),
            kv._dt, ptr(kv.scales), ptr(kv.tables_dev), kv.max_blocks_per_seq, ptr(sid_t), ptr(start_t),
            ptr(kv.lens_dev), ptr(kv.allocator.ctr), B, chunk,
            hq, kv.num_kv_heads, d, kv.block_size, int(layer), kv.allocator.capacity, int(max_ctx), scale)
    if plan is not None and plan.buf is not None:
        call("spv_verify_attn_planned", *args, ptr(plan.buf), ptr(ws), int(ws_bytes), stream)
    else:
        call("spv_verify_attn", *args, ptr(ws), int(ws_bytes), stream)
    # A read of unwritten keys is flagged on the device and raised (IndexError)
    # at the next metadata query, without a synchronisation here.
    kv._stale = True
    return out


def paged_attention_extend(query_3d: torch.Tensor, kv: PagedKVCache, layer: int,
                           seq_ids: Sequence[int], start_positions: Sequence[int],
                           num_q_heads: int) -> torch.Tensor:
    """Causal attention of a chunk over its paged prefix (attention.py:170-216).

    ``query_3d`` is ``(B, chunk, num_q_heads, d)``; row ``j`` of sequence ``b``
    attends positions ``0 .. start_positions[b] + j``. Returns
    ``(B, chunk, num_q_heads, d)`` in the query dtype.
    """
    B, chunk = int(query_3d.shape[0]), int(query_3d.shape[1])
    if int(query_3d.shape[2]) != int(num_q_heads):
        raise ValueError("query has {} heads, expected {}".format(query_3d.shape[2], num_q_heads))
    starts = [int(s) for s in start_positions]
    sids = [kv._check_sid(s) for s in seq_ids]
    if len(starts) != B or len(sids) != B:
        raise ValueError("one seq_id and start position per batch row")
    kv._refresh()
    for sid, st in zip(sids, starts):
        if st < 0 or -(-(st + chunk) // kv.block_size) > kv._nb[sid]:
            raise IndexError("sequence {} has no K/V written up to position {}".format(sid, st + chunk))
    max_ctx = max(starts) + chunk if B else chunk
    return verify_attention(query_3d, kv, layer, sids, starts, max_ctx)


def paged_attention_decode(query_2d: torch.Tensor, kv: PagedKVCache, layer: int,
                           seq_ids: Sequence[int], seq_token_lengths: Sequence[int],
                           num_q_heads: int) -> torch.Tensor:
    """One query row per sequence over its full stored prefix (attention.py:96-118)."""
    lengths = [int(x) for x in seq_token_lengths]
    if any(x < 1 for x in lengths):
        raise ValueError("decode needs at least one stored position per row")
    q3 = query_2d.unsqueeze(1)
    out = paged_attention_extend(q3, kv, layer, seq_ids, [x - 1 for x in lengths], num_q_heads)
    return out.squeeze(1)


def prefill_attention(query_3d: torch.Tensor, key_3d: torch.Tensor, value_3d: torch.Tensor,
                      lengths: Union[Sequence[int], torch.Tensor], scale: Optional[float] = None,
                      out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Device-argument form of ``paged_attention_prefill_chunk``: ``lengths`` may
    be an int32 device tensor (no host sync); values above the chunk length are
    clamped to it."""
    B, chunk, hq, d = query_3d.shape
    if tuple(key_3d.shape[:2]) != (B, chunk) or key_3d.shape != value_3d.shape or key_3d.shape[3] != d \
            or hq % key_3d.shape[2]:
        raise ValueError("query (B, chunk, Hq, d) and key / value (B, chunk, Hkv, d) do not match")
    dev = _hip.require_gpu(query_3d.device)
    if key_3d.device != dev or value_3d.device != dev or key_3d.dtype != query_3d.dtype or \
            value_3d.dtype != query_3d.dtype:
        raise ValueError("query, key and value must share a device and dtype")
    q, k, v = query_3d.contiguous(), key_3d.contiguous(), value_3d.contiguous()
    if out is None:
        out = torch.empty_like(q)
    if B == 0:
        return out
    lens = _hip.i32(lengths, dev)
    scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
    call("spv_prefill_attn", ptr(out), ptr(q), ptr(k), ptr(v), _hip.dtype_code(q.dtype), ptr(lens), B, chunk,
         hq, int(key_3d.shape[2]), d, scale, _hip.stream_of(dev))
    return out


def paged_attention_prefill_chunk(query_3d: torch.Tensor, key_3d: torch.Tensor, value_3d: torch.Tensor,
                                  num_q_heads: int, chunk_query_lengths: Sequence[int]) -> torch.Tensor:
    """Causal attention over a freshly prefilled prompt chunk (attention.py:121-167).

    ``query_3d`` (B, chunk, Hq, d), ``key_3d``/``value_3d`` (B, chunk, Hkv, d);
    row ``b`` position ``j < chunk_query_lengths[b]`` attends ``0 .. j``; the
    padded tail is zeros. Returns (B, chunk, Hq, d).
    """
    B, chunk = int(query_3d.shape[0]), int(query_3d.shape[1])
    if int(query_3d.shape[2]) != int(num_q_heads):
        raise ValueError("query has {} heads, expected {}".format(query_3d.shape[2], num_q_heads))
    lengths = [int(x) for x in chunk_query_lengths]
    if len(lengths) != B or any(not 0 <= n <= chunk for n in lengths):
        raise ValueError("one length in [0, chunk] per batch row")
    return prefill_attention(query_3d, key_3d, value_3d, lengths)
