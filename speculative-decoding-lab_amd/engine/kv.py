"""Paged KV cache whose pool, block tables and free list live in GPU memory.

Drop-in for the reference's engine/kv.py (same classes, constructor arguments,
methods, attributes and errors). What changes is where the state lives:

* the free list is a device stack (``free_stack[0:top]``, top = free count)
  with a per-block "is free" flag, so ``free`` keeps the reference's
  ignore-if-already-free rule (kv.py:73-74) without a list scan;
* block tables, table lengths and sequence lengths are device arrays; the host
  keeps mirrors of the lengths and the free count (exact: they follow from the
  arguments of every operation), refreshed from the device after operations
  whose inputs are device-computed (``rewind_device``);
* K pages are stored ``[layer][block][kv_head][token][d]`` and V pages
  transposed ``[layer][block][kv_head][d][token]`` so the verify-attention
  kernel feeds MFMA operands straight from HBM. ``key_map``/``value_map``
  return the reference layout ``(n, block_size, kv_heads, d)``.

Every batched operation (``write_block``, ``rewind``) is one or two kernel
launches on the current stream; there is no CPU path.
"""

from __future__ import annotations

from typing import Dict, List, Optional, Sequence

import torch

from . import _hip
from ._hip import call, ptr


class BlockExhaustedError(RuntimeError):
    """Raised when an allocation finds the free list empty (kv.py:41-42)."""


def _exhausted(capacity: int) -> BlockExhaustedError:
    return BlockExhaustedError(
        "paged KV block pool exhausted ({} blocks; raise max_num_blocks)".format(capacity))


class BlockAllocator:
    """Device LIFO free list of physical block ids (kv.py:45-76).

    ``alloc`` pops the stack top (the reference pops its list tail, so the first
    id handed out is ``capacity - 1``); ``free`` pushes unless the id is already
    free. Both return only after the device has answered (as the reference's
    return values require); batched paths never synchronise.
    """

    def __init__(self, capacity: int, device: torch.device, dtype: torch.dtype) -> None:
        if capacity < 1:
            raise ValueError("capacity_blocks must be >= 1")
        device = _hip.require_gpu(device)
        self.capacity = int(capacity)
        self._device = device
        self._dtype = dtype
        self.free_stack = torch.empty(self.capacity, dtype=torch.int32, device=device)
        self.free_flag = torch.empty(self.capacity, dtype=torch.int32, device=device)
        self.ctr = torch.zeros(_hip.SPV_CTR_WORDS, dtype=torch.int32, device=device)
        self._out = torch.zeros(2, dtype=torch.int32, device=device)
        self._free_count = self.capacity  # host mirror of ctr[0]
        self._stale = False
        # counts the calls that may free blocks (rewinds, clears, alignments,
        # frees, re-initialisation): a write plan's rows stay valid within the
        # epoch that recorded them (allocation never moves an existing row)
        self.epoch = 0
        self.reinit()

    # -- internal -------------------------------------------------------------
    def _stream(self) -> int:
        return _hip.stream_of(self._device)

    def reinit(self) -> None:
        """Free list back to ``[0 .. capacity-1]`` (kv.py:52)."""
        call("spv_pool_init", ptr(self.free_stack), ptr(self.free_flag), ptr(self.ctr),
             self.capacity, self._stream())
        self.epoch += 1
        self._free_count = self.capacity
        self._stale = False

    def _refresh(self) -> None:
        if self._stale:
            self._free_count = int(self.ctr[_hip.CTR_TOP].item())
            self._stale = False

    # -- reference API -----------------------------------------------------------
    @property
    def num_allocated(self) -> int:
        self._refresh()
        return self.capacity - self._free_count

    @property
    def num_free(self) -> int:
        self._refresh()
        return self._free_count

    def alloc(self) -> int:
        self._refresh()
        call("spv_pool_alloc_one", ptr(self.free_stack), ptr(self.free_flag), ptr(self.ctr),
             self.capacity, ptr(self._out), self._stream())
        block = int(self._out[0].item())
        if block < 0:
            self._free_count = 0
            raise _exhausted(self.capacity)
        self._free_count -= 1
        return block

    def free(self, block: int) -> None:
        block = int(block)
        if not 0 <= block < self.capacity:
            # The reference would append an out-of-range id to its list; a
            # device stack cannot hold it, so it is rejected instead.
            raise ValueError("block id {} outside the pool [0, {})".format(block, self.capacity))
        self._refresh()
        self.epoch += 1
        call("spv_pool_free_one", ptr(self.free_stack), ptr(self.free_flag), ptr(self.ctr),
             self.capacity, block, ptr(self._out[1:]), self._stream())
        if int(self._out[1].item()):
            self._free_count += 1

    # -- inspection --------------------------------------------------------------
    def free_list(self) -> List[int]:
        """The free list bottom -> top (the reference's ``_free`` list order)."""
        top = int(self.ctr[_hip.CTR_TOP].item())
        return self.free_stack[:top].tolist()

    def load_free_list(self, ids: Sequence[int]) -> None:
        """Install an explicit free list (bottom -> top); ids not listed are allocated."""
        ids_t = _hip.i32(ids, self._device)
        n = int(ids_t.numel())
        if n > self.capacity:
            raise ValueError("free list longer than the pool")
        flags = torch.zeros(self.capacity, dtype=torch.int32, device=self._device)
        if n:
            flags[ids_t.long()] = 1
            if int(flags.sum().item()) != n:
                raise ValueError("free list holds duplicate ids")
            self.free_stack[:n] = ids_t
        self.free_flag.copy_(flags)
        self.epoch += 1
        self.ctr.zero_()
        self.ctr[_hip.CTR_TOP] = n
        self._free_count = n
        self._stale = False


class PagedKVCache:
    """Physical KV pool plus per-sequence device metadata (kv.py:79-224)."""

    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int,
                 capacity_blocks: int, block_size: int, device: torch.device,
                 dtype: torch.dtype, max_seqs: int = 64,
                 max_blocks_per_seq: Optional[int] = None) -> None:
        device = _hip.require_gpu(device)
        if num_layers < 1 or num_kv_heads < 1 or head_dim < 1 or block_size < 1:
            raise ValueError("num_layers, num_kv_heads, head_dim and block_size must be >= 1")
        self.num_layers = int(num_layers)
        self.num_kv_heads = int(num_kv_heads)
        self.head_dim = int(head_dim)
        self.block_size = int(block_size)
        self.device = device
        self.dtype = dtype
        self._dt = _hip.dtype_code(dtype)
        self.allocator = BlockAllocator(capacity_blocks, device, dtype)
        cap = self.allocator.capacity
        self.fp8 = self._dt == _hip.SPV_FP8E4M3
        # fp8 pools hold e4m3 codes (zero bytes at start) and one fp32 scale
        # per (layer, block, K | V).
        store = torch.uint8 if self.fp8 else dtype
        self.k_pool = torch.zeros((num_layers, cap, num_kv_heads, block_size, head_dim),
                                  dtype=store, device=device)
        self.v_pool = torch.zeros((num_layers, cap, num_kv_heads, head_dim, block_size),
                                  dtype=store, device=device)
        if self.fp8:
            self.k_pool = self.k_pool.view(dtype)
            self.v_pool = self.v_pool.view(dtype)
        self.scales = torch.zeros((num_layers, cap, 2), dtype=torch.float32, device=device) if self.fp8 else None
        self._max_seqs = max(1, int(max_seqs))
        self._maxb = int(max_blocks_per_seq) if max_blocks_per_seq else min(cap, 64)
        self.tables_dev = torch.full((self._max_seqs, self._maxb), -1, dtype=torch.int32, device=device)
        self.nblocks_dev = torch.zeros(self._max_seqs, dtype=torch.int32, device=device)
        self.lens_dev = torch.zeros(self._max_seqs, dtype=torch.int32, device=device)
        self._nb: List[int] = []     # host mirror of table lengths
        self._lens: List[int] = []   # host mirror of sequence lengths
        self._stale = False

    # ----------------------------------------------------------- internals
    def _stream(self) -> int:
        return _hip.stream_of(self.device)

    @property
    def max_blocks_per_seq(self) -> int:
        return self._maxb

    def _refresh(self) -> None:
        if self._stale:
            n = len(self._nb)
            self._nb = self.nblocks_dev[:n].tolist()
            self._lens = self.lens_dev[:n].tolist()
            self.allocator._stale = True
            self.allocator._refresh()
            self._stale = False
            ctr = self.allocator.ctr.tolist()
            words = (_hip.CTR_EXHAUSTED, _hip.CTR_OVERFLOW, _hip.CTR_BAD_READ, _hip.CTR_ALIGN)
            if not any(ctr[w] for w in words):
                return
            # One error is raised; the others set since the last query follow
            # from it (an exhausted or full table leaves keys unwritten that a
            # later attention then reads), so all are cleared.
            for w in words:
                if ctr[w]:
                    self.allocator.ctr[w] = 0
            if ctr[_hip.CTR_EXHAUSTED]:
                raise _exhausted(self.allocator.capacity)
            if ctr[_hip.CTR_OVERFLOW]:
                raise IndexError("batch entry {}: the chunk needs more than max_blocks_per_seq={} blocks; "
                                 "its table was filled and the tokens beyond it were not written".format(
                                     ctr[_hip.CTR_OVERFLOW] - 1, self._maxb))
            if ctr[_hip.CTR_BAD_READ]:
                raise IndexError("batch entry {}: verify attention read positions that were never written "
                                 "(or a block id outside the pool, or beyond max_ctx)".format(
                                     ctr[_hip.CTR_BAD_READ] - 1))
            raise ValueError("batch entry {}: the draft cache is shorter than the round's start position; "
                             "its catch-up needs tokens from before the round".format(ctr[_hip.CTR_ALIGN] - 1))

    def _grow_rows(self, n: int) -> None:
        if n <= self._max_seqs:
            return
        new = max(n, 2 * self._max_seqs)
        t = torch.full((new, self._maxb), -1, dtype=torch.int32, device=self.device)
        t[: self._max_seqs] = self.tables_dev
        nb = torch.zeros(new, dtype=torch.int32, device=self.device)
        nb[: self._max_seqs] = self.nblocks_dev
        ln = torch.zeros(new, dtype=torch.int32, device=self.device)
        ln[: self._max_seqs] = self.lens_dev
        self.tables_dev, self.nblocks_dev, self.lens_dev = t, nb, ln
        self._max_seqs = new

    def _grow_width(self, blocks: int) -> None:
        if blocks <= self._maxb:
            return
        new = min(max(blocks, 2 * self._maxb), max(blocks, self.allocator.capacity))
        t = torch.full((self._max_seqs, new), -1, dtype=torch.int32, device=self.device)
        t[:, : self._maxb] = self.tables_dev
        self.tables_dev = t
        self._maxb = new

    def _check_sid(self, seq_id: int) -> int:
        seq_id = int(seq_id)
        if not 0 <= seq_id < len(self._nb):
            raise IndexError("sequence {} was never added".format(seq_id))
        return seq_id

    # ------------------------------------------------------------- sequences
    def add_sequence(self, seq_id: int) -> None:
        """Register an empty sequence (kv.py:108-112)."""
        self._refresh()
        seq_id = int(seq_id)
        if seq_id >= len(self._nb):
            self._grow_rows(seq_id + 1)
            grow = seq_id + 1 - len(self._nb)
            self._nb.extend([0] * grow)
            self._lens.extend([0] * grow)

    @property
    def num_sequences(self) -> int:
        return len(self._nb)

    @property
    def seq_lengths(self) -> List[int]:
        """Valid logical positions per sequence (kv.py:104-105); a snapshot list."""
        self._refresh()
        return list(self._lens)

    @property
    def block_tables(self) -> List[List[int]]:
        """Physical blocks per sequence in logical order (kv.py:102-103); reads the device."""
        self._refresh()
        n = len(self._nb)
        if n == 0:
            return []
        rows = self.tables_dev[:n].tolist()
        return [row[: self._nb[i]] for i, row in enumerate(rows)]

    # ------------------------------------------------------------ write path
    def _plan_alloc(self, seq_ids: Sequence[int], starts: Sequence[int], chunk: int):
        """Host mirror of the device allocation: per-sequence grants and the failing index."""
        bs = self.block_size
        free = self.allocator.num_free
        grants, fail = [], len(seq_ids)
        for b, sid in enumerate(seq_ids):
            need = max(0, (int(starts[b]) + chunk - 1) // bs + 1 - self._nb[sid])
            got = min(need, free)
            free -= got
            grants.append(got)
            if got < need and fail == len(seq_ids):
                fail = b
        return grants, fail

    def _append(self, layer: int, seq_ids: Sequence[int], starts: Sequence[int],
                k_new: Optional[torch.Tensor], v_new: Optional[torch.Tensor], chunk: int) -> None:
        self._refresh()
        if not 0 <= int(layer) < self.num_layers:
            raise IndexError("layer {} out of range".format(layer))
        seq_ids = [self._check_sid(s) for s in seq_ids]
        if len(set(seq_ids)) != len(seq_ids):
            raise ValueError("a batched write needs distinct sequence ids")
        starts = [int(s) for s in starts]
        if any(s < 0 for s in starts):
            raise ValueError("start positions must be >= 0")
        B = len(seq_ids)
        if B == 0 or chunk == 0:
            return
        bs = self.block_size
        grants, fail = self._plan_alloc(seq_ids, starts, chunk)
        self._grow_width(max(self._nb[s] + g for s, g in zip(seq_ids, grants)))
        if k_new is not None:
            shape = (B, chunk, self.num_kv_heads, self.head_dim)
            if tuple(k_new.shape) != shape or tuple(v_new.shape) != shape:
                raise ValueError("k/v must have shape {}".format(shape))
            if k_new.device != self.device or v_new.device != self.device:
                raise ValueError("k/v must live on {}".format(self.device))
            k_new, v_new = self._new_kv(k_new, v_new)
        sid_t = _hip.i32(seq_ids, self.device)
        start_t = _hip.i32(starts, self.device)
        self._launch_append(layer, sid_t, start_t, k_new, v_new, B, chunk, 1 if sum(grants) else 0, fail)
        # Mirrors: allocation, then the lengths the (possibly truncated) writes reach.
        for b, sid in enumerate(seq_ids):
            self._nb[sid] += grants[b]
            self.allocator._free_count -= grants[b]
            if k_new is None or b > fail:
                continue
            last = min(chunk - 1, self._nb[sid] * bs - 1 - starts[b])
            if last >= 0:
                self._lens[sid] = max(self._lens[sid], starts[b] + last + 1)
        if fail < B:
            raise _exhausted(self.allocator.capacity)

    def write_block_device(self, layer: int, seq_ids: torch.Tensor, start_positions: torch.Tensor,
                           k_new: torch.Tensor, v_new: torch.Tensor, alloc: bool = True,
                           plan: Optional["WritePlan"] = None) -> None:
        """``write_block`` with int32 device ``seq_ids``/``start_positions`` and no host sync.

        The allocation decides on the device which sequence (if any) exhausts
        the pool and limits the writes exactly as ``write_block`` does; the host
        learns of it -- ``BlockExhaustedError`` -- at the next metadata query. The
        caller guarantees distinct, added sequence ids and that every table fits
        ``max_blocks_per_seq`` blocks. ``alloc=False`` skips the allocation for
        a chunk whose blocks an earlier call allocated (the same ids and starts
        in an earlier layer) and applies that call's exhaustion verdict.

        ``plan`` (a ``WritePlan``): with ``alloc`` the call records the rows of
        the chunk's tokens into it; without, a recorded plan of the same chunk
        replaces the table lookups (the round's later layers: one round trip,
        ``spv_kv_write_planned``). fp8 pools, and chunks the planned copy does
        not take, ignore it.
        """
        B, chunk = int(k_new.shape[0]), int(k_new.shape[1])
        if B == 0:
            return
        k_new, v_new = self._new_kv(k_new, v_new)
        if plan is not None and not self.fp8 and self._plannable(chunk):
            if alloc:
                plan._reserve(B, chunk, self.device)
                a = self.allocator
                call("spv_kv_append_plan", ptr(self.k_pool), ptr(self.v_pool), self._dt, ptr(k_new), ptr(v_new),
                     ptr(self.tables_dev), self._maxb, ptr(self.nblocks_dev), ptr(self.lens_dev),
                     ptr(a.free_stack), ptr(a.free_flag), ptr(a.ctr), ptr(seq_ids), ptr(start_positions), B, chunk,
                     int(layer), a.capacity, self.block_size, self.num_kv_heads, self.head_dim, 1, -1,
                     ptr(plan.rows), self._stream())
                plan._record(self.allocator.epoch, seq_ids, start_positions)
                self._stale = True
                self.allocator._stale = True
                return
            if plan.ready:
                if (B, chunk) != (plan.B, plan.C):
                    raise ValueError("the chunk ({}, {}) does not match its write plan ({}, {})".format(
                        B, chunk, plan.B, plan.C))
                if plan.epoch != self.allocator.epoch or plan.key != WritePlan._key(seq_ids, start_positions):
                    raise ValueError("the write plan was recorded for another chunk, or before a later "
                                     "call that may have freed its blocks")
                call("spv_kv_write_planned", ptr(self.k_pool), ptr(self.v_pool), self._dt, ptr(k_new), ptr(v_new),
                     ptr(plan.rows), B, chunk, int(layer), self.allocator.capacity, self.block_size,
                     self.num_kv_heads, self.head_dim, self._stream())
                return
        self._launch_append(layer, seq_ids, start_positions, k_new, v_new, B, chunk, 1 if alloc else 0, -1)
        self._stale = True
        self.allocator._stale = True

    def _plannable(self, chunk: int) -> bool:
        """Whether spv_kv_write_planned takes this pool's chunks of ``chunk`` tokens."""
        es = self.k_pool.element_size()
        return (chunk <= 64 and (self.head_dim * es) % 16 == 0 and chunk * self.head_dim * es <= 16384
                and self.allocator.capacity * self.block_size < 2 ** 31)

    def _new_kv(self, k_new: torch.Tensor, v_new: torch.Tensor):
        """New keys / values as the append takes them: the pool dtype, or for an
        fp8 pool the caller's f32 / bf16 / f16 (quantised on the device)."""
        if self.fp8:
            if k_new.dtype not in (torch.float32, torch.bfloat16, torch.float16) or v_new.dtype != k_new.dtype:
                raise ValueError("an fp8 pool takes new keys / values in float32, bfloat16 or float16")
            return k_new.contiguous(), v_new.contiguous()
        return k_new.to(self.dtype).contiguous(), v_new.to(self.dtype).contiguous()

    def _launch_append(self, layer, sid_t, start_t, k_new, v_new, B, chunk, may_alloc, limit) -> None:
        a = self.allocator
        if self.fp8:
            new_dt = _hip.dtype_code(k_new.dtype) if k_new is not None else 0
            call("spv_kv_append_fp8", ptr(self.k_pool), ptr(self.v_pool), ptr(self.scales), new_dt, ptr(k_new),
                 ptr(v_new), ptr(self.tables_dev), self._maxb, ptr(self.nblocks_dev), ptr(self.lens_dev),
                 ptr(a.free_stack), ptr(a.free_flag), ptr(a.ctr), ptr(sid_t), ptr(start_t), B, chunk, int(layer),
                 self.num_layers, a.capacity, self.block_size, self.num_kv_heads, self.head_dim, may_alloc, limit,
                 self._stream())
            return
        call("spv_kv_append", ptr(self.k_pool), ptr(self.v_pool), self._dt, ptr(k_new), ptr(v_new),
             ptr(self.tables_dev), self._maxb, ptr(self.nblocks_dev), ptr(self.lens_dev),
             ptr(a.free_stack), ptr(a.free_flag), ptr(a.ctr), ptr(sid_t), ptr(start_t), B, chunk, int(layer),
             a.capacity, self.block_size, self.num_kv_heads, self.head_dim, may_alloc, limit, self._stream())

    def _ensure_blocks_up_to(self, seq_id: int, max_block_index: int) -> None:
        """Lazily extend a table to cover ``max_block_index`` (kv.py:119-122)."""
        self._append(0, [seq_id], [int(max_block_index) * self.block_size], None, None, 1)

    def write(self, layer: int, seq_id: int, token_pos: int, kvec: torch.Tensor,
              vvec: torch.Tensor) -> None:
        """Store one token's ``(num_kv_heads, head_dim)`` K/V (kv.py:125-147)."""
        self._append(layer, [seq_id], [token_pos], kvec.reshape(1, 1, *kvec.shape[-2:]),
                     vvec.reshape(1, 1, *vvec.shape[-2:]), 1)

    def write_block(self, layer: int, seq_ids: Sequence[int], start_positions: Sequence[int],
                    k_new: torch.Tensor, v_new: torch.Tensor) -> None:
        """The whole per-token write loop of an extend block (model.py:184-187) in one launch.

        ``k_new``/``v_new`` are ``(B, chunk, num_kv_heads, head_dim)``. Sequence
        ``b`` writes positions ``start_positions[b] + j``; on pool exhaustion the
        state is exactly what the per-token loop leaves when ``write`` raises.
        """
        self._append(layer, seq_ids, start_positions, k_new, v_new, int(k_new.shape[1]))

    # ------------------------------------------------------------ rollback
    def rewind(self, seq_ids: Sequence[int], new_lens: Optional[Sequence[int]] = None,
               finished: Optional[Sequence[int]] = None, shrink_only: bool = False) -> None:
        """Per entry, in order: truncate to ``new_lens[i]`` (skipped when < 0), then
        clear if ``finished[i]`` -- the commit of engine/spec_scheduler.py:302-322."""
        self._refresh()
        seq_ids = [self._check_sid(s) for s in seq_ids]
        if len(set(seq_ids)) != len(seq_ids):
            raise ValueError("a batched rewind needs distinct sequence ids")
        n = len(seq_ids)
        if n == 0:
            return
        nl = [-1] * n if new_lens is None else [int(x) for x in new_lens]
        fin = [0] * n if finished is None else [1 if f else 0 for f in finished]
        sid_t = _hip.i32(seq_ids, self.device)
        nl_t = _hip.i32(nl, self.device)
        fin_t = _hip.i32(fin, self.device)
        self.allocator.epoch += 1
        call("spv_kv_rewind", ptr(self.tables_dev), self._maxb, ptr(self.nblocks_dev),
             ptr(self.lens_dev), ptr(self.allocator.free_stack), ptr(self.allocator.free_flag),
             ptr(self.allocator.ctr), ptr(sid_t), ptr(nl_t), ptr(fin_t), n, self.allocator.capacity, self.block_size,
             1 if shrink_only else 0, self._stream())
        bs = self.block_size
        for i, sid in enumerate(seq_ids):
            nb, ln = self._nb[sid], self._lens[sid]
            freed = 0
            if nl[i] >= 0 and (not shrink_only or ln > nl[i]):
                need = 0 if nl[i] <= 0 else -(-nl[i] // bs)
                freed = max(0, nb - need)
                nb -= freed
                ln = max(0, nl[i])
            if fin[i]:
                freed += nb
                nb, ln = 0, 0
            self._nb[sid], self._lens[sid] = nb, ln
            self.allocator._free_count += freed

    def rewind_device(self, seq_ids: torch.Tensor, new_lens: torch.Tensor,
                      finished: torch.Tensor, shrink_only: bool = False) -> None:
        """``rewind`` with device-resident inputs (e.g. the outputs of verify sampling).

        No host synchronisation; the host mirrors are refreshed lazily on the next
        query. ``seq_ids`` must be distinct and already added.
        """
        n = int(seq_ids.numel())
        if n == 0:
            return
        self.allocator.epoch += 1
        call("spv_kv_rewind", ptr(self.tables_dev), self._maxb, ptr(self.nblocks_dev),
             ptr(self.lens_dev), ptr(self.allocator.free_stack), ptr(self.allocator.free_flag),
             ptr(self.allocator.ctr), ptr(seq_ids), ptr(new_lens), ptr(finished), n,
             self.allocator.capacity, self.block_size, 1 if shrink_only else 0, self._stream())
        self._stale = True
        self.allocator._stale = True

    def rewind_append_device(self, seq_ids: torch.Tensor, new_lens: Optional[torch.Tensor],
                             finished: Optional[torch.Tensor], start_positions: torch.Tensor,
                             k_new: torch.Tensor, v_new: torch.Tensor, layer: int = 0,
                             plan: Optional["WritePlan"] = None) -> None:
        """``rewind_device(seq_ids, new_lens, finished)`` followed by the allocating
        ``write_block_device(layer, seq_ids, start_positions, k_new, v_new, plan=plan)``
        of the same batch, in one launch (``spv_kv_rewind_append``).

        The commit of one round (engine/spec_scheduler.py:296-322) meets the next
        round's first-layer append (engine/model.py:184-187) when no request is
        admitted in between. Tables, lengths, free list, stored keys and values
        and the write plan equal the two calls' results in every case. No host
        sync; distinct, added sequence ids; not for fp8 pools.
        """
        if self.fp8:
            raise ValueError("rewind_append_device does not take fp8 pools; use rewind_device + write_block_device")
        if not 0 <= int(layer) < self.num_layers:
            raise IndexError("layer {} out of range".format(layer))
        B, chunk = int(k_new.shape[0]), int(k_new.shape[1])
        shape = (B, chunk, self.num_kv_heads, self.head_dim)
        if tuple(k_new.shape) != shape or tuple(v_new.shape) != shape:
            raise ValueError("k/v must have shape {}".format(shape))
        for name, t in (("seq_ids", seq_ids), ("start_positions", start_positions), ("new_lens", new_lens),
                        ("finished", finished)):
            if t is not None and (t.dtype != torch.int32 or t.numel() != B or t.device != self.device):
                raise ValueError("{} must be {} int32 entries on {}".format(name, B, self.device))
        if B == 0:
            return
        k_new, v_new = self._new_kv(k_new, v_new)
        rows = None
        if plan is not None and self._plannable(chunk):
            plan._reserve(B, chunk, self.device)
            rows = plan.rows
        a = self.allocator
        a.epoch += 1
        call("spv_kv_rewind_append", ptr(self.k_pool), ptr(self.v_pool), self._dt, ptr(k_new), ptr(v_new),
             ptr(self.tables_dev), self._maxb, ptr(self.nblocks_dev), ptr(self.lens_dev),
             ptr(a.free_stack), ptr(a.free_flag), ptr(a.ctr), ptr(seq_ids), ptr(new_lens), ptr(finished),
             ptr(start_positions), B, chunk, int(layer), a.capacity, self.block_size, self.num_kv_heads,
             self.head_dim, ptr(rows), self._stream())
        if rows is not None:
            plan._record(a.epoch, seq_ids, start_positions)
        self._stale = True
        self.allocator._stale = True

    def align_device(self, seq_ids: torch.Tensor, start_pos: torch.Tensor, n_commit: torch.Tensor,
                     finished: torch.Tensor, chunk_tokens: torch.Tensor, catch_n: torch.Tensor,
                     catch_pos: torch.Tensor, catch_tok: torch.Tensor, max_len: Optional[int] = None) -> None:
        """Align this (draft) cache with a round's commit on the device
        (engine/spec_scheduler.py:296-322): truncate to ``start + n_commit``,
        or allocate and lengthen for the catch-up positions (reported in
        ``catch_*`` for the draft model to decode), then clear the finished
        sequences -- in the reference's per-sequence order. ``max_len`` (a bound
        on ``start + n_commit``) widens the tables beforehand; without it a
        catch-up beyond the table width is capped and reported. No host
        synchronisation."""
        n = int(seq_ids.numel())
        if n == 0:
            return
        if n > 1024:
            raise ValueError("draft alignment takes at most 1024 sequences per call")
        C = int(chunk_tokens.shape[1])
        if max_len is not None:
            self._grow_width(-(-int(max_len) // self.block_size))
        self.allocator.epoch += 1
        call("spv_kv_draft_align", ptr(self.tables_dev), self._maxb, ptr(self.nblocks_dev), ptr(self.lens_dev),
             ptr(self.allocator.free_stack), ptr(self.allocator.free_flag), ptr(self.allocator.ctr), ptr(self.scales),
             self.num_layers, ptr(seq_ids), ptr(start_pos), ptr(n_commit), ptr(finished), ptr(chunk_tokens), C,
             ptr(catch_n), ptr(catch_pos), ptr(catch_tok), n, self.allocator.capacity, self.block_size,
             self._stream())
        self._stale = True
        self.allocator._stale = True

    def metrics_device(self, record: torch.Tensor, peak: Optional[torch.Tensor] = None,
                       n_commit: Optional[torch.Tensor] = None, finished: Optional[torch.Tensor] = None,
                       batch: int = 0) -> None:
        """Write one round's metrics record on the device (no host read):
        ``record`` (6 int64) = allocated blocks, logical tokens, longest
        sequence, ``batch``, sum of ``n_commit``, finished count; ``peak`` (1
        int64) tracks the most blocks allocated (engine/spec_scheduler.py:200-205,
        engine/kv.py:186-224)."""
        rows = len(self._nb)
        call("spv_pool_metrics", ptr(self.allocator.ctr), ptr(self.lens_dev), rows, self.allocator.capacity,
             ptr(n_commit), ptr(finished), int(batch), ptr(record), ptr(peak), self._stream())

    def truncate(self, seq_id: int, new_len: int) -> None:
        """Rewind to ``new_len`` positions, freeing the table tail tail-first (kv.py:150-162)."""
        self.rewind([seq_id], [int(new_len)], None)
        self._sync_pushes()

    def clear(self, seq_id: int) -> None:
        """Free every block of a sequence in forward order (kv.py:164-171)."""
        self._refresh()
        if int(seq_id) >= len(self._nb):
            return
        self.rewind([seq_id], None, [1])
        self._sync_pushes()

    def reset(self) -> None:
        """Free every table in sequence order and forget all sequences (kv.py:173-183)."""
        self._refresh()
        n = len(self._nb)
        if n:
            self.rewind(list(range(n)), None, [1] * n)
            self._sync_pushes()
        self._nb, self._lens = [], []

    def _sync_pushes(self) -> None:
        # Single-sequence calls are synchronous in the reference; reading the
        # device count back here also keeps the mirror exact if a block was freed
        # through the allocator while still listed in a table.
        self.allocator._stale = True
        self.allocator._refresh()

    # --------------------------------------------------------------- metrics
    @property
    def num_allocated_blocks(self) -> int:
        return self.allocator.num_allocated

    @property
    def logical_tokens(self) -> int:
        self._refresh()
        return sum(self._lens)

    @property
    def block_utilization(self) -> float:
        """Fraction of allocated block slots holding a token (kv.py:194-201)."""
        allocated = self.num_allocated_blocks
        if allocated == 0:
            return 0.0
        return float(self.logical_tokens) / float(allocated * self.block_size)

    @property
    def kv_memory_bytes(self) -> int:
        scales = 0 if self.scales is None else self.scales.numel() * 4
        return 2 * self.k_pool.numel() * self.k_pool.element_size() + scales

    # ------------------------------------------------------ read (for attention)
    def _read_blocks(self, layer: int, phys: List[int], is_value: int) -> torch.Tensor:
        ids = _hip.i32(phys, self.device)
        out = torch.empty((len(phys), self.block_size, self.num_kv_heads, self.head_dim),
                          dtype=self.dtype, device=self.device)
        pool = self.v_pool if is_value else self.k_pool
        call("spv_kv_read_blocks", ptr(pool), is_value, self._dt, ptr(ids), len(phys), int(layer),
             self.allocator.capacity, self.block_size, self.num_kv_heads, self.head_dim, ptr(out),
             self._stream())
        return out

    def key_map(self, layer: int, phys: List[int]) -> torch.Tensor:
        """K of the listed blocks, ``(n, block_size, kv_heads, d)`` (kv.py:208-210)."""
        return self._read_blocks(layer, list(phys), 0)

    def value_map(self, layer: int, phys: List[int]) -> torch.Tensor:
        """V of the listed blocks, ``(n, block_size, kv_heads, d)`` (kv.py:212-213)."""
        return self._read_blocks(layer, list(phys), 1)

    def kv_stats(self) -> Optional[Dict[str, float]]:
        if self.num_sequences == 0:
            return None
        return {
            "num_allocated_blocks": self.num_allocated_blocks,
            "logical_tokens": self.logical_tokens,
            "block_utilization": round(self.block_utilization, 4),
            "kv_memory_bytes": self.kv_memory_bytes,
            "max_seq_len": max(self.seq_lengths),
        }

    # ----------------------------------------------------------- harness
    def load_state(self, tables: Sequence[Sequence[int]], lengths: Sequence[int],
                   free_list: Sequence[int]) -> None:
        """Install a pool state (e.g. random-permutation tables) on the device.

        ``tables[s]`` lists sequence s's blocks; ``free_list`` is bottom -> top.
        """
        n = len(tables)
        self._nb, self._lens = [], []
        self.add_sequence(n - 1) if n else None
        width = max([len(t) for t in tables] + [1])
        self._grow_width(width)
        rows = torch.full((self._max_seqs, self._maxb), -1, dtype=torch.int32)
        for s, t in enumerate(tables):
            if len(t):
                rows[s, : len(t)] = torch.tensor(list(t), dtype=torch.int32)
        self.tables_dev.copy_(rows.to(self.device))
        nb = torch.zeros(self._max_seqs, dtype=torch.int32)
        nb[:n] = torch.tensor([len(t) for t in tables], dtype=torch.int32)
        ln = torch.zeros(self._max_seqs, dtype=torch.int32)
        ln[:n] = torch.tensor([int(x) for x in lengths], dtype=torch.int32)
        self.nblocks_dev.copy_(nb.to(self.device))
        self.lens_dev.copy_(ln.to(self.device))
        self._nb = [len(t) for t in tables]
        self._lens = [int(x) for x in lengths]
        self.allocator.load_free_list(free_list)
        self._stale = False


class WritePlan:
    """The pool rows one round's chunk was written to by its first layer's
    append (``write_block_device(..., alloc=True, plan=...)``), for the same
    chunk's appends into the round's later layers. A buffer of B x C int32 on
    the device, reused across rounds; ``ready`` once recorded. A planned write
    must pass the very ``seq_ids`` / ``start_positions`` tensors the recording
    call took (unchanged since) and come before any later call that may free
    blocks (a rewind, clear, alignment or free); otherwise it raises instead of
    copying into rows that belong to another chunk."""

    def __init__(self):
        self.rows: Optional[torch.Tensor] = None
        self.B = self.C = 0
        self.ready = False
        self.epoch = -1
        self.key = None

    @staticmethod
    def _key(seq_ids: torch.Tensor, starts: torch.Tensor):
        return (seq_ids.data_ptr(), seq_ids._version, starts.data_ptr(), starts._version)

    def _reserve(self, B: int, C: int, device) -> None:
        if self.rows is None or self.rows.numel() < B * C or self.rows.device != device:
            self.rows = torch.empty(max(B * C, 64), dtype=torch.int32, device=device)
        self.B, self.C = B, C
        self.ready = False

    def _record(self, epoch: int, seq_ids: torch.Tensor, starts: torch.Tensor) -> None:
        self.epoch = epoch
        self.key = WritePlan._key(seq_ids, starts)
        self.ready = True
