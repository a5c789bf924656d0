"""CPU restatement of the reference paged KV pool (test infrastructure only).

Follows engine/kv.py of the reference:

* ``BlockAllocator``  -- kv.py:45-76. The free list starts as ``[0 .. cap-1]``
  (kv.py:52); ``alloc`` pops the list TAIL (kv.py:68), so the first id handed out
  is ``cap-1``; ``free`` ignores ids already on the list (kv.py:73-74) and
  otherwise appends (kv.py:75). Exhaustion raises ``BlockExhaustedError``
  (kv.py:41-42, 62-67).
* ``PagedKVCache``    -- kv.py:79-224: lazy allocation in logical order
  (kv.py:119-122), per-token write (kv.py:125-147), tail-first ``truncate``
  (kv.py:150-162), forward-order ``clear`` (kv.py:164-171), table-by-table
  ``reset`` (kv.py:173-183) and the metrics (kv.py:186-224).

K/V are stored in the reference layout ``(layers, cap, block_size, kv_heads, d)``
as CPU torch tensors. The free-list membership test is the reference's linear
list scan, kept on purpose so the CPU baseline times the same algorithm.

Pinned by tests/test_oracle_kv.py: every assertion of the reference's
tests/test_kv.py:44-183 and tests/test_spec_accept.py:258-280, plus invariants
(free list + tables partition the pool, ``num_allocated == cap - len(free)``)
over random operation traces checked against an independent set-based model.
"""

from __future__ import annotations

from typing import Dict, List, Optional, Sequence, Tuple

import torch


class BlockExhaustedError(RuntimeError):
    """Raised when an allocation finds the free list empty (kv.py:41-42)."""


class BlockAllocator:
    """LIFO free list of physical block ids (kv.py:45-76)."""

    def __init__(self, capacity: int) -> None:
        if capacity < 1:
            raise ValueError("capacity_blocks must be >= 1")
        self.capacity = capacity
        self.free_list: List[int] = list(range(capacity))
        self.allocated = 0

    @property
    def num_allocated(self) -> int:
        return self.allocated

    def alloc(self) -> int:
        if not self.free_list:
            raise BlockExhaustedError(
                "paged KV block pool exhausted ({} blocks)".format(self.capacity))
        self.allocated += 1
        return self.free_list.pop()

    def free(self, block: int) -> None:
        # Linear membership scan, as in the reference (kv.py:73).
        if block in self.free_list:
            return
        self.free_list.append(block)
        self.allocated -= 1


class PagedKVCache:
    """Block tables + K/V pools (kv.py:79-224), CPU only."""

    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int,
                 capacity_blocks: int, block_size: int,
                 dtype: torch.dtype = torch.float32, store: bool = True) -> None:
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.block_size = block_size
        self.dtype = dtype
        self.allocator = BlockAllocator(capacity_blocks)
        shape = (num_layers, capacity_blocks, block_size, num_kv_heads, head_dim)
        # ``store=False`` keeps only the metadata (pool-only parity checks at
        # full pool sizes would otherwise allocate GBs of zeros on the host).
        self.k = torch.zeros(shape, dtype=dtype) if store else None
        self.v = torch.zeros(shape, dtype=dtype) if store else None
        self.block_tables: List[List[int]] = []
        self.seq_lengths: List[int] = []

    # kv.py:108-112
    def add_sequence(self, seq_id: int) -> None:
        while len(self.block_tables) <= seq_id:
            self.block_tables.append([])
            self.seq_lengths.append(0)

    @property
    def num_sequences(self) -> int:
        return len(self.seq_lengths)

    # kv.py:119-122
    def _ensure_blocks_up_to(self, seq_id: int, max_block_index: int) -> None:
        table = self.block_tables[seq_id]
        while len(table) <= max_block_index:
            table.append(self.allocator.alloc())

    # kv.py:125-147
    def write(self, layer: int, seq_id: int, token_pos: int,
              kvec: Optional[torch.Tensor], vvec: Optional[torch.Tensor]) -> None:
        bi, off = divmod(token_pos, self.block_size)
        self._ensure_blocks_up_to(seq_id, bi)
        phys = self.block_tables[seq_id][bi]
        if self.k is not None:
            self.k[layer, phys, off] = kvec
            self.v[layer, phys, off] = vvec
        if self.seq_lengths[seq_id] <= token_pos:
            self.seq_lengths[seq_id] = token_pos + 1

    def write_block(self, layer: int, seq_ids: Sequence[int],
                    start_positions: Sequence[int],
                    k_new: Optional[torch.Tensor], v_new: Optional[torch.Tensor],
                    chunk: Optional[int] = None) -> None:
        """The write loop of a verify/extend block (model.py:184-187).

        Sequences in batch order, then positions ``start+j`` in order; an
        exhausted pool raises from inside the loop, leaving earlier writes and
        allocations in place exactly as the per-token loop does.
        """
        C = int(k_new.shape[1]) if chunk is None else int(chunk)
        for b, sid in enumerate(seq_ids):
            base = int(start_positions[b])
            for j in range(C):
                kv = None if k_new is None else k_new[b, j]
                vv = None if v_new is None else v_new[b, j]
                self.write(layer, sid, base + j, kv, vv)

    # kv.py:150-162
    def truncate(self, seq_id: int, new_len: int) -> None:
        need = 0 if new_len <= 0 else -(-new_len // self.block_size)
        table = self.block_tables[seq_id]
        while len(table) > need:
            self.allocator.free(table.pop())
        self.seq_lengths[seq_id] = max(0, new_len)

    # kv.py:164-171
    def clear(self, seq_id: int) -> None:
        table = self.block_tables[seq_id] if seq_id < len(self.block_tables) else []
        for phys in table:
            self.allocator.free(phys)
        self.block_tables[seq_id] = []
        self.seq_lengths[seq_id] = 0

    # kv.py:173-183
    def reset(self) -> None:
        for table in self.block_tables:
            for phys in table:
                self.allocator.free(phys)
        self.block_tables[:] = []
        self.seq_lengths[:] = []

    # kv.py:186-205
    @property
    def num_allocated_blocks(self) -> int:
        return self.allocator.num_allocated

    @property
    def logical_tokens(self) -> int:
        return sum(self.seq_lengths)

    @property
    def block_utilization(self) -> float:
        if self.num_allocated_blocks == 0:
            return 0.0
        return float(self.logical_tokens) / float(self.num_allocated_blocks * self.block_size)

    @property
    def kv_memory_bytes(self) -> int:
        n = self.num_layers * self.allocator.capacity * self.block_size
        n *= self.num_kv_heads * self.head_dim
        return 2 * n * torch.tensor([], dtype=self.dtype).element_size()

    # kv.py:208-213
    def key_map(self, layer: int, phys: List[int]) -> torch.Tensor:
        return self.k[layer][phys]

    def value_map(self, layer: int, phys: List[int]) -> torch.Tensor:
        return self.v[layer][phys]

    # kv.py:215-224
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

    # ------------------------------------------------------------ harness
    def snapshot(self) -> Tuple[List[List[int]], List[int], List[int]]:
        """(block tables, sequence lengths, free list bottom->top) for parity."""
        return ([list(t) for t in self.block_tables], list(self.seq_lengths),
                list(self.allocator.free_list))

    def load_state(self, tables: Sequence[Sequence[int]], lengths: Sequence[int],
                   free_list: Sequence[int]) -> None:
        """Install a synthetic pool state (random-permutation tables etc.)."""
        self.block_tables = [list(map(int, t)) for t in tables]
        self.seq_lengths = [int(x) for x in lengths]
        self.allocator.free_list = [int(x) for x in free_list]
        self.allocator.allocated = self.allocator.capacity - len(self.allocator.free_list)
