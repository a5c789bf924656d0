"""gfx950 paged-KV speculative-verify engine (reference: engine/)."""

from .kv import BlockAllocator, BlockExhaustedError, PagedKVCache

__all__ = ["BlockAllocator", "BlockExhaustedError", "PagedKVCache"]
