"""Physical KV-cache blocks of the end-to-end harness, with prefix caching.

Restates the block semantics of the reference's BlockPool (core/block.py:
20-158) and of its full-attention prefix cache (core/cache_group_manager.py:
98-132, 235-253; core/kv_cache_manager.py:113-222):

* ids ``[0, num_blocks - 1)`` are allocatable; the last id is the null block
  that pads block tables and is never handed out;
* every allocated block carries a reference count; a block whose count drops
  to zero goes to the tail of the free list but keeps its digest, so a later
  request can still hit it until an allocation takes it from the head of the
  free list (that allocation drops the digest);
* a request's complete blocks are indexed by their chained digest
  (``prefix_hash.hash_block``) after each step; if the digest is already
  indexed under another block, the request switches to that canonical block
  and releases its own;
* admission looks up the longest run of indexed digests over the request's
  first ``(known tokens - 1) // block_size`` blocks and starts the request
  after them (the scheduler's ``num_computed_tokens`` = the hit length).

The free list is an insertion-ordered dict, so taking a cached free block
out of the middle (a hit on a block nobody holds) costs O(1).
"""

from __future__ import annotations

from collections import OrderedDict
from collections.abc import Iterable, Sequence


class BlockPool:
    __slots__ = ("null_block_id", "_ref", "_digest", "_index", "_free")

    def __init__(self, num_blocks: int) -> None:
        if num_blocks < 2:
            raise ValueError("a block pool needs at least one block besides the null block")
        self.null_block_id = num_blocks - 1
        self._ref = [0] * self.null_block_id
        self._digest: list[bytes | None] = [None] * self.null_block_id
        self._index: dict[bytes, int] = {}
        self._free: OrderedDict[int, None] = OrderedDict.fromkeys(range(self.null_block_id))

    @property
    def num_free_blocks(self) -> int:
        return len(self._free)

    @property
    def num_cached_blocks(self) -> int:
        return len(self._index)

    def ref_count(self, block_id: int) -> int:
        return self._ref[block_id]

    def lookup(self, digest: bytes) -> int | None:
        """The block indexed under ``digest``, if any."""

        return self._index.get(digest)

    def can_allocate(self, count: int, cached: Sequence[int] = ()) -> bool:
        held_free = sum(1 for b in cached if self._ref[b] == 0)
        return count + held_free <= len(self._free)

    def allocate(self, count: int, cached: Sequence[int] = ()) -> list[int] | None:
        """Take a reference to every ``cached`` block and ``count`` new blocks
        from the head of the free list, or change nothing and return None."""

        if not self.can_allocate(count, cached):
            return None
        for b in cached:
            self.acquire(b)
        new = []
        for _ in range(count):
            b, _ = self._free.popitem(last=False)
            old = self._digest[b]
            if old is not None:
                if self._index.get(old) == b:
                    del self._index[old]
                self._digest[b] = None
            self._ref[b] = 1
            new.append(b)
        return new

    def acquire(self, block_id: int) -> None:
        if self._ref[block_id] == 0:
            del self._free[block_id]
        self._ref[block_id] += 1

    def release(self, block_id: int) -> None:
        self._ref[block_id] -= 1
        if self._ref[block_id] == 0:
            self._free[block_id] = None

    def release_all(self, block_ids: Iterable[int]) -> None:
        for b in block_ids:
            self.release(b)

    def index(self, block_id: int, digest: bytes) -> None:
        """Index an allocated block under ``digest`` (no reference taken)."""

        old = self._digest[block_id]
        if old is not None and self._index.get(old) == block_id:
            del self._index[old]
        self._digest[block_id] = digest
        self._index[digest] = block_id
