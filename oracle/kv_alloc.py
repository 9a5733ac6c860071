"""Restatement of the reference's paged KV block allocator, as a checker.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  Follows
auto_infer/engine/kv_cache_manager.py:4-124 method by method (same state
dictionaries and the same order of operations), so that a seeded trace
replayed through it yields the reference's block ids.  The product
allocator, ``auto_infer_amd.block_allocator.KVCacheManager``, is an
array-based design of the same policy and is checked against this class on
random traces (tests/test_block_allocator.py).

Policy: a LIFO free list initialised to 0..N-1 (``pop()`` from the tail,
:12,41-44); refcounts; full-block prefix hashes ``hash((prev_hash, chunk))``
with a token-tuple collision guard (:78-111); freed blocks that carry a
registered hash go to an LRU pool instead of the free list (:63-73) and are
evicted oldest-first only when the free list is empty (:34-40).
"""
from collections import OrderedDict


class RefKVCacheManager:

    def __init__(self, num_blocks: int, block_size: int):
        self.num_blocks = num_blocks
        self.block_size = block_size
        self._free = list(range(num_blocks))
        self._cached = OrderedDict()       # block -> hash, oldest first
        self._ref = {}
        self._hash_to_block = {}
        self._block_hash = {}
        self._block_tokens = {}
        self.prefix_queried_blocks = 0
        self.prefix_hit_blocks = 0

    def record_prefix_stats(self, queried_blocks: int, hit_blocks: int) -> None:
        self.prefix_queried_blocks += queried_blocks
        self.prefix_hit_blocks += hit_blocks

    def num_free_blocks(self) -> int:
        return len(self._free) + len(self._cached)

    def blocks_needed(self, num_tokens: int) -> int:
        return -(-num_tokens // self.block_size)

    def can_allocate(self, num_tokens: int) -> bool:
        return self.blocks_needed(num_tokens) <= self.num_free_blocks()

    def _take(self) -> int:
        if self._free:
            blk = self._free.pop()
        else:
            blk, h = self._cached.popitem(last=False)
            if self._hash_to_block.get(h) == blk:
                del self._hash_to_block[h]
            self._block_hash.pop(blk, None)
            self._block_tokens.pop(blk, None)
        self._ref[blk] = 1
        return blk

    def allocate(self, num_tokens: int) -> list:
        need = self.blocks_needed(num_tokens)
        if need > self.num_free_blocks():
            raise MemoryError(f"need {need} blocks, {self.num_free_blocks()} free")
        return [self._take() for _ in range(need)]

    def append_slots(self, block_ids: list, cur_num_tokens: int, num_new_tokens: int) -> list:
        extra = self.blocks_needed(cur_num_tokens + num_new_tokens) - len(block_ids)
        if extra <= 0:
            return []
        if extra > self.num_free_blocks():
            raise MemoryError(f"need {extra} more blocks, {self.num_free_blocks()} free")
        new = [self._take() for _ in range(extra)]
        block_ids.extend(new)
        return new

    def free(self, block_ids: list) -> None:
        for b in block_ids:
            if b not in self._ref:
                continue
            self._ref[b] -= 1
            if self._ref[b] > 0:
                continue
            del self._ref[b]
            if b in self._block_hash:
                self._cached[b] = self._block_hash[b]
            else:
                self._free.append(b)

    @staticmethod
    def _chunk_hash(prev: int, chunk: tuple) -> int:
        return hash((prev, chunk))

    def match_prefix(self, token_ids: list) -> list:
        bs = self.block_size
        matched, prev = [], 0
        for start in range(0, (len(token_ids) // bs) * bs, bs):
            chunk = tuple(token_ids[start:start + bs])
            h = self._chunk_hash(prev, chunk)
            blk = self._hash_to_block.get(h)
            if blk is None or self._block_tokens.get(blk) != chunk:
                break
            if blk in self._cached:
                del self._cached[blk]
                self._ref[blk] = 1
            elif blk in self._ref:
                self._ref[blk] += 1
            else:
                break
            matched.append(blk)
            prev = h
        return matched

    def register_prefix(self, token_ids: list, block_ids: list) -> None:
        bs = self.block_size
        prev = 0
        for idx in range(len(token_ids) // bs):
            chunk = tuple(token_ids[idx * bs:(idx + 1) * bs])
            h = self._chunk_hash(prev, chunk)
            blk = block_ids[idx]
            self._hash_to_block.setdefault(h, blk)
            self._block_hash.setdefault(blk, h)
            self._block_tokens[blk] = chunk
            prev = h
