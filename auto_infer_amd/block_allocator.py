"""Paged KV block allocator with prefix caching (host side).

Produces the block tables that the packers upload.  The public surface is
the reference's ``KVCacheManager`` (auto_infer/engine/kv_cache_manager.py:
4-124): the same method names, arguments, return values and ``MemoryError``
text, and the same allocation policy, so that a seeded allocate/free trace
hands out the same block ids:

* unused blocks are taken last-freed-first, starting from the highest id
  (the reference pops the tail of ``list(range(N))``, :12,41-44);
* a block whose last reference is dropped while it carries a registered
  prefix hash stays revivable, in least-recently-freed order, and is
  reclaimed oldest-first only when no unused block is left (:34-40, 63-73);
* a full block's hash chains its predecessor's, ``hash((prev, chunk))``,
  and a match also compares the stored token chunk (:78-111).

The state lives in flat per-block arrays instead of dictionaries: a state
code and refcount per block, a stack of unused ids, and an intrusive
doubly linked list (``_prev``/``_next``, sentinel ``N``) that keeps the
revivable blocks in freeing order.  Every operation is O(1) per block, so
an 80 GB pool (150 k blocks of 512 KiB) costs a few MB of host memory and
no per-operation rehashing.
"""

_UNUSED, _ACTIVE, _CACHED = 0, 1, 2


class KVCacheManager:

    def __init__(self, num_blocks: int, block_size: int):
        n = int(num_blocks)
        self.num_blocks = n
        self.block_size = int(block_size)
        self._state = [_UNUSED] * n
        self._refs = [0] * n
        self._stack = list(range(n))      # unused ids; the top is the end
        self._prev = [n] * (n + 1)        # LRU ring of revivable blocks, sentinel n
        self._next = [n] * (n + 1)
        self._num_cached = 0
        self._hash_of = [None] * n        # registered prefix hash per block
        self._chunk_of = [None] * n       # the token chunk that hash was made from
        self._owner = {}                  # prefix hash -> block holding it
        self.prefix_queried_blocks = 0
        self.prefix_hit_blocks = 0

    # ------------------------------------------------------------ counters

    def record_prefix_stats(self, queried_blocks: int, hit_blocks: int) -> None:
        self.prefix_queried_blocks += queried_blocks
        self.prefix_hit_blocks += hit_blocks

    def num_free_blocks(self) -> int:
        return len(self._stack) + self._num_cached

    def blocks_needed(self, num_tokens: int) -> int:
        return -(-num_tokens // self.block_size)

    def can_allocate(self, num_tokens: int) -> bool:
        return self.blocks_needed(num_tokens) <= self.num_free_blocks()

    # ------------------------------------------------------ LRU ring links

    def _ring_push(self, b):
        s = self.num_blocks
        last = self._prev[s]
        self._next[last], self._prev[b] = b, last
        self._next[b], self._prev[s] = s, b
        self._num_cached += 1

    def _ring_unlink(self, b):
        p, q = self._prev[b], self._next[b]
        self._next[p], self._prev[q] = q, p
        self._num_cached -= 1

    # ---------------------------------------------------------- allocation

    def _grab(self, count):
        """``count`` blocks, each with one reference: unused ones first,
        then the least recently freed revivable ones (their registration
        is dropped)."""
        out = []
        state, refs, stack = self._state, self._refs, self._stack
        for _ in range(count):
            if stack:
                b = stack.pop()
            else:
                b = self._next[self.num_blocks]
                self._ring_unlink(b)
                h = self._hash_of[b]
                if self._owner.get(h) == b:
                    del self._owner[h]
                self._hash_of[b] = None
                self._chunk_of[b] = None
            state[b] = _ACTIVE
            refs[b] = 1
            out.append(b)
        return out

    def allocate(self, num_tokens: int) -> list:
        need = self.blocks_needed(num_tokens)
        have = self.num_free_blocks()
        if need > have:
            raise MemoryError(f"need {need} blocks, {have} free")
        return self._grab(need)

    def append_slots(self, block_ids: list, cur_num_tokens: int, num_new_tokens: int) -> list:
        """Grow ``block_ids`` in place to cover ``cur + new`` tokens; returns
        the blocks added."""
        extra = self.blocks_needed(cur_num_tokens + num_new_tokens) - len(block_ids)
        if extra <= 0:
            return []
        have = self.num_free_blocks()
        if extra > have:
            raise MemoryError(f"need {extra} more blocks, {have} free")
        added = self._grab(extra)
        block_ids.extend(added)
        return added

    def free(self, block_ids: list) -> None:
        """Drop one reference per listed block; ids that hold none are
        ignored."""
        state, refs = self._state, self._refs
        for b in block_ids:
            if not 0 <= b < self.num_blocks or state[b] != _ACTIVE:
                continue
            refs[b] -= 1
            if refs[b]:
                continue
            if self._hash_of[b] is not None:
                state[b] = _CACHED
                self._ring_push(b)
            else:
                state[b] = _UNUSED
                self._stack.append(b)

    # ----------------------------------------------------- prefix caching

    def match_prefix(self, token_ids: list) -> list:
        """Blocks holding the longest registered full-block prefix of
        ``token_ids``; each gains a reference (revivable ones come back into
        use)."""
        bs = self.block_size
        state, refs = self._state, self._refs
        hits, prev = [], 0
        for start in range(0, len(token_ids) - bs + 1, bs):
            chunk = tuple(token_ids[start:start + bs])
            h = hash((prev, chunk))
            b = self._owner.get(h)
            # an id outside the pool (registered by the caller) never matches
            if b is None or not 0 <= b < self.num_blocks or self._chunk_of[b] != chunk \
                    or state[b] == _UNUSED:
                break
            if state[b] == _CACHED:
                self._ring_unlink(b)
                state[b] = _ACTIVE
                refs[b] = 1
            else:
                refs[b] += 1
            hits.append(b)
            prev = h
        return hits

    def register_prefix(self, token_ids: list, block_ids: list) -> None:
        """Make the full blocks of ``token_ids`` (held in ``block_ids``)
        findable by ``match_prefix``.  A hash keeps its first block and a
        block its first hash; the stored chunk is always the latest."""
        bs = self.block_size
        prev = 0
        for i in range(len(token_ids) // bs):
            chunk = tuple(token_ids[i * bs:(i + 1) * bs])
            h = hash((prev, chunk))
            b = block_ids[i]
            # An id outside the pool still claims the hash (as a dict keyed by
            # block id would), but has no per-block state to update and is
            # never matched: negative ids must not alias the pool's last
            # blocks.
            self._owner.setdefault(h, b)
            if 0 <= b < self.num_blocks:
                if self._hash_of[b] is None:
                    self._hash_of[b] = h
                self._chunk_of[b] = chunk
            prev = h
