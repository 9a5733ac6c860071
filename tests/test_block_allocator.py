"""The product block allocator (auto_infer_amd.block_allocator) against
(1) the reference's allocator test cases, kept as data in
tests/golden/allocator.json, replayed by a small interpreter on both the
product and the oracle restatement, and (2) the oracle restatement of
auto_infer/engine/kv_cache_manager.py:4-124 on seeded random traces that
mix every operation, compared block id by block id."""
import json
import os
import re

import numpy as np
import pytest

from auto_infer_amd.block_allocator import KVCacheManager
from oracle.kv_alloc import RefKVCacheManager

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "allocator.json")
CASES = json.load(open(GOLDEN))["cases"]


def _resolve(v, saved):
    if isinstance(v, str) and v.startswith("$"):
        m = re.fullmatch(r"\$(\w+)(?:\[(\d+)\])?", v)
        val = saved[m.group(1)]
        return val[int(m.group(2))] if m.group(2) is not None else val
    if isinstance(v, list):
        return [_resolve(x, saved) for x in v]
    return v


def _replay(cls, case):
    m = cls(case["num_blocks"], case["block_size"])
    saved = {}
    for op in case["ops"]:
        args = [_resolve(a, saved) for a in op.get("args", [])]
        if "raises" in op:
            with pytest.raises(getattr(__builtins__, op["raises"], None) or eval(op["raises"])):
                getattr(m, op["op"])(*args)
            continue
        got = getattr(m, op["op"])(*args)
        if "save" in op:
            saved[op["save"]] = got
        if "expect" in op:
            assert got == _resolve(op["expect"], saved), (case["name"], op)
        if "expect_len" in op:
            assert len(got) == op["expect_len"], (case["name"], op)


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
@pytest.mark.parametrize("cls", [KVCacheManager, RefKVCacheManager], ids=["product", "oracle"])
def test_reference_allocator_cases(cls, case):
    _replay(cls, case)


def test_highest_id_first_and_last_freed_first():
    m = KVCacheManager(10, 4)
    assert m.allocate(8) == [9, 8]
    a = m.allocate(4)
    m.free(a)
    assert m.allocate(4) == a


def test_memory_error_text_matches_reference():
    m = KVCacheManager(3, 4)
    with pytest.raises(MemoryError, match=r"need 4 blocks, 3 free"):
        m.allocate(16)
    b = m.allocate(4)
    with pytest.raises(MemoryError, match=r"need 3 more blocks, 2 free"):
        m.append_slots(b, 4, 12)


def _random_trace(seed, steps, num_blocks, block_size):
    """Yield (method, args) tuples: allocate/append/free/register/match with
    prompts drawn from a few shared prefixes so hashes hit, collide in chains
    and get evicted."""
    rng = np.random.default_rng(seed)
    prefixes = [[int(x) for x in rng.integers(0, 5, size=block_size * 4)] for _ in range(4)]
    for _ in range(steps):
        r = rng.random()
        if r < 0.35:
            n = int(rng.integers(0, block_size * 6))
            base = prefixes[int(rng.integers(len(prefixes)))]
            toks = (base + [int(x) for x in rng.integers(0, 5, size=n)])[:max(n, 1)]
            yield "new", toks
        elif r < 0.55:
            yield "free", int(rng.integers(1 << 30))
        elif r < 0.70:
            yield "grow", (int(rng.integers(1 << 30)), int(rng.integers(1, block_size * 3)))
        elif r < 0.85:
            yield "register", int(rng.integers(1 << 30))
        else:
            yield "double_free", int(rng.integers(1 << 30))


def _drive(m, trace, block_size):
    """Apply a trace to allocator m; return the log of every result."""
    live, log = [], []
    for kind, arg in trace:
        if kind == "new":
            toks = list(arg)
            hit = m.match_prefix(toks)
            try:
                rest = m.allocate(max(0, len(toks) - len(hit) * block_size))
            except MemoryError as e:
                m.free(hit)
                log.append(("oom", str(e)))
                continue
            live.append([toks, hit + rest])
            log.append(("new", hit, rest, m.num_free_blocks()))
        elif not live:
            continue
        elif kind == "free":
            toks, blocks = live.pop(arg % len(live))
            m.free(blocks)
            log.append(("free", m.num_free_blocks()))
        elif kind == "double_free":
            toks, blocks = live[arg % len(live)]
            m.free([blocks[0], -1, m.num_blocks + 5] if blocks else [])
            blocks[:1] = []
            log.append(("dfree", m.num_free_blocks()))
        elif kind == "grow":
            i, n = arg
            toks, blocks = live[i % len(live)]
            try:
                add = m.append_slots(blocks, len(toks), n)
                toks.extend([7] * n)
                log.append(("grow", add))
            except MemoryError as e:
                log.append(("oom", str(e)))
        elif kind == "register":
            toks, blocks = live[arg % len(live)]
            try:
                m.register_prefix(toks, blocks)
            except IndexError:          # fewer blocks than full chunks: both raise
                log.append(("short",))
            log.append(("reg", m.num_free_blocks()))
    return log


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("num_blocks,block_size", [(24, 4), (64, 8), (200, 16)])
def test_matches_oracle_on_random_traces(seed, num_blocks, block_size):
    trace = list(_random_trace(seed, 600, num_blocks, block_size))
    got = _drive(KVCacheManager(num_blocks, block_size), trace, block_size)
    want = _drive(RefKVCacheManager(num_blocks, block_size), trace, block_size)
    assert got == want


def test_config5_fragmentation_trace_matches_oracle():
    """The allocator trace behind BASELINE config 5's block tables, at a
    reduced pool: identical block ids from both."""
    from auto_infer_amd import workloads
    lks = workloads.config5_contexts(seed=0, batch=32)
    got, _ = workloads.fragmented_block_tables(lks, num_blocks=8192, block_size=128, ops=1500)
    want, _ = workloads.fragmented_block_tables(lks, num_blocks=8192, block_size=128, ops=1500,
                                                allocator=RefKVCacheManager)
    assert got == want


@pytest.mark.parametrize("cls", [KVCacheManager, RefKVCacheManager], ids=["product", "oracle"])
def test_out_of_range_ids_in_register_prefix(cls):
    """Block ids outside the pool handed to register_prefix claim their
    hashes (as the reference's dicts keyed by block id do) but never match,
    and a negative id does not alias the pool's last block: the same log
    from the product and the oracle."""
    def drive(m):
        log = []
        toks = [1, 2, 3, 4, 5, 6]
        m.register_prefix(toks[:2], [-1])
        m.register_prefix(toks, [-1, m.num_blocks, m.num_blocks + 3])
        a = m.allocate(2)                  # the highest id: the slot -1 would alias
        log.append(a)
        m.register_prefix([9, 9], a)
        log.append(m.match_prefix(toks))   # hashes held by foreign ids: no hit
        m.free(a)
        b = m.allocate(6)
        log.append(b)
        m.register_prefix(toks, b)
        log.append(m.match_prefix(toks))
        m.free(b)
        log.append(m.allocate(8))
        log.append(m.num_free_blocks())
        return log
    got = drive(cls(8, 2))
    assert got == drive(RefKVCacheManager(8, 2))
