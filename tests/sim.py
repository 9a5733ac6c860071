"""A tiny seeded continuous-batching simulator producing BatchPlans.

Requests arrive with random prompts, are prefilled in chunks under a token
budget (decode rows first, like the reference scheduler,
auto_infer/engine/scheduler.py:83-222), decode one token per step, may carry
MTP drafts and finish after a random number of outputs; blocks come from the
allocator mirror.  Used to drive the packers over many steps.
"""
import numpy as np

from auto_infer_amd.execution import BatchPlan, RequestView, ScheduledRequest
from auto_infer_amd.block_allocator import KVCacheManager


class _Req:
    def __init__(self, rid, prompt, max_out):
        self.rid = rid
        self.tokens = list(prompt)
        self.num_prompt = len(prompt)
        self.computed = 0
        self.max_out = max_out
        self.blocks = []
        self.draft = ()


def simulate(steps, *, seed=0, block_size=16, num_blocks=4096, budget=96, max_running=12,
             draft_depth=0, max_prompt=70):
    rng = np.random.default_rng(seed)
    kv = KVCacheManager(num_blocks, block_size)
    waiting, running, nid = [], [], 0
    for _ in range(steps):
        for _ in range(int(rng.integers(0, 3))):
            p = [int(x) for x in rng.integers(1, 30000, size=int(rng.integers(1, max_prompt)))]
            waiting.append(_Req(f"r{nid}", p, int(rng.integers(1, 12))))
            nid += 1
        sched, tok = [], 0
        for r in list(running):                    # decode rows first
            if r.computed < r.num_prompt:
                continue
            k = draft_depth if draft_depth else 0
            r.draft = tuple(int(x) for x in rng.integers(1, 30000, size=k)) if k else ()
            n = 1 + k
            kv.append_slots(r.blocks, r.computed, n)
            sched.append((r, n, False))
            tok += n
        for r in running + waiting:                # then (chunked) prefill
            if r.computed >= r.num_prompt or tok >= budget:
                continue
            if r in waiting:
                if len(running) >= max_running:
                    continue
                waiting.remove(r)
                running.append(r)
            n = min(r.num_prompt - r.computed, budget - tok)
            kv.append_slots(r.blocks, r.computed, n)
            r.draft = ()
            sched.append((r, n, True))
            tok += n
        if not sched:
            continue
        views = {r.rid: RequestView(r.rid, tuple(r.tokens), r.computed, r.num_prompt,
                                    r.num_prompt, tuple(r.draft)) for r, _, _ in sched}
        plan = BatchPlan.make([ScheduledRequest(r.rid, n, p, tuple(r.blocks)) for r, n, p in sched],
                              views, {r.rid: tuple(r.blocks) for r, _, _ in sched})
        yield plan
        for r, n, is_prefill in sched:             # commit (engine_core.py:152-192)
            if is_prefill:
                r.computed += n
                if r.computed >= r.num_prompt:
                    r.tokens.append(int(rng.integers(1, 30000)))
            else:
                accepted = int(rng.integers(0, len(r.draft) + 1)) if r.draft else 0
                r.tokens.extend(r.draft[:accepted])
                r.tokens.append(int(rng.integers(1, 30000)))
                r.computed = len(r.tokens) - 1
            if len(r.tokens) - r.num_prompt >= r.max_out:
                running.remove(r)
                kv.free(r.blocks)
