"""Seeded random steps through the whole GQA path (planner routing, split-K
segments and their padding, row blocks, prefill items and their key chunks,
merge) against the oracle, plus the fused KV write against the oracle write.

Each case draws: heads (group 1..32, 20 and 24 among them), block size, a batch mixing decode,
verify (2-4 tokens) and prefill chunks (with and without a prefix), and
optionally a forced range count.  Sizes keep the float32 oracle to well
under a second per case.
"""
import math
import random

import pytest
import torch

from auto_infer_amd import ops, workloads
from oracle.paged_attn import kv_write, paged_attention

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 2e-2

HEADS = [(8, 8), (16, 8), (16, 4), (28, 4), (32, 8), (64, 4), (32, 1), (64, 2), (40, 2), (24, 1)]
BLOCKS = [4, 16, 32, 64, 128, 256]


def draw(seed):
    r = random.Random(seed)
    hq, hkv = r.choice(HEADS)
    bs = r.choice(BLOCKS)
    B = r.randint(1, 12)
    lqs, lks = [], []
    for _ in range(B):
        kind = r.random()
        if kind < 0.45:
            lq = 1
        elif kind < 0.65:
            lq = r.randint(2, 4)
        else:
            lq = r.randint(5, 300)
        prefix = 0 if r.random() < 0.2 else r.randint(0, 3000)
        lqs.append(lq)
        lks.append(lq + prefix)
    waves = r.choice([0, 0, 0, 1, 3, 64, 700])
    fused = r.random() < 0.5
    return dict(hq=hq, hkv=hkv, bs=bs, lqs=lqs, lks=lks, waves=waves, fused=fused)


@pytest.mark.parametrize("seed", range(120))
def test_random_steps_match_the_oracle(seed):
    c = draw(1000 + seed)
    print(f"case {seed}: {c}", flush=True)
    step = workloads.make_gqa_step(lqs=c["lqs"], lks=c["lks"], num_q_heads=c["hq"],
                                   num_kv_heads=c["hkv"], block_size=c["bs"], seed=seed,
                                   extra_blocks=3)
    kc, vc = step.k_cache.to(DEV), step.v_cache.to(DEV)
    plan = ops.AttentionPlan.from_lists(step.block_table.to(DEV), step.cu_seqlens_q,
                                        step.seqlens_kv, c["hq"], c["hkv"], 128, c["bs"],
                                        num_waves=c["waves"])
    ek, ev = step.k_cache, step.v_cache
    if c["fused"]:
        ek, ev = ek.clone(), ev.clone()
        kv_write(step.k_new, step.v_new, ek, ev, step.slot_mapping)
        out = ops.paged_attention_gqa(step.q.to(DEV), kc, vc, plan, step.scale,
                                      key_new=step.k_new.to(DEV), value_new=step.v_new.to(DEV))
    else:
        out = ops.paged_attention_gqa(step.q.to(DEV), kc, vc, plan, step.scale)
    torch.cuda.synchronize()
    if c["fused"]:
        assert torch.equal(kc.cpu(), ek) and torch.equal(vc.cpu(), ev)
    exp = paged_attention(step.q, ek, ev, step.block_table, step.cu_seqlens_q, step.seqlens_kv,
                          step.scale)
    err = (out.float().cpu() - exp).abs().max().item()
    print(f"max-abs err {err:.3e}", flush=True)
    assert err <= TOL


def draw_small_decode(seed):
    r = random.Random(seed)
    hq, hkv = r.choice(HEADS + [(16, 8), (16, 8), (24, 12), (8, 4)])
    bs = r.choice(BLOCKS)
    B = r.randint(1, 24)
    lqs = [1 if r.random() < 0.7 else r.randint(2, 3) for _ in range(B)]
    lks = [lq + r.randint(0, 2500) for lq in lqs]
    waves = r.choice([0, 0, 5, 32, 128, 256, 1000])
    return dict(hq=hq, hkv=hkv, bs=bs, lqs=lqs, lks=lks, waves=waves, fused=r.random() < 0.5)


@pytest.mark.parametrize("seed", range(60))
def test_random_small_decode_steps_match_the_oracle(seed):
    """Decode and short-verify steps of at most 24 requests: the small-step
    planner, its fixed partial slots (header word 10) where every segment has
    at most 32 ranges, and the fixed-slot or record-driven merge."""
    c = draw_small_decode(5000 + seed)
    step = workloads.make_gqa_step(lqs=c["lqs"], lks=c["lks"], num_q_heads=c["hq"],
                                   num_kv_heads=c["hkv"], block_size=c["bs"], seed=seed,
                                   extra_blocks=3)
    kc, vc = step.k_cache.to(DEV), step.v_cache.to(DEV)
    plan = ops.AttentionPlan.from_lists(step.block_table.to(DEV), step.cu_seqlens_q,
                                        step.seqlens_kv, c["hq"], c["hkv"], 128, c["bs"],
                                        num_waves=c["waves"])
    ek, ev = step.k_cache, step.v_cache
    if c["fused"]:
        ek, ev = ek.clone(), ev.clone()
        kv_write(step.k_new, step.v_new, ek, ev, step.slot_mapping)
        out = ops.paged_attention_gqa(step.q.to(DEV), kc, vc, plan, step.scale,
                                      key_new=step.k_new.to(DEV), value_new=step.v_new.to(DEV))
    else:
        out = ops.paged_attention_gqa(step.q.to(DEV), kc, vc, plan, step.scale)
    torch.cuda.synchronize()
    fixed = int(plan.workspace[:64].cpu().view(torch.int32)[10])
    print(f"case {seed}: {c}, fixed slots {fixed}", flush=True)
    if c["fused"]:
        assert torch.equal(kc.cpu(), ek) and torch.equal(vc.cpu(), ev)
    exp = paged_attention(step.q, ek, ev, step.block_table, step.cu_seqlens_q, step.seqlens_kv,
                          step.scale)
    err = (out.float().cpu() - exp).abs().max().item()
    print(f"max-abs err {err:.3e}", flush=True)
    assert err <= TOL


def draw_mla(seed):
    r = random.Random(seed)
    bs = r.choice(BLOCKS)
    B = r.randint(1, 10)
    lqs, lks = [], []
    for _ in range(B):
        lq = 1 if r.random() < 0.6 else r.randint(2, 40)
        lqs.append(lq)
        lks.append(lq + (0 if r.random() < 0.15 else r.randint(0, 2500)))
    return dict(bs=bs, lqs=lqs, lks=lks, waves=r.choice([0, 0, 1, 5, 100]))


@pytest.mark.parametrize("seed", range(40))
def test_random_mla_steps_match_the_oracle(seed):
    from oracle.paged_attn import mla_absorbed_attention
    c = draw_mla(2000 + seed)
    print(f"case {seed}: {c}", flush=True)
    step = workloads.make_mla_step(lqs=c["lqs"], lks=c["lks"], block_size=c["bs"], seed=seed)
    plan = ops.AttentionPlan.from_lists(step.block_table.to(DEV), step.cu_seqlens_q,
                                        step.seqlens_kv, step.q_latent.shape[1], 1, 512,
                                        c["bs"], num_waves=c["waves"])
    out = ops.paged_attention_mla(step.q_latent.to(DEV), step.cache.to(DEV), plan, step.scale)
    torch.cuda.synchronize()
    exp = mla_absorbed_attention(step.q_latent, step.cache, step.block_table, step.cu_seqlens_q,
                                 step.seqlens_kv, step.scale, 512)
    err = (out.float().cpu() - exp).abs().max().item()
    print(f"max-abs err {err:.3e}", flush=True)
    assert err <= TOL


HEADS_64 = [(14, 2), (16, 2), (8, 8), (32, 4), (12, 2), (16, 16), (64, 8)]


@pytest.mark.parametrize("seed", range(40))
def test_random_steps_head_dim_64_match_the_oracle(seed):
    """head_dim 64 (Qwen2 / Qwen2.5 0.5B: hidden 896 over 14 heads): the
    same random steps on the split-K kernel, fused KV write included."""
    c = draw(4000 + seed)
    c["hq"], c["hkv"] = random.Random(seed).choice(HEADS_64)
    print(f"case {seed}: {c}", flush=True)
    step = workloads.make_gqa_step(lqs=c["lqs"], lks=c["lks"], num_q_heads=c["hq"],
                                   num_kv_heads=c["hkv"], head_dim=64, block_size=c["bs"],
                                   seed=seed, extra_blocks=3)
    kc, vc = step.k_cache.to(DEV), step.v_cache.to(DEV)
    plan = ops.AttentionPlan.from_lists(step.block_table.to(DEV), step.cu_seqlens_q,
                                        step.seqlens_kv, c["hq"], c["hkv"], 64, c["bs"],
                                        num_waves=c["waves"])
    ek, ev = step.k_cache, step.v_cache
    if c["fused"]:
        ek, ev = ek.clone(), ev.clone()
        kv_write(step.k_new, step.v_new, ek, ev, step.slot_mapping)
        out = ops.paged_attention_gqa(step.q.to(DEV), kc, vc, plan, step.scale,
                                      key_new=step.k_new.to(DEV), value_new=step.v_new.to(DEV))
    else:
        out = ops.paged_attention_gqa(step.q.to(DEV), kc, vc, plan, step.scale)
    torch.cuda.synchronize()
    if c["fused"]:
        assert torch.equal(kc.cpu(), ek) and torch.equal(vc.cpu(), ev)
    exp = paged_attention(step.q, ek, ev, step.block_table, step.cu_seqlens_q, step.seqlens_kv,
                          step.scale)
    err = (out.float().cpu() - exp.float()).abs().max().item()
    print(f"max-abs err {err:.3e}", flush=True)
    assert err <= TOL


@pytest.mark.parametrize("seed", range(12))
def test_random_mla_steps_other_head_counts(seed):
    """Absorbed MLA at head counts other than configs[2]'s 16: fewer heads
    than a 16-row block (1, 8), several head blocks per token (32, 128 as in
    DeepSeek-V2), with decode, verify and prefill-sized rows."""
    from oracle.paged_attn import mla_absorbed_attention
    heads = [1, 8, 32, 128][seed % 4]
    c = draw_mla(5000 + seed)
    print(f"case {seed}: heads {heads} {c}", flush=True)
    step = workloads.make_mla_step(lqs=c["lqs"], lks=c["lks"], num_heads=heads, block_size=c["bs"],
                                   seed=seed)
    plan = ops.AttentionPlan.from_lists(step.block_table.to(DEV), step.cu_seqlens_q,
                                        step.seqlens_kv, heads, 1, 512, c["bs"],
                                        num_waves=c["waves"])
    out = ops.paged_attention_mla(step.q_latent.to(DEV), step.cache.to(DEV), plan, step.scale)
    torch.cuda.synchronize()
    exp = mla_absorbed_attention(step.q_latent, step.cache, step.block_table, step.cu_seqlens_q,
                                 step.seqlens_kv, step.scale, 512)
    err = (out.float().cpu() - exp).abs().max().item()
    print(f"max-abs err {err:.3e}", flush=True)
    assert err <= TOL


def draw_mla_large(seed):
    r = random.Random(seed)
    B = r.randint(32, 128)
    lqs = [1 if r.random() < 0.9 else r.randint(2, 4) for _ in range(B)]
    lks = [lq + int(math.exp(r.uniform(0, math.log(8192)))) for lq in lqs]
    return dict(bs=r.choice([16, 64, 128]), lqs=lqs, lks=lks,
                waves=r.choice([0, 0, 256, 512, 1024, 300]))


@pytest.mark.parametrize("seed", range(12))
def test_random_large_mla_batches_match_the_oracle(seed):
    """Batches of 32-128 requests (contexts log-uniform up to 8K, a few
    verify rows) at several range counts: the balanced-plan path at the
    sizes the benchmark runs."""
    from oracle.paged_attn import mla_absorbed_attention
    c = draw_mla_large(6000 + seed)
    print(f"case {seed}: B {len(c['lqs'])} bs {c['bs']} waves {c['waves']}", flush=True)
    step = workloads.make_mla_step(lqs=c["lqs"], lks=c["lks"], block_size=c["bs"], seed=seed)
    plan = ops.AttentionPlan.from_lists(step.block_table.to(DEV), step.cu_seqlens_q,
                                        step.seqlens_kv, step.q_latent.shape[1], 1, 512,
                                        c["bs"], num_waves=c["waves"])
    out = ops.paged_attention_mla(step.q_latent.to(DEV), step.cache.to(DEV), plan, step.scale)
    torch.cuda.synchronize()
    exp = mla_absorbed_attention(step.q_latent, step.cache, step.block_table, step.cu_seqlens_q,
                                 step.seqlens_kv, step.scale, 512)
    err = (out.float().cpu() - exp).abs().max().item()
    print(f"max-abs err {err:.3e}", flush=True)
    assert err <= TOL


# Two cases that failed once each (max-abs 0.187 and 0.093) on an
# intermediate build of the prefill path and passed on every build since:
# group 32 (Hq 64 / Hkv 2), block sizes below the 64-key prefill tile, the
# fused KV write, and prefill-routed requests with and without a prefix.
# They were drawn by an earlier head list of draw(); kept verbatim.
PINNED = {
    79: dict(hq=64, hkv=2, bs=4, lqs=[1, 1, 1, 295, 1, 4, 1, 3, 2, 216, 1, 140],
             lks=[2549, 1748, 1899, 295, 404, 288, 283, 860, 2319, 216, 1098, 2874], waves=0),
    88: dict(hq=64, hkv=2, bs=32, lqs=[76, 183, 1, 1, 1, 4, 150],
             lks=[2806, 545, 260, 814, 1, 382, 596], waves=1),
}


def check_prefill_plan(plan, c):
    """The plan read back, on the CPU: the routed requests' prefill items
    (128 rows of (query token, group head)) are covered by units whose key
    tiles partition [0, tiles of the item) exactly once, in order; every cut
    item has one merge record naming its units and rows; nothing
    overflowed."""
    hq, hkv = c["hq"], c["hkv"]
    group, B, T = hq // hkv, len(c["lqs"]), sum(c["lqs"])
    L = ops.workspace_layout(B, T, hq, hkv, 128, c["waves"])
    ws = plan.workspace.cpu()
    hdr = ws[:256].view(torch.int32).tolist()
    assert hdr[8] == 0, hdr[:10]
    units, pmerges = hdr[6], hdr[7]
    rows_pf, keys = L["pf_rows"], L["pf_keys"]
    u = ws[L["pf"]: L["pf"] + units * 32].view(torch.int32).view(units, 8).tolist()
    m = ws[L["pfm"]: L["pfm"] + pmerges * 16].view(torch.int32).view(pmerges, 4).tolist()
    cu = [0]
    for lq in c["lqs"]:
        cu.append(cu[-1] + lq)
    items = {}
    for rec in u:
        b, r0, t0, t1, c0, lq, lk = rec[:7]
        assert c0 == cu[b] and lq == c["lqs"][b] and lk == c["lks"][b]
        items.setdefault((b, r0), []).append((t0, t1))
    want = set()
    for b, (lq, lk) in enumerate(zip(c["lqs"], c["lks"])):
        if lq * group < rows_pf:
            continue
        for r0 in range(0, lq * group, rows_pf):
            want.add((b, r0))
    assert set(items) == want
    for (b, r0), spans in items.items():
        lq, lk = c["lqs"][b], c["lks"][b]
        last = min(lq * group, r0 + rows_pf) - 1
        kend = max(0, min(lk, lk - lq + last // group + 1))
        nt = -(-kend // keys)
        spans.sort()
        assert spans[0][0] == 0 and spans[-1][1] == nt, (b, r0, spans, nt)
        assert all(spans[i][1] == spans[i + 1][0] for i in range(len(spans) - 1))
    cut = {k for k, v in items.items() if len(v) > 1}
    assert len(m) == len(cut)
    for c0, r0, u0, kr in m:
        k, rows = kr & 0xffff, kr >> 16
        b = cu.index(c0)
        assert (b, r0) in cut and len(items[(b, r0)]) == k
        assert all(u[u0 + j][0] == b and u[u0 + j][1] == r0 for j in range(k))
        assert rows == min(rows_pf, c["lqs"][b] * group - r0)


@pytest.mark.parametrize("case", sorted(PINNED))
def test_pinned_prefill_cases(case):
    """The two pinned cases with ten data seeds each, fused KV write,
    against the oracle; and their plans read back and checked."""
    c = PINNED[case]
    for seed in range(10):
        print(f"pinned case {case}, data seed {seed}", flush=True)
        step = workloads.make_gqa_step(lqs=c["lqs"], lks=c["lks"], num_q_heads=c["hq"],
                                       num_kv_heads=c["hkv"], block_size=c["bs"], seed=seed,
                                       extra_blocks=3)
        kc, vc = step.k_cache.to(DEV), step.v_cache.to(DEV)
        plan = ops.AttentionPlan.from_lists(step.block_table.to(DEV), step.cu_seqlens_q,
                                            step.seqlens_kv, c["hq"], c["hkv"], 128, c["bs"],
                                            num_waves=c["waves"])
        ek, ev = step.k_cache.clone(), step.v_cache.clone()
        kv_write(step.k_new, step.v_new, ek, ev, step.slot_mapping)
        out = ops.paged_attention_gqa(step.q.to(DEV), kc, vc, plan, step.scale,
                                      key_new=step.k_new.to(DEV), value_new=step.v_new.to(DEV))
        torch.cuda.synchronize()
        assert torch.equal(kc.cpu(), ek) and torch.equal(vc.cpu(), ev)
        if seed == 0:
            check_prefill_plan(plan, c)
        exp = paged_attention(step.q, ek, ev, step.block_table, step.cu_seqlens_q,
                              step.seqlens_kv, step.scale)
        err = (out.float().cpu() - exp).abs().max().item()
        print(f"max-abs err {err:.3e}", flush=True)
        assert err <= TOL


@pytest.mark.parametrize("seed", range(40))
def test_random_steps_nz_layout_equal_the_standard_layout(seed):
    """The same random steps (head_dim 128 or 64) over caches in the NZ
    layout of the reference's graph mode: outputs bit-identical to the
    standard layout over the same values, and after a fused write the NZ
    caches are the NZ image of the standard ones."""
    from oracle.paged_attn import nz_from_nd
    c = draw(6000 + seed)
    d = 64 if seed % 3 == 2 else 128
    if d == 64:
        c["hq"], c["hkv"] = random.Random(seed).choice(HEADS_64)
    print(f"case {seed}: d={d} {c}", flush=True)
    step = workloads.make_gqa_step(lqs=c["lqs"], lks=c["lks"], num_q_heads=c["hq"],
                                   num_kv_heads=c["hkv"], head_dim=d, block_size=c["bs"],
                                   seed=seed, extra_blocks=3)
    plan = ops.AttentionPlan.from_lists(step.block_table.to(DEV), step.cu_seqlens_q,
                                        step.seqlens_kv, c["hq"], c["hkv"], d, c["bs"],
                                        num_waves=c["waves"])
    kw = {}
    if c["fused"]:
        kw = dict(key_new=step.k_new.to(DEV), value_new=step.v_new.to(DEV))
    kc, vc = step.k_cache.to(DEV), step.v_cache.to(DEV)
    nd = ops.paged_attention_gqa(step.q.to(DEV), kc, vc, plan, step.scale, **kw)
    kz, vz = nz_from_nd(step.k_cache).to(DEV), nz_from_nd(step.v_cache).to(DEV)
    nz = ops.paged_attention_gqa(step.q.to(DEV), kz, vz, plan, step.scale, kv_layout="nz", **kw)
    torch.cuda.synchronize()
    assert torch.equal(nz.view(torch.int16), nd.view(torch.int16))
    assert torch.equal(kz.cpu(), nz_from_nd(kc.cpu())) and torch.equal(vz.cpu(), nz_from_nd(vc.cpu()))
