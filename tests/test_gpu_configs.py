"""BASELINE configs 2, 4 and 5 at their full sizes on the GPU.

The oracle runs on a sample of requests (attention rows of a request depend
only on that request, pinned by tests/test_workloads.py); the KV write is
checked bit-exact on every written slot; packing of the config-5 plan is
checked bit-exact against the packing oracle.
"""
import numpy as np
import pytest
import torch

from auto_infer_amd import ops, packing, workloads
from auto_infer_amd.execution import BatchPlan, RequestView, ScheduledRequest
from oracle import pack
from oracle.paged_attn import kv_write, paged_attention

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TOL = 2e-2


def attend(step):
    plan = ops.AttentionPlan.from_lists(step.block_table, step.cu_seqlens_q, step.seqlens_kv,
                                        step.q.shape[1], step.k_cache.shape[2], step.q.shape[2],
                                        step.k_cache.shape[1])
    out = ops.paged_attention_gqa(step.q, step.k_cache, step.v_cache, plan, step.scale)
    torch.cuda.synchronize()
    return out


def check_sample(step, out, requests):
    sub, rows = workloads.subset(step, requests)
    exp = paged_attention(sub.q, sub.k_cache, sub.v_cache, sub.block_table, sub.cu_seqlens_q,
                          sub.seqlens_kv, step.scale)
    got = out[torch.tensor(rows, device=out.device)].float().cpu()
    err = (got - exp).abs().max().item()
    print(f"sampled {len(requests)} requests, max-abs err {err:.3e}", flush=True)
    assert err <= TOL


def test_config2_mixed_prefill_decode():
    print("config2: building on GPU", flush=True)
    step = workloads.config2_mixed(seed=0, device=DEV)
    ops.write_kv(step.k_new, step.v_new, step.k_cache, step.v_cache, step.slot_mapping)
    out = attend(step)
    # every written slot holds the new row (bit-exact)
    slots = step.slot_mapping.long()
    assert torch.equal(step.k_cache.view(-1, 4, 128)[slots], step.k_new)
    assert torch.equal(step.v_cache.view(-1, 4, 128)[slots], step.v_new)
    rng = np.random.default_rng(0)
    sample = [0, 1, 2] + sorted(rng.choice(np.arange(3, 515), 29, replace=False).tolist())
    check_sample(step, out, sample)


@pytest.mark.parametrize("fused", [False, True])
def test_config2_prefill_chunks_alone_dealt_by_size(fused):
    """configs[1]'s three 512-token chunks alone: every request goes to the
    prefill units, the planner takes the least chunk size whose units fit
    one round and deals the work-groups by size in CU pairs (hdr[9]).
    Checked against the oracle, with and without the fused KV write."""
    full = workloads.config2_mixed(seed=0)
    sub, _ = workloads.subset(full, [0, 1, 2])
    exp_k, exp_v = sub.k_cache.clone(), sub.v_cache.clone()
    bs, starts = sub.k_cache.shape[1], [0] + list(sub.cu_seqlens_q[:-1])
    slots = [int(sub.block_table[b, p // bs]) * bs + p % bs
             for b, (c0, c1, lk) in enumerate(zip(starts, sub.cu_seqlens_q, sub.seqlens_kv))
             for p in range(lk - (c1 - c0), lk)]
    kv_write(sub.k_new, sub.v_new, exp_k, exp_v, slots)
    exp = paged_attention(sub.q, exp_k, exp_v, sub.block_table, sub.cu_seqlens_q,
                          sub.seqlens_kv, sub.scale)
    kc, vc = (exp_k if not fused else sub.k_cache).to(DEV), (exp_v if not fused else sub.v_cache).to(DEV)
    plan = ops.AttentionPlan.from_lists(sub.block_table.to(DEV), sub.cu_seqlens_q, sub.seqlens_kv,
                                        28, 4, 128, sub.k_cache.shape[1])
    kw = dict(key_new=sub.k_new.to(DEV), value_new=sub.v_new.to(DEV)) if fused else {}
    out = ops.paged_attention_gqa(sub.q.to(DEV), kc, vc, plan, sub.scale, **kw)
    torch.cuda.synchronize()
    hdr = plan.workspace[:64].cpu().view(torch.int32).tolist()
    units, ncu = hdr[6], torch.cuda.get_device_properties(DEV).multi_processor_count
    jobs = units * 4
    assert hdr[8] == 0 and jobs > 256, hdr[:10]
    # every work-group's record written at its id (dealt by size when they
    # fit one round of two per CU, as all of them do on a 256-CU MI355X)
    assert hdr[9] == jobs, (hdr[:10], ncu)
    err = (out.float().cpu() - exp).abs().max().item()
    print(f"units {units}, max-abs err {err:.3e}", flush=True)
    assert err <= TOL
    if fused:
        assert torch.equal(kc.cpu(), exp_k) and torch.equal(vc.cpu(), exp_v)


@pytest.mark.parametrize("fused", [False, True])
def test_config4_mtp_verify_full(fused):
    """configs[3] at full size, with the separate KV write or with the write
    fused into the attention kernel (the bench's and the backend's default):
    the caches are bit-exact against the separate write at slot_mapping, and
    the output within 2e-2 of the oracle on every request."""
    step = workloads.config4_mtp(seed=0, device=DEV)
    if not fused:
        ops.write_kv(step.k_new, step.v_new, step.k_cache, step.v_cache, step.slot_mapping)
        out = attend(step)
    else:
        ek, ev = step.k_cache.clone(), step.v_cache.clone()
        ops.write_kv(step.k_new, step.v_new, ek, ev, step.slot_mapping)
        plan = ops.AttentionPlan.from_lists(step.block_table, step.cu_seqlens_q, step.seqlens_kv,
                                            32, 8, 128, step.k_cache.shape[1])
        out = ops.paged_attention_gqa(step.q, step.k_cache, step.v_cache, plan, step.scale,
                                      key_new=step.k_new, value_new=step.v_new)
        torch.cuda.synchronize()
        assert torch.equal(step.k_cache, ek) and torch.equal(step.v_cache, ev), \
            "fused KV write differs from the write at slot_mapping"
    check_sample(step, out, list(range(16)))


def _spec_plan(reqs, blocks):
    views = {rid: RequestView(rid, tuple(r["tokens"]), r["computed"], r["prompt"], r["prompt"],
                              tuple(r["draft"])) for rid, r in reqs.items()}
    sched = [ScheduledRequest(rid, 1 + len(r["draft"]), False, tuple(blocks[rid]))
             for rid, r in reqs.items()]
    return BatchPlan.make(sched, views, {rid: tuple(b) for rid, b in blocks.items()})


def test_config4_mtp_rollback_of_rejected_drafts():
    """Two verify steps through the GPU packer: 30% of drafts rejected
    (seeded).  A rejected draft's KV stays in its slot, is excluded from the
    next step's context (num_computed_tokens = num_tokens - 1,
    engine_core.py:172) and is overwritten by the next write; the cache and
    the attention must match a sequential oracle replay."""
    rng = np.random.default_rng(4)
    B, bs, hq, hkv, d = 16, 128, 32, 8, 128
    lks = rng.integers(1024, 4096, size=B, endpoint=True).tolist()
    nb = sum((lk + 4 + bs - 1) // bs for lk in lks) + 4
    perm = rng.permutation(nb).tolist()
    blocks, cur = {}, 0
    reqs = {}
    for i, lk in enumerate(lks):
        n = (lk + 4 + bs - 1) // bs
        blocks[f"r{i}"] = perm[cur:cur + n]
        cur += n
        toks = rng.integers(1, 30000, size=lk - 1).tolist()        # positions 0..lk-2
        reqs[f"r{i}"] = dict(tokens=toks, computed=lk - 2, prompt=64,
                             draft=[int(rng.integers(1, 30000))])
    g = torch.Generator(device=DEV).manual_seed(1)
    kc = torch.randn(nb, bs, hkv, d, generator=g, device=DEV, dtype=torch.bfloat16)
    vc = torch.randn(nb, bs, hkv, d, generator=g, device=DEV, dtype=torch.bfloat16)
    ek, ev = kc.cpu(), vc.cpu()
    packer = packing.DeviceBatchPacker(bs, DEV)
    for step_i in range(2):
        plan = _spec_plan(reqs, blocks)
        ctx, _, _ = packer.build(plan)
        exp = pack.build(plan, bs)
        assert ctx.slot_mapping.cpu().numpy().tolist() == exp["slot_mapping"].tolist()
        T = ctx.slot_mapping.shape[0]
        q = torch.randn(T, hq, d, generator=g, device=DEV, dtype=torch.bfloat16)
        k = torch.randn(T, hkv, d, generator=g, device=DEV, dtype=torch.bfloat16)
        v = torch.randn(T, hkv, d, generator=g, device=DEV, dtype=torch.bfloat16)
        ops.write_kv(k, v, kc, vc, ctx.slot_mapping)
        kv_write(k.cpu(), v.cpu(), ek, ev, ctx.slot_mapping.cpu())
        plan_a = ops.AttentionPlan(ctx.block_table, ctx.aia_cu_seqlens_q, ctx.aia_seqlens_kv, T,
                                   hq, hkv, d, bs)
        out = ops.paged_attention_gqa(q, kc, vc, plan_a, d ** -0.5)
        torch.cuda.synchronize()
        assert torch.equal(kc.cpu(), ek) and torch.equal(vc.cpu(), ev)
        ref = paged_attention(q.cpu(), ek, ev, exp["block_table"], exp["cu_seqlens_q"],
                              exp["seqlens_kv"], d ** -0.5)
        err = (out.float().cpu() - ref).abs().max().item()
        print(f"mtp step {step_i}: max-abs err {err:.3e}", flush=True)
        assert err <= TOL
        for rid, r in reqs.items():                 # verify outcome
            if rng.random() < 0.3:                 # rejected: corrected token only
                r["tokens"] = r["tokens"] + [int(rng.integers(1, 30000))]
            else:                                   # accepted draft + bonus token
                r["tokens"] = r["tokens"] + r["draft"] + [int(rng.integers(1, 30000))]
            r["computed"] = len(r["tokens"]) - 1
            r["draft"] = [int(rng.integers(1, 30000))]


def test_config5_stress_packing_and_attention():
    """256 requests, lognormal contexts, an 80 GB pool fragmented by a 10k-op
    allocate/free trace; the decode plan is packed on the GPU (bit-exact vs
    the packing oracle) and attended (sampled oracle)."""
    bs, hkv, d, hq = 128, 8, 128, 64
    nb = int(80e9) // (bs * hkv * d * 2 * 2)
    lks = workloads.config5_contexts(seed=0)
    print(f"config5: pool {nb} blocks, tokens {sum(lks)}", flush=True)
    tables, _ = workloads.fragmented_block_tables(lks, num_blocks=nb, block_size=bs,
                                                  ops=10000, seed=0)
    reqs = {f"r{i}": dict(tokens=list(range(lk)), computed=lk - 1, prompt=1, draft=[])
            for i, lk in enumerate(lks)}
    views = {rid: RequestView(rid, tuple(r["tokens"]), r["computed"], 1, 1, ())
             for rid, r in reqs.items()}
    plan = BatchPlan.make([ScheduledRequest(f"r{i}", 1, False, tuple(t))
                           for i, t in enumerate(tables)], views,
                          {f"r{i}": t for i, t in enumerate(tables)})
    packer = packing.DeviceBatchPacker(bs, DEV)
    ctx, _, _ = packer.build(plan)
    exp = pack.build(plan, bs)
    torch.cuda.synchronize()
    assert np.array_equal(ctx.block_table.cpu().numpy(), exp["block_table"])
    assert np.array_equal(ctx.slot_mapping.cpu().numpy(), exp["slot_mapping"])
    assert np.array_equal(ctx.token_ids.cpu().numpy(), exp["token_ids"])
    step = workloads.make_gqa_step(lqs=[1] * 256, lks=lks, num_q_heads=hq, num_kv_heads=hkv,
                                   block_size=bs, num_blocks=nb, seed=2, device=DEV,
                                   tables=tables)
    ops.write_kv(step.k_new, step.v_new, step.k_cache, step.v_cache, ctx.slot_mapping)
    plan_a = ops.AttentionPlan(ctx.block_table, ctx.aia_cu_seqlens_q, ctx.aia_seqlens_kv, 256,
                               hq, hkv, d, bs)
    out = ops.paged_attention_gqa(step.q, step.k_cache, step.v_cache, plan_a, step.scale)
    torch.cuda.synchronize()
    rng = np.random.default_rng(1)
    longest = int(np.argmax(lks))
    sample = sorted(set([longest] + rng.choice(256, 15, replace=False).tolist()))
    check_sample(step, out, sample)
    del step
    torch.cuda.empty_cache()
