"""HIP-graph decode (capture once per gear, replay per step) on the GPU: each
step restages the fixed-address metadata and replays the captured planner +
layers; outputs and caches are checked against a sequential oracle replay."""
import numpy as np
import pytest
import torch

from auto_infer_amd import packing
from auto_infer_amd.execution import BatchPlan, RequestView, ScheduledRequest
from auto_infer_amd.graph import DecodeGraph
from oracle import pack
from oracle.paged_attn import kv_write, nd_from_nz, nz_from_nd, paged_attention

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.mark.parametrize("kv_layout", ["nd", "nz"])
def test_decode_graph_replays_across_steps(kv_layout):
    rng = np.random.default_rng(0)
    gear, maxb, bs, nb, hq, hkv, d, L = 8, 16, 16, 200, 16, 8, 128, 2
    stager = packing.DecodeInputStager(
        tid=torch.zeros(gear, dtype=torch.long, device=DEV),
        positions=torch.zeros(gear, dtype=torch.long, device=DEV),
        slots=torch.zeros(gear, dtype=torch.int32, device=DEV),
        block_table=torch.zeros(gear, maxb, dtype=torch.int32, device=DEV),
        block_size=bs, scratch0=nb - gear)
    g = torch.Generator(device=DEV).manual_seed(3)
    caches = [(torch.randn(nb, bs, hkv, d, generator=g, device=DEV, dtype=torch.bfloat16),
               torch.randn(nb, bs, hkv, d, generator=g, device=DEV, dtype=torch.bfloat16))
              for _ in range(L)]
    ref = [(k.cpu(), v.cpu()) for k, v in caches]
    if kv_layout == "nz":      # the same values, in the graph mode's NZ memory layout
        caches = [(nz_from_nd(k).to(DEV), nz_from_nd(v).to(DEV)) for k, v in ref]
    view = nd_from_nz if kv_layout == "nz" else (lambda c: c)
    dg = DecodeGraph(stager, caches, num_q_heads=hq, num_kv_heads=hkv, kv_layout=kv_layout)
    free = list(range(nb - gear))
    rng.shuffle(free)
    reqs = {}
    for i, lk in enumerate([5, 40, 17, 100, 63]):
        nblk = (lk + 3 + bs - 1) // bs
        reqs[f"r{i}"] = dict(pos=lk - 1, blocks=[free.pop() for _ in range(nblk)])
    for step in range(4):
        views = {rid: RequestView(rid, tuple(range(r["pos"] + 1)), r["pos"], 1, 1, ())
                 for rid, r in reqs.items()}
        plan = BatchPlan.make([ScheduledRequest(rid, 1, False, tuple(r["blocks"]))
                               for rid, r in reqs.items()], views,
                              {rid: r["blocks"] for rid, r in reqs.items()})
        for buf in (dg.q, dg.k_new, dg.v_new):
            buf.copy_(torch.randn(buf.shape, generator=g, device=DEV, dtype=torch.bfloat16))
        staged = dg.stage(plan)
        if dg.graph is None:
            dg.capture()
        else:
            dg.replay()
        torch.cuda.synchronize()
        exp = pack.decode_stage(plan, gear=gear, max_blocks=maxb, block_size=bs,
                                scratch0=nb - gear)
        assert staged.slots.cpu().tolist() == exp["slots"].tolist()
        for layer in range(L):
            kv_write(dg.k_new[layer].cpu(), dg.v_new[layer].cpu(), ref[layer][0], ref[layer][1],
                     torch.from_numpy(exp["slots"]))
            o = paged_attention(dg.q[layer].cpu(), ref[layer][0], ref[layer][1],
                                exp["block_table"], list(range(1, gear + 1)),
                                exp["kv_lengths"], d ** -0.5)
            err = (dg.out[layer].float().cpu() - o).abs().max().item()
            print(f"step {step} layer {layer}: max-abs err {err:.3e}", flush=True)
            assert err <= 2e-2
            assert torch.equal(view(caches[layer][0].cpu()), ref[layer][0])
            assert torch.equal(view(caches[layer][1].cpu()), ref[layer][1])
        for r in reqs.values():
            r["pos"] += 1


@pytest.mark.parametrize("depth", [0, 1])
def test_latent_decode_graph_replays_across_steps(depth):
    """Absorbed-MLA gear in a HIP graph (decode, and MTP verify with one
    draft): per step the stager restages the fixed buffers and the captured
    planner + latent write + latent attention replay; the latent caches stay
    bit-exact with the oracle's write and the outputs within 2e-2."""
    from auto_infer_amd.attention.mla import MlaHipBackend
    from auto_infer_amd.graph import LatentDecodeGraph
    from oracle.paged_attn import mla_absorbed_attention
    rng = np.random.default_rng(4 + depth)
    gear, maxb, bs, nb, H, L = 8, 72, 16, 240, 16, 2
    w = depth + 1
    common = dict(positions=torch.zeros(gear * w, dtype=torch.long, device=DEV),
                  slots=torch.zeros(gear * w, dtype=torch.int32, device=DEV),
                  block_table=torch.zeros(gear, maxb, dtype=torch.int32, device=DEV),
                  block_size=bs, scratch0=nb - gear)
    tid = torch.zeros(gear * w, dtype=torch.long, device=DEV)
    if depth:
        stager = packing.SpecDecodeInputStager(
            tid=tid, drafts=torch.zeros(gear, depth, dtype=torch.long, device=DEV),
            draft_depth=depth, **common)
    else:
        stager = packing.DecodeInputStager(tid=tid, **common)
    backend = MlaHipBackend({}, num_heads=H, qk_nope=128, qk_rope=64, v_head_dim=128,
                            kv_lora_rank=512, q_lora_rank=None, rms_eps=1e-6,
                            softmax_scale=192 ** -0.5, num_layers=L, device=DEV,
                            dtype=torch.bfloat16)
    caches = backend.alloc_kv_caches(nb, bs)
    g = torch.Generator(device=DEV).manual_seed(8)
    for latent, _ in caches:
        latent.copy_(torch.randn(latent.shape, generator=g, device=DEV, dtype=torch.bfloat16))
    ref = [c[0].cpu() for c in caches]
    dg = LatentDecodeGraph(stager, caches, num_heads=H)
    free = list(range(nb - gear))
    rng.shuffle(free)
    reqs = {}
    for i, lk in enumerate([5, 400, 17, 100, 63, 1000]):
        nblk = (lk + 5 * w + bs - 1) // bs
        reqs[f"r{i}"] = dict(pos=lk - 1, blocks=[free.pop() for _ in range(nblk)])
    for step in range(4):
        views = {rid: RequestView(rid, tuple(range(r["pos"] + 1)), r["pos"], 1, 1,
                                  tuple(range(depth)))
                 for rid, r in reqs.items()}
        plan = BatchPlan.make([ScheduledRequest(rid, w, False, tuple(r["blocks"]))
                               for rid, r in reqs.items()], views,
                              {rid: r["blocks"] for rid, r in reqs.items()})
        for buf in (dg.q, dg.latent_new):
            buf.copy_(torch.randn(buf.shape, generator=g, device=DEV, dtype=torch.bfloat16))
        staged = dg.stage(plan)
        if dg.graph is None:
            dg.capture()
        else:
            dg.replay()
        torch.cuda.synchronize()
        slots = staged.slots.cpu()
        cu = list(range(w, gear * w + 1, w))
        for layer in range(L):
            kv_write(dg.latent_new[layer].cpu(), None, ref[layer], None, slots)
            assert torch.equal(caches[layer][0].cpu(), ref[layer])
            o = mla_absorbed_attention(dg.q[layer].cpu(), ref[layer], staged.block_table.cpu(),
                                       cu, staged.kv_lengths, 192 ** -0.5, 512)
            err = (dg.out[layer].float().cpu() - o).abs().max().item()
            print(f"step {step} layer {layer}: max-abs err {err:.3e}", flush=True)
            assert err <= 2e-2
        for r in reqs.values():
            r["pos"] += 1
