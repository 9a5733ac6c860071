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
from oracle.paged_attn import kv_write, paged_attention

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def test_decode_graph_replays_across_steps():
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
    dg = DecodeGraph(stager, caches, num_q_heads=hq, num_kv_heads=hkv)
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
            assert torch.equal(caches[layer][0].cpu(), ref[layer][0])
            assert torch.equal(caches[layer][1].cpu(), ref[layer][1])
        for r in reqs.values():
            r["pos"] += 1
