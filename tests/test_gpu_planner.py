"""The small-step planner (one wave for the per-request and per-segment
phases, used for GQA steps of at most 64 segments without prefill routing)
against the one-work-group planner on the same steps: the header, segment
records, range records and merge records read back from both workspaces
are identical.  The large planner runs in a subprocess with
AIA_PLANNER=large (read once per process)."""
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

from auto_infer_amd import ops, workloads

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# (lqs, lks, hq, hkv, head_dim, block_size, num_waves)
CASES = [
    ("config1", None),
    ("config4", None),
    ("mixed-small", ([1, 3, 1, 2, 1, 4], [700, 90, 1500, 33, 1, 300], 16, 8, 128, 16, 0)),
    ("group32", ([1, 2, 1], [200, 513, 40], 64, 2, 128, 128, 0)),
    ("hkv16", ([1, 1, 2], [900, 17, 3000], 32, 16, 128, 64, 0)),
    ("d64", ([1, 1, 1, 1, 2], [130, 7, 300, 1000, 64], 14, 2, 64, 16, 0)),
    ("waves1", ([1, 1, 1], [300, 17, 1000], 8, 2, 128, 16, 1)),
    ("waves7", ([1, 2, 1], [300, 17, 1000], 8, 2, 128, 16, 7)),
    ("waves700", ([1, 1, 1, 3], [3000, 17, 1000, 4], 8, 2, 128, 4, 700)),
    ("batch56", ([1] * 56, [((i * 37) % 2000) + 1 for i in range(56)], 16, 8, 128, 128, 0)),
    ("zero-len", ([1, 0, 1], [10, 0, 20], 8, 2, 128, 16, 0)),
]


def _step(name, spec):
    if name == "config1":
        s = workloads.config1_decode(seed=2)
        return s, 16, 8, 128, 128, 0
    if name == "config4":
        s = workloads.config4_mtp(seed=1)
        return s, 32, 8, 128, s.k_cache.shape[1], 0
    lqs, lks, hq, hkv, d, bs, waves = spec
    s = workloads.make_gqa_step(lqs=lqs, lks=lks, num_q_heads=hq, num_kv_heads=hkv, head_dim=d,
                                block_size=bs, seed=3)
    return s, hq, hkv, d, bs, waves


def plans():
    """Every case's plan regions as int32 arrays (name -> dict)."""
    out = {}
    for name, spec in CASES:
        s, hq, hkv, d, bs, waves = _step(name, spec)
        plan = ops.AttentionPlan.from_lists(s.block_table.to(DEV), s.cu_seqlens_q, s.seqlens_kv,
                                            hq, hkv, d, bs, num_waves=waves)
        torch.cuda.synchronize()
        L = ops.workspace_layout(len(s.seqlens_kv), s.num_tokens, hq, hkv, d, waves)
        ws = plan.workspace.cpu().view(torch.int32).numpy()
        hdr = ws[:16].copy()
        nseg, nmrg = int(hdr[0]), int(hdr[5])
        out[name + ".hdr"] = hdr[:11]
        out[name + ".seg"] = ws[L["seg"] // 4: L["seg"] // 4 + (nseg + 1) * 8].copy()
        rec = ws[L["wave"] // 4: L["wave"] // 4 + L["waves"] * 32].copy().reshape(-1, 32)
        rec[rec[:, 0] < 0, 4:] = 0        # an unused slot's record is its first 4 ints
        out[name + ".rec"] = rec
        out[name + ".mrg"] = ws[L["mrg"] // 4: L["mrg"] // 4 + nmrg * 8].copy()
    return out


def test_small_planner_matches_the_work_group_planner(tmp_path):
    path = str(tmp_path / "large.npz")
    code = ("import sys, numpy as np; sys.path.insert(0, %r); "
            "from tests.test_gpu_planner import plans; np.savez(%r, **plans())" % (ROOT, path))
    env = dict(os.environ, AIA_PLANNER="large")
    r = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env, capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    large = np.load(path)
    small = plans()
    for name, _ in CASES:
        print(f"case {name}: header {small[name + '.hdr'].tolist()}", flush=True)
        for part in ("hdr", "seg", "rec", "mrg"):
            a, b = small[f"{name}.{part}"], large[f"{name}.{part}"]
            assert a.shape == b.shape and np.array_equal(a, b), (name, part)


@pytest.mark.parametrize("waves, fixed", [(0, 1), (7, 1), (2048, 0)])
def test_fixed_partial_slots(waves, fixed):
    """Small steps whose segments have at most 32 ranges each put segment s's
    partials at slots 32 s .. 32 s + 31 (header word 10 = 1), so the merge
    finds them without a record; more ranges per segment fall back to the
    packed slots and the merge records.  The output matches the oracle either
    way."""
    from oracle.paged_attn import paged_attention
    s = workloads.config1_decode(seed=5)
    plan = ops.AttentionPlan.from_lists(s.block_table.to(DEV), s.cu_seqlens_q, s.seqlens_kv,
                                        16, 8, 128, 128, num_waves=waves)
    out = ops.paged_attention_gqa(s.q.to(DEV), s.k_cache.to(DEV), s.v_cache.to(DEV), plan, s.scale)
    torch.cuda.synchronize()
    L = ops.workspace_layout(len(s.seqlens_kv), s.num_tokens, 16, 8, 128, waves)
    ws = plan.workspace.cpu().view(torch.int32).numpy()
    hdr = ws[:16]
    nseg, tpw = int(hdr[0]), int(hdr[2])
    seg = ws[L["seg"] // 4: L["seg"] // 4 + nseg * 8].reshape(nseg, 8)
    nparts = (seg[:, 6] - 1) // tpw - seg[:, 5] // tpw + 1
    print(f"waves {waves}: header {hdr[:11].tolist()}, ranges per segment {nparts.tolist()}",
          flush=True)
    assert int(hdr[10]) == fixed
    assert (int(nparts.max()) <= 32) == bool(fixed)
    if fixed:
        assert np.array_equal(seg[:, 7], 32 * np.arange(nseg))
    else:
        assert np.array_equal(seg[:, 7], np.concatenate([[0], np.cumsum(nparts)[:-1]]))
    ref = paged_attention(s.q, s.k_cache, s.v_cache, s.block_table, s.cu_seqlens_q,
                          s.seqlens_kv, s.scale)
    err = (out.float().cpu() - ref).abs().max().item()
    assert err <= 2e-2, err
