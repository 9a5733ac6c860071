"""Host logic of the synthetic workloads (CPU)."""
import torch

from auto_infer_amd import workloads
from oracle.paged_attn import paged_attention


def test_subset_matches_full_batch_rows():
    s = workloads.make_gqa_step(lqs=[2, 1, 3, 1], lks=[40, 9, 60, 17], num_q_heads=4,
                                num_kv_heads=2, block_size=16, seed=1, extra_blocks=5,
                                shared_prefix_blocks=1, share_frac=0.9)
    full = paged_attention(s.q, s.k_cache, s.v_cache, s.block_table, s.cu_seqlens_q,
                           s.seqlens_kv, s.scale)
    sub, rows = workloads.subset(s, [3, 0, 2])
    part = paged_attention(sub.q, sub.k_cache, sub.v_cache, sub.block_table, sub.cu_seqlens_q,
                           sub.seqlens_kv, s.scale)
    assert torch.equal(full[rows], part)


def test_config_generators_shapes():
    c4 = workloads.config4_mtp()
    assert c4.q.shape == (32, 32, 128) and c4.k_cache.shape[2] == 8
    assert all(1024 <= lk <= 4096 for lk in c4.seqlens_kv)
    lks = workloads.config5_contexts()
    assert len(lks) == 256 and min(lks) >= 64 and max(lks) <= 32768


def test_fragmented_tables_are_disjoint_and_noncontiguous():
    lks = [3000, 100, 7000, 64]
    tables, kv = workloads.fragmented_block_tables(lks, num_blocks=4000, block_size=128,
                                                   ops=2000, seed=3)
    flat = [b for t in tables for b in t]
    assert len(flat) == len(set(flat))
    assert [len(t) for t in tables] == [(lk + 127) // 128 for lk in lks]
    steps = [abs(t[i + 1] - t[i]) for t in tables for i in range(len(t) - 1)]
    assert any(d != 1 for d in steps)
