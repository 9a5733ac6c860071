"""Absorbed-MLA paged attention on the GPU vs the float32 oracle (2e-2)."""
import pytest
import torch

from auto_infer_amd import ops, workloads
from oracle.paged_attn import kv_write, mla_absorbed_attention

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 2e-2


def run(step, num_waves=0):
    plan = ops.AttentionPlan.from_lists(step.block_table.to(DEV), step.cu_seqlens_q,
                                        step.seqlens_kv, step.q_latent.shape[1], 1, 512,
                                        step.cache.shape[1],
                                        num_waves=num_waves)
    out = ops.paged_attention_mla(step.q_latent.to(DEV), step.cache.to(DEV), plan, step.scale)
    torch.cuda.synchronize()
    return out.float().cpu()


def check(step, num_waves=0):
    got = run(step, num_waves)
    exp = mla_absorbed_attention(step.q_latent, step.cache, step.block_table,
                                 step.cu_seqlens_q, step.seqlens_kv, step.scale, 512)
    err = (got - exp).abs().max().item()
    print(f"max-abs err {err:.3e}", flush=True)
    assert err <= TOL, err


def test_mla_config3_shape_small():
    step = workloads.make_mla_step(lqs=[1] * 8, lks=[512, 700, 1, 129, 2000, 33, 8192, 3000],
                                   seed=3)
    check(step)


@pytest.mark.parametrize("waves", [1, 5, 0])
def test_mla_split_invariance(waves):
    step = workloads.make_mla_step(lqs=[1, 1], lks=[900, 77], block_size=16, seed=8)
    check(step, waves)


def test_mla_multi_token_query_causal():
    step = workloads.make_mla_step(lqs=[2, 3, 1], lks=[300, 40, 5], block_size=64, seed=6)
    check(step)


def test_mla_write_then_attend_single_cache():
    """The absorbed path writes one latent row per token into the one cache
    that serves as both K and V (mla.py:111-113), then attends."""
    step = workloads.make_mla_step(lqs=[1] * 4, lks=[10, 200, 130, 1], block_size=128, seed=12)
    cache = step.cache.to(DEV)
    ops.write_kv(step.latent_new.to(DEV), None, cache, None, step.slot_mapping.to(DEV))
    exp_cache = step.cache.clone()
    kv_write(step.latent_new, None, exp_cache, None, step.slot_mapping)
    torch.cuda.synchronize()
    assert torch.equal(cache.cpu(), exp_cache)
    step.cache = exp_cache
    check(step)
