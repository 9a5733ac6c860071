"""Pins for the attention oracle (CPU): the float32 gather-softmax against an
independent float64 brute force, the closed forms the reference fixes, and
invariants a wrong index or transposed operand would break."""
import math

import torch

from auto_infer_amd import workloads
from oracle.paged_attn import (kv_write, mla_absorbed_attention, paged_attention,
                               paged_attention_f64_bruteforce)


def _dense_causal(q, k, v, scale):
    """The reference's own fp32 oracle shape (base.py:64-80) for one segment,
    written out: full causal softmax with Lq == Lk."""
    t = q.shape[0]
    s = (q.float() @ k.float().t()) * scale
    s = s + torch.triu(torch.full((t, t), float("-inf")), diagonal=1)
    return torch.softmax(s, dim=-1) @ v.float()


def test_matches_float64_bruteforce_ragged_gqa():
    step = workloads.make_gqa_step(lqs=[3, 1, 2], lks=[7, 5, 9], num_q_heads=4, num_kv_heads=2,
                                   head_dim=16, block_size=4, seed=1, dtype=torch.float32)
    a = paged_attention(step.q, step.k_cache, step.v_cache, step.block_table,
                        step.cu_seqlens_q, step.seqlens_kv, 0.3)
    b = paged_attention_f64_bruteforce(step.q, step.k_cache, step.v_cache, step.block_table,
                                       step.cu_seqlens_q, step.seqlens_kv, 0.3)
    assert torch.allclose(a.double(), b, atol=1e-5)


def test_full_prefill_equals_dense_causal_per_head():
    """Lq == Lk: bottom-right causal is ordinary causal attention; head h
    reads KV head h // (Hq / Hkv)."""
    step = workloads.make_gqa_step(lqs=[6], lks=[6], num_q_heads=4, num_kv_heads=2,
                                   head_dim=8, block_size=4, seed=2, dtype=torch.float32)
    out = paged_attention(step.q, step.k_cache, step.v_cache, step.block_table,
                          step.cu_seqlens_q, step.seqlens_kv, 0.5)
    bt = step.block_table[0].long()
    j = torch.arange(6)
    k = step.k_cache[bt[j // 4], j % 4]
    v = step.v_cache[bt[j // 4], j % 4]
    for h in range(4):
        exp = _dense_causal(step.q[:, h], k[:, h // 2], v[:, h // 2], 0.5)
        assert torch.allclose(out[:, h], exp, atol=1e-6)


def test_decode_is_plain_softmax_over_all_keys():
    step = workloads.make_gqa_step(lqs=[1], lks=[11], num_q_heads=2, num_kv_heads=1,
                                   head_dim=8, block_size=4, seed=3, dtype=torch.float32)
    out = paged_attention(step.q, step.k_cache, step.v_cache, step.block_table,
                          step.cu_seqlens_q, step.seqlens_kv, 1.0)
    bt = step.block_table[0].long()
    j = torch.arange(11)
    k, v = step.k_cache[bt[j // 4], j % 4, 0], step.v_cache[bt[j // 4], j % 4, 0]
    for h in range(2):
        w = torch.softmax(step.q[0, h] @ k.t(), dim=0)
        assert torch.allclose(out[0, h], w @ v, atol=1e-6)


def test_single_key_returns_its_value():
    step = workloads.make_gqa_step(lqs=[1], lks=[1], num_q_heads=2, num_kv_heads=1,
                                   head_dim=8, block_size=4, seed=4, dtype=torch.float32)
    out = paged_attention(step.q, step.k_cache, step.v_cache, step.block_table,
                          step.cu_seqlens_q, step.seqlens_kv, 1.0)
    blk = int(step.block_table[0, 0])
    assert torch.allclose(out[0, 0], step.v_cache[blk, 0, 0])


def test_segment_isolation():
    step = workloads.make_gqa_step(lqs=[2, 3], lks=[5, 8], num_q_heads=2, num_kv_heads=2,
                                   head_dim=8, block_size=4, seed=5, dtype=torch.float32)
    both = paged_attention(step.q, step.k_cache, step.v_cache, step.block_table,
                           step.cu_seqlens_q, step.seqlens_kv, 0.4)
    second = paged_attention(step.q[2:], step.k_cache, step.v_cache, step.block_table[1:],
                             [3], [8], 0.4)
    assert torch.equal(both[2:], second)


def test_block_permutation_invariance():
    step = workloads.make_gqa_step(lqs=[1, 2], lks=[9, 6], num_q_heads=2, num_kv_heads=1,
                                   head_dim=8, block_size=4, seed=6, dtype=torch.float32,
                                   extra_blocks=3)
    a = paged_attention(step.q, step.k_cache, step.v_cache, step.block_table,
                        step.cu_seqlens_q, step.seqlens_kv, 0.4)
    nb = step.k_cache.shape[0]
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(0))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(nb)
    b = paged_attention(step.q, step.k_cache[perm], step.v_cache[perm],
                        inv[step.block_table.long()], step.cu_seqlens_q, step.seqlens_kv, 0.4)
    assert torch.allclose(a, b, atol=1e-7)


def test_kv_write_closed_form_and_untouched_slots():
    cache = torch.arange(2 * 4 * 3 * 2, dtype=torch.float32).view(2, 4, 3, 2)
    before = cache.clone()
    key = -torch.ones(2, 3, 2)
    key[1] *= 2
    kv_write(key, None, cache, None, torch.tensor([5, 0]))
    flat, fb = cache.view(-1, 3, 2), before.view(-1, 3, 2)
    assert torch.equal(flat[5], key[0]) and torch.equal(flat[0], key[1])
    keep = [i for i in range(8) if i not in (0, 5)]
    assert torch.equal(flat[keep], fb[keep])


def test_absorbed_mla_equals_non_absorbed():
    """Absorbed latent attention (mla.py:76-122) equals materialising
    K = [W_UK^T ckv, k_pe] and V = W_UV^T ckv per head (mla.py:23-64) -- the
    identity the reference checks on NPU (scripts/verify_mla_absorb.py)."""
    g = torch.Generator().manual_seed(7)
    H, nope, rope, vd, kvl, L, bs = 3, 8, 4, 6, 16, 7, 4
    ckv = torch.randn(L, kvl, generator=g, dtype=torch.float64)
    kpe = torch.randn(L, rope, generator=g, dtype=torch.float64)
    w_uk = torch.randn(H, nope, kvl, generator=g, dtype=torch.float64)
    w_uv = torch.randn(H, vd, kvl, generator=g, dtype=torch.float64)
    q_nope = torch.randn(1, H, nope, generator=g, dtype=torch.float64)
    q_pe = torch.randn(1, H, rope, generator=g, dtype=torch.float64)
    scale = (nope + rope) ** -0.5
    nb = (L + bs - 1) // bs
    bt = torch.arange(nb).view(1, nb)
    # absorbed
    q_lat = torch.cat([torch.einsum("tnp,npl->tnl", q_nope, w_uk), q_pe], dim=-1)
    lat = torch.zeros(nb * bs, 1, kvl + rope, dtype=torch.float64)
    lat[:L, 0] = torch.cat([ckv, kpe], dim=-1)
    o_lat = mla_absorbed_attention(q_lat, lat.view(nb, bs, 1, -1), bt, [1], [L], scale, kvl)
    o_abs = torch.einsum("tnl,nvl->tnv", o_lat.double(), w_uv)
    # non-absorbed
    k_nope = torch.einsum("jl,npl->jnp", ckv, w_uk)
    k = torch.cat([k_nope, kpe[:, None].expand(L, H, rope)], dim=-1)
    v = torch.einsum("jl,nvl->jnv", ckv, w_uv)
    kc = torch.zeros(nb * bs, H, nope + rope, dtype=torch.float64)
    vc = torch.zeros(nb * bs, H, vd, dtype=torch.float64)
    kc[:L], vc[:L] = k, v
    q = torch.cat([q_nope, q_pe], dim=-1)
    o_full = paged_attention(q, kc.view(nb, bs, H, -1), vc.view(nb, bs, H, -1), bt, [1], [L],
                             scale)
    assert torch.allclose(o_abs.float(), o_full, atol=1e-5)
