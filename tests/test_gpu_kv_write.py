"""KV slot write on the GPU vs the oracle's index assignment: bit-exact."""
import pytest
import torch

from auto_infer_amd import ops
from oracle.paged_attn import kv_write as oracle_kv_write

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.mark.parametrize("T,hkv,d,nb,bs", [(16, 8, 128, 512, 128), (1, 1, 576, 64, 128),
                                           (37, 4, 128, 40, 16), (0, 8, 128, 8, 4)])
def test_kv_write_bit_exact(T, hkv, d, nb, bs):
    g = torch.Generator().manual_seed(T * 31 + d)
    kc = torch.randn(nb, bs, hkv, d, generator=g).bfloat16()
    vc = torch.randn(nb, bs, hkv, d, generator=g).bfloat16()
    k = torch.randn(T, hkv, d, generator=g).bfloat16()
    v = torch.randn(T, hkv, d, generator=g).bfloat16()
    slots = torch.randperm(nb * bs, generator=g)[:T].to(torch.int32)
    ek, ev = kc.clone(), vc.clone()
    oracle_kv_write(k, v, ek, ev, slots)
    gk, gv = kc.to(DEV), vc.to(DEV)
    ops.write_kv(k.to(DEV), v.to(DEV), gk, gv, slots.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(gk.cpu().view(torch.int16), ek.view(torch.int16))
    assert torch.equal(gv.cpu().view(torch.int16), ev.view(torch.int16))


def test_kv_write_strided_views_of_a_packed_projection():
    """k/v as column slices of a packed qkv projection (gqa.py:14-16, 36-39)."""
    T, hq, hkv, d, nb, bs = 9, 16, 8, 128, 16, 16
    g = torch.Generator().manual_seed(5)
    qkv = torch.randn(T, (hq + 2 * hkv) * d, generator=g).bfloat16()
    _, k, v = qkv.split((hq * d, hkv * d, hkv * d), dim=-1)
    k, v = k.view(T, hkv, d), v.view(T, hkv, d)
    kc = torch.zeros(nb, bs, hkv, d).bfloat16()
    vc = torch.zeros(nb, bs, hkv, d).bfloat16()
    slots = torch.tensor([3, 17, 40, 41, 42, 100, 200, 255, 0], dtype=torch.int32)
    ek, ev = kc.clone(), vc.clone()
    oracle_kv_write(k, v, ek, ev, slots)
    gqkv = qkv.to(DEV)
    _, gk, gv = gqkv.split((hq * d, hkv * d, hkv * d), dim=-1)
    gkc, gvc = kc.to(DEV), vc.to(DEV)
    ops.write_kv(gk.view(T, hkv, d), gv.view(T, hkv, d), gkc, gvc, slots.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(gkc.cpu(), ek) and torch.equal(gvc.cpu(), ev)


def test_kv_write_single_cache_and_padding_slots():
    """Absorbed MLA writes one 576-wide latent row; negative slots are skipped."""
    T, d, nb, bs = 6, 576, 8, 16
    g = torch.Generator().manual_seed(7)
    cache = torch.randn(nb, bs, 1, d, generator=g).bfloat16()
    lat = torch.randn(T, 1, d, generator=g).bfloat16()
    slots = torch.tensor([5, -1, 33, 127, -7, 64], dtype=torch.int32)
    exp = cache.clone()
    keep = slots >= 0
    oracle_kv_write(lat[keep], None, exp, None, slots[keep])
    gc = cache.to(DEV)
    ops.write_kv(lat.to(DEV), None, gc, None, slots.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(gc.cpu(), exp)
