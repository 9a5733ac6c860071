"""Pins for the oracle's NZ-layout helpers (CPU).  The reference's graph mode
keeps each KV cache as a (NB, bs, Hkv, D) tensor whose memory
npu_scatter_pa_kv_cache and FIA-v2 view as (NB, Hkv*D/16, bs, 16)
(auto_infer/layers/attention/gqa.py:202-226).  The checks below index that
view element by element from its definition -- the flat offset of
[blk, c, t, j] is ((blk*C + c)*bs + t)*16 + j -- so a transposed tile or a
wrong chunk index fails them."""
import torch

from oracle.paged_attn import NZ, kv_write, kv_write_nz, nd_from_nz, nz_from_nd


def _bruteforce_nz(nd):
    nb, bs, h, d = nd.shape
    c_n = h * d // NZ
    flat = torch.empty(nd.numel(), dtype=nd.dtype)
    for blk in range(nb):
        for c in range(c_n):
            for t in range(bs):
                for j in range(NZ):
                    e = c * NZ + j
                    flat[((blk * c_n + c) * bs + t) * NZ + j] = nd[blk, t, e // d, e % d]
    return flat.view(nb, bs, h, d)


def test_nz_image_matches_the_view_definition():
    for shape in ((2, 4, 2, 32), (3, 16, 1, 64), (1, 5, 3, 16)):
        nd = torch.arange(torch.Size(shape).numel(), dtype=torch.float32).view(shape)
        assert torch.equal(nz_from_nd(nd), _bruteforce_nz(nd))


def test_round_trip_and_block_size_one_is_identity():
    g = torch.Generator().manual_seed(3)
    nd = torch.randn(4, 8, 2, 64, generator=g)
    assert torch.equal(nd_from_nz(nz_from_nd(nd)), nd)
    # one slot per block: the (Hkv*D/16, 1, 16) view is the row itself
    one = torch.randn(6, 1, 4, 32, generator=g)
    assert torch.equal(nz_from_nd(one), one)
    # more than one slot: the layouts differ
    assert not torch.equal(nz_from_nd(nd), nd)


def test_kv_write_nz_is_kv_write_then_nz_image():
    """Scattering rows into the NZ view equals writing them in the standard
    layout and taking the NZ image; out-of-range slots are skipped."""
    g = torch.Generator().manual_seed(5)
    nb, bs, h, d, t = 5, 16, 2, 128, 11
    base = torch.randn(nb, bs, h, d, generator=g)
    k = torch.randn(t, h, d, generator=g)
    v = torch.randn(t, h, d, generator=g)
    slots = torch.tensor([0, 17, 79, -1, 33, 40, 41, nb * bs, 2, 15, 64], dtype=torch.int32)
    ek, ev = base.clone(), base.clone() + 1
    keep = (slots >= 0) & (slots < nb * bs)
    kv_write(k[keep], v[keep], ek, ev, slots[keep])
    gk, gv = nz_from_nd(base), nz_from_nd(base + 1)
    kv_write_nz(k, v, gk, gv, slots)
    assert torch.equal(gk, nz_from_nd(ek)) and torch.equal(gv, nz_from_nd(ev))
    # a written row is readable back through the view at [slot//bs, :, slot%bs, :]
    view = gk.view(nb, h * d // NZ, bs, NZ)
    assert torch.equal(view[17 // bs, :, 17 % bs, :].reshape(-1), k[1].reshape(-1))
    # key only
    only = nz_from_nd(base)
    kv_write_nz(k, None, only, None, slots)
    assert torch.equal(only, gk)
