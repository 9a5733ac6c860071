"""Float32 torch-CPU restatement of the KV write and paged attention op.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The reference delegates both ops to closed torch_npu kernels; their
semantics are fixed by the call sites:

* KV write -- auto_infer/layers/attention/base.py:41-45
  (``_npu_reshape_and_cache``): ``cache.view(-1, Hkv, D)[slot[t]] = k[t]``
  for K and V.  Absorbed MLA writes the same 576-wide latent to both caches
  (auto_infer/layers/attention/mla.py:111-113).
* Paged attention -- base.py:48-61 (``npu_fused_infer_attention_score`` with
  input_layout="TND", sparse_mode=3): for request b with
  Lq = cu[b] - cu[b-1] query rows and Lk = seqlens_kv[b] keys, query row i
  sees keys j <= Lk - Lq + i (bottom-right causal); query head h reads KV
  head h // (Hq / Hkv) (gqa.py:81-94); KV row j lives at
  ``block_table[b, j // bs]``, offset ``j % bs``; scale is passed in
  (head_dim ** -0.5 for GQA, registry.py:42).  Absorbed MLA attends with one
  KV head, V = K and keeps the first kv_lora_rank outputs (mla.py:114-120).
"""
import math

import torch


def kv_write(key, value, key_cache, value_cache, slot_mapping):
    """In-place index assignment of this step's K/V rows (base.py:41-45)."""
    heads, dim = key.shape[1], key.shape[2]
    slots = torch.as_tensor(slot_mapping, dtype=torch.long)
    key_cache.view(-1, heads, dim)[slots] = key.to(key_cache.dtype)
    if value is not None and value_cache is not None:
        vh, vd = value.shape[1], value.shape[2]
        value_cache.view(-1, vh, vd)[slots] = value.to(value_cache.dtype)


# ---- NZ layout of the reference's graph-mode caches (gqa.py:163,195-226):
# a (NB, bs, Hkv, D) cache tensor whose memory is viewed (NB, Hkv*D/16, bs,
# 16) by npu_scatter_pa_kv_cache and FIA-v2.

NZ = 16   # gqa.py:163


def nz_from_nd(cache):
    """The NZ memory image of standard-layout values: the returned (NB, bs,
    Hkv, D) tensor, viewed (NB, Hkv*D/16, bs, 16), holds value d of head h of
    block offset t at [blk, (h*D + d) // 16, t, d % 16]."""
    nb, bs, h, d = cache.shape
    return (cache.reshape(nb, bs, h * d // NZ, NZ).permute(0, 2, 1, 3).contiguous()
            .reshape(nb, bs, h, d))


def nd_from_nz(cache):
    """Standard-layout values of a cache whose memory holds the NZ image."""
    nb, bs, h, d = cache.shape
    return cache.reshape(nb, h * d // NZ, bs, NZ).permute(0, 2, 1, 3).reshape(nb, bs, h, d)


def kv_write_nz(key, value, key_cache, value_cache, slot_mapping):
    """npu_scatter_pa_kv_cache(k, v, kc.view(NB, Hkv*D/16, bs, 16), ...,
    slot_mapping) (gqa.py:202-211), in place: token t's row, split into
    16-wide chunks, goes to [slot // bs, chunk, slot % bs, :]."""
    for src, cache in ((key, key_cache), (value, value_cache)):
        if src is None:
            continue
        nb, bs, h, d = cache.shape
        view = cache.view(nb, h * d // NZ, bs, NZ)
        rows = src.reshape(src.shape[0], h * d // NZ, NZ)
        for t, s in enumerate(torch.as_tensor(slot_mapping).tolist()):
            if 0 <= s < nb * bs:
                view[s // bs, :, s % bs, :] = rows[t]


def _segments(cu_seqlens_q):
    start = 0
    for end in cu_seqlens_q:
        yield start, end
        start = end


def paged_attention(query, key_cache, value_cache, block_table, cu_seqlens_q,
                    seqlens_kv, scale, value_dim=None):
    """Gather-softmax paged attention in float32 (base.py:48-61 semantics).

    query (T, Hq, D); key_cache (NB, bs, Hkv, D); value_cache (NB, bs, Hkv, Dv)
    (may be the key cache itself, e.g. absorbed MLA); block_table (B, W) int;
    cu_seqlens_q cumulative ends (len B); seqlens_kv per request (len B).
    Returns float32 (T, Hq, value_dim or Dv).
    """
    T, hq, _ = query.shape
    bs, hkv = key_cache.shape[1], key_cache.shape[2]
    dv = value_cache.shape[-1] if value_dim is None else value_dim
    group = hq // hkv
    out = torch.zeros(T, hq, dv, dtype=torch.float32)
    bt = torch.as_tensor(block_table, dtype=torch.long)
    for b, (s, e) in enumerate(_segments(cu_seqlens_q)):
        lq, lk = e - s, int(seqlens_kv[b])
        if lq == 0 or lk == 0:
            continue
        j = torch.arange(lk)
        blocks = bt[b, j // bs]
        k = key_cache[blocks, j % bs].float()                  # (Lk, Hkv, D)
        v = value_cache[blocks, j % bs].float()[..., :dv]       # (Lk, Hkv, Dv)
        k = k.repeat_interleave(group, dim=1).transpose(0, 1)  # (Hq, Lk, D)
        v = v.repeat_interleave(group, dim=1).transpose(0, 1)
        q = query[s:e].float().transpose(0, 1)                 # (Hq, Lq, D)
        scores = (q @ k.transpose(-1, -2)) * scale              # (Hq, Lq, Lk)
        limit = lk - lq + torch.arange(lq)                      # bottom-right
        masked = j[None, :] > limit[:, None]
        scores = scores.masked_fill(masked, float("-inf"))
        prob = torch.softmax(scores, dim=-1)
        prob = torch.nan_to_num(prob, nan=0.0)                  # fully masked rows -> 0
        out[s:e] = (prob @ v).transpose(0, 1)
    return out


def mla_absorbed_attention(q_latent, latent_cache, block_table, cu_seqlens_q,
                           seqlens_kv, scale, kv_lora_rank):
    """Absorbed-MLA latent attention (mla.py:76-122): one KV head of width
    kv_lora_rank + rope, V = K, output keeps the first kv_lora_rank values."""
    return paged_attention(q_latent, latent_cache, latent_cache, block_table,
                           cu_seqlens_q, seqlens_kv, scale,
                           value_dim=kv_lora_rank)


def paged_attention_f64_bruteforce(query, key_cache, value_cache, block_table,
                                   cu_seqlens_q, seqlens_kv, scale,
                                   value_dim=None):
    """Scalar-loop float64 version of the same definition, for tiny inputs.

    Written independently of ``paged_attention`` (explicit per-key loop,
    max-subtracted exponentials, no tensor masking) so that a slip in one
    does not repeat in the other.
    """
    T, hq, d = query.shape
    bs, hkv = key_cache.shape[1], key_cache.shape[2]
    dv = value_cache.shape[-1] if value_dim is None else value_dim
    group = hq // hkv
    out = torch.zeros(T, hq, dv, dtype=torch.float64)
    for b, (s, e) in enumerate(_segments(cu_seqlens_q)):
        lq, lk = e - s, int(seqlens_kv[b])
        for i in range(lq):
            visible = lk - lq + i + 1
            for h in range(hq):
                kh = h // group
                qv = query[s + i, h].double()
                logits = []
                for jj in range(max(visible, 0)):
                    blk = int(block_table[b][jj // bs])
                    kvec = key_cache[blk, jj % bs, kh].double()
                    logits.append(float((qv * kvec).sum()) * scale)
                if not logits:
                    continue
                mx = max(logits)
                w = [math.exp(x - mx) for x in logits]
                z = sum(w)
                acc = torch.zeros(dv, dtype=torch.float64)
                for jj, wj in enumerate(w):
                    blk = int(block_table[b][jj // bs])
                    acc += wj * value_cache[blk, jj % bs, kh, :dv].double()
                out[s + i, h] = acc / z
    return out
