"""Seeded synthetic steps for the benchmark configurations.

Each generator returns plain tensors shaped like one layer's inputs for one
step of the reference's paged path: query rows (T, Hq, D), this step's new
K/V rows, the paged caches (reference layout (NB, bs, Hkv, D) per cache,
gqa.py:69-74), block tables, the cumulative query lengths / per-request KV
lengths lists (ForwardContext, forward_context.py:14-15) and the slot
mapping of the new rows (token_layout.py:1-4).
"""
import math
from dataclasses import dataclass, field

import numpy as np
import torch


@dataclass
class GqaStep:
    q: torch.Tensor
    k_new: torch.Tensor
    v_new: torch.Tensor
    k_cache: torch.Tensor
    v_cache: torch.Tensor
    block_table: torch.Tensor      # (B, max_blocks) int32, zero padded
    cu_seqlens_q: list             # cumulative ends, no leading 0
    seqlens_kv: list
    slot_mapping: torch.Tensor     # (T,) int32
    scale: float
    meta: dict = field(default_factory=dict)

    @property
    def num_tokens(self):
        return self.q.shape[0]

    def kv_bytes_read(self):
        """Logical KV bytes one attention pass reads (no dedup of shared blocks)."""
        _, _, hkv, d = self.k_cache.shape
        return sum(self.seqlens_kv) * 2 * hkv * d * self.k_cache.element_size()


def _block_tables(rng, lks, bs, num_blocks, shared_prefix_blocks=0, share_frac=0.0):
    """Disjoint random block assignment (a permutation of the pool); a
    fraction of requests may share their first ``shared_prefix_blocks``."""
    need = [(lk + bs - 1) // bs for lk in lks]
    perm = rng.permutation(num_blocks)
    if sum(need) > num_blocks:
        raise ValueError(f"pool of {num_blocks} blocks cannot hold {sum(need)}")
    tables, cur = [], 0
    shared = None
    for i, n in enumerate(need):
        row = perm[cur:cur + n].tolist()
        cur += n
        if shared_prefix_blocks and rng.random() < share_frac and n > shared_prefix_blocks:
            if shared is None:
                shared = row[:shared_prefix_blocks]
            else:
                row[:shared_prefix_blocks] = shared
        tables.append(row)
    return tables


def make_gqa_step(*, lqs, lks, num_q_heads, num_kv_heads, head_dim=128, block_size=128,
                  num_blocks=None, seed=0, device="cpu", value_scale=1.0,
                  dtype=torch.bfloat16, shared_prefix_blocks=0, share_frac=0.0,
                  extra_blocks=0, tables=None):
    """One GQA step: request b has lqs[b] query rows at the end of its
    lks[b]-long context (new K/V rows are the last lqs[b] positions)."""
    rng = np.random.default_rng(seed)
    B = len(lks)
    need = sum((lk + block_size - 1) // block_size for lk in lks)
    if num_blocks is None:
        num_blocks = need + extra_blocks
    if tables is None:
        tables = _block_tables(rng, lks, block_size, num_blocks, shared_prefix_blocks,
                               share_frac)
    width = max((len(t) for t in tables), default=0)
    bt = np.zeros((B, max(width, 1)), dtype=np.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = t
    dev = torch.device(device)
    gen = torch.Generator(device=dev).manual_seed(seed)
    T = sum(lqs)

    def rnd(*shape):
        if dev.type == "cpu":
            return (torch.randn(*shape, generator=gen) * value_scale).to(dtype)
        # on the GPU: generate in the target dtype (no fp32 temporary of the pool)
        t = torch.randn(*shape, generator=gen, device=dev, dtype=dtype)
        return t.mul_(value_scale) if value_scale != 1.0 else t
    q = rnd(T, num_q_heads, head_dim)
    k_new = rnd(T, num_kv_heads, head_dim)
    v_new = rnd(T, num_kv_heads, head_dim)
    shape = (num_blocks, block_size, num_kv_heads, head_dim)
    k_cache = rnd(*shape)
    v_cache = rnd(*shape)
    slots, cu, acc = [], [], 0
    for b, (lq, lk) in enumerate(zip(lqs, lks)):
        for p in range(lk - lq, lk):
            slots.append(bt[b, p // block_size] * block_size + p % block_size)
        acc += lq
        cu.append(acc)
    return GqaStep(q=q, k_new=k_new, v_new=v_new, k_cache=k_cache, v_cache=v_cache,
                   block_table=torch.from_numpy(bt).to(dev), cu_seqlens_q=cu,
                   seqlens_kv=list(lks),
                   slot_mapping=torch.tensor(slots, dtype=torch.int32, device=dev),
                   scale=head_dim ** -0.5)


def _to(self, device):
    for name in ("q", "k_new", "v_new", "k_cache", "v_cache", "block_table", "slot_mapping"):
        setattr(self, name, getattr(self, name).to(device))
    return self


GqaStep.to = _to


def subset(step, requests):
    """A self-contained CPU copy of the given requests of a GQA step: only
    their blocks, renumbered, with their query rows (attention rows of a
    request depend only on that request).  Returns (step, query row index)."""
    bt = step.block_table.cpu()
    rows, cu, kv, acc = [], [], [], 0
    starts = [0] + list(step.cu_seqlens_q[:-1])
    for r in requests:
        lq = step.cu_seqlens_q[r] - starts[r]
        rows.extend(range(starts[r], starts[r] + lq))
        acc += lq
        cu.append(acc)
        kv.append(step.seqlens_kv[r])
    bs = step.k_cache.shape[1]
    used = sorted({int(bt[r, c]) for r in requests
                   for c in range((step.seqlens_kv[r] + bs - 1) // bs)})
    remap = {b: i for i, b in enumerate(used)}
    idx = torch.tensor(used, dtype=torch.long, device=step.k_cache.device)
    width = max((step.seqlens_kv[r] + bs - 1) // bs for r in requests)
    nbt = torch.zeros(len(requests), max(width, 1), dtype=torch.int32)
    for i, r in enumerate(requests):
        for c in range((step.seqlens_kv[r] + bs - 1) // bs):
            nbt[i, c] = remap[int(bt[r, c])]
    ridx = torch.tensor(rows, dtype=torch.long, device=step.q.device)
    sub = GqaStep(q=step.q[ridx].cpu(), k_new=step.k_new[ridx].cpu(),
                  v_new=step.v_new[ridx].cpu(), k_cache=step.k_cache[idx].cpu(),
                  v_cache=step.v_cache[idx].cpu(), block_table=nbt, cu_seqlens_q=cu,
                  seqlens_kv=kv, slot_mapping=None, scale=step.scale)
    return sub, rows


def config1_decode(seed=0, device="cpu", num_blocks=512):
    """Qwen3-0.6B heads (16 q / 8 kv / 128), bf16, batch 16,
    query length 1, contexts U[128, 2048], block 128, pool 512 blocks, values
    N(0,1)/sqrt(128)."""
    rng = np.random.default_rng(seed)
    lks = rng.integers(128, 2048, size=16, endpoint=True).tolist()
    return make_gqa_step(lqs=[1] * 16, lks=lks, num_q_heads=16, num_kv_heads=8,
                         block_size=128, num_blocks=num_blocks, seed=seed + 1,
                         device=device, value_scale=1.0 / math.sqrt(128))


@dataclass
class MlaStep:
    q_latent: torch.Tensor        # (T, H, 576) = [absorbed nope (512), rope (64)]
    latent_new: torch.Tensor      # (T, 1, 576) this step's latent rows
    cache: torch.Tensor           # (NB, bs, 1, 576)
    block_table: torch.Tensor
    cu_seqlens_q: list
    seqlens_kv: list
    slot_mapping: torch.Tensor
    scale: float

    @property
    def num_tokens(self):
        return self.q_latent.shape[0]

    def kv_bytes_read(self):
        return sum(self.seqlens_kv) * self.cache.shape[-1] * self.cache.element_size()

    def to(self, device):
        for name in ("q_latent", "latent_new", "cache", "block_table", "slot_mapping"):
            setattr(self, name, getattr(self, name).to(device))
        return self


def make_mla_step(*, lqs, lks, num_heads=16, block_size=128, num_blocks=None, seed=0,
                  extra_blocks=0, dtype=torch.bfloat16, scale=192 ** -0.5, device="cpu"):
    """Absorbed-MLA step (latent 512 + rope 64 per token, one KV head)."""
    rng = np.random.default_rng(seed)
    need = sum((lk + block_size - 1) // block_size for lk in lks)
    if num_blocks is None:
        num_blocks = need + extra_blocks
    tables = _block_tables(rng, lks, block_size, num_blocks)
    width = max((len(t) for t in tables), default=0)
    bt = np.zeros((len(lks), max(width, 1)), dtype=np.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = t
    dev = torch.device(device)
    gen = torch.Generator(device=dev).manual_seed(seed)
    T = sum(lqs)
    if dev.type == "cpu":
        q = torch.randn(T, num_heads, 576, generator=gen).to(dtype)
        lat = torch.randn(T, 1, 576, generator=gen).to(dtype)
        cache = torch.randn(num_blocks, block_size, 1, 576, generator=gen).to(dtype)
    else:
        q = torch.randn(T, num_heads, 576, generator=gen, device=dev, dtype=dtype)
        lat = torch.randn(T, 1, 576, generator=gen, device=dev, dtype=dtype)
        cache = torch.randn(num_blocks, block_size, 1, 576, generator=gen, device=dev, dtype=dtype)
    slots, cu, acc = [], [], 0
    for b, (lq, lk) in enumerate(zip(lqs, lks)):
        for p in range(lk - lq, lk):
            slots.append(bt[b, p // block_size] * block_size + p % block_size)
        acc += lq
        cu.append(acc)
    return MlaStep(q_latent=q, latent_new=lat, cache=cache,
                   block_table=torch.from_numpy(bt).to(dev), cu_seqlens_q=cu,
                   seqlens_kv=list(lks),
                   slot_mapping=torch.tensor(slots, dtype=torch.int32, device=dev), scale=scale)


def config3_mla(seed=0, device="cpu"):
    """absorbed MLA, 16 heads, latent 512 + rope 64,
    block 128, batch 64, query length 1, contexts log-uniform [512, 8192],
    values N(0,1), scale 1/sqrt(192)."""
    rng = np.random.default_rng(seed)
    lks = np.exp(rng.uniform(np.log(512), np.log(8192), size=64)).astype(int).tolist()
    return make_mla_step(lqs=[1] * 64, lks=lks, num_heads=16, block_size=128, seed=seed + 1,
                         device=device)


def fragmented_block_tables(lks, *, num_blocks, block_size, ops=10000, seed=0, allocator=None):
    """Block tables for requests of context lengths ``lks`` drawn from an
    allocator that first ran a seeded trace of ``ops`` allocate/free
    operations, so the tables are non-contiguous.
    ``allocator``: the allocator class (default: the product's)."""
    from auto_infer_amd.block_allocator import KVCacheManager
    rng = np.random.default_rng(seed)
    kv = (allocator or KVCacheManager)(num_blocks, block_size)
    live = []
    for _ in range(ops):
        if live and (rng.random() < 0.45 or kv.num_free_blocks() < num_blocks // 4):
            kv.free(live.pop(int(rng.integers(len(live)))))
        else:
            n = int(min(32768, max(1, rng.lognormal(np.log(2048), 1.0))))
            if kv.can_allocate(n):
                live.append(kv.allocate(n))
    return [kv.allocate(lk) for lk in lks], kv


def config2_mixed(seed=0, device="cpu"):
    """Qwen2-7B heads (28 q / 4 kv / 128), block 128,
    token budget 2048 = 3 prefill chunks of 512 continuing a prefix
    U[0, 1024] (causal inside the chunk) + 512 decode rows with contexts
    U[256, 4096]; 25% of requests share their first 4 blocks; values N(0,1)."""
    rng = np.random.default_rng(seed)
    prefix = rng.integers(0, 1024, size=3, endpoint=True).tolist()
    dec = rng.integers(256, 4096, size=512, endpoint=True).tolist()
    lqs = [512] * 3 + [1] * 512
    lks = [p + 512 for p in prefix] + dec
    return make_gqa_step(lqs=lqs, lks=lks, num_q_heads=28, num_kv_heads=4, block_size=128,
                         seed=seed + 1, shared_prefix_blocks=4, share_frac=0.25, device=device)


def config4_mtp(seed=0, device="cpu"):
    """MiMo-7B heads (32 q / 8 kv / 128), block 128, batch
    16, query length 2 (accepted token + one draft, causal in the pair),
    contexts U[1024, 4096]; values N(0,1)."""
    rng = np.random.default_rng(seed)
    lks = rng.integers(1024, 4096, size=16, endpoint=True).tolist()
    return make_gqa_step(lqs=[2] * 16, lks=lks, num_q_heads=32, num_kv_heads=8,
                         block_size=128, seed=seed + 1, device=device)


def config5_contexts(seed=0, batch=256):
    """BASELINE config 5 contexts: lognormal (median 2048, sigma 1), clipped
    to [64, 32768]."""
    rng = np.random.default_rng(seed)
    return np.clip(rng.lognormal(np.log(2048), 1.0, size=batch), 64, 32768).astype(int).tolist()
