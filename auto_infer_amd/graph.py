"""HIP-graph decode: capture once per gear, replay every step.

The reference captures an ACL graph per decode gear and, after every replay,
re-issues each layer's attention op with the step's new ``seqlens_kv`` on a
side thread (auto_infer/worker/graph_decode_runner.py:416-541,
layers/attention/graph_fia.py:66-95).  The kernels here read all step
metadata from device buffers, so a captured graph needs no updates: the
stager rewrites its fixed-address buffers in place (one upload + the packing
kernel, outside the graph), and the graph -- planner once, then every
layer's attention with the fused KV write -- is replayed as is.
"""
import torch

from auto_infer_amd import ops


class _GearGraph:
    """Capture / stage / replay shared by the GQA and latent gears."""

    def _body(self):
        raise NotImplementedError

    def capture(self):
        """Capture after one staged step (the buffers hold valid metadata)."""
        with torch.cuda.stream(self.stream):
            self._body()                       # warm-up outside the graph
            torch.cuda.synchronize()
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph, stream=self.stream):
                self._body()
        return self

    def stage(self, plan, scheduled=None):
        with torch.cuda.stream(self.stream):
            return self.stager.stage(plan, scheduled)

    def replay(self):
        with torch.cuda.stream(self.stream):
            self.graph.replay()


class DecodeGraph(_GearGraph):
    """One decode gear of GQA layers captured in a HIP graph.

    ``stager``: a ``packing.DecodeInputStager`` or ``SpecDecodeInputStager``
    whose buffers (slots, block table, cu/kv lengths) the graph reads.
    ``caches``: per-layer (key_cache, value_cache).  ``q``, ``k_new``,
    ``v_new``: fixed-address per-layer input buffers (T, H, D) the caller
    fills before each replay (the projections' outputs); ``out`` receives
    each layer's attention output.  ``kv_layout="nz"``: the caches are in the
    NZ layout of the reference's graph mode (``GraphGqaBackend``,
    gqa.py:192-226), as ``GqaHipBackend(kv_layout="nz")`` allocates them.
    """

    def __init__(self, stager, caches, *, num_q_heads, num_kv_heads, head_dim=128, scale=None,
                 stream=None, kv_layout="nd"):
        if kv_layout not in ops.KV_LAYOUTS:
            raise ValueError(f"kv_layout must be one of {sorted(ops.KV_LAYOUTS)}")
        self.kv_layout = kv_layout
        self.stager = stager
        self.caches = caches
        dev = stager.block_table.device
        T = stager.slots.shape[0]
        L = len(caches)
        self.q = torch.zeros(L, T, num_q_heads, head_dim, dtype=torch.bfloat16, device=dev)
        self.k_new = torch.zeros(L, T, num_kv_heads, head_dim, dtype=torch.bfloat16, device=dev)
        self.v_new = torch.zeros_like(self.k_new)
        self.out = torch.zeros_like(self.q)
        self.scale = head_dim ** -0.5 if scale is None else scale
        self.stream = stream or torch.cuda.Stream(device=dev)
        block_size = caches[0][0].shape[1]
        with torch.cuda.stream(self.stream):
            self.plan = ops.AttentionPlan(stager.block_table, stager._cu, stager._kv, T,
                                          num_q_heads, num_kv_heads, head_dim, block_size)
        self.graph = None

    def _body(self):
        self.plan.replan()
        for layer, (kc, vc) in enumerate(self.caches):
            ops.paged_attention_gqa(self.q[layer], kc, vc, self.plan, self.scale,
                                    out=self.out[layer], key_new=self.k_new[layer],
                                    value_new=self.v_new[layer], kv_layout=self.kv_layout)


class LatentDecodeGraph(_GearGraph):
    """One decode (or MTP verify) gear of absorbed-MLA layers in a HIP graph
    -- the latent-cache counterpart of the reference's GraphMlaBackend
    (auto_infer/layers/attention/mla.py:258-366), whose graph replays the
    latent write and the 576-wide attention per layer.

    ``caches``: per layer the latent cache (NB, bs, 1, 576), or the
    (latent, latent) pair ``MlaHipBackend.alloc_kv_caches`` returns.
    ``q``: (L, T, H, 576) latent queries, ``latent_new``: (L, T, 1, 576) this
    step's latent rows, both filled by the caller before each replay;
    ``out``: (L, T, H, 512) latent attention outputs.  Per layer the graph
    writes the new rows at the stager's slots, then attends; the planner
    runs once per replay on the stager's device metadata.
    """

    def __init__(self, stager, caches, *, num_heads, scale=192 ** -0.5, stream=None):
        self.stager = stager
        self.caches = [c[0] if isinstance(c, (tuple, list)) else c for c in caches]
        dev = stager.block_table.device
        T = stager.slots.shape[0]
        L = len(self.caches)
        width = ops.MLA_LATENT + ops.MLA_ROPE
        self.q = torch.zeros(L, T, num_heads, width, dtype=torch.bfloat16, device=dev)
        self.latent_new = torch.zeros(L, T, 1, width, dtype=torch.bfloat16, device=dev)
        self.out = torch.zeros(L, T, num_heads, ops.MLA_LATENT, dtype=torch.bfloat16, device=dev)
        self.scale = scale
        self.stream = stream or torch.cuda.Stream(device=dev)
        block_size = self.caches[0].shape[1]
        with torch.cuda.stream(self.stream):
            self.plan = ops.AttentionPlan(stager.block_table, stager._cu, stager._kv, T,
                                          num_heads, 1, ops.MLA_LATENT, block_size)
        self.graph = None

    def _body(self):
        self.plan.replan()
        for layer, latent in enumerate(self.caches):
            ops.write_kv(self.latent_new[layer], None, latent, None, self.stager.slots)
            ops.paged_attention_mla(self.q[layer], latent, self.plan, self.scale,
                                    out=self.out[layer])
