"""Torch-facing wrappers of the gfx950 kernels.

PyTorch owns every buffer (caches, metadata, workspace); these functions
check shapes/dtypes/devices on the host, then hand raw pointers and the
current HIP stream to the C ABI.  Nothing here computes on the CPU.
"""
import ctypes

import torch

from auto_infer_amd import _native

_BF16 = torch.bfloat16


# Pointers and streams go to the C-ABI as plain ints: every pointer
# parameter is declared c_void_p, which converts them (and None -> NULL).
def _stream(device):
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t):
    return t.data_ptr() if t is not None else None


def _require(cond, msg):
    if not cond:
        raise ValueError(msg)


def _check_device_tensor(t, name, dtype=None):
    _require(isinstance(t, torch.Tensor), f"{name} must be a tensor")
    _require(t.is_cuda, f"{name} must be on the GPU (no CPU fallback)")
    if dtype is not None:
        _require(t.dtype == dtype, f"{name} must be {dtype}, got {t.dtype}")


def _row_stride(t, name):
    """Token stride of a (T, heads, dim) tensor whose (heads, dim) part is
    one contiguous row."""
    _require(t.dim() == 3, f"{name} must be (tokens, heads, dim)")
    _require(t.stride(2) == 1 and t.stride(1) == t.shape[2],
             f"{name} rows (heads, dim) must be contiguous")
    return t.stride(0)


# ---------------------------------------------------------------- KV write

def qk_norm_rope(qkv, num_q_heads, num_kv_heads, cos, sin, q_norm_weight=None,
                 k_norm_weight=None, eps=1e-6, head_dim=128):
    """Fused pre-attention over a packed qkv projection, in place: optional
    per-head RMSNorm of the Q and K heads (Qwen3 QK-Norm) and NeoX RoPE with
    ``cos``/``sin`` of shape (T, 1, D) or (T, D), D = ``head_dim`` (128 or
    64).  Returns the (q, k, v) views of ``qkv`` -- (T, Hq, D), (T, Hkv, D),
    (T, Hkv, D) -- ready for ``paged_attention_gqa(q, ..., key_new=k,
    value_new=v)``.

    Replaces the split / rms_norm / rotary steps of the reference's
    ``_GqaProjRopeMixin.attention`` (auto_infer/layers/attention/gqa.py:
    27-49) with one kernel that rounds to bf16 where those ops round."""
    _check_device_tensor(qkv, "qkv", _BF16)
    _require(qkv.dim() == 2 and qkv.stride(1) == 1, "qkv must be (T, width) with unit inner stride")
    T, width = qkv.shape
    D = int(head_dim)
    if D not in (128, 64):
        raise NotImplementedError(f"qk_norm_rope: head_dim {D} (128 or 64)")
    _require(width == (num_q_heads + 2 * num_kv_heads) * D,
             f"qkv width {width} != (Hq + 2 Hkv) x {D}")
    cs = []
    for t, name in ((cos, "cos"), (sin, "sin")):
        _check_device_tensor(t, name, _BF16)
        _require(t.shape[0] == T and t.shape[-1] == D and t.numel() == T * D and t.stride(-1) == 1,
                 f"{name} must hold one {D}-wide row per token")
        cs.append(t.stride(0))
    for t, name in ((q_norm_weight, "q_norm_weight"), (k_norm_weight, "k_norm_weight")):
        if t is not None:
            _check_device_tensor(t, name, _BF16)
            _require(t.numel() == D and t.is_contiguous(), f"{name} must be {D} contiguous values")
    _native.call("aia_qk_norm_rope", _ptr(qkv), qkv.stride(0), T, num_q_heads, num_kv_heads, D,
                 _ptr(cos), cs[0], _ptr(sin), cs[1], _ptr(q_norm_weight), _ptr(k_norm_weight),
                 float(eps), _stream(qkv.device))
    q, k, v = qkv.split((num_q_heads * D, num_kv_heads * D, num_kv_heads * D), dim=-1)
    return q.view(T, num_q_heads, D), k.view(T, num_kv_heads, D), v.view(T, num_kv_heads, D)


def _rope_rows(t, name, T, width):
    _check_device_tensor(t, name, _BF16)
    _require(t.shape[0] == T and t.shape[-1] == width and t.numel() == T * width and
             t.stride(-1) == 1, f"{name} must hold one {width}-wide row per token")
    return t.stride(0)


def mla_kv_latent(ckv_full, norm_weight, eps, cos, sin, out=None):
    """Absorbed-MLA latent KV rows, one launch: ``[rms_norm(ckv), rope(
    interleave(k_pe))]`` of the kv_a_proj_with_mqa output ``ckv_full`` (T,
    576) with ``cos``/``sin`` (T, 1, 64).  Returns ``out`` (T, 1, 576), the
    reference's ``k_latent`` (auto_infer/layers/attention/mla.py:97-111)."""
    _check_device_tensor(ckv_full, "ckv_full", _BF16)
    _require(ckv_full.dim() == 2 and ckv_full.shape[1] == MLA_LATENT + MLA_ROPE and
             ckv_full.stride(1) == 1, "ckv_full must be (T, 576) with unit inner stride")
    T = ckv_full.shape[0]
    cts, sts = _rope_rows(cos, "cos", T, MLA_ROPE), _rope_rows(sin, "sin", T, MLA_ROPE)
    _check_device_tensor(norm_weight, "norm_weight", _BF16)
    _require(norm_weight.numel() == MLA_LATENT and norm_weight.is_contiguous(),
             "norm_weight must be 512 contiguous values")
    if out is None:
        out = torch.empty(T, 1, MLA_LATENT + MLA_ROPE, dtype=_BF16, device=ckv_full.device)
    _check_out(out, "out", (T, 1, MLA_LATENT + MLA_ROPE), ckv_full.device)
    _require(out.is_contiguous(), "out must be a contiguous (T, 1, 576) tensor")
    _native.call("aia_mla_kv_latent", _ptr(ckv_full), ckv_full.stride(0), T, _ptr(norm_weight),
                 float(eps), _ptr(cos), cts, _ptr(sin), sts, _ptr(out), MLA_LATENT + MLA_ROPE,
                 _stream(ckv_full.device))
    return out


def mla_q_latent(q, w_uk_t, cos, sin, out=None):
    """Absorbed-MLA latent query, one launch: ``[q_nope . W_UK, rope(
    interleave(q_pe))]`` for ``q`` (T, H, 192) = [nope 128, pe 64], with
    ``w_uk_t`` = W_UK transposed, (H, 512, 128) contiguous, and ``cos``/``sin``
    (T, 1, 64).  Returns ``out`` (T, H, 576), the reference's ``q_latent``
    (auto_infer/layers/attention/mla.py:93-107)."""
    _check_device_tensor(q, "q", _BF16)
    _require(q.dim() == 3 and q.shape[2] == 128 + MLA_ROPE and q.stride(2) == 1,
             "q must be (T, H, 192) with unit inner stride")
    T, H, _ = q.shape
    _check_device_tensor(w_uk_t, "w_uk_t", _BF16)
    _require(tuple(w_uk_t.shape) == (H, MLA_LATENT, 128) and w_uk_t.is_contiguous(),
             "w_uk_t must be a contiguous (H, 512, 128) tensor")
    cts, sts = _rope_rows(cos, "cos", T, MLA_ROPE), _rope_rows(sin, "sin", T, MLA_ROPE)
    if out is None:
        out = torch.empty(T, H, MLA_LATENT + MLA_ROPE, dtype=_BF16, device=q.device)
    _check_out(out, "out", (T, H, MLA_LATENT + MLA_ROPE), q.device)
    _native.call("aia_mla_q_latent", _ptr(q), q.stride(0), q.stride(1), T, H, _ptr(w_uk_t),
                 _ptr(cos), cts, _ptr(sin), sts, _ptr(out), out.stride(0), out.stride(1),
                 _stream(q.device))
    return out


# Query rows (tokens x heads) up to which mla_v_up beats the library GEMM
# (measured at 16 heads: 7.3 against 11.3 us at 256 tokens; from 320 tokens
# the library switches algorithm and wins, 6.9 against 8.6 us).
MLA_V_UP_MAX_ROWS = 4096


def mla_v_up(o_latent, w_uv, out=None):
    """Absorbed-MLA value up-projection, one launch: ``einsum("tnl,nvl->tnv",
    o_latent[..., :512], W_UV)`` (auto_infer/layers/attention/mla.py:120-121)
    for ``o_latent`` (T, H, >= 512) and ``w_uv`` (H, 128, 512) contiguous.
    Returns ``out`` (T, H, 128); its (T, H * 128) view feeds o_proj.  Every
    16-token work-group reads its share of W_UV, so the kernel is for decode
    and verify batches (up to ``MLA_V_UP_MAX_ROWS`` rows); it is correct at
    any size."""
    _check_device_tensor(o_latent, "o_latent", _BF16)
    _require(o_latent.dim() == 3 and o_latent.shape[2] >= MLA_LATENT and o_latent.stride(2) == 1,
             "o_latent must be (T, H, >= 512) with unit inner stride")
    T, H, _ = o_latent.shape
    _check_device_tensor(w_uv, "w_uv", _BF16)
    _require(tuple(w_uv.shape) == (H, 128, MLA_LATENT) and w_uv.is_contiguous(),
             "w_uv must be a contiguous (H, 128, 512) tensor")
    if out is None:
        out = torch.empty(T, H, 128, dtype=_BF16, device=o_latent.device)
    _check_out(out, "out", (T, H, 128), o_latent.device)
    _native.call("aia_mla_v_up", _ptr(o_latent), o_latent.stride(0), o_latent.stride(1), T, H,
                 _ptr(w_uv), _ptr(out), out.stride(0), out.stride(1), _stream(o_latent.device))
    return out


def mtp_compact(preds, drafts, active_mask, hidden, positions, slots, scratch_positions,
                scratch_slots, *, accepted=None, out_hidden=None, out_tokens=None,
                out_positions=None, out_slots=None):
    """Accepted draft counts and the compaction of confirmed target rows for
    the MTP drafter, in one launch (reference: GraphMtpRunner._target_body,
    auto_infer/worker/graph_mtp_runner.py:224-248).  Shapes: preds (g, w)
    int64, drafts (g, w - 1) int64, active_mask (g,), hidden (g * w, H) bf16,
    positions / scratch_positions (g * w,) int64, slots / scratch_slots
    (g * w,) int32.  Outputs (allocated unless given, so a graph can pass
    fixed buffers): accepted (g,) int64, hidden (g * w, H), tokens and
    positions (g * w,) int64, slots (g * w,) int32.  Returns them as a tuple
    (accepted, hidden, tokens, positions, slots)."""
    _check_device_tensor(preds, "preds", torch.int64)
    _require(preds.dim() == 2 and preds.is_contiguous(), "preds must be a contiguous (g, w) tensor")
    g, w = preds.shape
    _require(1 <= g <= 64 and w >= 2, "gear must be in [1, 64] and query width >= 2")
    _check_device_tensor(drafts, "drafts", torch.int64)
    _require(tuple(drafts.shape) == (g, w - 1) and drafts.is_contiguous(),
             "drafts must be a contiguous (g, w - 1) tensor")
    _check_device_tensor(active_mask, "active_mask")
    active = active_mask.to(torch.int32).contiguous()
    _require(active.numel() == g, "active_mask must have g entries")
    _check_device_tensor(hidden, "hidden", _BF16)
    _require(hidden.dim() == 2 and hidden.shape[0] == g * w and hidden.stride(1) == 1,
             "hidden must be (g * w, H) with unit inner stride")
    H = hidden.shape[1]
    for t, name, dt in ((positions, "positions", torch.int64), (slots, "slots", torch.int32),
                        (scratch_positions, "scratch_positions", torch.int64),
                        (scratch_slots, "scratch_slots", torch.int32)):
        _check_device_tensor(t, name, dt)
        _require(t.numel() == g * w and t.is_contiguous(), f"{name} must hold g * w entries")
    dev = preds.device
    accepted = accepted if accepted is not None else torch.empty(g, dtype=torch.int64, device=dev)
    out_hidden = out_hidden if out_hidden is not None else torch.empty(g * w, H, dtype=_BF16, device=dev)
    out_tokens = out_tokens if out_tokens is not None else torch.empty(g * w, dtype=torch.int64, device=dev)
    out_positions = (out_positions if out_positions is not None
                     else torch.empty(g * w, dtype=torch.int64, device=dev))
    out_slots = out_slots if out_slots is not None else torch.empty(g * w, dtype=torch.int32, device=dev)
    _require(out_hidden.shape == (g * w, H) and out_hidden.stride(1) == 1 and out_hidden.dtype == _BF16,
             "out_hidden must be (g * w, H) bf16 with unit inner stride")
    _native.call("aia_mtp_compact", _ptr(preds), _ptr(drafts), _ptr(active), _ptr(hidden),
                 hidden.stride(0), _ptr(positions), _ptr(slots), _ptr(scratch_positions),
                 _ptr(scratch_slots), g, w, H, _ptr(accepted), _ptr(out_hidden),
                 out_hidden.stride(0), _ptr(out_tokens), _ptr(out_positions), _ptr(out_slots),
                 _stream(dev))
    return accepted, out_hidden, out_tokens, out_positions, out_slots


def write_kv(key, value, key_cache, value_cache, slot_mapping):
    """Scatter this step's K/V into the paged cache by slot index.

    Same call shape and semantics as the reference's ``write_kv``
    (auto_infer/layers/attention/base.py:41-45):
    ``key_cache.view(-1, Hkv, D)[slot_mapping[t]] = key[t]`` and the same for
    ``value``.  ``value``/``value_cache`` may be None to write a single
    cache (absorbed MLA).  Slots outside the cache are skipped.
    """
    _check_device_tensor(key, "key", _BF16)
    _check_device_tensor(key_cache, "key_cache", _BF16)
    _check_device_tensor(slot_mapping, "slot_mapping", torch.int32)
    _require(key_cache.is_contiguous(), "key_cache must be contiguous")
    _require(slot_mapping.dim() == 1 and slot_mapping.is_contiguous(),
             "slot_mapping must be a contiguous 1-D tensor")
    T = key.shape[0]
    _require(slot_mapping.shape[0] == T, "slot_mapping length must equal the token count")
    krow = key.shape[1] * key.shape[2]
    _require(key_cache.numel() % krow == 0 and key_cache.shape[-1] * key_cache.shape[-2] == krow,
             "key rows do not match the key cache's (heads, dim)")
    num_slots = key_cache.numel() // krow
    kts = _row_stride(key, "key")
    if value is not None:
        _check_device_tensor(value, "value", _BF16)
        _check_device_tensor(value_cache, "value_cache", _BF16)
        _require(value_cache.is_contiguous(), "value_cache must be contiguous")
        _require(value.shape[0] == T, "value must have as many tokens as key")
        vrow = value.shape[1] * value.shape[2]
        _require(value_cache.numel() // vrow == num_slots and
                 value_cache.shape[-1] * value_cache.shape[-2] == vrow,
                 "value rows do not match the value cache")
        vts = _row_stride(value, "value")
    else:
        _require(value_cache is None, "value_cache given without value")
        vrow, vts = 0, 0
    _native.call("aia_kv_write", _ptr(key), kts, _ptr(value), vts, _ptr(key_cache),
                 _ptr(value_cache), _ptr(slot_mapping), T, krow, vrow, num_slots,
                 _stream(key.device))


def write_kv_nz(key, value, key_cache, value_cache, slot_mapping):
    """The KV slot write into caches in the NZ layout of the reference's
    graph-mode backend (``npu_scatter_pa_kv_cache``, auto_infer/layers/
    attention/gqa.py:202-211): the caches are (NB, bs, Hkv, D) tensors whose
    memory is viewed (NB, Hkv*D/16, bs, 16).  ``value``/``value_cache`` may
    be None.  Slots outside the cache are skipped."""
    _check_device_tensor(key, "key", _BF16)
    _check_device_tensor(key_cache, "key_cache", _BF16)
    _check_device_tensor(slot_mapping, "slot_mapping", torch.int32)
    _require(key_cache.dim() == 4 and key_cache.is_contiguous(),
             "key_cache must be a contiguous (num_blocks, block_size, Hkv, D) tensor")
    _require(slot_mapping.dim() == 1 and slot_mapping.is_contiguous() and
             slot_mapping.shape[0] == key.shape[0], "slot_mapping must hold one slot per token")
    nb, bs, hkv, d = key_cache.shape
    row = hkv * d
    _require(key.dim() == 3 and key.shape[1] * key.shape[2] == row, "key rows do not match the cache")
    kts = _row_stride(key, "key")
    vts = 0
    if value is not None:
        _check_device_tensor(value, "value", _BF16)
        _check_device_tensor(value_cache, "value_cache", _BF16)
        _require(tuple(value_cache.shape) == tuple(key_cache.shape) and value_cache.is_contiguous(),
                 "value_cache must match key_cache")
        _require(tuple(value.shape) == tuple(key.shape), "value must match key")
        vts = _row_stride(value, "value")
    else:
        _require(value_cache is None, "value_cache given without value")
    _native.call("aia_kv_write_nz", _ptr(key), kts, _ptr(value), vts, _ptr(key_cache),
                 _ptr(value_cache), _ptr(slot_mapping), key.shape[0], row, bs, nb * bs,
                 _stream(key.device))


KV_LAYOUTS = {"nd": 0, "nz": 1}   # nz: AIA_ATTN_KV_NZ


# ---------------------------------------------------------------- attention

def workspace_bytes(batch, num_tokens, num_q_heads, num_kv_heads, head_dim_v, num_waves=0):
    out = ctypes.c_int64(0)
    _native.call("aia_attn_workspace_bytes", batch, num_tokens, num_q_heads, num_kv_heads,
                 head_dim_v, num_waves, ctypes.byref(out))
    return out.value


_LAYOUT_KEYS = ("hdr", "seg", "wave", "part_ml", "part_o", "req", "mrg", "pf", "pfm", "pfw",
                "pf_ml", "pf_o", "total", "seg_cap", "mrg_cap", "pf_cap", "pf_unit_cap",
                "pf_mrg_cap", "waves", "pf_rows", "pf_keys")


def workspace_layout(batch, num_tokens, num_q_heads, num_kv_heads, head_dim_v, num_waves=0):
    """Byte offsets of a plan's parts in its workspace and the plan's
    capacities (``aia_attn_workspace_layout``), as a dict: for tools and
    tests that read a plan back."""
    vals = (ctypes.c_int64 * len(_LAYOUT_KEYS))()
    _native.call("aia_attn_workspace_layout", batch, num_tokens, num_q_heads, num_kv_heads,
                 head_dim_v, num_waves, vals, len(_LAYOUT_KEYS))
    return dict(zip(_LAYOUT_KEYS, vals))


class AttentionPlan:
    """Device metadata + split-K work plan of one step.

    Built once per step (all layers share it): ``cu_seqlens_q`` is the
    reference's cumulative query-length list with a leading 0 (B + 1
    entries), ``seqlens_kv`` the per-request KV lengths
    (forward_context.py:14-15), both int32 on the device.  The planner runs
    on the GPU, so device-produced metadata (the packing kernel) needs no
    host round trip.
    """

    def __init__(self, block_table, cu_seqlens_q, seqlens_kv, num_tokens, num_q_heads,
                 num_kv_heads, head_dim_v, block_size, num_waves=0, workspace=None, owned=None):
        _check_device_tensor(block_table, "block_table", torch.int32)
        _check_device_tensor(cu_seqlens_q, "cu_seqlens_q", torch.int32)
        _check_device_tensor(seqlens_kv, "seqlens_kv", torch.int32)
        _require(block_table.dim() == 2 and block_table.stride(1) == 1,
                 "block_table must be (batch, max_blocks) with unit column stride")
        batch = seqlens_kv.shape[0]
        _require(cu_seqlens_q.shape[0] == batch + 1, "cu_seqlens_q must have batch + 1 entries")
        _require(block_table.shape[0] >= batch, "block_table has fewer rows than requests")
        _require(cu_seqlens_q.is_contiguous() and seqlens_kv.is_contiguous(),
                 "metadata tensors must be contiguous")
        self.block_table = block_table
        self.cu_seqlens_q = cu_seqlens_q
        self.seqlens_kv = seqlens_kv
        self.batch = batch
        self.num_tokens = int(num_tokens)
        self.num_q_heads = num_q_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim_v = head_dim_v
        self.num_waves = num_waves
        self.block_size = int(block_size)
        nbytes = workspace_bytes(batch, self.num_tokens, num_q_heads, num_kv_heads, head_dim_v,
                                 num_waves)
        if workspace is None:
            workspace = torch.empty(nbytes, dtype=torch.uint8, device=block_table.device)
        _check_device_tensor(workspace, "workspace", torch.uint8)
        _require(workspace.numel() >= nbytes, "attention workspace too small")
        self.workspace = workspace
        # streams the plan's own device tensors are known to be used on: the
        # caching allocator may hand their memory to the allocating stream's
        # next allocation once they are dropped, so every other stream that
        # reads or writes them is recorded (Tensor.record_stream)
        self._streams = {torch.cuda.current_stream(block_table.device)}
        self._owned = [workspace] if owned is None else [workspace, *owned]
        self.replan()

    def replan(self):
        """Re-run the device planner on the (possibly updated in place)
        metadata tensors; graph-capturable.  The plan is then valid on the
        current stream (attention calls on another stream wait for it)."""
        self.stream = torch.cuda.current_stream(self.block_table.device)
        self._use_on(self.stream)
        _native.call("aia_attn_plan", _ptr(self.cu_seqlens_q), _ptr(self.seqlens_kv),
                     _ptr(self.block_table), self.block_table.stride(0), self.block_size,
                     self.batch, self.num_tokens, self.num_q_heads, self.num_kv_heads,
                     self.head_dim_v, self.num_waves, _ptr(self.workspace),
                     self.workspace.numel(), _stream(self.block_table.device))

    def _use_on(self, stream):
        if stream not in self._streams:
            self._streams.add(stream)
            for t in self._owned:
                t.record_stream(stream)

    def status(self):
        """Synchronising check of the last plan: raises ValueError if the
        planner found more work than the workspace was sized for (query
        lengths that do not add up to ``num_tokens``); the kernels then ran
        an empty plan and the attention calls filled their outputs with
        NaN."""
        code = int(self.workspace[32:36].view(torch.int32).item())
        if code != 0:
            raise ValueError(f"attention planner overflow (status {code}): cu_seqlens_q does "
                             f"not describe {self.num_tokens} query tokens")

    @classmethod
    def from_lists(cls, block_table, cu_seqlens_q, seqlens_kv, num_q_heads, num_kv_heads,
                   head_dim_v, block_size, **kw):
        """From the reference's host lists (cumulative ends without the
        leading 0, per-request KV lengths)."""
        dev = block_table.device
        check_lists(cu_seqlens_q, seqlens_kv, block_table.shape[1] * block_size)
        cu = torch.tensor([0, *cu_seqlens_q], dtype=torch.int32).to(dev, non_blocking=True)
        kv = torch.tensor(list(seqlens_kv), dtype=torch.int32).to(dev, non_blocking=True)
        total = cu_seqlens_q[-1] if len(cu_seqlens_q) else 0
        return cls(block_table, cu, kv, total, num_q_heads, num_kv_heads, head_dim_v, block_size,
                   owned=[cu, kv], **kw)


def check_lists(cu_seqlens_q, seqlens_kv, max_context):
    """Host check of the reference's metadata lists (cumulative query ends,
    per-request KV lengths; forward_context.py:14-15): same length,
    non-decreasing ends, every KV length within the block table (the
    kernels read block ids up to it)."""
    _require(len(cu_seqlens_q) == len(seqlens_kv),
             "cu_seqlens_q and seqlens_kv must have one entry per request")
    prev = 0
    for end, lk in zip(cu_seqlens_q, seqlens_kv):
        _require(end >= prev, "cu_seqlens_q must be non-decreasing")
        _require(0 <= lk <= max_context,
                 f"KV length {lk} does not fit the block table ({max_context} slots)")
        prev = end


def _ready(plan, device):
    """Order the attention launch after the planner: on another stream, make
    the current stream wait for the plan's stream (not allowed while
    capturing a graph, where the plan must be made on the capturing stream)
    and record the plan's buffers as in use there."""
    cur = torch.cuda.current_stream(device)
    if cur != plan.stream:
        if torch.cuda.is_current_stream_capturing():
            raise ValueError("attention plan was made on another stream than the one being "
                             "captured; call plan.replan() on the capturing stream")
        cur.wait_stream(plan.stream)
        plan._use_on(cur)


def _check_out(out, name, shape, device):
    """A caller-supplied output: bf16 on the same GPU, of ``shape``, unit
    inner stride, rows (heads, dim) not overlapping."""
    _check_device_tensor(out, name, _BF16)
    _require(out.device == device, f"{name} must be on {device}")
    _require(tuple(out.shape) == tuple(shape), f"{name} must have shape {tuple(shape)}, "
             f"got {tuple(out.shape)}")
    _require(out.stride(-1) == 1, f"{name} must have unit inner stride")
    if out.dim() == 3:
        _require(out.stride(1) >= out.shape[2] and out.stride(0) >= out.shape[1] * out.stride(1),
                 f"{name} rows must not overlap")


def paged_attention_gqa(query, key_cache, value_cache, plan, scale, out=None, flags=0,
                        key_new=None, value_new=None, kv_layout="nd"):
    """Paged GQA attention (reference base.py:48-61 FIA semantics).

    query (T, Hq, D) bf16 with D = 128 or 64; key/value caches (NB, bs, Hkv,
    D) bf16 contiguous; ``plan`` an ``AttentionPlan`` of this step (head_dim_v
    D).  Returns (T, Hq, D) bf16.  With ``key_new`` / ``value_new`` (this
    step's new rows, (T, Hkv, D)) the kernel also writes them into the caches
    at the slots the block table assigns (the fused form of ``write_kv``).
    ``kv_layout="nz"``: the caches hold the NZ layout of the reference's
    graph mode (see ``write_kv_nz``); results are the same as for the same
    values in the standard layout.
    """
    _require(kv_layout in KV_LAYOUTS, f"kv_layout must be one of {sorted(KV_LAYOUTS)}")
    flags |= KV_LAYOUTS[kv_layout]
    _check_device_tensor(query, "query", _BF16)
    _check_device_tensor(key_cache, "key_cache", _BF16)
    _check_device_tensor(value_cache, "value_cache", _BF16)
    _require(query.dim() == 3 and query.stride(2) == 1, "query must be (T, Hq, D), D contiguous")
    T, hq, d = query.shape
    _require(key_cache.dim() == 4 and key_cache.is_contiguous() and value_cache.is_contiguous(),
             "caches must be contiguous (num_blocks, block_size, Hkv, D)")
    nb, bs, hkv, dk = key_cache.shape
    _require(tuple(value_cache.shape) == (nb, bs, hkv, dk), "value cache shape differs from key cache")
    _require(dk == d, "query head_dim differs from the cache's")
    _require(hq == plan.num_q_heads and hkv == plan.num_kv_heads and T == plan.num_tokens
             and bs == plan.block_size, "plan was made for another shape")
    if out is None:
        out = torch.empty(T, hq, d, dtype=_BF16, device=query.device)
    else:
        _check_out(out, "out", (T, hq, d), query.device)
    kn_ts = vn_ts = 0
    if key_new is not None or value_new is not None:
        _check_device_tensor(key_new, "key_new", _BF16)
        _check_device_tensor(value_new, "value_new", _BF16)
        _require(tuple(key_new.shape) == (T, hkv, d) and tuple(value_new.shape) == (T, hkv, d),
                 "new K/V rows must be (tokens, Hkv, D)")
        kn_ts, vn_ts = _row_stride(key_new, "key_new"), _row_stride(value_new, "value_new")
    _ready(plan, query.device)
    _native.call("aia_paged_attention_gqa", _ptr(query), query.stride(0), query.stride(1),
                 _ptr(key_cache), _ptr(value_cache), _ptr(plan.block_table),
                 plan.block_table.stride(0), _ptr(plan.cu_seqlens_q), _ptr(plan.seqlens_kv),
                 plan.batch, T, hq, hkv, d, bs, nb, float(scale), _ptr(out), out.stride(0),
                 out.stride(1), _ptr(key_new), _ptr(value_new), kn_ts, vn_ts, plan.num_waves,
                 flags, _ptr(plan.workspace), plan.workspace.numel(), _stream(query.device))
    return out


MLA_LATENT, MLA_ROPE = 512, 64


def paged_attention_mla(q_latent, latent_cache, plan, scale, out=None, flags=0):
    """Absorbed-MLA latent attention (reference mla.py:76-122 semantics).

    q_latent (T, H, 576) bf16 = [W_UK-absorbed nope (512), rope (64)];
    latent_cache (NB, bs, 1, 576) bf16 contiguous; ``plan`` an
    ``AttentionPlan`` made with (num_q_heads=H, num_kv_heads=1,
    head_dim_v=512).  Returns the latent output (T, H, 512) bf16, i.e. the
    first kv_lora_rank values of attention with V = K.
    """
    _check_device_tensor(q_latent, "q_latent", _BF16)
    _check_device_tensor(latent_cache, "latent_cache", _BF16)
    _require(q_latent.dim() == 3 and q_latent.stride(2) == 1,
             "q_latent must be (T, H, 576), last dim contiguous")
    T, h, dk = q_latent.shape
    _require(dk == MLA_LATENT + MLA_ROPE, "q_latent last dim must be 576")
    _require(latent_cache.dim() == 4 and latent_cache.is_contiguous() and
             latent_cache.shape[2] == 1 and latent_cache.shape[3] == dk,
             "latent_cache must be contiguous (num_blocks, block_size, 1, 576)")
    nb, bs = latent_cache.shape[0], latent_cache.shape[1]
    _require(h == plan.num_q_heads and plan.num_kv_heads == 1 and plan.head_dim_v == MLA_LATENT
             and T == plan.num_tokens and bs == plan.block_size,
             "plan was not made for this MLA shape")
    if out is None:
        out = torch.empty(T, h, MLA_LATENT, dtype=_BF16, device=q_latent.device)
    else:
        _check_out(out, "out", (T, h, MLA_LATENT), q_latent.device)
    _ready(plan, q_latent.device)
    _native.call("aia_paged_attention_mla", _ptr(q_latent), q_latent.stride(0),
                 q_latent.stride(1), _ptr(latent_cache), _ptr(plan.block_table),
                 plan.block_table.stride(0), _ptr(plan.cu_seqlens_q), _ptr(plan.seqlens_kv),
                 plan.batch, T, h, MLA_LATENT, MLA_ROPE, bs, nb, float(scale), _ptr(out),
                 out.stride(0), out.stride(1), plan.num_waves, flags, _ptr(plan.workspace),
                 plan.workspace.numel(), _stream(q_latent.device))
    return out
