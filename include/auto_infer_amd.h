/* C ABI of the MI355X (gfx950) ragged paged-attention path.
 *
 * Every entry point returns an int status (AIA_OK = 0, negative = error; no
 * exception crosses the ABI) and records a message readable through
 * aia_last_error() (thread local).  All tensor arguments are DEVICE pointers
 * owned by the caller; the library never allocates: scratch space is a
 * caller-provided workspace.  Work is enqueued on the caller's stream
 * (a hipStream_t passed as void*, NULL = the default stream) and nothing
 * synchronises the host.  No global mutable state: calls are reentrant and
 * may come from several host threads on different streams.
 *
 * Element type of query/key/value/output tensors is bf16 (passed as raw
 * 16-bit words).  Indices are int32.
 */
#ifndef AUTO_INFER_AMD_H
#define AUTO_INFER_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AIA_OK 0
#define AIA_ERR_INVALID (-1)     /* bad argument (maps to ValueError) */
#define AIA_ERR_HIP (-2)         /* HIP runtime error (RuntimeError) */
#define AIA_ERR_CAPACITY (-3)    /* exceeds a gear / workspace (ValueError) */
#define AIA_ERR_UNSUPPORTED (-4) /* shape not supported (NotImplementedError) */

/* Library ABI version (major * 10000 + minor * 100 + patch). */
int aia_version(void);

/* Message of the last failing call on this host thread ("" if none). */
const char* aia_last_error(void);

/* KV slot write.  Replaces torch_npu._npu_reshape_and_cache
 * (reference auto_infer/layers/attention/base.py:41-45, called from
 * gqa.py:76-79 and mla.py:111-113):
 *   key_cache.view(-1, row)[slot_mapping[t]] = key[t]   (and value).
 * key:   (num_tokens, key_row_elems) rows, token stride key_token_stride
 *        elements, each row contiguous (heads * head_dim).
 * value: same with value_row_elems / value_token_stride; may be NULL (with
 *        value_cache NULL) to write only one cache (absorbed MLA aliases).
 * caches: contiguous (num_slots, row) = (num_blocks * block_size, heads, dim).
 * Slots < 0 or >= num_slots are skipped (padding rows). */
int aia_kv_write(const void* key, int64_t key_token_stride,
                 const void* value, int64_t value_token_stride,
                 void* key_cache, void* value_cache,
                 const int32_t* slot_mapping, int32_t num_tokens,
                 int32_t key_row_elems, int32_t value_row_elems,
                 int64_t num_slots, void* stream);

/* KV slot write into caches in the NZ layout.  Replaces
 * torch_npu.npu_scatter_pa_kv_cache of the reference's graph-mode backend
 * (auto_infer/layers/attention/gqa.py:202-211), which scatters by
 * slot_mapping into each cache viewed (num_blocks, Hkv * D / 16,
 * block_size, 16): value d of head h of the token at slot s = blk *
 * block_size + off sits at [blk][(h * D + d) / 16][off][d % 16].
 * key / value: (num_tokens, row_elems) rows (row_elems = Hkv * D, a
 * multiple of 16), 16-byte aligned, token strides a multiple of 8 values;
 * value may be NULL (with value_cache NULL).  caches: num_slots = num_blocks
 * * block_size token slots.  Slots < 0 or >= num_slots are skipped. */
int aia_kv_write_nz(const void* key, int64_t key_token_stride, const void* value,
                    int64_t value_token_stride, void* key_cache, void* value_cache,
                    const int32_t* slot_mapping, int32_t num_tokens, int32_t row_elems,
                    int32_t block_size, int64_t num_slots, void* stream);

/* Bytes of workspace the attention planner/kernels need for a step of at
 * most `batch` requests and `num_tokens` query rows, planned with
 * `num_waves` key ranges (0 = the default, as in aia_attn_plan).  No
 * reference counterpart (the vendor op hides its workspace). */
int aia_attn_workspace_bytes(int32_t batch, int32_t num_tokens,
                             int32_t num_q_heads, int32_t num_kv_heads,
                             int32_t head_dim_v, int32_t num_waves, int64_t* bytes);

/* Where a plan keeps its parts in the workspace, for tools and tests that
 * read a plan back (no counterpart in the reference, whose plan is the host
 * lists themselves).  Writes up to `count` int64 values, -1 past the end:
 * byte offsets of the header, segment records, range records, split
 * partials (max/sum, values), request offsets, merge records, prefill unit
 * records, prefill merge records, dealt prefill work-groups, prefill
 * partials (max/sum, values) and the total size; then the capacities
 * (segments, merge records, prefill items, prefill units, prefill merges),
 * the range count, and the prefill item rows and tile keys. */
int aia_attn_workspace_layout(int32_t batch, int32_t num_tokens, int32_t num_q_heads,
                              int32_t num_kv_heads, int32_t head_dim_v, int32_t num_waves,
                              int64_t* offsets, int32_t count);

/* Split-K work plan for one step: reads the device copies of
 * cu_seqlens_q (batch + 1 entries, leading 0 -- the reference keeps the
 * cumulative ends as a host list, model_runner.py:137 / ForwardContext
 * .cu_seqlens_q), seqlens_kv (batch entries, forward_context.py:15) and the
 * block table (batch rows, block_table_stride apart) and writes a flat list
 * of (request, kv-head group, query block, key range) work items into
 * `workspace` (256-byte aligned, aia_attn_workspace_bytes long), each
 * carrying the first block ids it reads.  GQA requests whose query rows
 * (tokens x group) fill a 128-row item become prefill items instead (cut
 * into key chunks when they are too few to fill the chip).  The plan depends
 * only on step metadata, so one plan serves every layer of the step.
 * num_waves: number of key ranges (work-groups); 0 picks the default (about
 * 2048 waves in flight for GQA; three four-wave groups per compute unit of the
 * current device for MLA, 768 on the MI355X).
 * Status: the int32 at byte offset 32 of the workspace is 0 after a good
 * plan and -1 when the query lengths ask for more work than a step of
 * num_tokens rows can hold (cu_seqlens_q not ending at num_tokens, or
 * decreasing); the plan is then empty and the attention calls leave `out`
 * unwritten.  Reading it is the caller's choice (it costs a sync). */
int aia_attn_plan(const int32_t* cu_seqlens_q, const int32_t* seqlens_kv,
                  const int32_t* block_table, int32_t block_table_stride,
                  int32_t block_size, int32_t batch, int32_t num_tokens,
                  int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim_v,
                  int32_t num_waves, void* workspace, int64_t workspace_bytes,
                  void* stream);

/* Paged GQA attention over a planned step.  Replaces the FIA call of
 * GqaFIABackend._attn (reference auto_infer/layers/attention/gqa.py:81-94 ->
 * base.py:48-61, npu_fused_infer_attention_score, TND layout, sparse_mode 3):
 * query row i of request b attends keys j <= Lk - Lq + i (bottom-right
 * causal), query head h reads KV head h / (Hq / Hkv), KV row j at
 * block_table[b, j / block_size], offset j % block_size.
 * query:  (num_tokens, Hq, head_dim) with the given token/head strides.
 * caches: contiguous (num_blocks, block_size, Hkv, head_dim), with
 *         num_blocks * block_size < 2^31 (the int32 slot_mapping's range;
 *         AIA_ERR_INVALID otherwise, here and in aia_paged_attention_mla).
 * out:    (num_tokens, Hq, head_dim) with the given strides.
 * head_dim must be 128 (Qwen2-7B, Qwen3) or 64 (Qwen2 / Qwen2.5 0.5B:
 * hidden 896 over 14 heads), AIA_ERR_UNSUPPORTED otherwise; scale must be
 * positive (AIA_ERR_INVALID otherwise).  Requests whose query rows fill
 * 128-row items run on the prefill kernel at both head dims.
 * The workspace must hold a plan made by
 * aia_attn_plan with the same metadata, head counts and num_waves.
 * key_new / value_new (optional, both or neither): this step's new K/V rows
 * (num_tokens, Hkv, head_dim), query token t being position Lk - Lq + i of its
 * request.  When given, the kernel also performs the KV slot write of those
 * rows (what aia_kv_write would do, at slot block_table[b, pos / bs] * bs +
 * pos % bs -- the slot_mapping every packer produces) and reads the new keys
 * from the rows themselves, saving the separate write launch.
 * Rows whose keys were split over several work-groups are merged by
 * log-sum-exp in a second kernel, from fp16 partials y = O / c scaled per
 * row (c = the row's largest |O|) with fp32 (max + log2 c, sum / c).
 * flags: AIA_ATTN_KV_NZ -- the caches are in the NZ layout of the
 * reference's graph mode (gqa.py:163,202-226; see aia_kv_write_nz); the
 * fused KV write then writes that layout too.  Results are the same as with
 * the same values in the standard layout.
 * If the plan overflowed (query lengths that do not add up to num_tokens:
 * the planner plans nothing and sets status -1 in the workspace header), the
 * output is filled with NaN.
 * Other flag bits must be 0. */
#define AIA_ATTN_KV_NZ 1
int aia_paged_attention_gqa(const void* query, int64_t q_token_stride,
                            int64_t q_head_stride,
                            const void* key_cache, const void* value_cache,
                            const int32_t* block_table, int32_t block_table_stride,
                            const int32_t* cu_seqlens_q, const int32_t* seqlens_kv,
                            int32_t batch, int32_t num_tokens,
                            int32_t num_q_heads, int32_t num_kv_heads,
                            int32_t head_dim, int32_t block_size,
                            int32_t num_blocks, float scale,
                            void* out, int64_t out_token_stride,
                            int64_t out_head_stride,
                            const void* key_new, const void* value_new,
                            int64_t new_key_token_stride,
                            int64_t new_value_token_stride, int32_t num_waves,
                            int32_t flags, void* workspace, int64_t workspace_bytes,
                            void* stream);

/* Allocation-free paged GQA attention: aia_attn_plan + aia_paged_attention_gqa
 * in one call, with the plan and the split partials in a static device array
 * of the library (aia_noalloc_scratch_bytes: 96 MiB; one per GPU, held until
 * the process ends) instead of a caller workspace.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation).  The array sits in its own code object, which the runtime
 * loads onto a GPU only on the first call there: processes that never call
 * this entry point do not hold it.  Same arguments as
 * aia_paged_attention_gqa without the workspace; steps whose plan needs
 * more than the array (aia_attn_workspace_bytes) fail with
 * AIA_ERR_CAPACITY.  It plans on every call (one planner launch per call).
 * All calls on one GPU share the array: calls that overlap on one GPU (two
 * streams, two host threads) race and must be ordered by the caller. */
int aia_paged_attention_gqa_noalloc(const void* query, int64_t q_token_stride,
                                    int64_t q_head_stride,
                                    const void* key_cache, const void* value_cache,
                                    const int32_t* block_table, int32_t block_table_stride,
                                    const int32_t* cu_seqlens_q, const int32_t* seqlens_kv,
                                    int32_t batch, int32_t num_tokens,
                                    int32_t num_q_heads, int32_t num_kv_heads,
                                    int32_t head_dim, int32_t block_size,
                                    int32_t num_blocks, float scale,
                                    void* out, int64_t out_token_stride,
                                    int64_t out_head_stride,
                                    const void* key_new, const void* value_new,
                                    int64_t new_key_token_stride,
                                    int64_t new_value_token_stride, int32_t num_waves,
                                    int32_t flags, void* stream);

/* Size in bytes of the allocation-free entry point's static array.  No
 * counterpart in the reference (see aia_paged_attention_gqa_noalloc). */
int aia_noalloc_scratch_bytes(int64_t* bytes);

/* Absorbed-MLA paged attention over a planned step.  Replaces the FIA call of
 * mla_paged_absorbed (reference auto_infer/layers/attention/mla.py:76-122,
 * from MlaFIABackend.attention :221-241): one KV head holding the 576-wide
 * latent (kv_lora_rank 512 + rope 64) per token, V = K, output keeps the
 * first kv_lora_rank values (mla.py:114-120); same causal / paging rules as
 * the GQA entry.
 * q_latent:     (num_tokens, num_heads, 576), token/head strides given.
 * latent_cache: contiguous (num_blocks, block_size, 1, 576).
 * out:          (num_tokens, num_heads, 512).
 * Requests of 8+ tokens (in steps of 4+ tokens per request on average) run
 * on prefill units, the rest on split-K ranges; the caller sees one call.
 * The plan must come from aia_attn_plan(num_q_heads = num_heads,
 * num_kv_heads = 1, head_dim_v = 512, same num_waves).  flags must be 0. */
int aia_paged_attention_mla(const void* q_latent, int64_t q_token_stride,
                            int64_t q_head_stride, const void* latent_cache,
                            const int32_t* block_table, int32_t block_table_stride,
                            const int32_t* cu_seqlens_q, const int32_t* seqlens_kv,
                            int32_t batch, int32_t num_tokens, int32_t num_heads,
                            int32_t kv_lora_rank, int32_t rope_dim,
                            int32_t block_size, int32_t num_blocks, float scale,
                            void* out, int64_t out_token_stride,
                            int64_t out_head_stride, int32_t num_waves,
                            int32_t flags, void* workspace, int64_t workspace_bytes,
                            void* stream);

/* Ragged-batch packing of one step's rows into attention metadata.
 * Replaces the host packing loops of the reference: NpuModelRunner._build
 * (auto_infer/worker/model_runner.py:111-188), DecodeInputStager.stage
 * (worker/decode_input_stager.py:74-123), SpecDecodeInputStager.stage
 * (:304-373) and PrefillInputStager.stage (worker/prefill_input_stager.py:
 * 72-162), with slot = block_table[pos / bs] * bs + pos % bs
 * (engine/token_layout.py:1-4).
 * Pools (device, caller-owned): token_pool int64 [slots][token_pool_stride],
 * block_pool int32 [slots][block_pool_stride].  First the given updates are
 * scattered (flat indices into the pools), then each row is packed.
 * rows: device int32 [num_rows][8] =
 *   {slot (-1 = synthetic scratch row), start, n, num_blocks, first scratch
 *    block (synthetic rows), first query row (cumulative offset),
 *    zero_tokens, sample slot (-1 = none)}.
 * Outputs: token_ids/positions int64 [T], slot_mapping int32 [T],
 * block_table int32 [num_rows][block_table_width] zero padded,
 * cu_seqlens_q int32 [num_rows + 1] (leading 0), seqlens_kv int32
 * [num_rows] = start + n, last_rows int64 [num_rows] (may be NULL),
 * sample_rows int64 [sample_cap]: row q_off + n - 1 at each row's sample
 * slot, zeros from sample_count on. */
int aia_pack_rows(const int64_t* token_update_index, const int64_t* token_update_value,
                  int32_t num_token_updates, const int64_t* block_update_index,
                  const int32_t* block_update_value, int32_t num_block_updates,
                  int64_t* token_pool, int64_t token_pool_stride,
                  int32_t* block_pool, int64_t block_pool_stride,
                  const int32_t* rows, int32_t num_rows, int32_t block_size,
                  int32_t block_table_width, int64_t* token_ids, int64_t* positions,
                  int32_t* slot_mapping, int32_t* block_table, int32_t* cu_seqlens_q,
                  int32_t* seqlens_kv, int64_t* last_rows, int64_t* sample_rows,
                  int32_t sample_count, int32_t sample_cap, void* stream);

/* aia_pack_rows for small steps, with no staging copy: the updates and row
 * descriptors come in `blob`, HOST memory that the call copies into the
 * kernel launch's arguments, and one work-group scatters the updates and
 * packs the rows.  blob layout (8-byte words): token_update_index [nt]
 * int64, token_update_value [nt] int64, block_update_index [nb] int64,
 * block_update_value [nb] int32 (padded to a whole word), rows [num_rows][8]
 * int32; at most AIA_PACK_INLINE_BYTES bytes (AIA_ERR_CAPACITY otherwise).
 * Other arguments and the outputs as in aia_pack_rows.  No reference
 * counterpart beyond aia_pack_rows' (it is the same packing, launched without
 * the host-to-device copy). */
#define AIA_PACK_INLINE_BYTES 3072
int aia_pack_rows_inline(const void* blob, int32_t num_token_updates,
                         int32_t num_block_updates, int32_t num_rows,
                         int64_t* token_pool, int64_t token_pool_stride,
                         int32_t* block_pool, int64_t block_pool_stride,
                         int32_t block_size, int32_t block_table_width,
                         int64_t* token_ids, int64_t* positions, int32_t* slot_mapping,
                         int32_t* block_table, int32_t* cu_seqlens_q, int32_t* seqlens_kv,
                         int64_t* last_rows, int64_t* sample_rows, int32_t sample_count,
                         int32_t sample_cap, void* stream);

/* Device token splice, one launch.  Replaces splice_device_tokens
 * (reference auto_infer/worker/staging.py:51-70) and the stager's
 * prepare_splice / apply_splice pair (worker/decode_input_stager.py:125-170),
 * which move last step's sampled tokens (still on the device) into this
 * step's token-id buffer with one index_select + index_copy_ per owning
 * tensor: target[pairs[i][1]] = *(const int64_t*)pairs[i][0] for i < count.
 * pairs: device int64 [count][2] = {address of the source token id (an
 * element of any int64 device tensor), target row}; rows outside
 * [0, target_len) are skipped. */
int aia_splice_tokens(const int64_t* pairs, int32_t count, int64_t* target, int64_t target_len,
                      void* stream);

/* Fused pre-attention, in place over a packed qkv projection (T rows of
 * (Hq + 2 Hkv) x head_dim bf16 values, token stride qkv_token_stride): per-head
 * RMSNorm of the Q and K heads with the given weights (both or neither;
 * Qwen3 QK-Norm) and NeoX RoPE x * cos + rotate_half(x) * sin with cos/sin
 * (T, head_dim) bf16 rows.  V is left as is.  Replaces the split / rms_norm /
 * rotary steps of _GqaProjRopeMixin.attention (auto_infer/layers/attention/
 * gqa.py:27-49; auto_infer/layers/norm.py:5-8; auto_infer/layers/
 * rotary_embedding/__init__.py:10-13), rounding to bf16 where those bf16
 * ops round.  The Q, K and V slices then go to aia_paged_attention_gqa as
 * query / key_new / value_new through their strides.  head_dim must be 128
 * or 64 (AIA_ERR_UNSUPPORTED otherwise). */
int aia_qk_norm_rope(void* qkv, int64_t qkv_token_stride, int32_t num_tokens,
                     int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                     const void* cos, int64_t cos_token_stride, const void* sin,
                     int64_t sin_token_stride, const void* q_norm_weight,
                     const void* k_norm_weight, float eps, void* stream);

/* Absorbed-MLA latent KV row, one launch.  Replaces the ckv RMSNorm, the
 * k_pe ds_rope_interleave + NeoX RoPE and the cat of mla_paged_absorbed
 * (auto_infer/layers/attention/mla.py:97-111; rotary_embedding/__init__.py:
 * 10-23): out[t] = [rms_norm(ckv_full[t][:512], norm_weight, eps) (512),
 * rope(interleave(ckv_full[t][512:576])) (64)], rounding to bf16 where those
 * bf16 ops round.  ckv_full rows of 576 bf16 (the kv_a_proj_with_mqa output),
 * cos/sin one 64-wide row per token; out rows of 576 (the k_latent that
 * aia_kv_write stores). */
int aia_mla_kv_latent(const void* ckv_full, int64_t ckv_token_stride, int32_t num_tokens,
                      const void* norm_weight, float eps, const void* cos,
                      int64_t cos_token_stride, const void* sin, int64_t sin_token_stride,
                      void* out, int64_t out_token_stride, void* stream);

/* Absorbed-MLA latent query, one launch.  Replaces the q_pe interleave +
 * RoPE, the einsum("tnp,npl->tnl", q_nope, W_UK) and the cat of
 * mla_paged_absorbed (mla.py:93-107): out[t][h] = [q_nope[t][h] . W_UK[h]
 * (512, fp32 accumulation on MFMA, one bf16 rounding), rope(interleave(
 * q_pe[t][h])) (64)].  q (T, H, 192) = [nope 128, pe 64]; w_uk_t is W_UK
 * transposed, (H, 512, 128) contiguous; out (T, H, 576). */
int aia_mla_q_latent(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                     int32_t num_tokens, int32_t num_heads, const void* w_uk_t, const void* cos,
                     int64_t cos_token_stride, const void* sin, int64_t sin_token_stride,
                     void* out, int64_t out_token_stride, int64_t out_head_stride, void* stream);

/* Absorbed-MLA value up-projection, one launch.  Replaces
 * einsum("tnl,nvl->tnv", o_latent, W_UV) of mla_paged_absorbed (mla.py:121):
 * out[t][h][v] = sum_l o_latent[t][h][l] * W_UV[h][v][l] with fp32
 * accumulation on MFMA and one bf16 rounding.  o_latent (T, H, >= 512) bf16
 * (the attention output; the first 512 dims are read), w_uv (H, 128, 512)
 * contiguous (build_absorb_weights, mla.py:67-73), out (T, H, 128): with
 * out_token_stride = H * 128 it is the (T, H * 128) input of o_proj. */
int aia_mla_v_up(const void* o_latent, int64_t o_token_stride, int64_t o_head_stride,
                 int32_t num_tokens, int32_t num_heads, const void* w_uv, void* out,
                 int64_t out_token_stride, int64_t out_head_stride, void* stream);

/* On-device MTP verify compaction, one launch.  Replaces the accept/compact
 * block of GraphMtpRunner._target_body (auto_infer/worker/
 * graph_mtp_runner.py:224-248): for a gear of `gear` (<= 64) requests of
 * query_width rows each (draft depth + 1), accepted[r] = the number of
 * leading drafts equal to the target's predictions, times active_mask[r];
 * then each request's 1 + accepted[r] confirmed rows are packed in request
 * order (confirmed_layout, spec_decode/layout.py:17-43) into out_hidden /
 * out_tokens / out_positions / out_slots (gear * query_width rows); rows past
 * the confirmed total get zero hidden/token and the scratch position/slot.
 * preds int64 [gear][query_width], drafts int64 [gear][query_width - 1],
 * active_mask int32 [gear] (0/1, active requests a prefix), hidden bf16
 * [gear * query_width][hidden_dim] (row stride in elements), positions
 * int64 / slots int32 / scratch_* [gear * query_width], accepted int64
 * [gear]. */
int aia_mtp_compact(const int64_t* preds, const int64_t* drafts, const int32_t* active_mask,
                    const void* hidden, int64_t hidden_row_stride, const int64_t* positions,
                    const int32_t* slots, const int64_t* scratch_positions,
                    const int32_t* scratch_slots, int32_t gear, int32_t query_width,
                    int32_t hidden_dim, int64_t* accepted, void* out_hidden,
                    int64_t out_hidden_row_stride, int64_t* out_tokens,
                    int64_t* out_positions, int32_t* out_slots, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AUTO_INFER_AMD_H */
