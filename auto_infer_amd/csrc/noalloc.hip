// Allocation-free paged GQA attention: aia_attn_plan + aia_paged_attention_gqa
// with the plan and the split partials in a file-scope device array instead of
// a caller workspace.
//
// The array lives in this translation unit on purpose: each HIP source is its
// own code object, and the runtime loads a code object onto a device when one
// of its kernels or variables is first used there.  So the array is reserved
// on a GPU only once a process calls the allocation-free entry point on it;
// processes that use only the workspace entry points never hold it.
#include <mutex>

#include "common.h"

namespace {

// Every BASELINE config's step fits (configs[1], the largest, needs about
// 63 MiB at its default range count); a step that needs more is rejected.
constexpr int64_t kScratchBytes = 96ll << 20;
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices];

}  // namespace

// One copy per GPU, held until the process ends.  Host code uses the
// per-device address that hipGetSymbolAddress returns, never the array's name.
static __device__ __align__(256) char scratch[kScratchBytes];

static int scratch_address(void** out) {
  int dev = 0;
  if (int rc = aia::check_hip(hipGetDevice(&dev), "aia_paged_attention_gqa_noalloc: hipGetDevice"))
    return rc;
  if (dev < 0 || dev >= kMaxScratchDevices)
    return aia::fail(AIA_ERR_UNSUPPORTED, "aia_paged_attention_gqa_noalloc: device %d", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (int rc = aia::check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)),
                                "aia_paged_attention_gqa_noalloc: scratch address"))
      return rc;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return AIA_OK;
}

extern "C" int aia_noalloc_scratch_bytes(int64_t* bytes) {
  if (!bytes) return aia::fail(AIA_ERR_INVALID, "aia_noalloc_scratch_bytes: null pointer");
  *bytes = kScratchBytes;
  return AIA_OK;
}

extern "C" int aia_paged_attention_gqa_noalloc(
    const void* query, int64_t q_token_stride, int64_t q_head_stride, const void* key_cache,
    const void* value_cache, const int32_t* block_table, int32_t block_table_stride,
    const int32_t* cu_seqlens_q, const int32_t* seqlens_kv, int32_t batch, int32_t num_tokens,
    int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
    int32_t num_blocks, float scale, void* out, int64_t out_token_stride, int64_t out_head_stride,
    const void* key_new, const void* value_new, int64_t new_key_token_stride,
    int64_t new_value_token_stride, int32_t num_waves, int32_t flags, void* stream) {
  using namespace aia;
  if (batch < 0 || num_tokens < 0)
    return fail(AIA_ERR_INVALID, "aia_paged_attention_gqa_noalloc: bad sizes");
  if (num_tokens == 0 || batch == 0) return AIA_OK;
  int64_t need = 0;
  if (int rc = aia_attn_workspace_bytes(batch, num_tokens, num_q_heads, num_kv_heads, head_dim,
                                        num_waves, &need))
    return rc;
  if (need > kScratchBytes)
    return fail(AIA_ERR_CAPACITY,
                "aia_paged_attention_gqa_noalloc: step needs %lld bytes of scratch, the static "
                "scratch holds %lld", (long long)need, (long long)kScratchBytes);
  void* ws = nullptr;
  if (int rc = scratch_address(&ws)) return rc;
  if (int rc = aia_attn_plan(cu_seqlens_q, seqlens_kv, block_table, block_table_stride,
                             block_size, batch, num_tokens, num_q_heads, num_kv_heads, head_dim,
                             num_waves, ws, kScratchBytes, stream))
    return rc;
  return aia_paged_attention_gqa(query, q_token_stride, q_head_stride, key_cache, value_cache,
                                 block_table, block_table_stride, cu_seqlens_q, seqlens_kv, batch,
                                 num_tokens, num_q_heads, num_kv_heads, head_dim, block_size,
                                 num_blocks, scale, out, out_token_stride, out_head_stride,
                                 key_new, value_new, new_key_token_stride, new_value_token_stride,
                                 num_waves, flags, ws, kScratchBytes, stream);
}
