// Ragged-batch packing: step rows -> the attention metadata of one step.
//
// Request state lives on the device: a block pool (one row of block ids per
// request slot) and a token pool (one row of token ids per request slot).
// Per step the host uploads only (a) the pool entries that changed since the
// last step (new blocks, new tokens, drafts) and (b) one 8-int descriptor per
// sequence row.  Two kernels then run:
//   pack_updates  scatter of the changed pool entries;
//   pack_rows     one wave per row: positions start..start+n-1, token ids
//                 gathered from the token pool, slot = block[pos / bs] * bs +
//                 pos % bs, the zero-padded block-table row, cu_seqlens_q,
//                 seqlens_kv = start + n, the last-row index of every row and
//                 the compacted sample rows.
// Synthetic rows (the stagers' scratch padding) take consecutive blocks
// block_base, block_base + 1, ... and token id 0.
#include <string.h>

#include "common.h"

namespace {

struct PackArgs {
  const int32_t* rows;       // [num_rows][8]
  int32_t num_rows;
  const int64_t* token_pool;
  int64_t token_stride;
  const int32_t* block_pool;
  int64_t block_stride;
  int32_t block_size;
  int32_t bt_width;
  int64_t* token_ids;
  int64_t* positions;
  int32_t* slot_mapping;
  int32_t* block_table;
  int32_t* cu_seqlens_q;
  int32_t* seqlens_kv;
  int64_t* last_rows;
  int64_t* sample_rows;
  int32_t sample_count, sample_cap;
};

__global__ __launch_bounds__(256) void pack_updates_kernel(
    const int64_t* __restrict__ tidx, const int64_t* __restrict__ tval, int32_t ntok,
    const int64_t* __restrict__ bidx, const int32_t* __restrict__ bval, int32_t nblk,
    int64_t* __restrict__ token_pool, int32_t* __restrict__ block_pool) {
  const int32_t total = ntok + nblk;
  for (int32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
    if (i < ntok) token_pool[tidx[i]] = tval[i];
    else block_pool[bidx[i - ntok]] = bval[i - ntok];
  }
}

// One row's outputs, by one wave.
__device__ __forceinline__ void pack_one_row(const PackArgs& a, int r, const int32_t* d, int lane) {
  const int src = d[0], start = d[1], n = d[2], nblocks = d[3], base = d[4], q_off = d[5];
  const int zero_tokens = d[6], sample_slot = d[7];
  const int32_t* prow = src >= 0 ? a.block_pool + (int64_t)src * a.block_stride : nullptr;
  const int64_t* trow = src >= 0 ? a.token_pool + (int64_t)src * a.token_stride : nullptr;
  const int max_col = (int)a.block_stride - 1;
  for (int j = lane; j < n; j += 64) {
    const int pos = start + j;
    const int bi = pos / a.block_size;
    const int blk = prow ? prow[min(bi, max_col)] : base + bi;
    const int64_t q = q_off + j;
    a.positions[q] = pos;
    a.slot_mapping[q] = blk * a.block_size + (pos - bi * a.block_size);
    a.token_ids[q] = (zero_tokens || !trow) ? 0 : trow[min((int64_t)pos, a.token_stride - 1)];
  }
  int32_t* bt = a.block_table + (int64_t)r * a.bt_width;
  for (int c = lane; c < a.bt_width; c += 64)
    bt[c] = c < nblocks ? (prow ? prow[min(c, max_col)] : base + c) : 0;
  if (lane == 0) {
    if (r == 0) a.cu_seqlens_q[0] = 0;
    a.cu_seqlens_q[r + 1] = q_off + n;
    a.seqlens_kv[r] = start + n;
    if (a.last_rows) a.last_rows[r] = q_off + n - 1;
    if (sample_slot >= 0 && sample_slot < a.sample_cap) a.sample_rows[sample_slot] = q_off + n - 1;
  }
}

__global__ __launch_bounds__(256) void pack_rows_kernel(PackArgs a) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  // zero the unused tail of the sample rows (prefill stager contract)
  for (int i = blockIdx.x * blockDim.x + threadIdx.x + a.sample_count; i < a.sample_cap;
       i += gridDim.x * blockDim.x)
    a.sample_rows[i] = 0;
  if (r >= a.num_rows) return;
  pack_one_row(a, r, a.rows + (int64_t)r * 8, lane);
}

// The whole step in one work-group, its updates and row descriptors carried
// in the kernel arguments (the launch copies them; no staging copy): the
// pool updates first, then, after a work-group barrier (one CU, so its
// stores are visible to the whole group), one wave per row; 16 waves, so a
// decode gear of up to 16 requests packs its rows in one pass.
template <int BYTES>
struct InlineBlob {
  int64_t w[BYTES / 8];
};
// a smaller argument block for the common small step (a decode gear of a
// dozen requests): the launch copies fewer argument bytes
constexpr int kInlineSmall = 1024;

template <int BYTES>
__global__ __launch_bounds__(1024) void pack_inline_kernel(PackArgs a, InlineBlob<BYTES> blob, int32_t nt,
                                                          int32_t nb, int64_t* token_pool,
                                                          int32_t* block_pool) {
  const int64_t* tidx = blob.w;
  const int64_t* tval = blob.w + nt;
  const int64_t* bidx = blob.w + 2 * nt;
  const int32_t* bval = reinterpret_cast<const int32_t*>(blob.w + 2 * nt + nb);
  const int32_t* rows = reinterpret_cast<const int32_t*>(blob.w + 2 * nt + nb + (nb + 1) / 2);
  for (int i = threadIdx.x; i < nt + nb; i += blockDim.x) {
    if (i < nt) token_pool[tidx[i]] = tval[i];
    else block_pool[bidx[i - nt]] = bval[i - nt];
  }
  for (int i = threadIdx.x + a.sample_count; i < a.sample_cap; i += blockDim.x) a.sample_rows[i] = 0;
  __syncthreads();
  const int lane = threadIdx.x & 63;
  for (int r = threadIdx.x >> 6; r < a.num_rows; r += blockDim.x >> 6)
    pack_one_row(a, r, rows + (int64_t)r * 8, lane);
}

// Token splice: target[pairs[i].row] = *pairs[i].source for every pair, one
// thread per pair.  Sources are addresses of int64 token ids inside the
// caller's sampled-token tensors, so rows of any number of tensors move in
// one launch.  Rows outside the target are skipped.
__global__ __launch_bounds__(256) void splice_tokens_kernel(const int64_t* __restrict__ pairs,
                                                            int32_t count, int64_t* __restrict__ target,
                                                            int64_t target_len) {
  const int32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count) return;
  const int64_t* src = reinterpret_cast<const int64_t*>(pairs[2 * i]);
  const int64_t row = pairs[2 * i + 1];
  if (src != nullptr && row >= 0 && row < target_len) target[row] = *src;
}

}  // namespace

extern "C" int aia_splice_tokens(const int64_t* pairs, int32_t count, int64_t* target,
                                 int64_t target_len, void* stream) {
  using namespace aia;
  if (count < 0 || target_len < 0) return fail(AIA_ERR_INVALID, "aia_splice_tokens: bad sizes");
  if (count == 0) return AIA_OK;
  if (!pairs || !target) return fail(AIA_ERR_INVALID, "aia_splice_tokens: null pointer argument");
  splice_tokens_kernel<<<(count + 255) / 256, 256, 0, (hipStream_t)stream>>>(pairs, count, target,
                                                                           target_len);
  return check_hip(hipGetLastError(), "aia_splice_tokens launch");
}

extern "C" int aia_pack_rows(const int64_t* token_update_index, const int64_t* token_update_value,
                             int32_t num_token_updates, const int64_t* block_update_index,
                             const int32_t* block_update_value, int32_t num_block_updates,
                             int64_t* token_pool, int64_t token_pool_stride, int32_t* block_pool,
                             int64_t block_pool_stride, const int32_t* rows, int32_t num_rows,
                             int32_t block_size, int32_t block_table_width, int64_t* token_ids,
                             int64_t* positions, int32_t* slot_mapping, int32_t* block_table,
                             int32_t* cu_seqlens_q, int32_t* seqlens_kv, int64_t* last_rows,
                             int64_t* sample_rows, int32_t sample_count, int32_t sample_cap,
                             void* stream) {
  using namespace aia;
  if (num_rows < 0 || block_size <= 0 || block_table_width < 0 || num_token_updates < 0 ||
      num_block_updates < 0 || sample_count < 0 || sample_cap < sample_count)
    return fail(AIA_ERR_INVALID, "aia_pack_rows: bad sizes");
  if (num_rows > 0 && (!rows || !positions || !slot_mapping || !token_ids || !cu_seqlens_q ||
                       !seqlens_kv || (block_table_width > 0 && !block_table)))
    return fail(AIA_ERR_INVALID, "aia_pack_rows: null output");
  if ((num_token_updates && (!token_pool || !token_update_index || !token_update_value)) ||
      (num_block_updates && (!block_pool || !block_update_index || !block_update_value)))
    return fail(AIA_ERR_INVALID, "aia_pack_rows: updates without a pool");
  if (sample_cap > 0 && !sample_rows) return fail(AIA_ERR_INVALID, "aia_pack_rows: null sample_rows");
  hipStream_t s = (hipStream_t)stream;
  const int32_t nupd = num_token_updates + num_block_updates;
  if (nupd > 0) {
    int blocks = (nupd + 255) / 256;
    if (blocks > 1024) blocks = 1024;
    pack_updates_kernel<<<blocks, 256, 0, s>>>(token_update_index, token_update_value,
                                               num_token_updates, block_update_index,
                                               block_update_value, num_block_updates, token_pool,
                                               block_pool);
    if (int rc = check_hip(hipGetLastError(), "pack_updates launch")) return rc;
  }
  if (num_rows == 0 && sample_cap == 0) return AIA_OK;
  PackArgs a;
  a.rows = rows; a.num_rows = num_rows;
  a.token_pool = token_pool; a.token_stride = token_pool_stride;
  a.block_pool = block_pool; a.block_stride = block_pool_stride > 0 ? block_pool_stride : 1;
  a.block_size = block_size; a.bt_width = block_table_width;
  a.token_ids = token_ids; a.positions = positions; a.slot_mapping = slot_mapping;
  a.block_table = block_table; a.cu_seqlens_q = cu_seqlens_q; a.seqlens_kv = seqlens_kv;
  a.last_rows = last_rows; a.sample_rows = sample_rows;
  a.sample_count = sample_count; a.sample_cap = sample_cap;
  const int grid = num_rows > 0 ? (num_rows + 3) / 4 : 1;
  pack_rows_kernel<<<grid, 256, 0, s>>>(a);
  return check_hip(hipGetLastError(), "pack_rows launch");
}

extern "C" int aia_pack_rows_inline(const void* blob, int32_t num_token_updates,
                                    int32_t num_block_updates, int32_t num_rows,
                                    int64_t* token_pool, int64_t token_pool_stride,
                                    int32_t* block_pool, int64_t block_pool_stride,
                                    int32_t block_size, int32_t block_table_width,
                                    int64_t* token_ids, int64_t* positions, int32_t* slot_mapping,
                                    int32_t* block_table, int32_t* cu_seqlens_q,
                                    int32_t* seqlens_kv, int64_t* last_rows, int64_t* sample_rows,
                                    int32_t sample_count, int32_t sample_cap, void* stream) {
  using namespace aia;
  const int64_t nt = num_token_updates, nb = num_block_updates, nr = num_rows;
  if (nt < 0 || nb < 0 || nr < 0 || block_size <= 0 || block_table_width < 0 || sample_count < 0 ||
      sample_cap < sample_count)
    return fail(AIA_ERR_INVALID, "aia_pack_rows_inline: bad sizes");
  const int64_t words = 2 * nt + nb + (nb + 1) / 2 + 4 * nr;
  if (words * 8 > AIA_PACK_INLINE_BYTES)
    return fail(AIA_ERR_CAPACITY, "aia_pack_rows_inline: %lld bytes exceed the %d inline bytes",
                (long long)(words * 8), AIA_PACK_INLINE_BYTES);
  if (nr > 0 && (!positions || !slot_mapping || !token_ids || !cu_seqlens_q || !seqlens_kv ||
                 (block_table_width > 0 && !block_table)))
    return fail(AIA_ERR_INVALID, "aia_pack_rows_inline: null output");
  if ((nt && !token_pool) || (nb && !block_pool) || (words && !blob))
    return fail(AIA_ERR_INVALID, "aia_pack_rows_inline: updates without a pool");
  if (sample_cap > 0 && !sample_rows)
    return fail(AIA_ERR_INVALID, "aia_pack_rows_inline: null sample_rows");
  if (words == 0 && sample_cap == 0) return AIA_OK;
  PackArgs a;
  a.rows = nullptr; a.num_rows = (int32_t)nr;
  a.token_pool = token_pool; a.token_stride = token_pool_stride;
  a.block_pool = block_pool; a.block_stride = block_pool_stride > 0 ? block_pool_stride : 1;
  a.block_size = block_size; a.bt_width = block_table_width;
  a.token_ids = token_ids; a.positions = positions; a.slot_mapping = slot_mapping;
  a.block_table = block_table; a.cu_seqlens_q = cu_seqlens_q; a.seqlens_kv = seqlens_kv;
  a.last_rows = last_rows; a.sample_rows = sample_rows;
  a.sample_count = sample_count; a.sample_cap = sample_cap;
  if (words * 8 <= kInlineSmall) {
    InlineBlob<kInlineSmall> b;
    memcpy(b.w, blob, (size_t)words * 8);
    pack_inline_kernel<kInlineSmall><<<1, 1024, 0, (hipStream_t)stream>>>(a, b, (int32_t)nt,
                                                                          (int32_t)nb, token_pool,
                                                                          block_pool);
  } else {
    InlineBlob<AIA_PACK_INLINE_BYTES> b;
    memcpy(b.w, blob, (size_t)words * 8);
    pack_inline_kernel<AIA_PACK_INLINE_BYTES><<<1, 1024, 0, (hipStream_t)stream>>>(
        a, b, (int32_t)nt, (int32_t)nb, token_pool, block_pool);
  }
  return check_hip(hipGetLastError(), "aia_pack_rows_inline launch");
}
