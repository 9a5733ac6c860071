// KV slot write: key_cache.view(-1, row)[slot[t]] = key[t] (and value).
//
// Pure copy, HBM bound: every thread moves one 16-byte chunk of one token
// row, consecutive threads take consecutive chunks of the same row, so each
// wave reads and writes whole contiguous rows (Hkv * D * 2 = 2048 B for the
// GQA configs, 1152 B for the MLA latent).
#include "common.h"

namespace {

__global__ __launch_bounds__(256) void kv_write_vec16(
    const uint4* __restrict__ key, int64_t key_ts16,
    const uint4* __restrict__ value, int64_t value_ts16,
    uint4* __restrict__ key_cache, uint4* __restrict__ value_cache,
    const int32_t* __restrict__ slots, int32_t num_tokens,
    int32_t kchunks, int32_t vchunks, int64_t num_slots) {
  const int64_t per_token = (int64_t)kchunks + vchunks;
  const int64_t total = per_token * num_tokens;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int32_t t = (int32_t)(i / per_token);
    const int32_t c = (int32_t)(i - (int64_t)t * per_token);
    const int32_t slot = slots[t];
    if (slot < 0 || slot >= num_slots) continue;
    if (c < kchunks) {
      key_cache[(int64_t)slot * kchunks + c] = key[t * key_ts16 + c];
    } else {
      const int32_t cv = c - kchunks;
      value_cache[(int64_t)slot * vchunks + cv] = value[t * value_ts16 + cv];
    }
  }
}

// Fallback for rows or strides that are not 16-byte aligned.
__global__ __launch_bounds__(256) void kv_write_scalar(
    const uint16_t* __restrict__ key, int64_t key_ts,
    const uint16_t* __restrict__ value, int64_t value_ts,
    uint16_t* __restrict__ key_cache, uint16_t* __restrict__ value_cache,
    const int32_t* __restrict__ slots, int32_t num_tokens,
    int32_t krow, int32_t vrow, int64_t num_slots) {
  const int64_t per_token = (int64_t)krow + vrow;
  const int64_t total = per_token * num_tokens;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int32_t t = (int32_t)(i / per_token);
    const int32_t c = (int32_t)(i - (int64_t)t * per_token);
    const int32_t slot = slots[t];
    if (slot < 0 || slot >= num_slots) continue;
    if (c < krow) key_cache[(int64_t)slot * krow + c] = key[t * key_ts + c];
    else value_cache[(int64_t)slot * vrow + (c - krow)] = value[t * value_ts + (c - krow)];
  }
}

// The same write into caches in the NZ layout of the reference's graph mode
// (each block viewed (row / 16, block_size, 16)): piece p (8 values) of a
// row goes to 16-wide chunk p / 2, half p % 2, of the token's offset in its
// block.
__global__ __launch_bounds__(256) void kv_write_nz_vec16(
    const uint4* __restrict__ key, int64_t key_ts16,
    const uint4* __restrict__ value, int64_t value_ts16,
    uint4* __restrict__ key_cache, uint4* __restrict__ value_cache,
    const int32_t* __restrict__ slots, int32_t num_tokens, int32_t pieces, int32_t block_size,
    int64_t num_slots) {
  const int64_t per_token = 2 * (int64_t)pieces;
  const int64_t total = per_token * num_tokens;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int32_t t = (int32_t)(i / per_token);
    int32_t c = (int32_t)(i - (int64_t)t * per_token);
    const int32_t slot = slots[t];
    if (slot < 0 || slot >= num_slots) continue;
    const bool is_v = c >= pieces;
    if (is_v) c -= pieces;
    if (is_v && !value) continue;
    const int64_t blk = slot / block_size, off = slot - blk * block_size;
    const int64_t dst = blk * block_size * pieces + ((int64_t)(c >> 1) * block_size + off) * 2 + (c & 1);
    if (is_v) value_cache[dst] = value[t * value_ts16 + c];
    else key_cache[dst] = key[t * key_ts16 + c];
  }
}

}  // namespace

extern "C" int aia_kv_write_nz(const void* key, int64_t key_token_stride, const void* value,
                               int64_t value_token_stride, void* key_cache, void* value_cache,
                               const int32_t* slot_mapping, int32_t num_tokens, int32_t row_elems,
                               int32_t block_size, int64_t num_slots, void* stream) {
  using namespace aia;
  if (num_tokens < 0 || row_elems <= 0 || block_size <= 0 || num_slots < 0 ||
      num_slots % block_size)
    return fail(AIA_ERR_INVALID, "aia_kv_write_nz: bad sizes (tokens %d, row %d, block %d, "
                "slots %lld)", num_tokens, row_elems, block_size, (long long)num_slots);
  if (row_elems % 16)
    return fail(AIA_ERR_UNSUPPORTED, "aia_kv_write_nz: row of %d values is not whole 16-wide "
                "chunks", row_elems);
  if (num_tokens == 0) return AIA_OK;
  if (!key || !key_cache || !slot_mapping)
    return fail(AIA_ERR_INVALID, "aia_kv_write_nz: null key/key_cache/slot_mapping");
  if ((value == nullptr) != (value_cache == nullptr))
    return fail(AIA_ERR_INVALID, "aia_kv_write_nz: value and value_cache must both be set or both NULL");
  auto aligned = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  if (!aligned(key) || !aligned(key_cache) || key_token_stride % 8 || key_token_stride < row_elems ||
      (value && (!aligned(value) || !aligned(value_cache) || value_token_stride % 8 ||
                 value_token_stride < row_elems)))
    return fail(AIA_ERR_INVALID, "aia_kv_write_nz: rows and caches must be 16-byte aligned with "
                "token strides a multiple of 8 values and at least a row");
  const int64_t total = 2LL * (row_elems / 8) * num_tokens;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  kv_write_nz_vec16<<<dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream>>>(
      (const uint4*)key, key_token_stride / 8, (const uint4*)value, value ? value_token_stride / 8 : 0,
      (uint4*)key_cache, (uint4*)value_cache, slot_mapping, num_tokens, row_elems / 8, block_size,
      num_slots);
  return check_hip(hipGetLastError(), "aia_kv_write_nz launch");
}

extern "C" int aia_kv_write(const void* key, int64_t key_token_stride,
                            const void* value, int64_t value_token_stride,
                            void* key_cache, void* value_cache,
                            const int32_t* slot_mapping, int32_t num_tokens,
                            int32_t key_row_elems, int32_t value_row_elems,
                            int64_t num_slots, void* stream) {
  using namespace aia;
  if (num_tokens < 0 || key_row_elems <= 0 || num_slots < 0)
    return fail(AIA_ERR_INVALID, "aia_kv_write: bad sizes (tokens %d, row %d, slots %lld)",
                num_tokens, key_row_elems, (long long)num_slots);
  if (num_tokens == 0) return AIA_OK;
  if (!key || !key_cache || !slot_mapping)
    return fail(AIA_ERR_INVALID, "aia_kv_write: null key/key_cache/slot_mapping");
  const bool has_v = value != nullptr;
  if (has_v != (value_cache != nullptr))
    return fail(AIA_ERR_INVALID, "aia_kv_write: value and value_cache must both be set or both NULL");
  if (has_v && value_row_elems <= 0)
    return fail(AIA_ERR_INVALID, "aia_kv_write: bad value_row_elems %d", value_row_elems);
  if (key_token_stride < key_row_elems || (has_v && value_token_stride < value_row_elems))
    return fail(AIA_ERR_INVALID, "aia_kv_write: token stride smaller than the row");
  const int32_t vrow = has_v ? value_row_elems : 0;
  hipStream_t s = (hipStream_t)stream;

  auto aligned = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  const bool vec = aligned(key) && aligned(key_cache) && key_row_elems % 8 == 0 &&
                   key_token_stride % 8 == 0 &&
                   (!has_v || (aligned(value) && aligned(value_cache) &&
                               value_row_elems % 8 == 0 && value_token_stride % 8 == 0));
  const int64_t per_token = vec ? (key_row_elems + vrow) / 8 : (key_row_elems + vrow);
  const int64_t total = per_token * num_tokens;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  if (vec) {
    kv_write_vec16<<<dim3((unsigned)blocks), dim3(256), 0, s>>>(
        (const uint4*)key, key_token_stride / 8, (const uint4*)value,
        has_v ? value_token_stride / 8 : 0, (uint4*)key_cache, (uint4*)value_cache,
        slot_mapping, num_tokens, key_row_elems / 8, vrow / 8, num_slots);
  } else {
    kv_write_scalar<<<dim3((unsigned)blocks), dim3(256), 0, s>>>(
        (const uint16_t*)key, key_token_stride, (const uint16_t*)value,
        has_v ? value_token_stride : 0, (uint16_t*)key_cache, (uint16_t*)value_cache,
        slot_mapping, num_tokens, key_row_elems, vrow, num_slots);
  }
  return check_hip(hipGetLastError(), "aia_kv_write launch");
}
