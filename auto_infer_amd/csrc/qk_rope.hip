// Fused pre-attention: per-head RMSNorm (optional, Qwen3 QK-Norm) + NeoX
// RoPE over the Q and K parts of a packed qkv projection, in place.
//
// Reference (auto_infer/layers/attention/gqa.py:27-49): split the packed
// projection into q (T, Hq, D), k (T, Hkv, D), v; if q_norm/k_norm weights
// exist, q = rms_norm(q, wq, eps), k = rms_norm(k, wk, eps)
// (auto_infer/layers/norm.py:5-8); then x = x * cos + rotate_half(x) * sin
// (auto_infer/layers/rotary_embedding/__init__.py:10-13) with cos/sin of
// shape (T, 1, D).  The reference runs these as separate bf16 torch ops, so
// results are rounded to bf16 after the norm, after x * cos, after
// rotate_half(x) * sin and after the sum; this kernel rounds at exactly the
// same points (a bf16 x bf16 product is exact in fp32, and a bf16 sum is the
// fp32 sum rounded once, as torch computes them), which makes the RoPE part
// bit-identical for identical inputs.
//
// Layout: a half-wave (32 lanes) owns one (token, head) row of 128 dims;
// lane j holds dims {2j, 2j+1} and their rotation partners {2j+64, 2j+65},
// so rotate_half needs no cross-lane traffic and every access is a 4-byte
// load/store of a contiguous pair.  V is not touched: the attention kernel
// reads it (and the rotated K) straight from the qkv buffer.
#include "common.h"

namespace {

constexpr int kDim = 128;

struct RopeArgs {
  uint16_t* qkv;
  int64_t qkv_ts;
  int32_t tokens, hq, hkv;
  const uint16_t* cos;
  const uint16_t* sin;
  int64_t cos_ts, sin_ts;
  const uint16_t* wq;
  const uint16_t* wk;
  float eps;
};

__device__ __forceinline__ float bf(uint32_t bits16) { return __uint_as_float(bits16 << 16); }
__device__ __forceinline__ uint32_t rnd(float x) { return aia::pack_bf16x2(x, 0.f) & 0xffffu; }
__device__ __forceinline__ float rbf(float x) { return bf(rnd(x)); }   // round to bf16

__global__ __launch_bounds__(256) void qk_norm_rope_kernel(RopeArgs a) {
  const int heads = a.hq + a.hkv;
  const int64_t row = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
  if (row >= (int64_t)a.tokens * heads) return;
  const int j = threadIdx.x & 31;
  const int t = (int)(row / heads), h = (int)(row - (int64_t)t * heads);
  uint16_t* x = a.qkv + (int64_t)t * a.qkv_ts + (int64_t)h * kDim;
  const uint32_t lo = *reinterpret_cast<const uint32_t*>(x + 2 * j);        // dims 2j, 2j+1
  const uint32_t hi = *reinterpret_cast<const uint32_t*>(x + 64 + 2 * j);   // dims 2j+64, +65
  float v[4] = {bf(lo & 0xffffu), bf(lo >> 16), bf(hi & 0xffffu), bf(hi >> 16)};
  const uint16_t* w = h < a.hq ? a.wq : a.wk;
  if (w) {
    float ss = (v[0] * v[0] + v[1] * v[1]) + (v[2] * v[2] + v[3] * v[3]);
#pragma unroll
    for (int d = 16; d >= 1; d >>= 1) ss += __shfl_xor(ss, d, 32);
    const float r = 1.0f / __builtin_sqrtf(ss * (1.0f / kDim) + a.eps);
    const uint32_t wlo = *reinterpret_cast<const uint32_t*>(w + 2 * j);
    const uint32_t whi = *reinterpret_cast<const uint32_t*>(w + 64 + 2 * j);
    const float wv[4] = {bf(wlo & 0xffffu), bf(wlo >> 16), bf(whi & 0xffffu), bf(whi >> 16)};
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = rbf((v[i] * r) * wv[i]);
  }
  const uint32_t clo = *reinterpret_cast<const uint32_t*>(a.cos + (int64_t)t * a.cos_ts + 2 * j);
  const uint32_t chi = *reinterpret_cast<const uint32_t*>(a.cos + (int64_t)t * a.cos_ts + 64 + 2 * j);
  const uint32_t slo = *reinterpret_cast<const uint32_t*>(a.sin + (int64_t)t * a.sin_ts + 2 * j);
  const uint32_t shi = *reinterpret_cast<const uint32_t*>(a.sin + (int64_t)t * a.sin_ts + 64 + 2 * j);
  const float c[4] = {bf(clo & 0xffffu), bf(clo >> 16), bf(chi & 0xffffu), bf(chi >> 16)};
  const float sn[4] = {bf(slo & 0xffffu), bf(slo >> 16), bf(shi & 0xffffu), bf(shi >> 16)};
  // rotate_half: first half takes -x[d + 64], second half x[d - 64]
  const float rot[4] = {-v[2], -v[3], v[0], v[1]};
  float o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = rbf(rbf(v[i] * c[i]) + rbf(rot[i] * sn[i]));
  *reinterpret_cast<uint32_t*>(x + 2 * j) = aia::pack_bf16x2(o[0], o[1]);
  *reinterpret_cast<uint32_t*>(x + 64 + 2 * j) = aia::pack_bf16x2(o[2], o[3]);
}

}  // namespace

extern "C" int aia_qk_norm_rope(void* qkv, int64_t qkv_token_stride, int32_t num_tokens,
                                int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                const void* cos, int64_t cos_token_stride, const void* sin,
                                int64_t sin_token_stride, const void* q_norm_weight,
                                const void* k_norm_weight, float eps, void* stream) {
  using namespace aia;
  if (head_dim != kDim)
    return fail(AIA_ERR_UNSUPPORTED, "aia_qk_norm_rope: head_dim %d (only 128)", head_dim);
  if (num_tokens < 0 || num_q_heads <= 0 || num_kv_heads <= 0)
    return fail(AIA_ERR_INVALID, "aia_qk_norm_rope: bad sizes");
  if ((q_norm_weight == nullptr) != (k_norm_weight == nullptr))
    return fail(AIA_ERR_INVALID, "aia_qk_norm_rope: q and k norm weights go together");
  if (num_tokens == 0) return AIA_OK;
  if (!qkv || !cos || !sin) return fail(AIA_ERR_INVALID, "aia_qk_norm_rope: null pointer argument");
  if (qkv_token_stride < (int64_t)(num_q_heads + 2 * num_kv_heads) * kDim ||
      qkv_token_stride % 2 || cos_token_stride % 2 || sin_token_stride % 2 ||
      ((uintptr_t)qkv & 3) || ((uintptr_t)cos & 3) || ((uintptr_t)sin & 3) ||
      ((uintptr_t)q_norm_weight & 3) || ((uintptr_t)k_norm_weight & 3))
    return fail(AIA_ERR_INVALID, "aia_qk_norm_rope: tensors must be 4-byte aligned with even "
                "strides, and a qkv row must hold (Hq + 2 Hkv) x 128 values");
  RopeArgs a;
  a.qkv = static_cast<uint16_t*>(qkv);
  a.qkv_ts = qkv_token_stride;
  a.tokens = num_tokens; a.hq = num_q_heads; a.hkv = num_kv_heads;
  a.cos = static_cast<const uint16_t*>(cos);
  a.sin = static_cast<const uint16_t*>(sin);
  a.cos_ts = cos_token_stride; a.sin_ts = sin_token_stride;
  a.wq = static_cast<const uint16_t*>(q_norm_weight);
  a.wk = static_cast<const uint16_t*>(k_norm_weight);
  a.eps = eps;
  const int64_t rows = (int64_t)num_tokens * (num_q_heads + num_kv_heads);
  const int64_t grid = (rows + 7) / 8;
  if (grid > 0x7fffffff) return fail(AIA_ERR_CAPACITY, "aia_qk_norm_rope: %lld rows", (long long)rows);
  qk_norm_rope_kernel<<<(unsigned)grid, 256, 0, (hipStream_t)stream>>>(a);
  return check_hip(hipGetLastError(), "qk_norm_rope launch");
}
