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
// Layout: D / 16 lanes own one (token, head) row of D dims (D = 128: 8
// lanes, D = 64: 4); lane j holds dims 8j .. 8j+7 and their rotation
// partners D/2 + 8j .. D/2 + 8j + 7, so rotate_half needs no cross-lane
// traffic and every access is a 16-byte load/store of 8 contiguous values.  V is not touched: the attention kernel
// reads it (and the rotated K) straight from the qkv buffer.
#include "common.h"

namespace {

constexpr int kThreads = 256;

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

__device__ __forceinline__ void unpack8(uint4 w, float (&v)[16], int at) {
  const uint32_t p[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) { v[at + 2 * i] = bf(p[i] & 0xffffu); v[at + 2 * i + 1] = bf(p[i] >> 16); }
}

// One work-group per token: its cos/sin (and the norm weights) are loaded
// once and reused by the row slots (256 / (D / 16) of them), which loop over
// the token's heads.
template <int D>
__global__ __launch_bounds__(kThreads) void qk_norm_rope_kernel(RopeArgs a) {
  constexpr int kLanes = D / 16, kHalf = D / 2, kRowsPerBlock = kThreads / kLanes;
  const int heads = a.hq + a.hkv;
  const int t = blockIdx.x;
  const int j = threadIdx.x & (kLanes - 1), slot = threadIdx.x / kLanes;
  const uint16_t* cp = a.cos + (int64_t)t * a.cos_ts;
  const uint16_t* sp = a.sin + (int64_t)t * a.sin_ts;
  // dims 8j .. 8j+7 and their rotation partners D/2 + 8j .. D/2 + 8j + 7
  float c[16], sn[16], wq[16], wk[16];
  unpack8(*reinterpret_cast<const uint4*>(cp + 8 * j), c, 0);
  unpack8(*reinterpret_cast<const uint4*>(cp + kHalf + 8 * j), c, 8);
  unpack8(*reinterpret_cast<const uint4*>(sp + 8 * j), sn, 0);
  unpack8(*reinterpret_cast<const uint4*>(sp + kHalf + 8 * j), sn, 8);
  const bool norm = a.wq != nullptr;
  if (norm) {
    unpack8(*reinterpret_cast<const uint4*>(a.wq + 8 * j), wq, 0);
    unpack8(*reinterpret_cast<const uint4*>(a.wq + kHalf + 8 * j), wq, 8);
    unpack8(*reinterpret_cast<const uint4*>(a.wk + 8 * j), wk, 0);
    unpack8(*reinterpret_cast<const uint4*>(a.wk + kHalf + 8 * j), wk, 8);
  }
  for (int h = slot; h < heads; h += kRowsPerBlock) {
    uint16_t* x = a.qkv + (int64_t)t * a.qkv_ts + (int64_t)h * D;
    float v[16];
    unpack8(*reinterpret_cast<const uint4*>(x + 8 * j), v, 0);
    unpack8(*reinterpret_cast<const uint4*>(x + kHalf + 8 * j), v, 8);
    if (norm) {
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) ss += v[i] * v[i];
#pragma unroll
      for (int d = kLanes / 2; d >= 1; d >>= 1) ss += __shfl_xor(ss, d, kLanes);
      const float r = 1.0f / __builtin_sqrtf(ss * (1.0f / D) + a.eps);
      const bool isq = h < a.hq;
#pragma unroll
      for (int i = 0; i < 16; ++i) v[i] = rbf((v[i] * r) * (isq ? wq[i] : wk[i]));
    }
    // rotate_half: first half takes -x[d + D/2], second half x[d - D/2]
    float o[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float rot = i < 8 ? -v[i + 8] : v[i - 8];
      o[i] = rbf(rbf(v[i] * c[i]) + rbf(rot * sn[i]));
    }
    uint4 lo, hi;
    lo.x = aia::pack_bf16x2(o[0], o[1]); lo.y = aia::pack_bf16x2(o[2], o[3]);
    lo.z = aia::pack_bf16x2(o[4], o[5]); lo.w = aia::pack_bf16x2(o[6], o[7]);
    hi.x = aia::pack_bf16x2(o[8], o[9]); hi.y = aia::pack_bf16x2(o[10], o[11]);
    hi.z = aia::pack_bf16x2(o[12], o[13]); hi.w = aia::pack_bf16x2(o[14], o[15]);
    *reinterpret_cast<uint4*>(x + 8 * j) = lo;
    *reinterpret_cast<uint4*>(x + kHalf + 8 * j) = hi;
  }
}

}  // namespace

extern "C" int aia_qk_norm_rope(void* qkv, int64_t qkv_token_stride, int32_t num_tokens,
                                int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                const void* cos, int64_t cos_token_stride, const void* sin,
                                int64_t sin_token_stride, const void* q_norm_weight,
                                const void* k_norm_weight, float eps, void* stream) {
  using namespace aia;
  if (head_dim != 128 && head_dim != 64)
    return fail(AIA_ERR_UNSUPPORTED, "aia_qk_norm_rope: head_dim %d (128 or 64)", head_dim);
  if (num_tokens < 0 || num_q_heads <= 0 || num_kv_heads <= 0)
    return fail(AIA_ERR_INVALID, "aia_qk_norm_rope: bad sizes");
  if ((q_norm_weight == nullptr) != (k_norm_weight == nullptr))
    return fail(AIA_ERR_INVALID, "aia_qk_norm_rope: q and k norm weights go together");
  if (num_tokens == 0) return AIA_OK;
  if (!qkv || !cos || !sin) return fail(AIA_ERR_INVALID, "aia_qk_norm_rope: null pointer argument");
  if (qkv_token_stride < (int64_t)(num_q_heads + 2 * num_kv_heads) * head_dim ||
      qkv_token_stride % 8 || cos_token_stride % 8 || sin_token_stride % 8 ||
      ((uintptr_t)qkv & 15) || ((uintptr_t)cos & 15) || ((uintptr_t)sin & 15) ||
      ((uintptr_t)q_norm_weight & 15) || ((uintptr_t)k_norm_weight & 15))
    return fail(AIA_ERR_INVALID, "aia_qk_norm_rope: tensors must be 16-byte aligned with strides "
                "a multiple of 8, and a qkv row must hold (Hq + 2 Hkv) x head_dim values");
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
  if (head_dim == 128)
    qk_norm_rope_kernel<128><<<(unsigned)num_tokens, kThreads, 0, (hipStream_t)stream>>>(a);
  else
    qk_norm_rope_kernel<64><<<(unsigned)num_tokens, kThreads, 0, (hipStream_t)stream>>>(a);
  return check_hip(hipGetLastError(), "qk_norm_rope launch");
}
