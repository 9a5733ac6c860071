// Absorbed-MLA pre- and post-attention: the latent query and the latent KV
// row of each token, each in one launch, and the W_UV value up-projection of
// the attention output (mla.py:120-121).
//
// Reference (auto_infer/layers/attention/mla.py:86-113, mla_paged_absorbed):
//   q_nope, q_pe = q.split([nope, rope])            q (T, H, nope + rope)
//   ckv, k_pe    = ckv_full.split([kvl, rope])      ckv_full (T, kvl + rope)
//   ckv          = rms_norm(ckv, kv_a_layernorm, eps)
//   q_pe, k_pe   = ds_rope_interleave(.)            (rotary_embedding:15-23)
//   q_pe, k_pe   = x * cos + rotate_half(x) * sin   (NeoX, cos/sin (T, 1, rope))
//   q_latent     = cat(einsum("tnp,npl->tnl", q_nope, W_UK), q_pe)
//   k_latent     = cat(ckv, k_pe)                   (T, 1, kvl + rope)
// with kvl = 512, rope = 64, nope = 128.  The torch ops round to bf16 after
// the norm, after x * cos, after rotate_half(x) * sin and after the sum; the
// kernels round at the same points, so the RoPE parts are bit-identical to
// them.  The norm is fp32 over the row with one rounding (its sum order
// differs from torch's); the W_UK product accumulates in fp32 on MFMA and
// rounds once, as a bf16 library GEMM does.
//
// ds_rope_interleave maps out[j] = in[2 j], out[32 + j] = in[2 j + 1], so the
// lane that loads input dims 2 j, 2 j + 1 holds both halves of rotation pair j:
// lane k (of 8) loads pe dims 8 k .. 8 k + 7 and writes output dims
// 4 k .. 4 k + 3 and 32 + 4 k .. 32 + 4 k + 3.
#include "common.h"

namespace {

constexpr int kLatent = 512, kRope = 64, kNope = 128, kRow = kLatent + kRope;

__device__ __forceinline__ float bfv(uint32_t bits16) { return __uint_as_float(bits16 << 16); }
__device__ __forceinline__ float rbf(float x) { return bfv(aia::pack_bf16x2(x, 0.f) & 0xffffu); }

// Rotated pe of one lane: in[8] = input dims 8 k .. 8 k + 7; c/s hold the
// cos/sin of output dims 4 k .. 4 k + 3 (lo) and 32 + 4 k .. (hi).
__device__ __forceinline__ void rope_pairs(const float (&in)[8], const float (&clo)[4],
                                           const float (&chi)[4], const float (&slo)[4],
                                           const float (&shi)[4], float (&lo)[4], float (&hi)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float x1 = in[2 * i], x2 = in[2 * i + 1];    // interleaved pair -> (j, 32 + j)
    lo[i] = rbf(rbf(x1 * clo[i]) + rbf(-x2 * slo[i]));
    hi[i] = rbf(rbf(x2 * chi[i]) + rbf(x1 * shi[i]));
  }
}

__device__ __forceinline__ void unpack4(uint2 w, float (&v)[4]) {
  v[0] = bfv(w.x & 0xffffu); v[1] = bfv(w.x >> 16); v[2] = bfv(w.y & 0xffffu); v[3] = bfv(w.y >> 16);
}
__device__ __forceinline__ void unpack8(uint4 w, float (&v)[8]) {
  const uint32_t p[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) { v[2 * i] = bfv(p[i] & 0xffffu); v[2 * i + 1] = bfv(p[i] >> 16); }
}
__device__ __forceinline__ uint2 pack4(const float (&v)[4]) {
  return make_uint2(aia::pack_bf16x2(v[0], v[1]), aia::pack_bf16x2(v[2], v[3]));
}

// Loads the rotation inputs of pe lane k for one token and writes its 2 x 4
// output dims at dst (dst[4 k..], dst[32 + 4 k..]).
__device__ __forceinline__ void rope_lane(const uint16_t* pe, const uint16_t* cs, const uint16_t* sn,
                                          uint16_t* dst, int k) {
  float in[8], clo[4], chi[4], slo[4], shi[4], lo[4], hi[4];
  unpack8(*reinterpret_cast<const uint4*>(pe + 8 * k), in);
  unpack4(*reinterpret_cast<const uint2*>(cs + 4 * k), clo);
  unpack4(*reinterpret_cast<const uint2*>(cs + 32 + 4 * k), chi);
  unpack4(*reinterpret_cast<const uint2*>(sn + 4 * k), slo);
  unpack4(*reinterpret_cast<const uint2*>(sn + 32 + 4 * k), shi);
  rope_pairs(in, clo, chi, slo, shi, lo, hi);
  *reinterpret_cast<uint2*>(dst + 4 * k) = pack4(lo);
  *reinterpret_cast<uint2*>(dst + 32 + 4 * k) = pack4(hi);
}

struct KvArgs {
  const uint16_t* ckv;      // (T, 576) rows, stride ckv_ts
  int64_t ckv_ts;
  const uint16_t* w;        // kv_a_layernorm weight (512)
  const uint16_t* cos;
  const uint16_t* sin;
  int64_t cos_ts, sin_ts;
  uint16_t* out;            // (T, 576) rows, stride out_ts
  int64_t out_ts;
  int32_t tokens;
  float eps;
};

// One wave per token: lane l normalises dims 8 l .. 8 l + 7 of the latent;
// lanes 0..7 rotate the pe part.
__global__ __launch_bounds__(256) void mla_kv_latent_kernel(KvArgs a) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= a.tokens) return;
  const uint16_t* x = a.ckv + (int64_t)t * a.ckv_ts;
  uint16_t* o = a.out + (int64_t)t * a.out_ts;
  float v[8], wv[8];
  unpack8(*reinterpret_cast<const uint4*>(x + 8 * lane), v);
  unpack8(*reinterpret_cast<const uint4*>(a.w + 8 * lane), wv);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss += v[i] * v[i];
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) ss += __shfl_xor(ss, d);
  const float r = 1.0f / __builtin_sqrtf(ss * (1.0f / kLatent) + a.eps);
  float y[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) y[i] = (v[i] * r) * wv[i];
  uint4 st;
  st.x = aia::pack_bf16x2(y[0], y[1]); st.y = aia::pack_bf16x2(y[2], y[3]);
  st.z = aia::pack_bf16x2(y[4], y[5]); st.w = aia::pack_bf16x2(y[6], y[7]);
  *reinterpret_cast<uint4*>(o + 8 * lane) = st;
  if (lane < 8)
    rope_lane(x + kLatent, a.cos + (int64_t)t * a.cos_ts, a.sin + (int64_t)t * a.sin_ts,
              o + kLatent, lane);
}

struct QArgs {
  const uint16_t* q;        // (T, H, 192): nope 128 + pe 64
  int64_t q_ts, q_hs;
  const uint16_t* wukt;     // W_UK transposed: (H, 512, 128)
  const uint16_t* cos;
  const uint16_t* sin;
  int64_t cos_ts, sin_ts;
  uint16_t* out;            // (T, H, 576)
  int64_t out_ts, out_hs;
  int32_t tokens, heads;
};

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ bf16x8_t as_b8(uint4 v) {
  return __builtin_bit_cast(bf16x8_t, u32x4_t{v.x, v.y, v.z, v.w});
}

// One work-group per (16 tokens, head, quarter of the latent).  q_latent^T
// (latent x tokens) = W_UK^T (latent x 128) . q_nope^T (128 x tokens) on
// v_mfma_f32_16x16x32_bf16: lane (latent m, group g) loads W_UK^T[h][m][32 j +
// 8 g, +8) (A) and lane (token n, g) loads q_nope[t][h][32 j + 8 g, +8) (B),
// both 16 contiguous bytes; wave w of quarter z owns latent columns
// 128 z + 32 w .. + 31 (2 tiles of 16), so a decode batch still spreads over
// the chip.  In quarter 0, threads (token tid / 16, lane tid % 16 < 8) rotate
// the pe part.
constexpr int kQTiles = 2;     // 16-column latent tiles per wave
__global__ __launch_bounds__(256) void mla_q_latent_kernel(QArgs a) {
  const int t0 = blockIdx.x * 16, h = blockIdx.y, z = blockIdx.z;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int tb = min(t0 + n, a.tokens - 1);           // rows past the end are not stored
  uint4 bq[4];
  const uint16_t* qrow = a.q + (int64_t)tb * a.q_ts + (int64_t)h * a.q_hs;
#pragma unroll
  for (int j = 0; j < 4; ++j) bq[j] = *reinterpret_cast<const uint4*>(qrow + 32 * j + 8 * g);
  const uint16_t* wh = a.wukt + (int64_t)h * kLatent * kNope;
#pragma unroll
  for (int c = 0; c < kQTiles; ++c) {
    const int l0 = 128 * z + 16 * kQTiles * wid + 16 * c;
    const uint16_t* wr = wh + (int64_t)(l0 + n) * kNope;
    uint4 aw[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) aw[j] = *reinterpret_cast<const uint4*>(wr + 32 * j + 8 * g);
    aia::float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_b8(aw[j]), as_b8(bq[j]), acc, 0, 0, 0);
    if (t0 + n < a.tokens) {
      uint16_t* dst = a.out + (int64_t)(t0 + n) * a.out_ts + (int64_t)h * a.out_hs + l0 + 4 * g;
      *reinterpret_cast<uint2*>(dst) =
          make_uint2(aia::pack_bf16x2(acc[0], acc[1]), aia::pack_bf16x2(acc[2], acc[3]));
    }
  }
  const int tt = t0 + (threadIdx.x >> 4), k = threadIdx.x & 15;
  if (z == 0 && k < 8 && tt < a.tokens)
    rope_lane(a.q + (int64_t)tt * a.q_ts + (int64_t)h * a.q_hs + kNope,
              a.cos + (int64_t)tt * a.cos_ts, a.sin + (int64_t)tt * a.sin_ts,
              a.out + (int64_t)tt * a.out_ts + (int64_t)h * a.out_hs + kLatent, k);
}

struct UvArgs {
  const uint16_t* o;        // o_latent rows (T, H, >= 512), strides o_ts / o_hs
  int64_t o_ts, o_hs;
  const uint16_t* w;        // W_UV (H, 128, 512) contiguous
  uint16_t* out;            // (T, H, 128) rows, strides out_ts / out_hs
  int64_t out_ts, out_hs;
  int32_t tokens;
};

// Value up-projection after absorbed attention, per head h:
// out[t][h][v] = sum_l o_latent[t][h][l] W_UV[h][v][l].  Computed as
// out^T (v x tokens) = W_UV[h] (v x 512) . o_latent^T (512 x tokens) on
// v_mfma_f32_16x16x32_bf16, both operands 16-byte contiguous along l:
// lane (v m, group g) loads W_UV[h][v0 + m][32 j + 8 g, +8) (A) and lane
// (token n, g) loads o_latent[t][h][32 j + 8 g, +8) (B).  A work-group owns
// 16 tokens x 32 v columns (grid z: quarter of 128) of one head; wave w sums
// latent dims 128 w .. 128 w + 127 and wave 0 adds the four slices through
// LDS, so every wave is short and a 64-token decode batch spreads over 256
// work-groups.  Each work-group reads its 32 KB of W_UV, so the W_UV reads
// grow with the token count: the kernel is for decode and verify batches.
__global__ __launch_bounds__(256) void mla_v_up_kernel(UvArgs a) {
  constexpr int KS = 4, kSteps = kLatent / 32 / KS;
  __shared__ aia::float4_t red[KS - 1][2][64];
  const int lane = threadIdx.x & 63, ks = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int h = blockIdx.y, v0 = 32 * blockIdx.z;
  const int t0 = blockIdx.x * 16;
  const int tb = min(t0 + n, a.tokens - 1);           // rows past the end are not stored
  const int l0 = ks * (kLatent / KS) + 8 * g;
  const uint16_t* orow = a.o + (int64_t)tb * a.o_ts + (int64_t)h * a.o_hs + l0;
  const uint16_t* w0 = a.w + ((int64_t)h * kNope + v0 + n) * kLatent + l0;
  const uint16_t* w1 = w0 + 16 * kLatent;
  // every operand load is issued before the first MFMA: one memory round
  // trip per wave instead of one per 32-dim step
  uint4 b[kSteps], x0[kSteps], x1[kSteps];
#pragma unroll
  for (int j = 0; j < kSteps; ++j) {
    b[j] = *reinterpret_cast<const uint4*>(orow + 32 * j);
    x0[j] = *reinterpret_cast<const uint4*>(w0 + 32 * j);
    x1[j] = *reinterpret_cast<const uint4*>(w1 + 32 * j);
  }
  __builtin_amdgcn_sched_barrier(0);
  aia::float4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < kSteps; ++j) {
    acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_b8(x0[j]), as_b8(b[j]), acc0, 0, 0, 0);
    acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_b8(x1[j]), as_b8(b[j]), acc1, 0, 0, 0);
  }
  if (ks > 0) {
    red[ks - 1][0][lane] = acc0;
    red[ks - 1][1][lane] = acc1;
  }
  __syncthreads();
  if (ks > 0) return;
#pragma unroll
  for (int k = 0; k < KS - 1; ++k) {
    const aia::float4_t r0 = red[k][0][lane], r1 = red[k][1][lane];
#pragma unroll
    for (int i = 0; i < 4; ++i) { acc0[i] += r0[i]; acc1[i] += r1[i]; }
  }
  if (t0 + n < a.tokens) {
    uint16_t* dst = a.out + (int64_t)(t0 + n) * a.out_ts + (int64_t)h * a.out_hs + v0 + 4 * g;
    *reinterpret_cast<uint2*>(dst) =
        make_uint2(aia::pack_bf16x2(acc0[0], acc0[1]), aia::pack_bf16x2(acc0[2], acc0[3]));
    *reinterpret_cast<uint2*>(dst + 16) =
        make_uint2(aia::pack_bf16x2(acc1[0], acc1[1]), aia::pack_bf16x2(acc1[2], acc1[3]));
  }
}

bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

extern "C" int aia_mla_kv_latent(const void* ckv_full, int64_t ckv_token_stride, int32_t num_tokens,
                                 const void* norm_weight, float eps, const void* cos,
                                 int64_t cos_token_stride, const void* sin, int64_t sin_token_stride,
                                 void* out, int64_t out_token_stride, void* stream) {
  using namespace aia;
  if (num_tokens < 0) return fail(AIA_ERR_INVALID, "aia_mla_kv_latent: num_tokens %d", num_tokens);
  if (num_tokens == 0) return AIA_OK;
  if (!ckv_full || !norm_weight || !cos || !sin || !out)
    return fail(AIA_ERR_INVALID, "aia_mla_kv_latent: null pointer argument");
  if (ckv_token_stride < kRow || out_token_stride < kRow || ckv_token_stride % 8 ||
      out_token_stride % 8 || cos_token_stride % 4 || sin_token_stride % 4 || !al16(ckv_full) ||
      !al16(out) || !al16(norm_weight) || ((uintptr_t)cos & 7) || ((uintptr_t)sin & 7))
    return fail(AIA_ERR_INVALID, "aia_mla_kv_latent: rows of 576 need 16-byte alignment with "
                "strides a multiple of 8 (cos/sin: 8-byte, stride a multiple of 4)");
  KvArgs a;
  a.ckv = static_cast<const uint16_t*>(ckv_full); a.ckv_ts = ckv_token_stride;
  a.w = static_cast<const uint16_t*>(norm_weight);
  a.cos = static_cast<const uint16_t*>(cos); a.sin = static_cast<const uint16_t*>(sin);
  a.cos_ts = cos_token_stride; a.sin_ts = sin_token_stride;
  a.out = static_cast<uint16_t*>(out); a.out_ts = out_token_stride;
  a.tokens = num_tokens; a.eps = eps;
  mla_kv_latent_kernel<<<(unsigned)((num_tokens + 3) / 4), 256, 0, (hipStream_t)stream>>>(a);
  return check_hip(hipGetLastError(), "mla_kv_latent launch");
}

extern "C" int aia_mla_q_latent(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                                int32_t num_tokens, int32_t num_heads, const void* w_uk_t,
                                const void* cos, int64_t cos_token_stride, const void* sin,
                                int64_t sin_token_stride, void* out, int64_t out_token_stride,
                                int64_t out_head_stride, void* stream) {
  using namespace aia;
  if (num_tokens < 0 || num_heads <= 0 || num_heads > 65535)
    return fail(AIA_ERR_INVALID, "aia_mla_q_latent: bad sizes");
  if (num_tokens == 0) return AIA_OK;
  if (!q || !w_uk_t || !cos || !sin || !out)
    return fail(AIA_ERR_INVALID, "aia_mla_q_latent: null pointer argument");
  if (q_head_stride < kNope + kRope || q_token_stride < (int64_t)num_heads * q_head_stride ||
      q_token_stride % 8 || q_head_stride % 8 || out_head_stride < kRow ||
      out_token_stride < (int64_t)num_heads * out_head_stride || out_token_stride % 4 ||
      out_head_stride % 4 || cos_token_stride % 4 || sin_token_stride % 4 || !al16(q) ||
      !al16(w_uk_t) || ((uintptr_t)out & 7) || ((uintptr_t)cos & 7) || ((uintptr_t)sin & 7))
    return fail(AIA_ERR_INVALID, "aia_mla_q_latent: q rows need 16-byte alignment with strides "
                "a multiple of 8; out / cos / sin 8-byte alignment with strides a multiple of 4");
  QArgs a;
  a.q = static_cast<const uint16_t*>(q); a.q_ts = q_token_stride; a.q_hs = q_head_stride;
  a.wukt = static_cast<const uint16_t*>(w_uk_t);
  a.cos = static_cast<const uint16_t*>(cos); a.sin = static_cast<const uint16_t*>(sin);
  a.cos_ts = cos_token_stride; a.sin_ts = sin_token_stride;
  a.out = static_cast<uint16_t*>(out); a.out_ts = out_token_stride; a.out_hs = out_head_stride;
  a.tokens = num_tokens; a.heads = num_heads;
  const dim3 grid((unsigned)((num_tokens + 15) / 16), (unsigned)num_heads, kLatent / 128);
  mla_q_latent_kernel<<<grid, 256, 0, (hipStream_t)stream>>>(a);
  return check_hip(hipGetLastError(), "mla_q_latent launch");
}

extern "C" int aia_mla_v_up(const void* o_latent, int64_t o_token_stride, int64_t o_head_stride,
                            int32_t num_tokens, int32_t num_heads, const void* w_uv, void* out,
                            int64_t out_token_stride, int64_t out_head_stride, void* stream) {
  using namespace aia;
  if (num_tokens < 0 || num_heads <= 0 || num_heads > 65535)
    return fail(AIA_ERR_INVALID, "aia_mla_v_up: bad sizes");
  if (num_tokens == 0) return AIA_OK;
  if (!o_latent || !w_uv || !out) return fail(AIA_ERR_INVALID, "aia_mla_v_up: null pointer argument");
  if (o_head_stride < kLatent || o_token_stride < (int64_t)num_heads * o_head_stride ||
      o_token_stride % 8 || o_head_stride % 8 || out_head_stride < kNope ||
      out_token_stride < (int64_t)num_heads * out_head_stride || out_token_stride % 4 ||
      out_head_stride % 4 || !al16(o_latent) || !al16(w_uv) || ((uintptr_t)out & 7))
    return fail(AIA_ERR_INVALID, "aia_mla_v_up: o_latent rows need 16-byte alignment with "
                "strides a multiple of 8; out 8-byte alignment with strides a multiple of 4");
  UvArgs a;
  a.o = static_cast<const uint16_t*>(o_latent); a.o_ts = o_token_stride; a.o_hs = o_head_stride;
  a.w = static_cast<const uint16_t*>(w_uv);
  a.out = static_cast<uint16_t*>(out); a.out_ts = out_token_stride; a.out_hs = out_head_stride;
  a.tokens = num_tokens;
  mla_v_up_kernel<<<dim3((unsigned)((num_tokens + 15) / 16), (unsigned)num_heads, 4), 256, 0,
                     (hipStream_t)stream>>>(a);
  return check_hip(hipGetLastError(), "mla_v_up launch");
}
