// HBM read-rate probes for gfx950: the measured ceilings that the decode
// kernels are compared against (bench.py --hbm-sweep).  Not part of the
// product ABI: built into their own library, libaia_probes.so, and loaded
// only by the bench.
//
//   probe_stream_read    every byte of a buffer read once with 16-byte loads,
//                        grid-stride over all CUs, 8 or 16 loads in flight
//                        per thread, plain or non-temporal: the plain
//                        streaming-read rate at a size.
//   probe_paged_gather   the decode kernels' access pattern with no math and
//                        no output: work-group w reads keys [k0, k1) of one
//                        request, `heads` kv heads from head0, K and V rows
//                        of the paged cache at the slots its block table
//                        gives -- the same bytes, in the same pages, as the
//                        attention kernel's range w.
//
// Both fold what they read into one word per work-group, so no load is dead.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int kUnroll = 8;

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load16(const uint4* p, bool nt) {
  if (!nt) return *p;
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// U loads in flight per thread; NT: non-temporal loads (streamed past the
// caches' normal replacement).
template <int U, bool NT>
__global__ __launch_bounds__(1024) void probe_stream_read(const uint4* __restrict__ src, int64_t n16,
                                                          uint32_t* __restrict__ sink) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t acc = 0;
  for (; i + (U - 1) * stride < n16; i += U * stride) {
    uint4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = load16(src + i + u * stride, NT);
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < n16; i += stride) {
    const uint4 v = src[i];
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  for (int d = 32; d >= 1; d >>= 1) acc ^= __shfl_xor(acc, d);
  if ((threadIdx.x & 63) == 0) atomicXor(sink + blockIdx.x, acc);
}

// rec[w] = {request, first key, end key, first kv head}
__global__ __launch_bounds__(1024) void probe_paged_gather(
    const uint4* __restrict__ kc, const uint4* __restrict__ vc, const int4* __restrict__ recs,
    const int32_t* __restrict__ bt, int64_t bt_stride, int32_t bs, int32_t row16,
    int32_t heads, int32_t d16, uint32_t* __restrict__ sink) {
  __shared__ int ids[256];
  const int4 r = recs[blockIdx.x];
  const int b = r.x, k0 = r.y, k1 = r.z, h0 = r.w;
  if (k1 <= k0) return;
  const int blk0 = k0 / bs, nblk = (k1 - 1) / bs - blk0 + 1;
  for (int i = threadIdx.x; i < nblk && i < 256; i += blockDim.x)
    ids[i] = bt[(int64_t)b * bt_stride + blk0 + i];
  __syncthreads();
  const int per_key = heads * d16;               // 16-byte chunks of one key's K (or V)
  const int kpi = blockDim.x / per_key;          // keys per pass of the work-group
  const int kl = threadIdx.x / per_key, c = threadIdx.x - kl * per_key;
  uint32_t acc = 0;
  if (kl < kpi) {
    for (int k = k0 + kl; k < k1; k += kUnroll / 2 * kpi) {
      uint4 v[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll / 2; ++u) {
        const int kk = min(k + u * kpi, k1 - 1);
        const int bi = kk / bs - blk0;
        const int id = ids[bi < 256 ? bi : 255];
        const int64_t off = ((int64_t)id * bs + kk % bs) * row16 + (int64_t)h0 * d16 + c;
        v[2 * u] = kc[off];
        v[2 * u + 1] = vc[off];
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
  }
  for (int d = 32; d >= 1; d >>= 1) acc ^= __shfl_xor(acc, d);
  if ((threadIdx.x & 63) == 0) atomicXor(sink + blockIdx.x, acc);
}

}  // namespace

// variant: bit 0 = 16 loads in flight per thread (else 8), bit 1 =
// non-temporal loads; threads per work-group 256, 512 or 1024.
extern "C" int aia_probe_stream_read(const void* src, int64_t bytes, int32_t grid, int32_t threads,
                                     int32_t variant, void* sink, void* stream) {
  if (!src || !sink || bytes < 16 || grid < 1 || ((uintptr_t)src & 15) || threads < 64 ||
      threads > 1024 || threads % 64)
    return 1;
  const uint4* p = static_cast<const uint4*>(src);
  uint32_t* o = static_cast<uint32_t*>(sink);
  hipStream_t s = (hipStream_t)stream;
  switch (variant & 3) {
    case 0: probe_stream_read<8, false><<<grid, threads, 0, s>>>(p, bytes / 16, o); break;
    case 1: probe_stream_read<16, false><<<grid, threads, 0, s>>>(p, bytes / 16, o); break;
    case 2: probe_stream_read<8, true><<<grid, threads, 0, s>>>(p, bytes / 16, o); break;
    default: probe_stream_read<16, true><<<grid, threads, 0, s>>>(p, bytes / 16, o); break;
  }
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// recs: nrec int4 {request, first key, end key, first kv head} (device);
// caches (num_blocks, bs, hkv, head_dim) bf16; sink: nrec words.
extern "C" int aia_probe_paged_gather(const void* key_cache, const void* value_cache,
                                      const void* recs, int32_t nrec, const int32_t* block_table,
                                      int64_t bt_stride, int32_t bs, int32_t hkv, int32_t head_dim,
                                      int32_t heads, int32_t threads, void* sink, void* stream) {
  if (!key_cache || !value_cache || !recs || !block_table || !sink || nrec < 1 || bs < 1 ||
      head_dim % 8 || heads < 1 || heads > hkv || threads < 64 || threads > 1024 ||
      threads % 64 || heads * head_dim / 8 > threads)
    return 1;
  probe_paged_gather<<<nrec, threads, 0, (hipStream_t)stream>>>(
      static_cast<const uint4*>(key_cache), static_cast<const uint4*>(value_cache),
      static_cast<const int4*>(recs), block_table, bt_stride, bs, hkv * head_dim / 8, heads,
      head_dim / 8, static_cast<uint32_t*>(sink));
  return hipGetLastError() == hipSuccess ? 0 : 2;
}
