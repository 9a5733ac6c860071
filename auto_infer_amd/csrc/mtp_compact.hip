// On-device MTP verify compaction: accepted draft counts and the packing of
// each request's confirmed target rows, in request order, for the drafter.
//
// Reference: GraphMtpRunner._target_body (auto_infer/worker/
// graph_mtp_runner.py:211-248).  For a gear of g requests with query width
// w = draft depth + 1:
//   accepted[r] = sum_j prod_{i<=j} (drafts[r][i] == preds[r][i])   (j < w-1)
//                 times active[r]
//   length[r]   = active[r] * (1 + accepted[r]),  start = exclusive cumsum
//   for each destination row d < g*w:
//     owner  = #{r : start[r] <= d} - 1 (at least 0)
//     source = clamp(w * owner + d - start[owner], 0, g*w - 1)
//     valid  = d < sum(length)
//     hidden[d] = valid ? h[source] : 0;   tokens[d] = valid ? preds[source] : 0
//     positions[d] = valid ? pos[source] : scratch_pos[d]
//     slots[d]     = valid ? slot[source] : scratch_slot[d]
// The valid rows are confirmed_layout's source rows (spec_decode/layout.py:
// 17-43).  The reference runs this as a chain of ~15 torch ops; here it is
// one launch: every work-group recomputes the (tiny) per-request counts in
// its first wave (lane r = request r, gear <= 64), then copies its row.
#include "common.h"

namespace {

constexpr int kMaxGear = 64;

struct CompactArgs {
  const int64_t* preds;          // [g][w]
  const int64_t* drafts;         // [g][w-1]
  const int32_t* active;         // [g]
  const uint16_t* hidden;        // [g*w][H], row stride h_rs
  int64_t h_rs;
  const int64_t* positions;      // [g*w]
  const int32_t* slots;          // [g*w]
  const int64_t* scratch_positions;
  const int32_t* scratch_slots;
  int32_t g, w, hdim;
  int64_t* accepted;             // [g]
  uint16_t* out_hidden;          // [g*w][H], row stride oh_rs
  int64_t oh_rs;
  int64_t* out_tokens;
  int64_t* out_positions;
  int32_t* out_slots;
};

__global__ __launch_bounds__(256) void mtp_compact_kernel(CompactArgs a) {
  __shared__ int s_source, s_valid;
  const int d = blockIdx.x;
  if (threadIdx.x < 64) {
    const int r = threadIdx.x;
    int acc = 0, len = 0;
    if (r < a.g) {
      int run = 1;
      for (int j = 0; j < a.w - 1; ++j) {
        run &= a.drafts[(int64_t)r * (a.w - 1) + j] == a.preds[(int64_t)r * a.w + j] ? 1 : 0;
        acc += run;
      }
      acc *= a.active[r];
      len = a.active[r] * (1 + acc);
    }
    // inclusive scan of the lengths across the wave
    int inc = len;
#pragma unroll
    for (int k = 1; k < 64; k <<= 1) {
      const int y = __shfl_up(inc, k);
      if (r >= k) inc += y;
    }
    const int start = inc - len;
    const int total = __shfl(inc, 63);
    // owner = #{r : start[r] <= d} - 1 over the g requests
    const unsigned long long le = __ballot(r < a.g && start <= d);
    const int owner = max(__popcll(le) - 1, 0);
    const int ostart = __shfl(start, owner);
    if (r == 0) {
      s_source = min(max(a.w * owner + d - ostart, 0), a.g * a.w - 1);
      s_valid = d < total;
    }
    if (d == 0 && r < a.g) a.accepted[r] = acc;
  }
  __syncthreads();
  const int src = s_source;
  const bool valid = s_valid;
  if (threadIdx.x == 0) {
    a.out_tokens[d] = valid ? a.preds[src] : 0;
    a.out_positions[d] = valid ? a.positions[src] : a.scratch_positions[d];
    a.out_slots[d] = valid ? a.slots[src] : a.scratch_slots[d];
  }
  const uint16_t* hs = a.hidden + (int64_t)src * a.h_rs;
  uint16_t* hd = a.out_hidden + (int64_t)d * a.oh_rs;
  if ((a.hdim & 7) == 0) {
    for (int c = threadIdx.x * 8; c < a.hdim; c += 256 * 8)
      *reinterpret_cast<uint4*>(hd + c) =
          valid ? *reinterpret_cast<const uint4*>(hs + c) : make_uint4(0, 0, 0, 0);
  } else {
    for (int c = threadIdx.x; c < a.hdim; c += 256) hd[c] = valid ? hs[c] : 0;
  }
}

}  // namespace

extern "C" int aia_mtp_compact(const int64_t* preds, const int64_t* drafts,
                               const int32_t* active_mask, const void* hidden,
                               int64_t hidden_row_stride, const int64_t* positions,
                               const int32_t* slots, const int64_t* scratch_positions,
                               const int32_t* scratch_slots, int32_t gear, int32_t query_width,
                               int32_t hidden_dim, int64_t* accepted, void* out_hidden,
                               int64_t out_hidden_row_stride, int64_t* out_tokens,
                               int64_t* out_positions, int32_t* out_slots, void* stream) {
  using namespace aia;
  if (gear <= 0 || gear > kMaxGear || query_width < 2 || hidden_dim <= 0)
    return fail(AIA_ERR_INVALID, "aia_mtp_compact: gear %d must be in [1, %d], query_width %d >= 2",
                gear, kMaxGear, query_width);
  if (!preds || !drafts || !active_mask || !hidden || !positions || !slots || !scratch_positions ||
      !scratch_slots || !accepted || !out_hidden || !out_tokens || !out_positions || !out_slots)
    return fail(AIA_ERR_INVALID, "aia_mtp_compact: null pointer argument");
  if (hidden_row_stride < hidden_dim || out_hidden_row_stride < hidden_dim)
    return fail(AIA_ERR_INVALID, "aia_mtp_compact: row strides shorter than hidden_dim");
  if ((hidden_dim & 7) == 0 &&
      (((uintptr_t)hidden & 15) || ((uintptr_t)out_hidden & 15) || (hidden_row_stride & 7) ||
       (out_hidden_row_stride & 7)))
    return fail(AIA_ERR_INVALID, "aia_mtp_compact: hidden rows must be 16-byte aligned");
  CompactArgs a;
  a.preds = preds; a.drafts = drafts; a.active = active_mask;
  a.hidden = static_cast<const uint16_t*>(hidden); a.h_rs = hidden_row_stride;
  a.positions = positions; a.slots = slots;
  a.scratch_positions = scratch_positions; a.scratch_slots = scratch_slots;
  a.g = gear; a.w = query_width; a.hdim = hidden_dim;
  a.accepted = accepted;
  a.out_hidden = static_cast<uint16_t*>(out_hidden); a.oh_rs = out_hidden_row_stride;
  a.out_tokens = out_tokens; a.out_positions = out_positions; a.out_slots = out_slots;
  mtp_compact_kernel<<<gear * query_width, 256, 0, (hipStream_t)stream>>>(a);
  return check_hip(hipGetLastError(), "mtp_compact launch");
}
