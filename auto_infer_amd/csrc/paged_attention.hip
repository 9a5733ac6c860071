// Paged attention for gfx950: GQA (head_dim 128 and 64) and absorbed MLA.
//
// Kernels:
//   plan_kernel         one work-group per step.  Turns (cu_seqlens_q,
//                       seqlens_kv) into segments (request, kv-head group,
//                       head block, query block) with their 16-key tiles and
//                       cuts the concatenated tile list into equal contiguous
//                       ranges (balanced split-K: every range streams the same
//                       number of KV bytes whatever the context-length mix).
//                       Requests whose query rows fill 128-row items go to the
//                       prefill units instead.  It also lists the merge work.
//   gqa_attn_kernel     split-K decode and verify rows, one wave per (range,
//                       kv head).  K rows go straight from HBM into MFMA
//                       fragments (S^T = K Q^T), online softmax on the S^T
//                       registers, V^T through LDS, O^T += V^T P^T with P^T
//                       taken from the S^T registers.  A wave that covers a
//                       whole segment writes bf16 output, otherwise an fp32
//                       partial (O, m, l).
//   gqa_prefill_kernel  prefill units: 128 query rows per work-group, 64-key
//                       K/V tiles loaded straight into LDS and used by all of
//                       them, QK^T and PV on MFMA.  A unit that covers only
//                       part of its item's keys writes an fp16 partial scaled
//                       per row.
//   gqa_mixed_kernel    both roles in one grid (Hkv = 4), so the compute-bound
//                       units run beside the HBM-bound ranges.
//   mla_attn_kernel     absorbed MLA over one latent cache (576-wide keys, V =
//                       their first 512 dims), four waves per range.
//   merge_kernel        log-sum-exp merge of the split segments and cut items.
#include <math.h>

#include <atomic>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <type_traits>

#include "common.h"

namespace {

using aia::float4_t;
using aia::short4_t;

constexpr int kHeadDim = 128;
constexpr int kTile = 16;         // keys per MFMA tile
constexpr int kRows = 16;         // query rows per segment (MFMA N)
// LDS row stride (elements) of a staged V tile: 288 bytes puts the 16 rows
// of a transposing read in distinct banks
constexpr int kVStride = 144;
constexpr int kMaxBatch = 8192;   // planner keeps the request offsets in LDS
constexpr int kDefaultWaves = 2048;
constexpr int kMaxWaves = 16384;
constexpr int kPlanThreads = 512;
// Per-range work record: {segment, first tile, end tile, tiles per range,
// the segment's 8-int record, first logical block, last segment of the
// range, 2 pad, the first 16 block ids of the range} -- everything a
// work-group needs to issue its first K/V loads after one load.
constexpr int kRecInts = 32;
constexpr int kRecBlocks = 16;

constexpr int kMaxGroupWaves = 8;  // kv heads (waves) per work-group

// A segment is (request, query block, kv-head group, head block): the
// work-group that owns one of its key ranges runs one wave per kv head of
// the group over the same keys, so every tile reads whole contiguous
// (block_size x Hkv x D) cache slots.
struct Geometry {
  int32_t hkv, group, hb, nhb, qb, nw, nkvg, rb, qs, pf;
  int32_t ncu;   // compute units of the current device (MLA range count and dealing)
};

// Compute units of the current device, queried once per device (256, the
// MI355X's count, when no device is visible, e.g. a size query on a host
// without a GPU).
constexpr int kMaxCuDevices = 64;
std::atomic<int> g_device_cus[kMaxCuDevices];
int32_t device_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxCuDevices) {
    (void)hipGetLastError();
    return 256;
  }
  int n = g_device_cus[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0) {
      (void)hipGetLastError();
      return 256;
    }
    g_device_cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Prefill routing: a GQA request whose query rows (query tokens x group
// heads) fill at least one prefill work item is planned for the prefill
// kernel (all its rows' keys staged once per 128 rows in LDS) instead of
// split-K segments.  AIA_PREFILL=0 builds the split-K-only planner.
#ifndef AIA_PREFILL
#define AIA_PREFILL 1
#endif
// AIA_MLA_PREFILL=0 keeps absorbed-MLA prefill steps on the split-K kernel.
#ifndef AIA_MLA_PREFILL
#define AIA_MLA_PREFILL 1
#endif
#ifndef AIA_PF_WAVES
#define AIA_PF_WAVES 4
#endif
#ifndef AIA_PF_KEYS
#define AIA_PF_KEYS 64
#endif
#ifndef AIA_PF_RT
#define AIA_PF_RT 2
#endif
constexpr int kPfWaves = AIA_PF_WAVES;       // waves per prefill work-group
constexpr int kPfRt = AIA_PF_RT;             // 16-row MFMA tiles per wave
constexpr int kPfRows = 16 * kPfRt * kPfWaves;   // rows per prefill work item
constexpr int kPfKeys = AIA_PF_KEYS;         // keys per staged K/V tile (32 or 64)
// Items alone fill the chip when items x kv heads reach kPfTargetWgs (a
// little under two resident work-groups per CU); below that, each item's key
// tiles are cut into chunks of at least kPfMinChunk tiles, sized so all units
// still fit in one round (fp16 partials scaled per row, merged with the
// split-K partials' rule).  448 rather than 512: fewer, longer chunks write
// fewer partials, and the CUs left with one work-group take the largest
// units (configs[1] prefill chunks, us per call: 43.1 at 448 or 416, 44.6 at
// 512, 44.1-44.5 at 384, 49.6-49.9 at 256-320; 416 is slower at 32K keys).
#ifndef AIA_PF_TARGET
#define AIA_PF_TARGET 448
#endif
constexpr int kPfTargetWgs = AIA_PF_TARGET;
#ifndef AIA_MLA_LPT
#define AIA_MLA_LPT 1
#endif

constexpr int kPfMinChunk = 8;

constexpr int64_t kMlaRb2Rows = 2048;

// rb: row blocks (of 16 query rows) per segment.  Two when a GQA launch's
// requests average more query tokens than one block holds (prefill chunks),
// so each K/V tile feeds 32 rows; one for decode and short verify steps.
// MLA gets two on steps with more tokens than requests and at least
// kMlaRb2Rows query rows.  Planner and kernels derive it from the same
// (heads, batch, tokens, head_dim_v), so they always agree.
Geometry geometry(int32_t hq, int32_t hkv, int32_t batch, int32_t tokens, int32_t dv) {
  Geometry g;
  g.hkv = hkv;
  g.group = hq / hkv;
  g.hb = g.group < kRows ? g.group : kRows;            // query heads per segment
  g.nhb = (g.group + g.hb - 1) / g.hb;                 // head blocks per kv head
  g.qb = kRows / g.hb;                                  // query tokens per segment
  g.nw = hkv < kMaxGroupWaves ? hkv : kMaxGroupWaves;   // waves per work-group
  g.nkvg = (hkv + g.nw - 1) / g.nw;                     // kv-head groups
  // Prefill routing is possible when some request can hold a full item of
  // rows: with at least one query token per request, none holds more than
  // tokens - batch + 1.  (The planner routes nothing when this says no, so a
  // batch that breaks the assumption still runs, on split-K.)
  // (absorbed MLA, whose 16 heads fill an item with 8 tokens, also needs an
  // average of 4 tokens per request, so verify steps of 2 or 3 make no
  // prefill launch that would find nothing routed)
  g.pf = (AIA_PREFILL && (dv == kHeadDim || dv == 64 || (dv == 512 && AIA_MLA_PREFILL)) &&
          batch > 0 && ((int64_t)tokens - batch + 1) * g.group >= kPfRows &&
          (dv != 512 || tokens >= 4LL * batch)) ? 1 : 0;
  // with prefill routing, requests with many query rows leave the split-K
  // kernel, whose segments are then decode / short-verify sized
  // (MLA, dv 512: a token's heads fill a block.  Two blocks halve the
  // latent reads per row but run two waves per SIMD instead of three, which
  // only pays once the step has kMlaRb2Rows query rows to fill the chip;
  // short verify steps of a few dozen requests stay at one block.)
  const bool mla_rb2 = dv == 512 && (int64_t)tokens * hq >= kMlaRb2Rows;
  g.rb = ((!g.pf && (dv == kHeadDim || dv == 64)) || mla_rb2) && tokens > (int64_t)batch * g.qb
             ? 2 : 1;
  g.qs = g.qb * g.rb;                                   // query tokens per segment
  g.ncu = device_cus();
  return g;
}

// Workspace layout (all offsets 256-byte aligned).
struct Layout {
  int64_t hdr, seg, wave, part_ml, part_o, req, mrg, pf, pfm, pfw, pf_o, pf_ml, total;
  int64_t seg_cap, part_cap, mrg_cap, pf_cap, pf_unit_cap, pf_mrg_cap, pf_slots;
};

constexpr int kMergeDims = 16;   // output dims per merge element
constexpr int kMrgInts = 8;      // merge record

// Merge slices (64 elements of kMergeDims dims) per (segment, kv head) at most.
int64_t merge_slices(const Geometry& g, int32_t dv) {
  return ((int64_t)kRows * g.rb * (dv / kMergeDims) + 63) / 64;
}

int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

// Fixed partial slots.  In a small step (the geometry the small planner
// serves, whose partial buffer is sized for kFixParts slots per segment)
// whose segments are each split over at most kFixParts ranges, segment s
// writes its partials to slots [kFixParts s, kFixParts s + np): the merge
// work-group of (segment, kv head) then knows where its partials are without
// reading a merge record, and issues those loads together with the
// header's, one round trip instead of two.  hdr[10] = 1 marks such a plan.
// Both planners decide it the same way, from the slot capacity the host
// passes (fix_cap, 0 outside the geometry) and the ranges.
constexpr int kFixParts = 32;
#ifndef AIA_FIX_WAVES
#define AIA_FIX_WAVES 2
#endif
constexpr int kFixWaves = AIA_FIX_WAVES;   // waves of a fixed-slot merge work-group
constexpr int kSmallPlanSegs = 64;

// The geometry of small steps: GQA without prefill routing, at most 64
// requests and segments.  Their plans may use fixed partial slots (see
// kFixParts), whichever planner makes them.
bool small_geometry(const Geometry& g, int32_t dv, int32_t batch, int64_t seg_cap) {
  return dv != 512 && !g.pf && batch >= 1 && batch <= 64 && seg_cap <= kSmallPlanSegs;
}


Layout layout(int32_t batch, int32_t tokens, const Geometry& g, int32_t dv, int32_t waves) {
  Layout L;
  L.seg_cap = (int64_t)g.nkvg * g.nhb * (batch + (tokens + g.qs - 1) / g.qs);
  L.part_cap = L.seg_cap + waves;
  // small steps: room for the fixed partial slots too
  if (small_geometry(g, dv, batch, L.seg_cap) && L.part_cap < kFixParts * L.seg_cap)
    L.part_cap = kFixParts * L.seg_cap;
  int64_t off = 0;
  L.hdr = off;      off = align256(off + 64 * 4);
  L.seg = off;      off = align256(off + (L.seg_cap + 1) * 8 * 4);
  L.wave = off;     off = align256(off + (int64_t)waves * kRecInts * 4);
  L.part_ml = off;  off = align256(off + L.part_cap * g.nw * kRows * g.rb * 8);
  // split partials are fp16, scaled per row
  L.part_o = off;   off = align256(off + L.part_cap * g.nw * kRows * g.rb * (int64_t)dv * 2);
  L.mrg_cap = L.seg_cap * g.nw * merge_slices(g, dv);
  L.mrg = off;      off = align256(off + L.mrg_cap * kMrgInts * 4);
  L.req = off;      off = align256(off + ((int64_t)batch + 1) * 8);   // request and item offsets
  // prefill items: a routed request has >= kPfRows rows, so at most
  // rows / kPfRows of them, each adding at most one partial item
  const int64_t pf_rows = g.pf ? (int64_t)tokens * g.group : 0;
  const int64_t pf_reqs = pf_rows / kPfRows < batch ? pf_rows / kPfRows : batch;
  L.pf_cap = (pf_rows + kPfRows - 1) / kPfRows + pf_reqs;
  // Chunked items exist only when items x kv heads < kPfTargetWgs; then the
  // units number at most items + total tiles / chunk < 2 kPfTargetWgs / Hkv.
  const int64_t split_units = g.pf ? 2 * ((kPfTargetWgs + g.hkv - 1) / g.hkv) + 1 : 0;
  L.pf_unit_cap = L.pf_cap > split_units ? L.pf_cap : split_units;
  L.pf_mrg_cap = g.pf ? (kPfTargetWgs + g.hkv - 1) / g.hkv : 0;
  L.pf_slots = split_units * g.hkv;             // partial row blocks
  L.pf = off;       off = align256(off + L.pf_unit_cap * 32);              // two int4 per unit
  L.pfm = off;      off = align256(off + L.pf_mrg_cap * 16);
  L.pfw = off;      off = align256(off + (g.pf ? kPfTargetWgs * 48 : 0));   // dealt work-groups
  L.pf_ml = off;    off = align256(off + L.pf_slots * kPfRows * 8);
  L.pf_o = off;     off = align256(off + L.pf_slots * kPfRows * (int64_t)dv * 2);
  L.total = off;
  return L;
}

// Number of key ranges (= work-groups).  Default: about kDefaultWaves waves
// in flight for GQA (one per kv head of a group), three four-wave groups per
// CU (768 on the MI355X) for the 576-wide MLA latent.
constexpr int kMlaRangesPerCu = 3;
int32_t resolve_waves(int32_t w, const Geometry& g, int32_t dv) {
  if (w <= 0) w = dv == 512 ? kMlaRangesPerCu * g.ncu : (kDefaultWaves + g.nw - 1) / g.nw;
  if (w > kMaxWaves) w = kMaxWaves;
  return w;
}

// ---------------------------------------------------------------- planner

constexpr int kXcdsPlan = 8;      // XCDs the hardware deals work-groups to, round-robin

// Inclusive prefix sum over the 64 lanes of a wave with DPP moves (VALU
// only, no LDS crossbar round trips): shifts by 1, 2, 4, 8 within each row of
// 16 lanes (lanes shifted in from outside the row read 0), then row 0's last
// lane is added to row 1 and row 2's to row 3 (row_bcast:15), and lane 31's
// total to rows 2 and 3 (row_bcast:31).  Rows a broadcast does not write keep
// the 0 passed as the old value.
__device__ __forceinline__ int wave_incl_scan(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, true);   // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, true);   // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, true);   // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, true);   // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return x;
}

// Exclusive scan of one value per thread across the planner work-group;
// returns the exclusive prefix and writes the block total to *total.
__device__ int block_exclusive_scan(int v, int* wave_sums, int* total) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int x = wave_incl_scan(v);
  if (lane == 63) wave_sums[wid] = x;
  __syncthreads();
  if (wid == 0) {
    const int s = wave_incl_scan(lane < kPlanThreads / 64 ? wave_sums[lane] : 0);
    if (lane < kPlanThreads / 64) wave_sums[lane] = s;  // inclusive
  }
  __syncthreads();
  const int before = wid ? wave_sums[wid - 1] : 0;
  *total = wave_sums[kPlanThreads / 64 - 1];
  __syncthreads();
  return before + x - v;
}

// The same for two values at once (one pass of barriers instead of two).
__device__ int2 block_exclusive_scan2(int2 v, int2* wave_sums2, int2* total) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int2 x = make_int2(wave_incl_scan(v.x), wave_incl_scan(v.y));
  if (lane == 63) wave_sums2[wid] = x;
  __syncthreads();
  if (wid == 0) {
    const int2 w = lane < kPlanThreads / 64 ? wave_sums2[lane] : make_int2(0, 0);
    const int2 s = make_int2(wave_incl_scan(w.x), wave_incl_scan(w.y));
    if (lane < kPlanThreads / 64) wave_sums2[lane] = s;  // inclusive
  }
  __syncthreads();
  const int2 before = wid ? wave_sums2[wid - 1] : make_int2(0, 0);
  *total = wave_sums2[kPlanThreads / 64 - 1];
  __syncthreads();
  return make_int2(before.x + x.x - v.x, before.y + x.y - v.y);
}

// Segment record, 8 ints: b, kv-head group | head block << 16 | (last query
// block of its request) << 30, first query
// token (global row), query tokens | q0 << 8 (q0 = first query of the block
// within its request), lim_base = Lk - Lq + q0 (last key of the block's first
// row), tile_begin, tile_end, part_base.
//
// The planner keeps the request metadata (request offsets, cu_seqlens_q,
// seqlens_kv) and later the segments' first tiles in LDS, and each thread
// keeps its own segments' tile counts in registers, so its phases cost one
// global round trip each (metadata in, block ids in) rather than one per
// dependent lookup.
constexpr int kPlanLds = 12288;          // ints of LDS scratch (48 KB)
constexpr int kPlanRegChunks = 2;        // segments kept in registers: 2 x 512
#ifndef AIA_PAD_BELOW
#define AIA_PAD_BELOW 16
#endif
constexpr int kPadBelow = AIA_PAD_BELOW;  // pad segments when ranges are shorter (tiles)


// Padded MLA plans: a request's tiles are split over its ranges evenly
// (sizes floor / ceil of nt / k, never crossing requests) and the ranges are
// dealt to work-group slots by size in a snake order over the CUs' slots
// (slots w, w + ncu, w + 2 ncu share a CU: work-groups go out one per CU per
// round), so every CU gets about the mean number of tiles.
#ifndef AIA_MLA_BALANCE
#define AIA_MLA_BALANCE 1
#endif

// Range placement over the segments' first tiles held in LDS (tb[0..nseg]):
// the last segment with first tile <= t0, and from it (galloping, then a
// bracket search) the last segment with first tile < t1.
__device__ __forceinline__ int range_first_seg(const int* tb, int nseg, int t0) {
  int lo = 0, hi = nseg - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (tb[mid] <= t0) lo = mid; else hi = mid - 1;
  }
  return lo;
}
__device__ __forceinline__ int range_last_seg(const int* tb, int nseg, int lo, int t1) {
  int lo2 = lo, step = 1;
  while (lo2 + step < nseg && tb[lo2 + step] < t1) { lo2 += step; step <<= 1; }
  int hi2 = min(nseg - 1, lo2 + step - 1);
  while (lo2 < hi2) {
    const int mid = (lo2 + hi2 + 1) >> 1;
    if (tb[mid] < t1) lo2 = mid; else hi2 = mid - 1;
  }
  return lo2;
}

__global__ __launch_bounds__(kPlanThreads) void plan_kernel(
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ kvlen,
    const int32_t* __restrict__ block_table, int64_t bt_stride, int32_t block_size,
    int32_t batch, Geometry g, int32_t waves, int32_t dv,
    int32_t* __restrict__ hdr, int32_t* __restrict__ seg, int32_t* __restrict__ wave_rec,
    int32_t* __restrict__ req_scratch,
    int32_t* __restrict__ mrg, int4* __restrict__ pf_units, int4* __restrict__ pf_mrg,
    int4* __restrict__ pf_wg, int32_t pf_cap, int32_t pf_unit_cap, int32_t pf_mrg_cap,
    int32_t seg_cap, int32_t fix_cap) {
  __shared__ __attribute__((aligned(16))) int lds[kPlanLds];
  __shared__ int wave_sums[kPlanThreads / 64];
  __shared__ int2 wave_sums2[kPlanThreads / 64];
  __shared__ int pf_hist[64];
  const int tid = threadIdx.x;
  const int per_req = g.nkvg * g.nhb;
  // request metadata in LDS when it fits, else in the workspace / inputs
  const bool req_lds = 4 * (batch + 1) <= kPlanLds;
  int* req_off = req_lds ? lds : req_scratch;
  int* cuv = req_lds ? lds + (batch + 1) : nullptr;
  int* kvv = req_lds ? lds + 2 * (batch + 1) : nullptr;
  int* item_off = req_lds ? lds + 3 * (batch + 1) : req_scratch + (batch + 1);

  // 1) segments per request -> request offsets; prefill-routed requests
  // get no segments and list their prefill items instead (last rows first:
  // under the causal mask they see the most keys)
  int carry = 0, pcarry = 0;
  for (int base = 0; base < batch; base += kPlanThreads) {
    const int b = base + tid;
    int cnt = 0, pcnt = 0;
    if (b < batch) {
      const int c0 = cu_q[b], c1 = cu_q[b + 1], lk = kvlen[b];
      if (req_lds) {
        cuv[b] = c0; kvv[b] = lk;
        if (b == batch - 1) cuv[batch] = c1;
      }
      const int lq = c1 - c0;
      if (g.pf && (int64_t)lq * g.group >= kPfRows)
        pcnt = (lq * g.group + kPfRows - 1) / kPfRows;
      else
        cnt = lq > 0 ? ((lq + g.qs - 1) / g.qs) * per_req : 0;
    }
    int2 tot2;
    const int2 ex2 = block_exclusive_scan2(make_int2(cnt, pcnt), wave_sums2, &tot2);
    if (b < batch) {
      req_off[b] = carry + ex2.x;
      item_off[b] = pcarry + ex2.y;
    }
    carry += tot2.x;
    pcarry += tot2.y;
  }
  // Query lengths that do not sum to the step's token count can ask for
  // more work than the workspace was sized for: plan nothing rather than
  // write past it.
  int overflow = 0;
  if (carry > seg_cap || pcarry > pf_cap) { carry = 0; pcarry = 0; overflow = 1; }
  if (tid == 0) req_off[batch] = carry;

  // 1b) prefill units.  Items are listed per request, last rows first (under
  // the causal mask they see the most keys).  When items x kv heads leave
  // the chip underfilled, an item's tiles are cut into k balanced chunks of
  // about `chunk` tiles; its k units write partials and get a merge record.
  // Every loop below runs over the flat item list (request-major, each
  // request's items last rows first), one item per thread.
  int units = 0, pmerges = 0, dealt = 0;
  // Fill target.  Absorbed-MLA units (158 KB of LDS) run one per CU: few
  // items are cut into one round of units (8 x 64 tokens at 4096 keys: 172
  // us against 205 at 448), many into about 1.75 rounds so the causal
  // items even out (1 x 2048 tokens: 218 against 280 at one round).
  const int pf_target = dv != 512 || g.ncu <= 0 || g.ncu >= kPfTargetWgs ? kPfTargetWgs
                        : (int64_t)pcarry * g.hkv <= g.ncu / 2 ? g.ncu : kPfTargetWgs;
  if (pcarry > 0) {
    __syncthreads();   // item offsets
    const int* cu_p = req_lds ? cuv : cu_q;
    const int* kv_p = req_lds ? kvv : kvlen;
    // item f: its request, first row and key tiles
    auto item_at = [&](int f, int& b, int& r0) {
      int lo = 0, hi = batch - 1;  // last b with item_off[b] <= f
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (item_off[mid] <= f) lo = mid; else hi = mid - 1;
      }
      b = lo;
      const int lq = cu_p[b + 1] - cu_p[b], lk = kv_p[b];
      const int nitems = (lq * g.group + kPfRows - 1) / kPfRows;
      r0 = (nitems - 1 - (f - item_off[b])) * kPfRows;
      const int last = min(lq * g.group, r0 + kPfRows) - 1;
      const int kend = max(0, min(lk, lk - lq + last / g.group + 1));
      return (kend + kPfKeys - 1) / kPfKeys;
    };
    int chunk = 0x7fffffff;
    if ((int64_t)pcarry * g.hkv < pf_target) {
      int mine = 0;
      for (int f = tid; f < pcarry; f += kPlanThreads) {
        int b, r0;
        mine += item_at(f, b, r0);
      }
      int wtot;
      block_exclusive_scan(mine, wave_sums, &wtot);
      // sum_i ceil(nt_i / c) <= W / c + P, so c = W Hkv / (target - P Hkv)
      // keeps units x kv heads within the target: one round of work-groups
      const int64_t room = pf_target - (int64_t)pcarry * g.hkv;
      chunk = max(kPfMinChunk, (int)(((int64_t)wtot * g.hkv + room - 1) / room));
      // That bound is loose.  In a step with no split-K segments the least
      // chunk whose units still fit evens the work-groups out (the slowest
      // one sets the kernel time), found by a binary search, one block
      // reduction per probe.  Beside split-K ranges the loose bound stays:
      // its fewer work-groups leave slots for the HBM-bound ranges.
      const int ucap = pf_target / g.hkv;
      int lo = carry > 0 ? chunk : max(kPfMinChunk, (wtot + ucap - 1) / ucap);
      while (lo < chunk) {
        const int mid = (lo + chunk) >> 1;
        int nu = 0;
        for (int f = tid; f < pcarry; f += kPlanThreads) {
          int b, r0;
          const int nt = item_at(f, b, r0);
          nu += nt > mid ? (nt + mid - 1) / mid : 1;
        }
        int utot;
        block_exclusive_scan(nu, wave_sums, &utot);
        if (utot <= ucap) chunk = mid; else lo = mid + 1;
      }
    }
    int ucarry = 0, mcarry2 = 0;
    for (int base = 0; base < pcarry; base += kPlanThreads) {
      const int f = base + tid;
      int b = 0, r0 = 0, nt = 0, k = 0;
      if (f < pcarry) {
        nt = item_at(f, b, r0);
        k = nt > chunk ? (nt + chunk - 1) / chunk : 1;
      }
      int2 tot2;
      const int2 ex2 = block_exclusive_scan2(make_int2(k, k > 1 ? 1 : 0), wave_sums2, &tot2);
      const int u = ucarry + ex2.x, mm = mcarry2 + ex2.y;
      if (f < pcarry && u + k <= pf_unit_cap && mm + (k > 1) <= pf_mrg_cap) {
        if (k > 1) {
          // {first query token, first row, first unit, units | item rows << 16}
          const int c0 = req_lds ? cuv[b] : cu_q[b];
          const int c1 = req_lds ? cuv[b + 1] : cu_q[b + 1];
          const int rows = min(kPfRows, (c1 - c0) * g.group - r0);
          pf_mrg[mm] = make_int4(c0, r0, u, k | (rows << 16));
        }
        // unit record: {request, first row, first tile, end tile}, then
        // {first query token, query tokens, keys, block id of the first
        // tile}, so a work-group starts its Q and first-tile loads as soon
        // as its record arrives (the id serves block sizes that are a
        // multiple of the tile)
        const int c0 = cu_p[b], lqb = cu_p[b + 1] - c0, lkb = kv_p[b];
        const int32_t* btr = block_table + (int64_t)b * bt_stride;
        for (int j = 0; j < k; ++j) {
          const int tj = (int)((int64_t)j * nt / k);
          pf_units[2 * (u + j)] = make_int4(b, r0, tj, (int)((int64_t)(j + 1) * nt / k));
          pf_units[2 * (u + j) + 1] = make_int4(c0, lqb, lkb, btr[(tj * kPfKeys) / block_size]);
        }
      }
      ucarry += tot2.x;
      mcarry2 += tot2.y;
    }
    units = ucarry;
    pmerges = mcarry2;
    if (units > pf_unit_cap || pmerges > pf_mrg_cap) { units = 0; pmerges = 0; overflow = 1; }

    // 1c) Work-group b's record at pf_wg[b]: its unit record (two int4),
    // then {unit, kv head}, so a work-group loads it beside the header
    // instead of after it; hdr[9] = the number written (0: too many
    // work-groups, they read the unit list).  When a step has only prefill
    // work-groups and they fit one round, two per CU (the hardware puts
    // work-groups b and b + ncu on one CU then), they are dealt by size so
    // every CU's pair sums evenly: the largest units alone on the CUs
    // without a partner, then the i-th largest of the rest beside the i-th
    // smallest.  Otherwise b takes (kv head, unit) pair xcd_range(b, pairs):
    // each XCD gets a contiguous run of pairs, kv-head major, so the items
    // that re-read one request's keys for one kv head share an XCD's L2.
    const int jobs = units * g.hkv;
    // Absorbed-MLA units run one per CU: in more than one round the next
    // work-group goes to whichever CU frees first, so they are dealt largest
    // first (the longest-processing-time order).
    const bool lpt = dv == 512 && AIA_MLA_LPT;
    const bool pair_deal = !lpt && carry == 0 && jobs > g.ncu && jobs <= 2 * g.ncu;
    if (jobs <= pf_target && !pair_deal && !lpt) {
      __syncthreads();   // publishes pf_units to the whole group
      const int q = jobs / kXcdsPlan, r = jobs - q * kXcdsPlan;
      for (int id = tid; id < jobs; id += kPlanThreads) {
        const int x = id % kXcdsPlan, i = id / kXcdsPlan;
        const int pair = x * q + min(x, r) + i;          // xcd_range(id, jobs)
        const int kvh = pair / units, u = pair - kvh * units;
        pf_wg[3 * id] = pf_units[2 * u];
        pf_wg[3 * id + 1] = pf_units[2 * u + 1];
        pf_wg[3 * id + 2] = make_int4(u, kvh, 0, 0);
      }
      dealt = jobs;
    }
    if ((pair_deal || lpt) && jobs <= pf_target) {
      if (tid < 64) pf_hist[tid] = 0;
      __syncthreads();   // also publishes pf_units to the whole group
      for (int p = tid; p < jobs; p += kPlanThreads) {
        const int4 e = pf_units[2 * (p % units)];
        atomicAdd(&pf_hist[63 - min(e.w - e.z, 63)], 1);   // bucket 0: the largest
      }
      __syncthreads();
      if (tid == 0) {
        int acc = 0;
        for (int k = 0; k < 64; ++k) { const int c = pf_hist[k]; pf_hist[k] = acc; acc += c; }
      }
      __syncthreads();
      const int n2 = jobs - g.ncu, lone = g.ncu - n2;
      for (int p = tid; p < jobs; p += kPlanThreads) {
        const int u = p % units, kvh = p / units;
        const int4 e = pf_units[2 * u];
        const int r = atomicAdd(&pf_hist[63 - min(e.w - e.z, 63)], 1);
        const int i = r - lone;
        const int id = lpt ? r : r < lone ? n2 + r : i < n2 ? i : g.ncu + (jobs - 1 - r);
        pf_wg[3 * id] = e;
        pf_wg[3 * id + 1] = pf_units[2 * u + 1];
        pf_wg[3 * id + 2] = make_int4(u, kvh, 0, 0);
      }
      dealt = jobs;
    }
  }
  __syncthreads();
  const int nseg = req_off[batch];
  const int* cu_r = req_lds ? cuv : cu_q;
  const int* kv_r = req_lds ? kvv : kvlen;
  const bool regs = nseg <= kPlanRegChunks * kPlanThreads;

  // 2) segment records and their key tiles
  int my_tb[kPlanRegChunks], my_nt[kPlanRegChunks], my_lim[kPlanRegChunks];
  int4 my_head[kPlanRegChunks];     // each own segment's record fields 0-3
  carry = 0;
  for (int base = 0, c = 0; base < nseg; base += kPlanThreads, ++c) {
    const int s = base + tid;
    int ntiles = 0;
    int rec[5];
    if (s < nseg) {
      int lo = 0, hi = batch - 1;  // last b with req_off[b] <= s
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (req_off[mid] <= s) lo = mid; else hi = mid - 1;
      }
      const int b = lo;
      const int local = s - req_off[b];
      // (one segment per query block in the common case: no divisions)
      const int hb = g.nhb == 1 ? 0 : local % g.nhb;
      const int kvg = g.nkvg == 1 ? 0 : (local / g.nhb) % g.nkvg;
      const int qblk = per_req == 1 ? local : local / per_req;
      const int q_begin = cu_r[b];
      const int lq = cu_r[b + 1] - q_begin;
      const int lk = kv_r[b];
      const int q0 = qblk * g.qs;
      const int nq = min(g.qs, lq - q0);
      const int lim_base = lk - lq + q0;
      const int visible = max(0, min(lk, lim_base + nq));
      // at least one (fully masked) tile, so the work-group that owns it
      // writes the zero output of rows that see no key
      ntiles = max(1, (visible + kTile - 1) / kTile);
      rec[0] = b; rec[1] = kvg | (hb << 16) | ((q0 + nq == lq) << 30);
      rec[2] = q_begin + q0; rec[3] = nq | (q0 << 8);
      rec[4] = lim_base;
    }
    int tot;
    const int ex = block_exclusive_scan(ntiles, wave_sums, &tot);
    if (s < nseg) {
      int4* r = reinterpret_cast<int4*>(seg + (int64_t)s * 8);   // field 7 follows in phase 3
      r[0] = make_int4(rec[0], rec[1], rec[2], rec[3]);
      r[1] = make_int4(rec[4], carry + ex, carry + ex + ntiles, 0);
    }
#pragma unroll
    for (int i = 0; i < kPlanRegChunks; ++i)
      if (i == c) {
        my_tb[i] = carry + ex; my_nt[i] = ntiles; my_lim[i] = rec[4];
        my_head[i] = make_int4(rec[0], rec[1], rec[2], rec[3]);
      }
    carry += tot;
  }
  // Range length.  With few segments and short ranges each segment's tile
  // span is padded to a multiple of it, so no range crosses a segment
  // boundary (a crossing costs the range's work-group further dependent
  // loads, and the slowest range sets the kernel time); waves - nseg ranges'
  // worth of tiles plus at most one partial range per segment still fit in
  // `waves` ranges.  Long ranges absorb a crossing and keep the even split.
  const int real_tiles = carry;
  int tpw = max(1, (real_tiles + waves - 1) / waves);
  const bool pad = 2 * nseg <= waves && tpw < kPadBelow;
  // Padded GQA plans aim at 7/8 of the range budget: with ranges this
  // short, fewer and slightly longer ones measured faster (config 1 22.7
  // against 23.1 us, configs[3] 40.7 against 41.0; 3/4 measured the same
  // on config 1, 5/8 and 1/2 slower), with the ranges spread over the XCDs
  // as below; MLA keeps its tuned budget.
  const int pw = (pad && dv != 512 && 2 * nseg <= waves * 7 / 8) ? waves * 7 / 8 : waves;
  if (pad) {
    // smallest length whose padded ranges fit in `pw`: the bound
    // ceil(tiles / (pw - nseg)) always fits, and a few block reductions
    // find the least one (an idle range slot is an idle work-group)
    tpw = max(1, (real_tiles + pw - 1) / pw);
    int hi = max(1, (real_tiles + pw - nseg - 1) / (pw - nseg));
    while (tpw < hi) {
      const int mid = (tpw + hi) >> 1;
      int mine = 0;
      for (int base = 0, c = 0; base < nseg; base += kPlanThreads, ++c) {
        const int s = base + tid;
        if (s >= nseg) break;
        int nt = 0;
        if (regs) {
#pragma unroll
          for (int i = 0; i < kPlanRegChunks; ++i)
            if (i == c) nt = my_nt[i];
        } else {
          nt = seg[(int64_t)s * 8 + 6] - seg[(int64_t)s * 8 + 5];
        }
        mine += (nt + mid - 1) / mid;
      }
      int tot;
      block_exclusive_scan(mine, wave_sums, &tot);
      if (tot <= pw) hi = mid; else tpw = mid + 1;
    }
  }
  int total_tiles = real_tiles;
  if (pad) {
    carry = 0;
    for (int base = 0, c = 0; base < nseg; base += kPlanThreads, ++c) {
      const int s = base + tid;
      int nt = 0;
      if (s < nseg) {
        if (regs) {
#pragma unroll
          for (int i = 0; i < kPlanRegChunks; ++i)
            if (i == c) nt = my_nt[i];
        } else {
          nt = seg[(int64_t)s * 8 + 6] - seg[(int64_t)s * 8 + 5];
        }
      }
      int tot;
      const int ex = block_exclusive_scan((nt + tpw - 1) / tpw * tpw, wave_sums, &tot);
      if (s < nseg) {
        *reinterpret_cast<int2*>(seg + (int64_t)s * 8 + 5) = make_int2(carry + ex, carry + ex + nt);
      }
#pragma unroll
      for (int i = 0; i < kPlanRegChunks; ++i)
        if (i == c) my_tb[i] = carry + ex;
      carry += tot;
    }
    total_tiles = carry;
  }
  __syncthreads();   // request metadata in LDS is no longer needed

  // segments' first tiles into LDS for the per-range search
  const bool tb_lds = regs && nseg + 1 <= kPlanLds;
  if (tb_lds) {
#pragma unroll
    for (int i = 0; i < kPlanRegChunks; ++i) {
      const int s = i * kPlanThreads + tid;
      if (s < nseg) lds[s] = my_tb[i];
    }
    if (tid == 0) lds[nseg] = total_tiles;
  }

  // 3) partial slots: a segment split over k ranges owns k consecutive slots
  const int pb0 = nseg + 1;     // LDS: segments' first partial slots (balanced MLA plans)
  const int ncu = g.ncu;
  const bool bal = AIA_MLA_BALANCE && pad && dv == 512 && ncu > 0 && waves % ncu == 0 &&
                   2 * (nseg + 1) + 32 <= kPlanLds;
  // The segment records are also kept in LDS (after the first tiles) for
  // the range records, which then need no global load before their block
  // ids.  With the galloping search below, config 5's plan went from
  // 11.8-12.3 to 11.0-11.8 us on one box (alternating runs).
  const int srec0 = (pb0 + 3) & ~3;
  const bool rec_lds = tb_lds && !bal && srec0 + 8 * nseg <= kPlanLds;
  int4* srec = reinterpret_cast<int4*>(lds + srec0);
  // GQA plans: each thread's first range is placed now, before phase 3, and
  // its block ids are loaded, so that load is in flight during phase 3's
  // scans and merge records instead of opening phase 4 (the partial base of
  // the LDS segment records follows in phase 3).
  const int nr_used_early = min(waves, (total_tiles + tpw - 1) / tpw);
  const bool early = rec_lds && tid < nr_used_early;
  int e_lo = 0, e_lo2 = 0, e_blk = 0;
  int e_bv[kRecBlocks];
  if (rec_lds) {
#pragma unroll
    for (int i = 0; i < kPlanRegChunks; ++i) {
      const int s = i * kPlanThreads + tid;
      if (s < nseg) {
        srec[2 * s] = my_head[i];
        srec[2 * s + 1] = make_int4(my_lim[i], my_tb[i], my_tb[i] + my_nt[i], 0);
      }
    }
    __syncthreads();   // first tiles and segment records
    if (early) {
      const int t0 = tid * tpw;
      const int t1 = min(total_tiles, t0 + tpw);
      e_lo = range_first_seg(lds, nseg, t0);
      e_lo2 = range_last_seg(lds, nseg, e_lo, t1);
      const int4 r0 = srec[2 * e_lo], r1 = srec[2 * e_lo + 1];
      const int nblk_vis = (max(0, r1.x + (r0.w & 0xff)) + block_size - 1) / block_size;
      e_blk = ((t0 - r1.y) * kTile) / block_size;
      const int32_t* btrow = block_table + (int64_t)r0.x * bt_stride;
#pragma unroll
      for (int i = 0; i < kRecBlocks; ++i) e_bv[i] = e_blk + i < nblk_vis ? btrow[e_blk + i] : 0;
    }
  }
  carry = 0;
  int mcarry = 0;
  bool fixed = false;
  for (int base = 0, c = 0; base < nseg; base += kPlanThreads, ++c) {
    const int s = base + tid;
    int np = 0;
    if (s < nseg) {
      int tb = 0, nt = 0;
      if (regs) {
#pragma unroll
        for (int i = 0; i < kPlanRegChunks; ++i)
          if (i == c) { tb = my_tb[i]; nt = my_nt[i]; }
      } else {
        tb = seg[(int64_t)s * 8 + 5];
        nt = seg[(int64_t)s * 8 + 6] - tb;
      }
      np = (tb + nt - 1) / tpw - tb / tpw + 1;
    }
    // merge work of a split segment: one record per (kv head, slice of 64
    // elements of its row span), so the merge kernel visits only real work
    int mcnt = 0, nwv = 0, nsl = 0, rows = 0;
    int r0[4] = {0, 0, 0, 0};
    if (s < nseg) {
      if (np > 1) {
        if (regs) {      // the segment's head, kept in registers since phase 2
#pragma unroll
          for (int i = 0; i < kPlanRegChunks; ++i)
            if (i == c) { r0[0] = my_head[i].x; r0[1] = my_head[i].y; r0[2] = my_head[i].z; r0[3] = my_head[i].w; }
        } else {
          for (int i = 0; i < 4; ++i) r0[i] = seg[(int64_t)s * 8 + i];
        }
        const int nq = r0[3] & 0xff;
        const int nblk = (nq + g.qb - 1) / g.qb;
        rows = (nblk - 1) * kRows + min(kRows, (nq - (nblk - 1) * g.qb) * g.hb);
        nwv = min(g.nw, g.hkv - (r0[1] & 0xffff) * g.nw);
        nsl = (rows * (dv / kMergeDims) + 63) / 64;
        mcnt = nwv * nsl;
      }
    }
    // fixed partial slots (see kFixParts), decided as the small planner does
    fixed = nseg <= kSmallPlanSegs && nseg * kFixParts <= fix_cap &&
            !__syncthreads_or(np > kFixParts);
    int2 tot2;
    const int2 ex2 = block_exclusive_scan2(make_int2(np, mcnt), wave_sums2, &tot2);
    const int ex = ex2.x, tot = tot2.x, mex = ex2.y, mtot = tot2.y;
    const int pbase = fixed ? kFixParts * s : carry + ex;   // the segment's first partial slot
    if (s < nseg) seg[(int64_t)s * 8 + 7] = pbase;
    if (bal && s < nseg) lds[pb0 + s] = carry + ex;
    if (rec_lds && s < nseg) lds[srec0 + 8 * s + 7] = pbase;   // srec[2 s + 1].w
    if (mcnt > 0) {
      const int seg_rows = kRows * g.rb;
      int4* m = reinterpret_cast<int4*>(mrg + (int64_t)(mcarry + mex) * kMrgInts);
      for (int w = 0; w < nwv; ++w)
        for (int sl = 0; sl < nsl; ++sl, m += kMrgInts / 4) {
          // {first query token, query tokens, kv head, head block; first
          // partial row, parts, slice, rows}, as two 16-byte stores
          m[0] = make_int4(r0[2], r0[3] & 0xff, (r0[1] & 0xffff) * g.nw + w, (r0[1] >> 16) & 0x3fff);
          m[1] = make_int4((pbase * g.nw + w) * seg_rows, np, sl, rows);
        }
    }
    mcarry += mtot;
    carry += tot;
  }
  if (tid == 0) {
    hdr[0] = nseg; hdr[1] = total_tiles; hdr[2] = tpw; hdr[3] = fixed ? kFixParts * nseg : carry;
    hdr[4] = waves; hdr[5] = mcarry; hdr[6] = units; hdr[7] = pmerges;
    hdr[8] = overflow ? -1 : 0;   // status: -1 = the metadata asked for more work than fits
    hdr[9] = overflow ? 0 : dealt;
    hdr[10] = fixed ? 1 : 0;
    // sentinel record so readers may look one past the end
    int* r = seg + (int64_t)nseg * 8;
    r[0] = 0; r[1] = 0; r[2] = 0; r[3] = 0; r[4] = 0;
    r[5] = total_tiles; r[6] = total_tiles; r[7] = fixed ? kFixParts * nseg : carry;
  }
  __syncthreads();

  // 4) per-range record (see kRecInts)
  // (records and segment records are 16-byte aligned: 16-byte stores and loads)
  auto write_rec = [&](int* out, int lo, int lo2, int t0, int t1, int j, int k) {
    int4* o4 = reinterpret_cast<int4*>(out);
    const int4* r = rec_lds ? srec + 2 * lo : reinterpret_cast<const int4*>(seg + (int64_t)lo * 8);
    const int4 r0 = r[0], r1 = r[1];
    o4[0] = make_int4(lo, t0, t1, tpw);
    o4[1] = r0;
    o4[2] = r1;
    const int b = r0.x, nq = r0.w & 0xff, lim_base = r1.x;
    const int visible = max(0, lim_base + nq);
    const int nblk_vis = (visible + block_size - 1) / block_size;
    const int blk_base = ((t0 - r1.y) * kTile) / block_size;
    o4[3] = make_int4(blk_base, lo2, j, k);
    const int32_t* btrow = block_table + (int64_t)b * bt_stride;
    int bv[kRecBlocks];
#pragma unroll
    for (int i = 0; i < kRecBlocks; ++i) bv[i] = blk_base + i < nblk_vis ? btrow[blk_base + i] : 0;
#pragma unroll
    for (int i = 0; i < kRecBlocks / 4; ++i)
      o4[4 + i] = make_int4(bv[4 * i], bv[4 * i + 1], bv[4 * i + 2], bv[4 * i + 3]);
  };
  if (bal) {
    // ranges = the partial slots of the padded plan; range r is number
    // r - pb[s] of segment s's k ranges, of floor / ceil (nt / k) tiles
    int* hist = lds + pb0 + nseg + 1;          // 16 size counters, then 16 offsets
    int* offs = hist + 16;
    if (tid == 0) lds[pb0 + nseg] = carry;
    if (tid < 32) hist[tid] = 0;
    __syncthreads();
    const int nr = carry;
    auto locate = [&](int r, int& s_, int& j_, int& k_, int& a_, int& b_) {
      int lo_ = 0, hi_ = nseg - 1;   // last s with pb[s] <= r (segments with k = 0 share it)
      while (lo_ < hi_) {
        const int mid = (lo_ + hi_ + 1) >> 1;
        if (lds[pb0 + mid] <= r) lo_ = mid; else hi_ = mid - 1;
      }
      s_ = lo_;
      j_ = r - lds[pb0 + lo_];
      k_ = lds[pb0 + lo_ + 1] - lds[pb0 + lo_];
      const int nt_ = seg[(int64_t)lo_ * 8 + 6] - seg[(int64_t)lo_ * 8 + 5];
      a_ = (int)((int64_t)j_ * nt_ / k_);
      b_ = (int)((int64_t)(j_ + 1) * nt_ / k_);
    };
    for (int r = tid; r < nr; r += kPlanThreads) {
      int s_, j_, k_, a_, b_;
      locate(r, s_, j_, k_, a_, b_);
      atomicAdd(&hist[min(b_ - a_, 15)], 1);
    }
    __syncthreads();
    if (tid == 0) {            // largest ranges first
      int acc = 0;
      for (int sz = 15; sz >= 0; --sz) { offs[sz] = acc; acc += hist[sz]; }
    }
    __syncthreads();
    for (int r = tid; r < nr; r += kPlanThreads) {
      int s_, j_, k_, a_, b_;
      locate(r, s_, j_, k_, a_, b_);
      const int rank = atomicAdd(&offs[min(b_ - a_, 15)], 1);
      const int round = rank / ncu, pos = rank - round * ncu;
      const int slot = round * ncu + ((round & 1) ? ncu - 1 - pos : pos);
      const int tb = seg[(int64_t)s_ * 8 + 5];
      write_rec(wave_rec + (int64_t)slot * kRecInts, s_, s_, tb + a_, tb + b_, j_, k_);
    }
    for (int w = tid; w < waves; w += kPlanThreads) {   // slots no rank maps to
      const int round = w / ncu, cu = w - round * ncu;
      const int rank = round * ncu + ((round & 1) ? ncu - 1 - cu : cu);
      if (rank >= nr) {
        int* out = wave_rec + (int64_t)w * kRecInts;
        *reinterpret_cast<int4*>(out) = make_int4(-1, 0, 0, tpw);
      }
    }
    return;
  }
  // GQA: work-group w runs the range in record slot w, and the hardware
  // deals work-groups to the 8 XCDs round-robin; the used ranges go to the
  // slots so that XCD x gets a contiguous run of about nr / 8 of them (a
  // padded plan's unused slots no longer pile up on the last XCDs: config 1
  // 22.8 against 23.2 us).  MLA work-groups read slot = range.
  const bool spread = dv != 512;
  const int nr_used = min(waves, (total_tiles + tpw - 1) / tpw);
  const int q8 = nr_used / kXcdsPlan, rem8 = nr_used - q8 * kXcdsPlan;
  // Range r goes to slot (i, x) = its place i in XCD x's run; threads walk
  // the ranges in order, so a wave's searches and record loads stay local.
  auto slot_of = [&](int r) {
    if (!spread) return r;
    const int big = (q8 + 1) * rem8;          // the first rem8 runs hold q8 + 1
    const int x = r < big ? r / (q8 + 1) : rem8 + (r - big) / q8;
    const int i = r < big ? r - x * (q8 + 1) : r - big - (x - rem8) * q8;
    return i * kXcdsPlan + x;
  };
  for (int r = tid; r < nr_used; r += kPlanThreads) {
    const int t0 = r * tpw;
    const int t1 = min(total_tiles, t0 + tpw);
    if (early && r == tid) {      // placed before phase 3, block ids loaded then
      int4* o4 = reinterpret_cast<int4*>(wave_rec + (int64_t)slot_of(r) * kRecInts);
      o4[0] = make_int4(e_lo, t0, t1, tpw);
      o4[1] = srec[2 * e_lo];
      o4[2] = srec[2 * e_lo + 1];
      o4[3] = make_int4(e_blk, e_lo2, 0, 0);
#pragma unroll
      for (int i = 0; i < kRecBlocks / 4; ++i)
        o4[4 + i] = make_int4(e_bv[4 * i], e_bv[4 * i + 1], e_bv[4 * i + 2], e_bv[4 * i + 3]);
      continue;
    }
    int lo = 0, hi = nseg - 1;  // last s with tile_begin <= t0
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      const int tb = tb_lds ? lds[mid] : seg[(int64_t)mid * 8 + 5];
      if (tb <= t0) lo = mid; else hi = mid - 1;
    }
    // last s with tile_begin < t1: a range ends a segment or two past
    // its first, so gallop from lo, then search the bracket
    auto tb_at = [&](int i) { return tb_lds ? lds[i] : seg[(int64_t)i * 8 + 5]; };
    int lo2 = lo, step = 1;
    while (lo2 + step < nseg && tb_at(lo2 + step) < t1) { lo2 += step; step <<= 1; }
    int hi2 = min(nseg - 1, lo2 + step - 1);
    while (lo2 < hi2) {
      const int mid = (lo2 + hi2 + 1) >> 1;
      if (tb_at(mid) < t1) lo2 = mid; else hi2 = mid - 1;
    }
    write_rec(wave_rec + (int64_t)slot_of(r) * kRecInts, lo, lo2, t0, t1, 0, 0);
  }
  // slots no range maps to
  for (int w = tid; w < waves; w += kPlanThreads) {
    const int x = w % kXcdsPlan, i = w / kXcdsPlan;
    const bool used = spread ? i < q8 + (x < rem8 ? 1 : 0) : w < nr_used;
    if (!used)
      *reinterpret_cast<int4*>(wave_rec + (int64_t)w * kRecInts) = make_int4(-1, 0, 0, tpw);
  }
}

// Small GQA steps (no prefill routing, at most 64 segments: config-1 and
// MTP-verify sized batches) are planned by one wave for the per-request and
// per-segment phases -- DPP scans and lane shuffles, no block barriers and
// no global round trip between phases -- and then by the whole work-group
// for the range records.  The plan is the one plan_kernel makes for the
// same step, record for record (tests compare the two workspaces).
constexpr int kSmallPlanThreads = 256;

__device__ __forceinline__ int wave_total(int x) {   // sum over the 64 lanes, in every lane
  return __builtin_amdgcn_readlane(wave_incl_scan(x), 63);
}

__global__ __launch_bounds__(kSmallPlanThreads) void plan_small_kernel(
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ kvlen,
    const int32_t* __restrict__ block_table, int64_t bt_stride, int32_t block_size,
    int32_t batch, Geometry g, int32_t waves, int32_t dv,
    int32_t* __restrict__ hdr, int32_t* __restrict__ seg, int32_t* __restrict__ wave_rec,
    int32_t* __restrict__ mrg, int32_t seg_cap, int32_t fix_cap) {
  __shared__ int4 srec[kSmallPlanSegs + 1][2];   // segment records (+ sentinel)
  __shared__ int sinfo[4];                        // nseg, total tiles, tpw
  const int tid = threadIdx.x, lane = tid & 63;
  const int per_req = g.nkvg * g.nhb;
  if (tid < 64) {
    // 1) segments per request (lane = request)
    int c0 = 0, c1 = 0, lk = 0, cnt = 0;
    if (lane < batch) {
      c0 = cu_q[lane]; c1 = cu_q[lane + 1]; lk = kvlen[lane];
      const int lq = c1 - c0;
      cnt = lq > 0 ? ((lq + g.qs - 1) / g.qs) * per_req : 0;
    }
    const int inc = wave_incl_scan(cnt);
    const int req_off = inc - cnt;
    int nseg = __builtin_amdgcn_readlane(inc, 63);
    int overflow = 0;
    if (nseg > seg_cap || nseg > kSmallPlanSegs) { nseg = 0; overflow = 1; }

    // 2) lane = segment: its request (last b with req_off[b] <= s), record
    // fields and key tiles
    const int s = lane;
    int rec0 = 0, rec1 = 0, rec2 = 0, rec3 = 0, lim_base = 0, nt = 0;
    {
      // a fixed number of steps with every lane active, so each shuffle
      // reads lanes that take part in it
      int lo = 0, hi = batch - 1;
#pragma unroll
      for (int it = 0; it < 6; ++it) {
        const int mid = (lo + hi + 1) >> 1;
        const bool le = __shfl(req_off, mid & 63) <= s;
        if (lo < hi) {
          if (le) lo = mid; else hi = mid - 1;
        }
      }
      const int b = lo;
      const int local = s - __shfl(req_off, b);
      const int q_begin = __shfl(c0, b), lq = __shfl(c1, b) - q_begin, lkb = __shfl(lk, b);
      if (s < nseg) {
        const int hb = g.nhb == 1 ? 0 : local % g.nhb;
        const int kvg = g.nkvg == 1 ? 0 : (local / g.nhb) % g.nkvg;
        const int qblk = per_req == 1 ? local : local / per_req;
        const int q0 = qblk * g.qs;
        const int nq = min(g.qs, lq - q0);
        lim_base = lkb - lq + q0;
        const int visible = max(0, min(lkb, lim_base + nq));
        nt = max(1, (visible + kTile - 1) / kTile);
        rec0 = b; rec1 = kvg | (hb << 16) | ((q0 + nq == lq) << 30);
        rec2 = q_begin + q0; rec3 = nq | (q0 << 8);
      }
    }
    const int real_tiles = wave_total(nt);
    // range length, padding as in plan_kernel
    int tpw = max(1, (real_tiles + waves - 1) / waves);
    const bool pad = 2 * nseg <= waves && tpw < kPadBelow;
    const int pw = (pad && 2 * nseg <= waves * 7 / 8) ? waves * 7 / 8 : waves;
    if (pad) {
      tpw = max(1, (real_tiles + pw - 1) / pw);
      int hi = max(1, (real_tiles + pw - nseg - 1) / (pw - nseg));
      while (tpw < hi) {
        const int mid = (tpw + hi) >> 1;
        const int tot = wave_total(s < nseg ? (nt + mid - 1) / mid : 0);
        if (tot <= pw) hi = mid; else tpw = mid + 1;
      }
    }
    const int span = s < nseg ? (pad ? (nt + tpw - 1) / tpw * tpw : nt) : 0;
    const int tinc = wave_incl_scan(span);
    const int tb = tinc - span;
    const int total_tiles = __builtin_amdgcn_readlane(tinc, 63);

    // 3) partial slots and merge records
    int np = 0, mcnt = 0, nwv = 0, nsl = 0, rows = 0;
    if (s < nseg) {
      np = (tb + nt - 1) / tpw - tb / tpw + 1;
      if (np > 1) {
        const int nq = rec3 & 0xff;
        const int nblk = (nq + g.qb - 1) / g.qb;
        rows = (nblk - 1) * kRows + min(kRows, (nq - (nblk - 1) * g.qb) * g.hb);
        nwv = min(g.nw, g.hkv - (rec1 & 0xffff) * g.nw);
        nsl = (rows * (dv / kMergeDims) + 63) / 64;
        mcnt = nwv * nsl;
      }
    }
    const int pinc = wave_incl_scan(np), minc = wave_incl_scan(mcnt);
    // fixed partial slots (see kFixParts)
    const bool fixed = nseg * kFixParts <= fix_cap && !__any(np > kFixParts);
    const int part_base = fixed ? kFixParts * s : pinc - np, mbase = minc - mcnt;
    const int nparts = fixed ? kFixParts * nseg : __builtin_amdgcn_readlane(pinc, 63);
    const int nmrg = __builtin_amdgcn_readlane(minc, 63);
    if (s < nseg) {
      const int4 r0 = make_int4(rec0, rec1, rec2, rec3);
      const int4 r1 = make_int4(lim_base, tb, tb + nt, part_base);
      int4* r = reinterpret_cast<int4*>(seg + (int64_t)s * 8);
      r[0] = r0; r[1] = r1;
      srec[s][0] = r0; srec[s][1] = r1;
      const int seg_rows = kRows * g.rb;
      int4* m = reinterpret_cast<int4*>(mrg + (int64_t)mbase * kMrgInts);
      for (int w = 0; w < nwv; ++w)
        for (int sl = 0; sl < nsl; ++sl, m += kMrgInts / 4) {
          m[0] = make_int4(rec2, rec3 & 0xff, (rec1 & 0xffff) * g.nw + w, (rec1 >> 16) & 0x3fff);
          m[1] = make_int4((part_base * g.nw + w) * seg_rows, np, sl, rows);
        }
    }
    if (lane == 0) {
      hdr[0] = nseg; hdr[1] = total_tiles; hdr[2] = tpw; hdr[3] = nparts; hdr[4] = waves;
      hdr[5] = nmrg; hdr[6] = 0; hdr[7] = 0;
      hdr[8] = overflow ? -1 : 0;
      hdr[9] = 0;
      hdr[10] = fixed ? 1 : 0;
      int4* r = reinterpret_cast<int4*>(seg + (int64_t)nseg * 8);   // sentinel
      r[0] = make_int4(0, 0, 0, 0);
      r[1] = make_int4(0, total_tiles, total_tiles, nparts);
      srec[nseg][1] = make_int4(0, total_tiles, total_tiles, nparts);
      sinfo[0] = nseg; sinfo[1] = total_tiles; sinfo[2] = tpw;
    }
  }
  __syncthreads();

  // 4) range records, spread over the XCDs as plan_kernel places them
  const int nseg = sinfo[0], total_tiles = sinfo[1], tpw = sinfo[2];
  const int nr_used = min(waves, (total_tiles + tpw - 1) / tpw);
  const int q8 = nr_used / kXcdsPlan, rem8 = nr_used - q8 * kXcdsPlan;
  for (int r = tid; r < nr_used && nseg > 0; r += kSmallPlanThreads) {
    const int t0 = r * tpw;
    const int t1 = min(total_tiles, t0 + tpw);
    int lo = 0, hi = nseg - 1;     // last s with tile_begin <= t0
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (srec[mid][1].y <= t0) lo = mid; else hi = mid - 1;
    }
    int lo2 = lo, hi2 = nseg - 1;  // last s with tile_begin < t1
    while (lo2 < hi2) {
      const int mid = (lo2 + hi2 + 1) >> 1;
      if (srec[mid][1].y < t1) lo2 = mid; else hi2 = mid - 1;
    }
    const int4 r0 = srec[lo][0], r1 = srec[lo][1];
    const int b = r0.x, nq = r0.w & 0xff;
    const int nblk_vis = (max(0, r1.x + nq) + block_size - 1) / block_size;
    const int blk_base = ((t0 - r1.y) * kTile) / block_size;
    const int32_t* btrow = block_table + (int64_t)b * bt_stride;
    int bv[kRecBlocks];
#pragma unroll
    for (int i = 0; i < kRecBlocks; ++i) bv[i] = blk_base + i < nblk_vis ? btrow[blk_base + i] : 0;
    const int big = (q8 + 1) * rem8;
    const int x = r < big ? r / (q8 + 1) : rem8 + (r - big) / q8;
    const int i8 = r < big ? r - x * (q8 + 1) : r - big - (x - rem8) * q8;
    int4* o4 = reinterpret_cast<int4*>(wave_rec + (int64_t)(i8 * kXcdsPlan + x) * kRecInts);
    o4[0] = make_int4(lo, t0, t1, tpw);
    o4[1] = r0;
    o4[2] = r1;
    o4[3] = make_int4(blk_base, lo2, 0, 0);
#pragma unroll
    for (int i = 0; i < kRecBlocks / 4; ++i)
      o4[4 + i] = make_int4(bv[4 * i], bv[4 * i + 1], bv[4 * i + 2], bv[4 * i + 3]);
  }
  for (int w = tid; w < waves; w += kSmallPlanThreads) {     // slots no range maps to
    const int x = w % kXcdsPlan, i = w / kXcdsPlan;
    if (nseg == 0 || i >= q8 + (x < rem8 ? 1 : 0))
      *reinterpret_cast<int4*>(wave_rec + (int64_t)w * kRecInts) = make_int4(-1, 0, 0, tpw);
  }
}

// ---------------------------------------------------------------- attention

struct AttnArgs {
  const uint16_t* q;
  int64_t q_ts, q_hs;
  uint16_t* kc;
  uint16_t* vc;
  // this step's new K/V rows (T, Hkv, D); when set, keys at the new
  // positions are read from them and written into the cache by the kernel
  const uint16_t* kn;
  const uint16_t* vn;
  int64_t kn_ts, vn_ts;
  const int32_t* bt;
  int64_t bt_stride;
  int32_t hkv, group, hb, bs, nb, nw;
  float scale_log2;
  const int32_t* seg;
  const int32_t* wave_rec;
  uint16_t* part_o;          // split partials (fp16, scaled per row)
  float2* part_ml;
  uint16_t* out;
  int64_t o_ts, o_hs;
  int32_t waves;
  const int32_t* hdr;
  int32_t batch, tokens;
};

// A record is used only if it lies inside the plan (defence against a plan
// read before its planner finished, e.g. from another stream).
__device__ __forceinline__ bool rec_ok(const int* r, int nseg_tiles, int batch, int tokens,
                                       int ngroups, int nhb) {
  return r[0] >= 0 && r[0] < batch && (r[1] & 0xffff) < ngroups && ((r[1] >> 16) & 0x3fff) < nhb &&
         r[2] >= 0 && (r[3] & 0xff) >= 1 && r[2] + (r[3] & 0xff) <= tokens && r[5] >= 0 && r[5] < r[6] &&
         r[6] <= nseg_tiles;
}

// s_waitcnt vmcnt(0) (expcnt / lgkmcnt left at their maxima), gfx9 encoding.
constexpr int kWaitVmcnt0 = 0x0F70;

__device__ __forceinline__ short4_t as_s4(uint32_t a, uint32_t b) {
  short4_t r;
  r[0] = (short)(a & 0xffff); r[1] = (short)(a >> 16);
  r[2] = (short)(b & 0xffff); r[3] = (short)(b >> 16);
  return r;
}

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) short4_t lds_short4_t;

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  const half2_t v = {(_Float16)lo, (_Float16)hi};
  return __builtin_bit_cast(uint32_t, v);
}


__device__ __forceinline__ u32x4_t as_u4(uint4 v) { return u32x4_t{v.x, v.y, v.z, v.w}; }

__device__ __forceinline__ bf16x8_t as_b8(uint4 v) { return __builtin_bit_cast(bf16x8_t, as_u4(v)); }

// S^T tile (16 keys x 16 rows) += K (16 keys x 32 dims) . Q^T: lane (key n,
// group g) holds dims [32 j + 8 g, +8) of its key in kk and of its row in q.
__device__ __forceinline__ float4_t qk_step(uint4 kk, uint4 q, float4_t acc) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_b8(kk), as_b8(q), acc, 0, 0, 0);
}

// A V tile is staged in LDS key-major (row stride kVStride elements): lane
// (key n, group g) stores its 16-byte pieces at dims 32 j + 8 g.  The
// transposing LDS read works within each 16-lane group: local lane l receives
// element l % 4 of the 8 bytes addressed by local lanes 4 k + l / 4, k = 0..3.
// Lane (n, g) addressing key 4 g + n / 4, dims 16 dt + 4 (n % 4) therefore
// receives V^T[16 dt + n][keys 4 g .. 4 g + 3], the A fragment of the
// 16x16x16 MFMA, in one instruction.  (The stores take vector values: an
// aggregate copy of the tile registers keeps them in a private array, which
// the compiler then places in LDS, serialising the load pipeline.)
template <int KJ>
__device__ __forceinline__ void stage_v(uint16_t* vs, int n, int g, const uint4 (&vv)[KJ]) {
#pragma unroll
  for (int j = 0; j < KJ; ++j) *reinterpret_cast<u32x4_t*>(vs + n * kVStride + 32 * j + 8 * g) = as_u4(vv[j]);
}
template <int STRIDE = kVStride>
__device__ __forceinline__ short4_t vt_frag(const uint16_t* vs, int n, int g, int dt) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_short4_t*)(vs + (4 * g + (n >> 2)) * STRIDE + 16 * dt + 4 * (n & 3)));
}

// Tiles kept in flight per GQA wave (registers: 32 VGPRs per tile).  One is
// fastest: with random blocks, more outstanding tiles per CU lowers the
// delivered bandwidth (measured on config-1 decode: 18.7 us at 1, 20.1 at 2,
// 24.9 at 5), and the planner keeps ranges short instead.
#ifndef AIA_PIPE
#define AIA_PIPE 1
#endif
constexpr int kPipe = AIA_PIPE;

// Processes key tiles [lt0, lt1) of one segment; rec = the segment record.
// A segment holds RB blocks of 16 query rows: block r has the segment's
// query tokens [r qb, r qb + qb), row n being token n / hb, head n % hb
// (qb = 16 / hb).  Every K/V tile is loaded once and used by all blocks, so a
// prefill chunk reads its keys 1/RB as often; blocks past the segment's last
// token are skipped (a uniform branch), so a decode segment costs one block.
// Cache layouts.  ND: (num_blocks, block_size, Hkv, D), a token slot's heads
// contiguous.  NZ: the 16-wide fractal layout of the reference's graph-mode
// caches (gqa.py:163,202-226): each block viewed (Hkv D / 16, block_size,
// 16), so 16 dims of all of a block's tokens are contiguous.  kv_piece gives
// the 16-byte index of piece p (8 dims) of head h of (block, offset).
template <bool NZ>
__device__ __forceinline__ int64_t kv_piece(int64_t blk, int off, int bs, int row_elems, int h,
                                            int D, int p) {
  if (!NZ) return (((blk * bs + off) * row_elems + (int64_t)h * D) >> 3) + p;
  return ((blk * bs * row_elems) >> 3) +
         (((int64_t)(h * (D / 16) + (p >> 1)) * bs + off) << 1) + (p & 1);
}

template <int RB, int D, bool NZ>
__device__ __forceinline__ void gqa_segment(const AttnArgs& a, const int* rec, int s, int lt0,
                                            int lt1, int w, int tpw, uint16_t* vt, int lane,
                                            int wid, bool use_pre, int pre) {
  constexpr int KJ = D / 32;   // 32-dim MFMA k-steps = 16-byte chunks per lane and row
  constexpr int DT = D / 16;   // 16-dim output tiles
  const int n = lane & 15, g = lane >> 4;
  const int b = rec[0], kvh = (rec[1] & 0xffff) * a.nw + wid, hbi = (rec[1] >> 16) & 0x3fff;
  const int qtok0 = rec[2], nq = rec[3] & 0xff, q0 = rec[3] >> 8, lim_base = rec[4];
  const int tile_begin = rec[5], tile_end = rec[6], part_base = rec[7];
  const int qb = kRows / a.hb;
  const int nt = n / a.hb, hh = n - nt * a.hb;
  const int nblk = (nq + qb - 1) / qb;               // row blocks holding tokens
  const int head = kvh * a.group + hbi * a.hb + hh;
  int qi[RB], lim[RB];
  bool rv[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    qi[r] = r * qb + nt;
    rv[r] = nt < qb && qi[r] < nq && hbi * a.hb + hh < a.group;
    lim[r] = rv[r] ? lim_base + qi[r] : -1;
  }
  const int visible = max(0, lim_base + nq);
  // smallest key limit of the valid rows (wave-uniform)
  int lim_lo = 0x7fffffff;
#pragma unroll
  for (int r = 0; r < RB; ++r) lim_lo = rv[r] ? min(lim_lo, lim[r]) : lim_lo;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) lim_lo = min(lim_lo, __shfl_xor(lim_lo, d));
  const int row_elems = a.hkv * D;
  // this step's new keys sit at positions [new_start, Lk); the request's last
  // query block (head block 0) owns writing them into the cache
  const int new_start = a.kn ? lim_base - q0 : 0x7fffffff;
  const int q_begin = qtok0 - q0;
  const bool writer = a.kn && ((rec[1] >> 30) & 1) && hbi == 0;

  const int32_t* btrow = a.bt + (int64_t)b * a.bt_stride;
  const int nblk_vis = (visible + a.bs - 1) / a.bs;
  int blk_base = 0, btv = 0, w1 = 0;
  // 16-byte pieces between MFMA k-steps j and j + 1 of a cached key (4 pieces
  // on in ND; two 16-dim chunks of block_size x 16 on in NZ)
  const int64_t jstride = NZ ? 4 * (int64_t)a.bs : 4;

  uint4 qf[RB][KJ];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    if (rv[r]) {
      const uint4* qp = reinterpret_cast<const uint4*>(
          a.q + (int64_t)(qtok0 + qi[r]) * a.q_ts + (int64_t)head * a.q_hs);
#pragma unroll
      for (int j = 0; j < KJ; ++j) qf[r][j] = qp[4 * j + g];
    } else {
#pragma unroll
      for (int j = 0; j < KJ; ++j) qf[r][j] = make_uint4(0, 0, 0, 0);
    }
  }

  float4_t o[RB][DT];
  float m[RB], lsum[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[r][dt] = float4_t{0.f, 0.f, 0.f, 0.f};
    m[r] = -1e30f;
    lsum[r] = 0.f;
  }

  // Block ids are held one per lane for a window of 64 logical blocks; the
  // window is (re)loaded only between pipelined runs, so the per-tile address
  // shuffle never waits on an outstanding global load.
  // Loads are issued unconditionally (tiles past the window read the
  // window's first key row, K and V, again: an L1 hit, and a different row
  // for every range, so no memory channel is hammered) so the load stream is
  // straight-line and the compiler can wait for each tile with an exact count.
  auto load = [&](int lt, uint4 (&kk)[KJ], uint4 (&vv)[KJ], int64_t& wdst) {
    const bool live = lt < w1;
    const int tok = live ? min(lt * kTile + n, visible - 1) : blk_base * a.bs;
    const int bi = tok / a.bs;
    // block ids outside the pool are clamped so a bad table cannot fault
    const int blk = min(max(__shfl(btv, bi - blk_base), 0), a.nb - 1);
    const int off = tok - bi * a.bs;
    // 16-byte index of this lane's first piece (4 g + 0) in the cache; piece
    // 4 j + g is jstride further on in either layout
    const int64_t base = kv_piece<NZ>(blk, off, a.bs, row_elems, kvh, D, g);
    const bool fresh = live && tok >= new_start;
    const int64_t nrow = (int64_t)(q_begin + tok - new_start);
    const uint4* kp = fresh ? reinterpret_cast<const uint4*>(a.kn + nrow * a.kn_ts + (int64_t)kvh * D) + g
                            : reinterpret_cast<const uint4*>(a.kc) + base;
    const uint4* vp = fresh ? reinterpret_cast<const uint4*>(a.vn + nrow * a.vn_ts + (int64_t)kvh * D) + g
                            : reinterpret_cast<const uint4*>(a.vc) + base;
    const int64_t js = fresh ? 4 : jstride;
    // cache slot this lane writes after the tile arrives (-1: nothing)
    wdst = (writer && fresh && lt * kTile + n < visible) ? base : (int64_t)-1;
#pragma unroll
    for (int j = 0; j < KJ; ++j) kk[j] = kp[j * js];
#pragma unroll
    for (int j = 0; j < KJ; ++j) vv[j] = vp[j * js];
  };

  auto compute = [&](int lt, const uint4 (&kk)[KJ], const uint4 (&vv)[KJ], int64_t wdst) {
    if (wdst >= 0) {   // KV slot write of a new row (its bytes just arrived)
      uint4* kd = reinterpret_cast<uint4*>(a.kc) + wdst;
      uint4* vd = reinterpret_cast<uint4*>(a.vc) + wdst;
#pragma unroll
      for (int j = 0; j < KJ; ++j) { kd[j * jstride] = kk[j]; vd[j * jstride] = vv[j]; }
    }
    float4_t acc[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      acc[r] = float4_t{0.f, 0.f, 0.f, 0.f};
      if (r == 0 || r < nblk) {
#pragma unroll
        for (int j = 0; j < KJ; ++j) acc[r] = qk_step(kk[j], qf[r][j], acc[r]);
      }
    }
    stage_v(vt, n, g, vv);
    const int tb = lt * kTile + 4 * g;
    // keys past a valid row's limit exist only in tiles that reach past the
    // smallest limit (causal diagonal, sequence end); rows that are not valid
    // are never written, so their scores need no mask
    const bool masked = lt * kTile + kTile - 1 > lim_lo;
    short4_t pb[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      // raw scores; scale (> 0) is applied inside the exponent
      float sv[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) sv[v] = (!masked || tb + v <= lim[r]) ? acc[r][v] : -INFINITY;
      float tmax = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
      tmax = aia::group4_max(tmax);
      const float mnew = fmaxf(m[r], tmax * a.scale_log2);
      float p[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) p[v] = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[v], a.scale_log2, -mnew));
      const float psum = (p[0] + p[1]) + (p[2] + p[3]);
      if (__any(mnew > m[r])) {   // rescale only when some row's max grew
        const float alpha = __builtin_amdgcn_exp2f(m[r] - mnew);
        lsum[r] = lsum[r] * alpha + psum;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[r][dt] *= alpha;
      } else {
        lsum[r] += psum;
      }
      m[r] = mnew;
      pb[r] = as_s4(aia::pack_bf16x2(p[0], p[1]), aia::pack_bf16x2(p[2], p[3]));
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const short4_t va = vt_frag(vt, n, g, dt);
#pragma unroll
      for (int r = 0; r < RB; ++r)
        if (r == 0 || r < nblk)
          o[r][dt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, pb[r], o[r][dt], 0, 0, 0);
    }
    __builtin_amdgcn_wave_barrier();
  };

  uint4 kbuf[kPipe][KJ], vbuf[kPipe][KJ];
  int64_t wbuf[kPipe];
  for (int w0 = lt0; w0 < lt1;) {
    blk_base = (w0 * kTile) / a.bs;
    // tiles whose keys all fall inside blocks [blk_base, blk_base + win);
    // the first window of a range uses the block ids of its work record
    const int win = use_pre ? kRecBlocks : 64;
    w1 = min(lt1, ((blk_base + win) * a.bs - kTile) / kTile + 1);
    if (use_pre) btv = lane < kRecBlocks ? pre : 0;
    else btv = blk_base + lane < nblk_vis ? btrow[blk_base + lane] : 0;
    use_pre = false;
#pragma unroll
    for (int i = 0; i < kPipe; ++i) {
      load(w0 + i, kbuf[i], vbuf[i], wbuf[i]);
      __builtin_amdgcn_sched_barrier(0);
    }
    for (int base = w0; base < w1; base += kPipe) {
#pragma unroll
      for (int i = 0; i < kPipe; ++i) {
        const int lt = base + i;
        if (lt < w1) compute(lt, kbuf[i], vbuf[i], wbuf[i]);
        load(lt + kPipe, kbuf[i], vbuf[i], wbuf[i]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    w0 = w1;
  }

#pragma unroll
  for (int r = 0; r < RB; ++r) {
    lsum[r] = aia::group4_sum(lsum[r]);
  }
  const int first_wave = tile_begin / tpw;
  const int nparts = (tile_end - 1) / tpw - first_wave + 1;
  constexpr int seg_rows = RB * kRows;
  if (nparts == 1) {
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      if (!rv[r]) continue;
      const float inv = lsum[r] > 0.f ? 1.f / lsum[r] : 0.f;
      uint16_t* op = a.out + (int64_t)(qtok0 + qi[r]) * a.o_ts + (int64_t)head * a.o_hs;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        uint2 wv;
        wv.x = aia::pack_bf16x2(o[r][dt][0] * inv, o[r][dt][1] * inv);
        wv.y = aia::pack_bf16x2(o[r][dt][2] * inv, o[r][dt][3] * inv);
        *reinterpret_cast<uint2*>(op + 16 * dt + 4 * g) = wv;
      }
    }
  } else {
    // fp16 partial y = O / c, c = the row's largest |O| (1 for a zero row),
    // with (m + log2 c, l / c) in place of (m, l): the merge's weights
    // exp2(m - M) carry c back, so y folds exactly as O would
    const int part = part_base + (w - first_wave);
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      float cmax = 0.f;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) cmax = fmaxf(cmax, fabsf(o[r][dt][i]));
      cmax = aia::group4_max(cmax);
      if (!rv[r]) continue;
      const float c = cmax > 0.f ? cmax : 1.f;
      const float inv = 1.f / c;
      const int64_t prow = ((int64_t)part * a.nw + wid) * seg_rows + r * kRows + n;
      uint16_t* pp = a.part_o + prow * D;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        uint2 hv;
        hv.x = pack_f16x2(o[r][dt][0] * inv, o[r][dt][1] * inv);
        hv.y = pack_f16x2(o[r][dt][2] * inv, o[r][dt][3] * inv);
        *reinterpret_cast<uint2*>(pp + 16 * dt + 4 * g) = hv;
      }
      if (g == 0) a.part_ml[prow] = make_float2(m[r] + __log2f(c), lsum[r] * inv);
    }
  }
}

// XCD-aware order of the prefill work items.  The hardware deals
// work-groups to the 8 XCDs round-robin by id; mapping work-group b to item
// x q + min(x, r) + b / 8 (x = b % 8, n = 8 q + r) gives each XCD a
// contiguous run of items, so the requests it serves -- and the keys their
// query blocks re-read -- stay in its own L2.  (The split-K ranges get the
// same order from the planner, which writes them into their slots.)
constexpr int kXcds = 8;
static_assert(kXcds == kXcdsPlan, "one XCD count for the planner and the kernels");
__device__ __forceinline__ int xcd_range(int b, int n) {
  const int q = n / kXcds, r = n - q * kXcds;
  const int x = b % kXcds, i = b / kXcds;
  return x * q + min(x, r) + i;
}

// One work-group per key range, one wave per kv head of the segment's group.
// D: head dim, 128 or 64.
template <int NW, int RB, int D, bool NZ>
#ifndef AIA_GQA_WAVES_PER_EU
#define AIA_GQA_WAVES_PER_EU 2
#endif
__device__ __forceinline__ void gqa_attn_body(const AttnArgs& a, int bid,
                                              uint16_t (*vt_all)[kTile * kVStride]) {
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (bid >= a.waves) return;
  // the planner placed the ranges in the slots, spread over the XCDs
  const int* wr = a.wave_rec + (int64_t)bid * kRecInts;
  const int pre = wr[16 + (lane & (kRecBlocks - 1))];   // issued with the header
  const int nseg = a.hdr[0], total_tiles = a.hdr[1];
  const int ngroups = (a.hkv + NW - 1) / NW, nhb = (a.group + a.hb - 1) / a.hb;
  int s = wr[0];
  int t = wr[1];
  const int t_end = wr[2], tpw = wr[3], s_last = wr[13];
  if (s < 0 || s >= nseg || t < 0 || t >= t_end || t_end > total_tiles || tpw < 1 ||
      s_last < s || s_last >= nseg)
    return;
  const int w = t / tpw;                                  // the range's index
  int rec[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) rec[i] = wr[4 + i];
  uint16_t* vt = vt_all[wid];
  bool first = true;
  while (true) {
    if (!rec_ok(rec, total_tiles, a.batch, a.tokens, ngroups, nhb)) return;
    if (rec[6] > t) {
      const int chunk_end = min(t_end, rec[6]);
      if ((rec[1] & 0xffff) * NW + wid < a.hkv)
        gqa_segment<RB, D, NZ>(a, rec, s, t - rec[5], chunk_end - rec[5], w, tpw, vt, lane, wid, first,
                        pre);
      first = false;
      t = chunk_end;
      if (t >= t_end) break;
    }
    if (++s > s_last) return;
    const int* r = a.seg + (int64_t)s * 8;
#pragma unroll
    for (int i = 0; i < 8; ++i) rec[i] = r[i];
  }
}

template <int NW, int RB, int D, bool NZ>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(AIA_GQA_WAVES_PER_EU, AIA_GQA_WAVES_PER_EU)))
void gqa_attn_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t vt_all[NW][kTile * kVStride];
  gqa_attn_body<NW, RB, D, NZ>(a, blockIdx.x, vt_all);
}

// ---------------------------------------------------------------- prefill

struct PrefillArgs {
  const uint16_t* q;
  int64_t q_ts, q_hs;
  uint16_t* kc;
  uint16_t* vc;
  const uint16_t* kn;
  const uint16_t* vn;
  int64_t kn_ts, vn_ts;
  const int32_t* bt;
  int64_t bt_stride;
  const int32_t* cu_q;
  const int32_t* kvlen;
  int32_t hkv, group, bs, nb, batch, tokens;
  float scale_log2;
  uint16_t* out;
  int64_t o_ts, o_hs;
  const int4* units;         // per unit: {request, first row, first tile, end tile},
                             // {first query token, query tokens, keys, first tile's block id}
  const int4* dealt;         // work-group b: its unit record (two int4), then {unit, kv head}
                             // (written when the work-groups fit kPfTargetWgs, hdr[9])
  const int32_t* hdr;
  uint16_t* part_o;          // partial row blocks of chunked items (fp16, scaled per row)
  float2* part_ml;
  int32_t part_units;        // units the partial buffer holds
};

// LDS rows of the staged K and V tiles are 2 D bytes, unpadded: the direct
// loads write whole 1 KB runs, so the chunks of each row are swizzled
// instead (see the loader).
constexpr int kKStride = kHeadDim;   // the mixed kernel's (D = 128) buffer rows
#ifndef AIA_PF_LAZY
#define AIA_PF_LAZY 8.0f
#endif
// Instruction order of the QK^T and PV blocks (sched_group_barrier): LDS
// reads kept kPfQkAhead 16-key sub-tiles (QK^T) and kPfPvAhead V^T fragments
// (PV) ahead of their MFMAs.  Left to itself the scheduler reuses one V^T
// fragment's registers and waits for each batch of reads before two MFMAs.
// (configs[1] prefill chunks, µs per call: 48.2 unordered; QK 2 / PV 4 46.0;
// PV 2, 6 or 8 and QK 3 or 4 the same within 0.1; QK 1 46.9; PV 16 46.6.)
constexpr int kPfQkAhead = 2;
constexpr int kPfPvAhead = 4;
constexpr int kSgMfma = 0x008, kSgDsRead = 0x100;    // sched_group_barrier masks
// One 16-byte direct load from global memory into LDS at byte lds + 16 lane
// (lds wave-uniform).  Issued as inline assembly on purpose: the compiler's
// counter-wait pass tracks the builtin form as an outstanding LDS access and
// then waits for the LDS counter to drain completely (lgkmcnt(0)) before
// every LDS read, which exposes each read's full latency (48.2 against 49.3
// µs per call, and it defeats the read-ahead order above: 47.6-47.9 against
// 46.0).  Completion is explicit instead: every step waits vmcnt(0) before its
// barrier.  Loads the compiler does not see can only make its own vmcnt waits
// stricter, never too weak (the counter retires in order).
// m0 (the LDS address of the load) is named as clobbered, which clang warns
// about for a register it reserves: the warning is silenced here because the
// clobber is what tells the compiler that m0 changed, and the compiler keeps
// no value of its own in m0 in these kernels (their device assembly sets m0
// only in front of these loads).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_load16(const uint16_t* src, uint16_t* lds) {
  const uint32_t la = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds;
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :: "s"(la), "v"(src) : "memory", "m0");
}
#pragma clang diagnostic pop
constexpr float kLazyLog2 = AIA_PF_LAZY;              // max growth (log2) before a rescale

// Prefill attention: one work-group per (prefill item, kv head).  An item is
// kPfRows consecutive rows of one request's (query token, group head) row
// list, row = token * group + head-in-group; each of the 4 waves owns 32
// rows (two 16-row MFMA tiles).  The work-group walks the keys its rows can
// see in tiles of 64: every K/V tile is loaded once (straight into one of
// two LDS buffers, one barrier per tile) and used by all 128 rows.
//   S^T = K Q^T   v_mfma_f32_16x16x32_bf16, K fragments ds_read_b128 from LDS
//                 (lane (key n, group g) reads dims 32 j + 8 g of key n), Q^T
//                 fragments held in registers for the whole item;
//   O^T += V^T P^T  v_mfma_f32_16x16x32_bf16 over 32 keys taken from two
//                 16-key sub-tiles s0, s1: operand position 8 g + i holds key
//                 16 s0 + 4 g + i (i < 4) or 16 s1 + 4 g + i - 4, which is
//                 exactly where the S^T accumulators of s0 and s1 leave P,
//                 and V^T comes from two transposing LDS reads.
// Online softmax per row with the scale inside exp2; masks only in tiles
// that reach past a wave's smallest row limit.  Outputs bf16 directly (a
// work-group covers all keys of its rows).  With new K/V rows, keys at this
// step's new positions are read from them, and the work-group writes the new
// rows of the tokens whose first row it holds into the cache.
#ifndef AIA_PF_WPE
#define AIA_PF_WPE 2
#endif
template <bool ONE_BLOCK, bool FUSED, int D, bool NZ>
__device__ __forceinline__ void gqa_prefill_body(const PrefillArgs& a, int wg,
                                                 uint16_t* k0, uint16_t* k1,
                                                 uint16_t* v0, uint16_t* v1) {
  constexpr int KJ = D / 32;        // 32-dim MFMA k-steps
  constexpr int DT = D / 16;        // 16-dim output tiles
  constexpr int RC = D / 8;         // 16-byte chunks per K / V row
  // The planner writes work-group b's record at dealt[b] when the
  // work-groups fit the fill target (hdr[9] = their number; dealt by size, or
  // in xcd_range order); it is loaded beside the header rather than after
  // it.  Past the target, work-group b takes (kv head, item) pair
  // xcd_range(b, pairs), kv-head major: each XCD gets a contiguous run of
  // pairs, so the items that re-read one request's keys for one kv head
  // share an XCD's L2.
  int4 w0 = make_int4(0, 0, 0, 0), w1 = w0, w2 = w0;
  if (wg < kPfTargetWgs) {
    w0 = a.dealt[3 * wg];
    w1 = a.dealt[3 * wg + 1];
    w2 = a.dealt[3 * wg + 2];
  }
  const int count = a.hdr[6];
  const int pairs = count * a.hkv;
  if (wg >= pairs) return;
  int kvh, unit;
  int4 it, iq;
  if (a.hdr[9] == pairs) {     // this work-group's record (see the planner)
    it = w0;
    iq = w1;
    unit = w2.x;
    kvh = w2.y;
    if (unit < 0 || unit >= count) return;
  } else {
    const int pair = xcd_range(wg, pairs);
    kvh = pair / count;
    unit = pair - kvh * count;
    it = a.units[2 * unit];
    iq = a.units[2 * unit + 1];
  }
  const int b = it.x, row0 = it.y, t0 = it.z, t1 = it.w;
  if (b < 0 || b >= a.batch || kvh >= a.hkv) return;
  const int q_begin = iq.x, lq = iq.y, lk = iq.z, bid0 = iq.w;
  const int G = a.group;
  const int nrows = lq * G;
  if (row0 < 0 || row0 >= nrows || q_begin < 0 || q_begin + lq > a.tokens) return;
  const int ctx0 = lk - lq;                       // position of the first query token
  const int row_end = min(nrows, row0 + kPfRows);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int row_elems = a.hkv * D;
  const int32_t* btrow = a.bt + (int64_t)b * a.bt_stride;

  // new K/V rows of the tokens whose first row lies in this item (written by
  // the item's first chunk)
  if (FUSED && t0 == 0) {
    const int t_lo = (row0 + G - 1) / G, t_hi = min(lq, (row_end - 1) / G + 1);
    for (int e = tid; e < (t_hi - t_lo) * RC; e += kPfWaves * 64) {
      const int t = t_lo + e / RC, c = e % RC;
      const int p = ctx0 + t;
      if (p < 0) continue;
      const int blk = min(max(btrow[p / a.bs], 0), a.nb - 1);
      const int64_t dst = kv_piece<NZ>(blk, p % a.bs, a.bs, row_elems, kvh, D, c);
      const int64_t tok = q_begin + t;
      reinterpret_cast<uint4*>(a.kc)[dst] =
          reinterpret_cast<const uint4*>(a.kn + tok * a.kn_ts + (int64_t)kvh * D)[c];
      reinterpret_cast<uint4*>(a.vc)[dst] =
          reinterpret_cast<const uint4*>(a.vn + tok * a.vn_ts + (int64_t)kvh * D)[c];
    }
  }

  // this wave's rows
  int lim[kPfRt], tokr[kPfRt], headr[kPfRt];
  bool rv[kPfRt];
  int wlim_lo = 0x7fffffff, wlim_hi = -1;
#pragma unroll
  for (int rt = 0; rt < kPfRt; ++rt) {
    const int row = row0 + (wid * kPfRt + rt) * kRows + n;
    rv[rt] = row < row_end;
    tokr[rt] = row / G;
    headr[rt] = kvh * G + (row - tokr[rt] * G);
    lim[rt] = rv[rt] ? min(ctx0 + tokr[rt], lk - 1) : -1;
    if (rv[rt]) { wlim_lo = min(wlim_lo, lim[rt]); wlim_hi = max(wlim_hi, lim[rt]); }
  }
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    wlim_lo = min(wlim_lo, __shfl_xor(wlim_lo, d));
    wlim_hi = max(wlim_hi, __shfl_xor(wlim_hi, d));
  }
  uint4 qf[kPfRt][KJ];
#pragma unroll
  for (int rt = 0; rt < kPfRt; ++rt) {
    if (rv[rt]) {
      const uint4* qp = reinterpret_cast<const uint4*>(
          a.q + (int64_t)(q_begin + tokr[rt]) * a.q_ts + (int64_t)headr[rt] * a.q_hs);
#pragma unroll
      for (int j = 0; j < KJ; ++j) qf[rt][j] = qp[4 * j + g];
    } else {
#pragma unroll
      for (int j = 0; j < KJ; ++j) qf[rt][j] = make_uint4(0, 0, 0, 0);
    }
  }

  // keys the work-group's last row sees
  const int kend = max(0, min(lk, ctx0 + (row_end - 1) / G + 1));
  const int ntiles = (kend + kPfKeys - 1) / kPfKeys;
  // this unit's tiles [t0, t1) of the item's [0, ntiles); a unit that does
  // not cover them all writes a partial
  if (t0 < 0 || t1 < t0 || t1 > ntiles) return;
  const bool whole = t0 == 0 && t1 == ntiles;
  if (!whole && unit >= a.part_units) return;

  // Loader: thread tid moves 16-byte chunk (tid % RC) of keys kLdKeys i + tid / RC
  // (RC = D / 8 chunks per row) straight from global memory into LDS (no
  // registers, no LDS stores).  Each wave's load writes one 1 KB run, 1024 /
  // (2 D) key rows of 2 D bytes with lane l at byte 16 l; lane l fetches the
  // chunk whose swizzled place that is: K chunk c of key r sits at
  // c ^ (r % RC) and V chunk c at c ^ 2 (r % (RC / 2)), so the K fragment
  // reads (16 keys, one chunk each) and the V^T transposing reads (8 keys, 32
  // bytes each) spread over the banks without padded rows.
  // When the block size is a multiple of the tile, a tile lies in one block
  // and a key's address is one multiply-add: lane l of every wave holds the
  // block id of tile tb + l, fetched 64 tiles at a time, and a tile takes its
  // id with one readlane.  (Fetched per tile, the id's load was waited for at
  // once to move it into a scalar register: a memory round trip every tile.)
  // Other block sizes fetch each key's id one tile ahead, so those loads are
  // in flight during a tile's math.  Keys past the last visible one re-read
  // it (never a slot that may hold stale bytes); keys at this step's new
  // positions come from the new rows.
  const int lkey = tid / RC, lc = tid % RC;
  const int64_t kvoff = (int64_t)kvh * D;
  const uint16_t* kcb = a.kc + kvoff;
  const uint16_t* vcb = a.vc + kvoff;
  const uint16_t* knb = FUSED ? a.kn + kvoff : nullptr;
  const uint16_t* vnb = FUSED ? a.vn + kvoff : nullptr;
  constexpr int kWaveKeys = 64 / RC;                   // key rows per wave per round
  constexpr int kLdKeys = kPfWaves * kWaveKeys;        // keys per loader round
  constexpr int kLdRounds = kPfKeys / kLdKeys;
  static_assert(kLdKeys % 16 == 0 && kPfKeys % kLdKeys == 0,
                "loader rounds of whole 16-key swizzle groups");
  int bid[kLdRounds];
  int tb = -64, vbid = 0;
  auto fetch_ids = [&](int t) {
    if (!ONE_BLOCK) {
#pragma unroll
      for (int i = 0; i < kLdRounds; ++i) bid[i] = btrow[min(t * kPfKeys + kLdKeys * i + lkey, kend - 1) / a.bs];
    }
  };
  auto tile_bid = [&](int t) {
    if (t == t0) return bid0;      // from the unit record
    if (t - tb >= 64) {
      tb = t;
      vbid = btrow[min((t + lane) * kPfKeys, kend - 1) / a.bs];
    }
    return __builtin_amdgcn_readlane(vbid, t - tb);
  };
  // key at position p, in block blk at offset boff
  auto load_row = [&](int i, int p, int blk, int boff, uint16_t* kdst, uint16_t* vdst) {
    // (rounds start at multiples of 16 keys, so lkey stands for the key mod RC)
    const int ck = lc ^ (lkey & (RC - 1)), cv = lc ^ (2 * (lkey & (RC / 2 - 1)));
    const uint16_t* kp;
    const uint16_t* vp;
    if (NZ) {
      kp = a.kc + 8 * kv_piece<true>(blk, boff, a.bs, row_elems, kvh, D, ck);
      vp = a.vc + 8 * kv_piece<true>(blk, boff, a.bs, row_elems, kvh, D, cv);
    } else {
      // (the slot in 32 bits: the entry points reject pools of 2^31 slots
      // or more, as the int32 slot_mapping cannot address them; the 64-bit
      // form of this address cost the 32K-key prefill 7%)
      const int64_t e = (int64_t)(blk * a.bs + boff) * row_elems;
      kp = kcb + e + 8 * ck;
      vp = vcb + e + 8 * cv;
    }
    if (FUSED) {
      const bool fresh = p >= ctx0;
      const int64_t tok = q_begin + (p - ctx0);
      kp = fresh ? knb + tok * a.kn_ts + 8 * ck : kp;
      vp = fresh ? vnb + tok * a.vn_ts + 8 * cv : vp;
    }
    const int rb = (kLdKeys * i + kWaveKeys * wid) * D;     // the wave's first row
    lds_load16(kp, kdst + rb);
    lds_load16(vp, vdst + rb);
  };
  auto load = [&](int t, auto buf_tag) {
    constexpr int B = decltype(buf_tag)::value;
    uint16_t* kdst = B ? k1 : k0;
    uint16_t* vdst = B ? v1 : v0;
    const int kb = t * kPfKeys;
    if (ONE_BLOCK) {
      const int blk = min(max(tile_bid(t), 0), a.nb - 1);
      const int boff0 = kb % a.bs;
      const int last = kend - 1 - kb;
#pragma unroll
      for (int i = 0; i < kLdRounds; ++i) {
        const int off = min(kLdKeys * i + lkey, last);
        load_row(i, kb + off, blk, boff0 + off, kdst, vdst);
      }
    } else {
#pragma unroll
      for (int i = 0; i < kLdRounds; ++i) {
        const int p = min(kb + kLdKeys * i + lkey, kend - 1);
        const int blk = min(max(bid[i], 0), a.nb - 1);
        load_row(i, p, blk, p % a.bs, kdst, vdst);
      }
    }
  };

  float4_t o[kPfRt][DT];
  float m[kPfRt], lsum[kPfRt];
#pragma unroll
  for (int rt = 0; rt < kPfRt; ++rt) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[rt][dt] = float4_t{0.f, 0.f, 0.f, 0.f};
    m[rt] = -INFINITY;
    lsum[rt] = 0.f;
  }

  // issue_next() issues the next tile's loads after the QK^T MFMAs, so that
  // the load addresses and issue overlap the MFMAs' execution: 0-1% faster
  // than issuing them first.  (A raised wave priority around each MFMA block,
  // 3% faster with register-staged loads, made this order 1-2% slower, and
  // either order is as fast without it, so no priority is set.)
  auto compute = [&](int t, auto buf_tag, auto mask_tag, auto issue_next) {
    constexpr bool MASK = decltype(mask_tag)::value;
    constexpr int B = decltype(buf_tag)::value;
    const int kbase = t * kPfKeys;
    if (MASK && kbase > wlim_hi) {               // no row of this wave sees these keys
      issue_next();
      return;
    }
    const uint16_t* kt = B ? k1 : k0;
    const uint16_t* vt = B ? v1 : v0;
    constexpr int kSt = kPfKeys / 16;      // 16-key sub-tiles
    float4_t acc[kPfRt][kSt];
    __builtin_amdgcn_sched_barrier(0);     // the block below is scheduled on its own
#pragma unroll
    for (int st = 0; st < kSt; ++st) {
      uint4 kf[KJ];
#pragma unroll
      for (int j = 0; j < KJ; ++j)
        kf[j] = *reinterpret_cast<const uint4*>(kt + (16 * st + n) * D + 8 * ((4 * j + g) ^ (n & (RC - 1))));
#pragma unroll
      for (int rt = 0; rt < kPfRt; ++rt) {
        // (a row tile with no valid row computes rows that are never written)
        acc[rt][st] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < KJ; ++j) acc[rt][st] = qk_step(kf[j], qf[rt][j], acc[rt][st]);
      }
    }
    __builtin_amdgcn_sched_group_barrier(kSgDsRead, KJ * kPfQkAhead, 0);
#pragma unroll
    for (int st = 0; st < kSt; ++st) {
      __builtin_amdgcn_sched_group_barrier(kSgMfma, KJ * kPfRt, 0);
      if (st + kPfQkAhead < kSt) __builtin_amdgcn_sched_group_barrier(kSgDsRead, KJ, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    issue_next();
    uint4 pb[kPfRt][kSt / 2];
#pragma unroll
    for (int rt = 0; rt < kPfRt; ++rt) {
      float sv[kSt][4];
      float tmax = -INFINITY;
      if (MASK) {     // causal diagonal / sequence end: per-key limits
        const int rel = lim[rt] - kbase - 4 * g;
#pragma unroll
        for (int st = 0; st < kSt; ++st)
#pragma unroll
          for (int v = 0; v < 4; ++v) sv[st][v] = 16 * st + v <= rel ? acc[rt][st][v] : -INFINITY;
      } else {
#pragma unroll
        for (int st = 0; st < kSt; ++st)
#pragma unroll
          for (int v = 0; v < 4; ++v) sv[st][v] = acc[rt][st][v];
      }
#pragma unroll
      for (int st = 0; st < kSt; ++st)
#pragma unroll
        for (int v = 0; v < 4; ++v) tmax = fmaxf(tmax, sv[st][v]);
      tmax = aia::group4_max(tmax);
      // Lazy rescale: the running max m only moves when some row's tile max
      // exceeds it by more than kLazyLog2, so P stays below 2^kLazyLog2 and O
      // and l (which share m) need no rescale on most tiles.  m = -inf until
      // a row sees a key; exp2(-inf) = 0 then.
      const float tm = tmax * a.scale_log2;
      const bool grow = __any(tm > m[rt] + kLazyLog2);
      const float mnew = grow ? fmaxf(m[rt], tm) : m[rt];
      const float msub = mnew == -INFINITY ? 0.f : mnew;
      float p[kSt][4];
      float psum = 0.f;
#pragma unroll
      for (int st = 0; st < kSt; ++st)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          p[st][v] = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[st][v], a.scale_log2, -msub));
          psum += p[st][v];
        }
      if (grow) {
        const float alpha = __builtin_amdgcn_exp2f(m[rt] - msub);
        lsum[rt] = lsum[rt] * alpha + psum;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[rt][dt] *= alpha;
      } else {
        lsum[rt] += psum;
      }
      m[rt] = mnew;
#pragma unroll
      for (int pp = 0; pp < kSt / 2; ++pp) {
        pb[rt][pp].x = aia::pack_bf16x2(p[2 * pp][0], p[2 * pp][1]);
        pb[rt][pp].y = aia::pack_bf16x2(p[2 * pp][2], p[2 * pp][3]);
        pb[rt][pp].z = aia::pack_bf16x2(p[2 * pp + 1][0], p[2 * pp + 1][1]);
        pb[rt][pp].w = aia::pack_bf16x2(p[2 * pp + 1][2], p[2 * pp + 1][3]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);     // the block below is scheduled on its own
    // PV over V^T fragments f = (32-key pair pp, 16 dims dt), read kPfPvAhead
    // fragments ahead of their MFMAs.  Lane (n, g) reads keys 4 g + n / 4
    // (+ 16), dims 16 dt + 4 (n % 4), at their swizzled place (the
    // transposing read as in vt_frag).
    const int vrow = 4 * g + (n >> 2);
#pragma unroll
    for (int f = 0; f < kSt / 2 * DT; ++f) {
      const int pp = f / DT, dt = f % DT;
      const int vsw = 16 * (dt ^ (vrow & (RC / 2 - 1)));
      const short4_t x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_short4_t*)(vt + (32 * pp + vrow) * D + vsw + 4 * (n & 3)));
      const short4_t x1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_short4_t*)(vt + (32 * pp + 16 + vrow) * D + vsw + 4 * (n & 3)));
      const bf16x8_t va = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
      for (int rt = 0; rt < kPfRt; ++rt)
        o[rt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, as_b8(pb[rt][pp]), o[rt][dt], 0, 0, 0);
    }
    __builtin_amdgcn_sched_group_barrier(kSgDsRead, 2 * kPfPvAhead, 0);
#pragma unroll
    for (int f = 0; f < kSt / 2 * DT; ++f) {
      __builtin_amdgcn_sched_group_barrier(kSgMfma, kPfRt, 0);
      if (f + kPfPvAhead < kSt / 2 * DT) __builtin_amdgcn_sched_group_barrier(kSgDsRead, 2, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  if (t1 > t0) {
    using buf0 = std::integral_constant<int, 0>;
    using buf1 = std::integral_constant<int, 1>;
    if (ONE_BLOCK) {   // the next 64 tiles' ids, in flight beside the first tile
      tb = t0;
      vbid = btrow[min((t0 + lane) * kPfKeys, kend - 1) / a.bs];
    }
    fetch_ids(t0);
    load(t0, buf0{});
    fetch_ids(t0 + 1);
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
    // Tiles below the wave's smallest row limit need no mask; the two runs
    // together take every tile, so all waves pass the same barriers.  The
    // buffer of each step is a compile-time choice (separate LDS arrays), so
    // the compiler sees that a step's reads and the next tile's direct loads
    // touch different memory and holds no read back for those loads; with a
    // buffer index chosen at run time it waits for the loads before each read.
    // The loop keeps one copy of each buffer's step (unrolled copies cost more
    // in instruction fetch than they save).
    const int t_um = max(t0, min(t1, (wlim_lo + 1) / kPfKeys));
    auto step = [&](int t, auto buf_tag, auto mask_tag) {
      constexpr int B = decltype(buf_tag)::value;
      using other = std::integral_constant<int, B ^ 1>;
      auto issue_next = [&]() {
        if (t + 1 < t1) {
          load(t + 1, other{});
          fetch_ids(t + 2);
        }
      };
      compute(t, buf_tag, mask_tag, issue_next);
      __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
      __syncthreads();
    };
    auto run = [&](int t, int t_end, auto mask_tag) {
      bool odd = ((t - t0) & 1) != 0;
#pragma clang loop unroll(disable)
      while (t < t_end) {
        if (!odd) {
          step(t, buf0{}, mask_tag);
          if (++t >= t_end) break;
        }
        step(t, buf1{}, mask_tag);
        ++t;
        odd = false;
      }
    };
    run(t0, t_um, std::false_type{});
    run(t_um, t1, std::true_type{});
  }

#pragma unroll
  for (int rt = 0; rt < kPfRt; ++rt) {
    lsum[rt] = aia::group4_sum(lsum[rt]);
    // a unit that does not cover all of its item's keys writes a partial:
    // y = O / c in fp16, c = the row's largest |O| (1 for an all-zero row),
    // with (m + log2 c, l / c) in place of (m, l).  The merge's log-sum-exp
    // rule then folds c back exactly (its weights are exp2(m - M)), and the
    // partials take half the bytes of fp32 ones.
    float cmax = 0.f;
    if (!whole) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int v = 0; v < 4; ++v) cmax = fmaxf(cmax, fabsf(o[rt][dt][v]));
      cmax = aia::group4_max(cmax);
    }
    if (!rv[rt]) continue;
    if (!whole) {
      const float c = cmax > 0.f ? cmax : 1.f, ic = 1.f / c;
      const int64_t prow = ((int64_t)unit * a.hkv + kvh) * kPfRows + (wid * kPfRt + rt) * kRows + n;
      uint16_t* pp = a.part_o + prow * D;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        uint2 hv;
        hv.x = pack_f16x2(o[rt][dt][0] * ic, o[rt][dt][1] * ic);
        hv.y = pack_f16x2(o[rt][dt][2] * ic, o[rt][dt][3] * ic);
        *reinterpret_cast<uint2*>(pp + 16 * dt + 4 * g) = hv;
      }
      if (g == 0) a.part_ml[prow] = make_float2(m[rt] + __log2f(c), lsum[rt] * ic);
      continue;
    }
    const float inv = lsum[rt] > 0.f ? 1.f / lsum[rt] : 0.f;
    uint16_t* op = a.out + (int64_t)(q_begin + tokr[rt]) * a.o_ts + (int64_t)headr[rt] * a.o_hs;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      uint2 wv;
      wv.x = aia::pack_bf16x2(o[rt][dt][0] * inv, o[rt][dt][1] * inv);
      wv.y = aia::pack_bf16x2(o[rt][dt][2] * inv, o[rt][dt][3] * inv);
      *reinterpret_cast<uint2*>(op + 16 * dt + 4 * g) = wv;
    }
  }
}

template <bool ONE_BLOCK, bool FUSED, int D, bool NZ>
__global__ __launch_bounds__(kPfWaves * 64) __attribute__((amdgpu_waves_per_eu(AIA_PF_WPE, AIA_PF_WPE)))
void gqa_prefill_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t k0[kPfKeys * D];
  __shared__ __attribute__((aligned(16))) uint16_t k1[kPfKeys * D];
  __shared__ __attribute__((aligned(16))) uint16_t v0[kPfKeys * D];
  __shared__ __attribute__((aligned(16))) uint16_t v1[kPfKeys * D];
  gqa_prefill_body<ONE_BLOCK, FUSED, D, NZ>(a, blockIdx.x, k0, k1, v0, v1);
}

// Mixed steps (prefill items beside split-K decode ranges) in one grid, for
// kPfWaves-wave decode groups (Hkv = kPfWaves).  Launched separately, the
// two kernels barely share a CU: one prefill wave (212-232 VGPRs, allocated
// in blocks of 8) plus two decode waves (2 x 144) fill or exceed a SIMD's
// 512, so the second kernel mostly waits for the first to drain.  In one grid every
// work-group gets the prefill budget and does one job or the other, so the
// compute-bound prefill runs while the HBM-bound decode streams beside it.
#ifndef AIA_MIXED
#define AIA_MIXED 1
#endif
// The decode role stages its V^T tiles in the first K buffer.
constexpr int kMixedK0 = kPfWaves * kTile * kVStride > kPfKeys * kKStride
                             ? kPfWaves * kTile * kVStride : kPfKeys * kKStride;
template <bool ONE_BLOCK, bool FUSED, bool NZ>
__global__ __launch_bounds__(kPfWaves * 64) __attribute__((amdgpu_waves_per_eu(AIA_PF_WPE, AIA_PF_WPE)))
void gqa_mixed_kernel(AttnArgs a, PrefillArgs pa, int npf) {
  __shared__ __attribute__((aligned(16))) uint16_t k0[kMixedK0];
  __shared__ __attribute__((aligned(16))) uint16_t k1[kPfKeys * kKStride];
  __shared__ __attribute__((aligned(16))) uint16_t v0[kPfKeys * kKStride];
  __shared__ __attribute__((aligned(16))) uint16_t v1[kPfKeys * kKStride];
  // Prefill units take the first npf block ids and the decode ranges the
  // rest: the units are dealt out first, one or two per CU, and the ranges
  // fill the remaining slots and every slot a unit frees.  (Alternating the
  // roles by block id measured slower: 590 us against 449 on configs[1] in
  // runs of 8 ids, 459-462 in runs of 64; runs of 256 matched.)
  const int b = blockIdx.x;
  const bool prefill = b < npf;
  const int idx = prefill ? b : b - npf;
  if (prefill)
    gqa_prefill_body<ONE_BLOCK, FUSED, kHeadDim, NZ>(pa, idx, k0, k1, v0, v1);
  else
    gqa_attn_body<kPfWaves, 1, kHeadDim, NZ>(a, idx,
                                         reinterpret_cast<uint16_t(*)[kTile * kVStride]>(&k0[0]));
}

struct MergeArgs {
  const int32_t* hdr;
  const int32_t* seg;
  const uint16_t* part_o;
  const float2* part_ml;
  uint16_t* out;
  int64_t o_ts, o_hs;
  int32_t group, hb, dv, nw, hkv, rb;
  const int32_t* mrg;
  int64_t mrg_cap;
  // prefill chunk merges: records {first query token, first row, first
  // unit, units | item rows << 16}
  const int4* pf_mrg;
  int64_t pf_items_cap;     // work items the records can hold
  const uint16_t* pf_o;
  const float2* pf_ml;
  int32_t tokens;           // output rows (query tokens); heads = group x hkv
  // fixed-slot merges (kFixParts): 1 when the launch has one work-group per
  // (segment, kv head) and the kernel a fixed-slot path, and the partial
  // slots the buffer holds
  int32_t fixed_slots;
  int64_t part_cap;
};

// Merge of split partials.  The planner lists the merge work: one record per
// (split segment, kv head, slice of 64 output elements), an element being 16
// dims of one row of the segment's row span (rows of a block past its qb
// tokens are skipped), and nothing for segments that one range covers.  The
// G waves of a work-group take every G-th partial each, so all partial loads
// of an item are in flight together, and combine their running (max, sum,
// accumulator) through LDS.  The item count is loaded together with the
// first record.
// Waves per merge work-group: 4, or 8 where items hold 64-element slices
// with a dozen or more partials (absorbed MLA, verify rows of 8+ heads x
// tokens, about 8+ ranges per segment), which then fold in one load round
// (configs[2] 52.1-52.7 -> 51.3-51.6 us, configs[3] 41.2-41.5 -> 40.6; with
// 8 everywhere config 1 went 22.7-22.9 -> 23.2, configs[1]'s prefill chunks
// 43.5 -> 45.8, and configs[4] (one or two partials per item) 605-607 ->
// 610).
#ifndef AIA_MERGE_WIDE
#define AIA_MERGE_WIDE 1
#endif
// FIXL: partial loads per thread of the fixed-slot path (0: none; see
// kFixParts), a compile-time count so that the loads are issued
// unconditionally and the compiler's counter waits for the header words
// leave them in flight.
template <int kMergeGroups, int FIXL>
__global__ __launch_bounds__(64 * kMergeGroups) void merge_kernel(MergeArgs a) {
  constexpr int kMergeThreads = 64 * kMergeGroups;
  constexpr int kLdsGroups = kMergeGroups > 1 ? kMergeGroups - 1 : 1;
  __shared__ float4 sacc[kLdsGroups][kMergeDims / 4][64];
  __shared__ float2 sml[kLdsGroups][64];
  const int lane = threadIdx.x & 63, kg = threadIdx.x >> 6;
  const int epr = a.dv / kMergeDims;                      // elements per row
  const int seg_rows = kRows * a.rb;
  const int qb = kRows / a.hb;
  const int64_t pstride = (int64_t)a.nw * seg_rows;
  // the first prefill record and the count go out with the first split-K
  // record, so a prefill work-group's chain is record, then partials
  // prefill chunk merges: a thread takes 8 dims of a row, so a pass of the
  // work-group covers 8 kMergeThreads / dv rows (16 at head_dim 128, 32 at 64)
  const int pf_tpr = a.dv / 8, pf_rpp = kMergeThreads / pf_tpr;
  const int kSlices = kPfRows / pf_rpp;
  const int per_rec = a.hkv * kSlices;
  // Every load the work-group's first step needs goes out before any of
  // them is waited for: the header words, its first merge record, its first
  // prefill record and, for fixed-slot plans (kFixParts), its segment record
  // and partials.  They are vector loads (indexed by an opaque zero), so the
  // in-order vector counter lets the header be waited for while the
  // partials are still in flight; as scalar loads they would share the
  // kernel arguments' counter, and the compiler's waits for those would
  // drain them.  An index past a list reads the header instead, and its
  // value is not used.
  int vz;
  asm volatile("v_mov_b32 %0, 0" : "=v"(vz));
  const int64_t item0 = blockIdx.x;
  const int4* mp = (item0 < a.mrg_cap ? reinterpret_cast<const int4*>(a.mrg + item0 * kMrgInts)
                                      : reinterpret_cast<const int4*>(a.hdr)) + vz;
  const int4* pp0 = (a.pf_mrg && item0 < a.pf_items_cap ? a.pf_mrg + (int)blockIdx.x / per_rec
                                                          : reinterpret_cast<const int4*>(a.hdr)) + vz;
  const int* hv = a.hdr + vz;
  const int4 m0_v = mp[0], m1_v = mp[1];
  const int4 pr_v = pp0[0];
  const int h0 = hv[0], h2 = hv[2], h5 = hv[5], h7 = hv[7], h8 = hv[8], h10 = hv[10];
  auto fold_into = [](float& mx, float& ls, float4 (&acc)[kMergeDims / 4], float2 ml,
                      const float4 (&x)[kMergeDims / 4]) {
    const float mn = fmaxf(mx, ml.x);
    const float sa = __builtin_amdgcn_exp2f(mx - mn), sb = __builtin_amdgcn_exp2f(ml.x - mn);
    ls = ls * sa + ml.y * sb;
#pragma unroll
    for (int i = 0; i < kMergeDims / 4; ++i) {
      acc[i].x = acc[i].x * sa + x[i].x * sb; acc[i].y = acc[i].y * sa + x[i].y * sb;
      acc[i].z = acc[i].z * sa + x[i].z * sb; acc[i].w = acc[i].w * sa + x[i].w * sb;
    }
    mx = mn;
  };
  auto unpack16 = [](uint4 h0, uint4 h1, float4 (&x)[kMergeDims / 4]) {
    const uint32_t hw[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
#pragma unroll
    for (int i = 0; i < kMergeDims / 4; ++i) {
      const half2_t a2 = __builtin_bit_cast(half2_t, hw[2 * i]);
      const half2_t b2 = __builtin_bit_cast(half2_t, hw[2 * i + 1]);
      x[i] = make_float4((float)a2[0], (float)a2[1], (float)b2[0], (float)b2[1]);
    }
  };
  // Fixed partial slots (kFixParts): work-group b merges (segment b / nw,
  // kv head b % nw), whose row span holds at most 16 elements (rows x dv /
  // 16: a decode segment's few rows).  Thread (wave kg, lane) takes element
  // lane % 16 and the slots q + 4 G r (q = 4 kg + lane / 16, G waves, r <
  // FIXL); a wave's four slot groups fold with two shuffles, the waves
  // through LDS.  Slots past a segment's parts hold stale values that are
  // not used.
  static_assert(FIXL == 0 || FIXL * 4 * kMergeGroups == kFixParts, "one load per slot");
  const int fb = blockIdx.x;
  const int fs = fb / a.nw, fw = fb - fs * a.nw;
  const int q = 4 * kg + (lane >> 4);
  int4 r0_v = make_int4(0, 0, 0, 0), r1_v = r0_v;
  float2 fml[FIXL > 0 ? FIXL : 1];
  uint4 fh0[FIXL > 0 ? FIXL : 1], fh1[FIXL > 0 ? FIXL : 1];
  if (FIXL > 0) {
    const int4* sr = reinterpret_cast<const int4*>(a.seg) + 2 * (int64_t)fs + vz;
    r0_v = sr[0];
    r1_v = sr[1];
    const int e = lane & 15;
    const int n = min(e / epr, seg_rows - 1);
    const int c = (e - (e / epr) * epr) * kMergeDims;
#pragma unroll
    for (int r = 0; r < FIXL; ++r) {
      const int64_t slot = (int64_t)kFixParts * fs + q + 4 * kMergeGroups * r;
      const int64_t prow = slot < a.part_cap ? (slot * a.nw + fw) * seg_rows + n : 0;
      fml[r] = a.part_ml[prow];
      const uint4* src = reinterpret_cast<const uint4*>(a.part_o + prow * a.dv + c);
      fh0[r] = src[0];
      fh1[r] = src[1];
    }
  }
  const int nmrg = __builtin_amdgcn_readfirstlane(h5);
  const int npm_hdr = __builtin_amdgcn_readfirstlane(h7);
  const int status = __builtin_amdgcn_readfirstlane(h8);   // planner status, used at the end
  const int npm = a.pf_mrg ? npm_hdr : 0;
  const int fixed_plan = FIXL > 0 ? __builtin_amdgcn_readfirstlane(h10) : 0;
  const int4 pr0 = make_int4(__builtin_amdgcn_readfirstlane(pr_v.x), __builtin_amdgcn_readfirstlane(pr_v.y),
                             __builtin_amdgcn_readfirstlane(pr_v.z), __builtin_amdgcn_readfirstlane(pr_v.w));
  const int4 m0_first = make_int4(__builtin_amdgcn_readfirstlane(m0_v.x), __builtin_amdgcn_readfirstlane(m0_v.y),
                                  __builtin_amdgcn_readfirstlane(m0_v.z), __builtin_amdgcn_readfirstlane(m0_v.w));
  const int4 m1_first = make_int4(__builtin_amdgcn_readfirstlane(m1_v.x), __builtin_amdgcn_readfirstlane(m1_v.y),
                                  __builtin_amdgcn_readfirstlane(m1_v.z), __builtin_amdgcn_readfirstlane(m1_v.w));
  if (FIXL > 0) {
    const int4 r0 = make_int4(__builtin_amdgcn_readfirstlane(r0_v.x), __builtin_amdgcn_readfirstlane(r0_v.y),
                              __builtin_amdgcn_readfirstlane(r0_v.z), __builtin_amdgcn_readfirstlane(r0_v.w));
    const int4 r1 = make_int4(__builtin_amdgcn_readfirstlane(r1_v.x), __builtin_amdgcn_readfirstlane(r1_v.y),
                              __builtin_amdgcn_readfirstlane(r1_v.z), __builtin_amdgcn_readfirstlane(r1_v.w));
    const int nseg = __builtin_amdgcn_readfirstlane(h0);
    const int tpw = max(1, __builtin_amdgcn_readfirstlane(h2));
    const int np = (r1.z - 1) / tpw - r1.y / tpw + 1;
    const int kvg = r0.y & 0xffff, hbi = (r0.y >> 16) & 0x3fff;
    const int nq = r0.w & 0xff;
    const int nblk = (nq + qb - 1) / qb;
    const int rows = (nblk - 1) * kRows + min(kRows, (nq - (nblk - 1) * qb) * a.hb);
    const bool use = fixed_plan == 1 && fs < nseg && np > 1 && fw < min(a.nw, a.hkv - kvg * a.nw);
    const int e = lane & 15;
    const int n = e / epr;
    const int c = (e - n * epr) * kMergeDims;
    const int rblk = n / kRows, t = (n - rblk * kRows) / a.hb;
    const int hh = n - rblk * kRows - t * a.hb;
    const bool live = use && e < rows * epr && t < qb && rblk * qb + t < nq &&
                      hbi * a.hb + hh < a.group;
    float4 acc[kMergeDims / 4];
#pragma unroll
    for (int i = 0; i < kMergeDims / 4; ++i) acc[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    float mx = -1e30f, ls = 0.f;
#pragma unroll
    for (int r = 0; r < FIXL; ++r) {
      if (live && q + 4 * kMergeGroups * r < np) {
        float4 x[kMergeDims / 4];
        unpack16(fh0[r], fh1[r], x);
        fold_into(mx, ls, acc, fml[r], x);
      }
    }
    // the wave's four slot groups of an element sit in lanes 16 apart
    for (int d = 16; d < 64; d <<= 1) {
      const float2 oml = make_float2(__shfl_xor(mx, d), __shfl_xor(ls, d));
      float4 ox[kMergeDims / 4];
#pragma unroll
      for (int i = 0; i < kMergeDims / 4; ++i)
        ox[i] = make_float4(__shfl_xor(acc[i].x, d), __shfl_xor(acc[i].y, d),
                            __shfl_xor(acc[i].z, d), __shfl_xor(acc[i].w, d));
      fold_into(mx, ls, acc, oml, ox);
    }
    // and the waves' results through LDS
    if (kg > 0 && lane < 16) {
#pragma unroll
      for (int i = 0; i < kMergeDims / 4; ++i) sacc[kg - 1][i][lane] = acc[i];
      sml[kg - 1][lane] = make_float2(mx, ls);
    }
    __syncthreads();
    if (kg == 0 && lane < 16 && live) {
#pragma unroll
      for (int j = 0; j < kMergeGroups - 1; ++j) {
        float4 x[kMergeDims / 4];
#pragma unroll
        for (int i = 0; i < kMergeDims / 4; ++i) x[i] = sacc[j][i][lane];
        fold_into(mx, ls, acc, sml[j][lane], x);
      }
      const float inv = ls > 0.f ? 1.f / ls : 0.f;
      const int qi = rblk * qb + t;
      const int head = (kvg * a.nw + fw) * a.group + hbi * a.hb + hh;
      uint16_t* op = a.out + (int64_t)(r0.z + qi) * a.o_ts + (int64_t)head * a.o_hs + c;
#pragma unroll
      for (int i = 0; i < kMergeDims / 4; ++i) {
        uint2 wv;
        wv.x = aia::pack_bf16x2(acc[i].x * inv, acc[i].y * inv);
        wv.y = aia::pack_bf16x2(acc[i].z * inv, acc[i].w * inv);
        *reinterpret_cast<uint2*>(op + 4 * i) = wv;
      }
    }
  }
  // the first test reads the first record too (a record has at least two
  // parts), which keeps its loads ahead of the first branch
  const bool first_live = (fixed_plan != 1) & (item0 < a.mrg_cap) & (item0 < nmrg) &
                          (m1_first.y >= 2);
  for (int64_t item = item0; first_live && item < a.mrg_cap; item += gridDim.x) {
    if (item >= nmrg) break;                               // uniform over the group
    const int4 m0 = item == item0 ? m0_first : *reinterpret_cast<const int4*>(a.mrg + item * kMrgInts);
    const int4 m1 = item == item0 ? m1_first : *reinterpret_cast<const int4*>(a.mrg + item * kMrgInts + 4);
    const int qtok0 = m0.x, nq = m0.y, kvh = m0.z, hbi = m0.w;
    const int row_base = m1.x, np = m1.y, sl = m1.z, rows = m1.w;
    // A slice of fewer than 64 elements (a decode segment's few rows) takes
    // the smallest power-of-two lane group that holds it, and the wave's
    // other lane groups fold other partials: all of an item's partial loads
    // then go out in one round (config 1: 16 elements, 16 partials at once).
    const int span = rows * epr - sl * 64;
    const int pw = span > 32 ? 64 : span > 16 ? 32 : span > 8 ? 16 : 8;
    const int pg = lane / pw, ng = 64 / pw;
    const int e = sl * 64 + (lane & (pw - 1));
    int n = e / epr;
    const int c = (e - n * epr) * kMergeDims;
    const int rblk = n / kRows, t = (n - rblk * kRows) / a.hb;
    const int hh = n - rblk * kRows - t * a.hb;
    // a group above 16 that 16 does not divide leaves its last head block
    // part-filled: rows past the group hold no partials and are skipped
    const bool live = e < rows * epr && t < qb && rblk * qb + t < nq && hbi * a.hb + hh < a.group;
    if (!live) n = 0;
    const int64_t row0 = (int64_t)row_base + n;
    float4 acc[kMergeDims / 4];
#pragma unroll
    for (int i = 0; i < kMergeDims / 4; ++i) acc[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    float mx = -1e30f, ls = 0.f;
    auto fold = [&](float2 ml, const float4 (&x)[kMergeDims / 4]) { fold_into(mx, ls, acc, ml, x); };
    if (live) {    // fp16 partials y = O / c, with (m + log2 c, l / c)
#pragma unroll 2
      for (int k = kg * ng + pg; k < np; k += kMergeGroups * ng) {
        const int64_t pr = row0 + k * pstride;
        const float2 ml = a.part_ml[pr];
        const uint4* src = reinterpret_cast<const uint4*>(
            a.part_o + pr * a.dv + c);
        float4 x[kMergeDims / 4];
        unpack16(src[0], src[1], x);
        fold(ml, x);
      }
    }
    // fold the wave's lane groups together (every lane of an element's
    // groups ends with the wave's result)
    for (int d = pw; d < 64; d <<= 1) {
      const float2 oml = make_float2(__shfl_xor(mx, d), __shfl_xor(ls, d));
      float4 ox[kMergeDims / 4];
#pragma unroll
      for (int i = 0; i < kMergeDims / 4; ++i)
        ox[i] = make_float4(__shfl_xor(acc[i].x, d), __shfl_xor(acc[i].y, d),
                            __shfl_xor(acc[i].z, d), __shfl_xor(acc[i].w, d));
      fold(oml, ox);
    }
    if (kg > 0) {
#pragma unroll
      for (int i = 0; i < kMergeDims / 4; ++i) sacc[kg - 1][i][lane] = acc[i];
      sml[kg - 1][lane] = make_float2(mx, ls);
    }
    __syncthreads();
    if (kg == 0 && live && pg == 0) {
#pragma unroll
      for (int j = 0; j < kMergeGroups - 1; ++j) {
        float4 x[kMergeDims / 4];
#pragma unroll
        for (int i = 0; i < kMergeDims / 4; ++i) x[i] = sacc[j][i][lane];
        fold(sml[j][lane], x);
      }
      const float inv = ls > 0.f ? 1.f / ls : 0.f;
      const int qi = rblk * qb + t;
      const int head = kvh * a.group + hbi * a.hb + hh;
      uint16_t* op = a.out + (int64_t)(qtok0 + qi) * a.o_ts + (int64_t)head * a.o_hs + c;
      // 8-byte stores: the GQA output token stride need only be a multiple of 4
#pragma unroll
      for (int i = 0; i < kMergeDims / 4; ++i) {
        uint2 wv;
        wv.x = aia::pack_bf16x2(acc[i].x * inv, acc[i].y * inv);
        wv.y = aia::pack_bf16x2(acc[i].z * inv, acc[i].w * inv);
        *reinterpret_cast<uint2*>(op + 4 * i) = wv;
      }
    }
    __syncthreads();
  }

  // Prefill chunk merges, one work item per (record, kv head, pf_rpp rows):
  // thread (row r, 8 dims) folds the record's fp16 partials (scaled per row,
  // see the prefill kernel) with the same rule, 8 at a time so a batch costs
  // one round trip.
  const int64_t pitems = (int64_t)npm * per_rec;
  for (int64_t it = blockIdx.x; it < pitems; it += gridDim.x) {
    const int rec = (int)(it / per_rec);
    const int rem = (int)(it - (int64_t)rec * per_rec);
    const int kvh = rem / kSlices, slice = rem - kvh * kSlices;
    const int4 r = it == blockIdx.x ? pr0 : a.pf_mrg[rec];
    const int q_begin = r.x, row0 = r.y, u0 = r.z, k = r.w & 0xffff, rows = r.w >> 16;
    const int rl = slice * pf_rpp + (int)threadIdx.x / pf_tpr, c = ((int)threadIdx.x % pf_tpr) * 8;
    const int row = row0 + rl;
    if (rl >= rows) continue;
    float4 acc[2] = {make_float4(0.f, 0.f, 0.f, 0.f), make_float4(0.f, 0.f, 0.f, 0.f)};
    float mx = -1e30f, ls = 0.f;
    for (int j0 = 0; j0 < k; j0 += 8) {
      float2 ml[8];
      float4 x[8][2];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (j0 + j >= k) break;                    // k is the same for the whole work-group
        const int64_t prow = ((int64_t)(u0 + j0 + j) * a.hkv + kvh) * kPfRows + rl;
        ml[j] = a.pf_ml[prow];
        const uint4 h = *reinterpret_cast<const uint4*>(a.pf_o + prow * a.dv + c);
        const half2_t h0 = __builtin_bit_cast(half2_t, h.x), h1 = __builtin_bit_cast(half2_t, h.y);
        const half2_t h2 = __builtin_bit_cast(half2_t, h.z), h3 = __builtin_bit_cast(half2_t, h.w);
        x[j][0] = make_float4((float)h0[0], (float)h0[1], (float)h1[0], (float)h1[1]);
        x[j][1] = make_float4((float)h2[0], (float)h2[1], (float)h3[0], (float)h3[1]);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (j0 + j >= k) break;
        const float mn = fmaxf(mx, ml[j].x);
        const float sa = __builtin_amdgcn_exp2f(mx - mn), sb = __builtin_amdgcn_exp2f(ml[j].x - mn);
        ls = ls * sa + ml[j].y * sb;
        acc[0].x = acc[0].x * sa + x[j][0].x * sb; acc[0].y = acc[0].y * sa + x[j][0].y * sb;
        acc[0].z = acc[0].z * sa + x[j][0].z * sb; acc[0].w = acc[0].w * sa + x[j][0].w * sb;
        acc[1].x = acc[1].x * sa + x[j][1].x * sb; acc[1].y = acc[1].y * sa + x[j][1].y * sb;
        acc[1].z = acc[1].z * sa + x[j][1].z * sb; acc[1].w = acc[1].w * sa + x[j][1].w * sb;
        mx = mn;
      }
    }
    const float inv = ls > 0.f ? 1.f / ls : 0.f;
    const int tok = row / a.group, head = kvh * a.group + (row - tok * a.group);
    uint16_t* op = a.out + (int64_t)(q_begin + tok) * a.o_ts + (int64_t)head * a.o_hs + c;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      uint2 wv;
      wv.x = aia::pack_bf16x2(acc[i].x * inv, acc[i].y * inv);
      wv.y = aia::pack_bf16x2(acc[i].z * inv, acc[i].w * inv);
      *reinterpret_cast<uint2*>(op + 4 * i) = wv;
    }
  }

  // A plan whose metadata asked for more work than the workspace holds
  // planned nothing (status -1): no kernel wrote the output, so it is filled
  // with NaN rather than left holding whatever the memory held.
  if (status < 0) {
    const int hq = a.group * a.hkv, per_row = a.dv / 4;   // 4 elements per 8-byte store
    const int64_t n = (int64_t)a.tokens * hq * per_row;
    const uint2 nan2 = make_uint2(0x7fc07fc0u, 0x7fc07fc0u);
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
      const int64_t row = i / per_row;
      const int tok = (int)(row / hq), h = (int)(row - (int64_t)tok * hq);
      const int d = (int)(i - row * per_row) * 4;
      *reinterpret_cast<uint2*>(a.out + (int64_t)tok * a.o_ts + (int64_t)h * a.o_hs + d) = nan2;
    }
  }
}

// ---------------------------------------------------------------- absorbed MLA
//
// One KV head of 576 bf16 per token (512 latent + 64 rope), V = the first 512
// values, Hq query heads share it.  A work-group of 4 waves owns one tile
// range: wave w loads latent dims [128w, 128w + 128) of every key (waves 0/1
// also one 32-dim rope chunk each), computes its partial S^T on MFMA, the
// four partials are summed through LDS (one barrier per tile), every wave
// runs the same softmax, and wave w accumulates output dims
// [128w, 128w + 128) from the K registers it already holds (V = K).
constexpr int kMlaK = 576, kMlaV = 512;
// MLA tiles kept in flight per wave (registers: 20 VGPRs per tile).  Its
// ranges are long and its work-groups small, so it keeps a deeper pipeline
// than the GQA kernel.
#ifndef AIA_MLA_PIPE
#define AIA_MLA_PIPE 3
#endif
constexpr int kMlaPipe = AIA_MLA_PIPE;

struct MlaArgs {
  const uint16_t* q;
  int64_t q_ts, q_hs;
  const uint16_t* cache;
  const int32_t* bt;
  int64_t bt_stride;
  int32_t group, hb, bs, nb;
  float scale_log2;
  const int32_t* seg;
  const int32_t* wave_rec;
  uint16_t* part_o;          // split partials (fp16, scaled per row)
  float2* part_ml;
  uint16_t* out;
  int64_t o_ts, o_hs;
  int32_t waves;
  const int32_t* hdr;
  int32_t batch, tokens;
};

// Processes key tiles [lt0, lt1) of one segment.  A segment holds RB blocks
// of 16 rows; block r is the segment's query token r (qb = 1: a token's 16
// heads fill a block), and every K tile (= V tile) feeds all blocks, so a
// verify or prefill step reads its keys 1/RB as often.
template <int RB>
__device__ __forceinline__ void mla_segment(const MlaArgs& a, const int* rec, int lt0, int lt1,
                                            int w, int tpw, int jrec, int krec, uint16_t* vt,
                                            float* sx, float* smax,
                                            int lane, int wid, bool use_pre, int pre) {
  const int n = lane & 15, g = lane >> 4;
  const int b = rec[0], hbi = (rec[1] >> 16) & 0x3fff;
  const int qtok0 = rec[2], nq = rec[3] & 0xff, q0 = rec[3] >> 8, lim_base = rec[4];
  const int tile_begin = rec[5], tile_end = rec[6], part_base = rec[7];
  const int qb = kRows / a.hb;
  const int nt = n / a.hb, hh = n - nt * a.hb;
  const int head = hbi * a.hb + hh;
  int qi[RB], lim[RB];
  bool rv[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    qi[r] = r * qb + nt;
    rv[r] = nt < qb && qi[r] < nq && head < a.group;
    lim[r] = rv[r] ? lim_base + qi[r] : -1;
  }
  const int nblk = (nq + qb - 1) / qb;                // row blocks holding tokens
  const int visible = max(0, lim_base + nq);
  const bool has_rope = wid < 2;
  // 16-byte chunk index (within a 576-element row) of this lane's pieces
  int cidx[5];
#pragma unroll
  for (int j = 0; j < 4; ++j) cidx[j] = 4 * (4 * wid + j) + g;
  cidx[4] = 4 * (16 + wid) + g;

  const int32_t* btrow = a.bt + (int64_t)b * a.bt_stride;
  const int nblk_vis = (visible + a.bs - 1) / a.bs;
  int blk_base = 0, btv = 0, w1 = 0;

  uint4 qf[RB][5];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    if (rv[r]) {
      const uint4* qp = reinterpret_cast<const uint4*>(
          a.q + (int64_t)(qtok0 + qi[r]) * a.q_ts + (int64_t)head * a.q_hs);
#pragma unroll
      for (int j = 0; j < 5; ++j) qf[r][j] = (j < 4 || has_rope) ? qp[cidx[j]] : make_uint4(0, 0, 0, 0);
    } else {
#pragma unroll
      for (int j = 0; j < 5; ++j) qf[r][j] = make_uint4(0, 0, 0, 0);
    }
  }

  float4_t o[RB][8];
  float m[RB], lsum[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[r][dt] = float4_t{0.f, 0.f, 0.f, 0.f};
    m[r] = -1e30f;
    lsum[r] = 0.f;
  }

  auto load = [&](int lt, uint4 (&kk)[5]) {
    const bool live = lt < w1;
    const int tok = live ? min(lt * kTile + n, visible - 1) : blk_base * a.bs;
    const int bi = tok / a.bs;
    const int blk = min(max(__shfl(btv, bi - blk_base), 0), a.nb - 1);
    const int off = tok - bi * a.bs;
    const uint4* kp = reinterpret_cast<const uint4*>(a.cache + ((int64_t)blk * a.bs + off) * kMlaK);
#pragma unroll
    for (int j = 0; j < 4; ++j) kk[j] = kp[cidx[j]];
    kk[4] = has_rope ? kp[cidx[4]] : make_uint4(0, 0, 0, 0);
  };

  int parity = 0;
  auto compute = [&](int lt, const uint4 (&kk)[5]) {
    // partial S^T over this wave's dims, one per row block; the 4 waves'
    // partials are summed through LDS (double-buffered by tile parity)
    float* xb = sx + parity * (4 * RB * 256);
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      float4_t acc = {0.f, 0.f, 0.f, 0.f};
      if (r == 0 || r < nblk) {
#pragma unroll
        for (int j = 0; j < 5; ++j) {
          if (j == 4 && !has_rope) break;
          acc = qk_step(kk[j], qf[r][j], acc);
        }
      }
      *reinterpret_cast<float4_t*>(xb + (wid * RB + r) * 256 + lane * 4) = acc;
    }
    // this wave's V slice (latent dims [128 w, +128)) is the K it holds
    stage_v(vt, n, g, reinterpret_cast<const uint4 (&)[4]>(kk));
    __syncthreads();
    parity ^= 1;
    const int tb = lt * kTile + 4 * g;
    short4_t pb[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      float4_t tot = *reinterpret_cast<const float4_t*>(xb + r * 256 + lane * 4);
#pragma unroll
      for (int ww = 1; ww < 4; ++ww)
        tot += *reinterpret_cast<const float4_t*>(xb + (ww * RB + r) * 256 + lane * 4);
      float sv[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) sv[v] = (tb + v <= lim[r]) ? tot[v] * a.scale_log2 : -INFINITY;
      float tmax = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
      tmax = aia::group4_max(tmax);
      const float mnew = fmaxf(m[r], tmax);
      const float alpha = __builtin_amdgcn_exp2f(m[r] - mnew);
      float p[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) p[v] = __builtin_amdgcn_exp2f(sv[v] - mnew);
      lsum[r] = lsum[r] * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
      m[r] = mnew;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) o[r][dt] *= alpha;
      pb[r] = as_s4(aia::pack_bf16x2(p[0], p[1]), aia::pack_bf16x2(p[2], p[3]));
    }
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const short4_t va = vt_frag(vt, n, g, dt);
#pragma unroll
      for (int r = 0; r < RB; ++r)
        if (r == 0 || r < nblk)
          o[r][dt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, pb[r], o[r][dt], 0, 0, 0);
    }
    __builtin_amdgcn_wave_barrier();
  };

  constexpr int kP = kMlaPipe;
  uint4 kbuf[kP][5];
  for (int w0 = lt0; w0 < lt1;) {
    blk_base = (w0 * kTile) / a.bs;
    const int win = use_pre ? kRecBlocks : 64;
    w1 = min(lt1, ((blk_base + win) * a.bs - kTile) / kTile + 1);
    if (use_pre) btv = lane < kRecBlocks ? pre : 0;
    else btv = blk_base + lane < nblk_vis ? btrow[blk_base + lane] : 0;
    use_pre = false;
#pragma unroll
    for (int i = 0; i < kP; ++i) {
      load(w0 + i, kbuf[i]);
      __builtin_amdgcn_sched_barrier(0);
    }
    for (int base = w0; base < w1; base += kP) {
#pragma unroll
      for (int i = 0; i < kP; ++i) {
        const int lt = base + i;
        if (lt < w1) compute(lt, kbuf[i]);
        load(lt + kP, kbuf[i]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    w0 = w1;
  }

#pragma unroll
  for (int r = 0; r < RB; ++r) lsum[r] = aia::group4_sum(lsum[r]);
  // balanced plans give the range's number within the segment and the
  // segment's range count in its record; otherwise ranges are tpw tiles
  const int first_wave = krec > 0 ? w - jrec : tile_begin / tpw;
  const int nparts = krec > 0 ? krec : (tile_end - 1) / tpw - first_wave + 1;
  const int d0 = 128 * wid;
  constexpr int seg_rows = RB * kRows;
  if (nparts == 1) {
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      if (!rv[r]) continue;
      const float inv = lsum[r] > 0.f ? 1.f / lsum[r] : 0.f;
      uint16_t* op = a.out + (int64_t)(qtok0 + qi[r]) * a.o_ts + (int64_t)head * a.o_hs + d0;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        uint2 wv;
        wv.x = aia::pack_bf16x2(o[r][dt][0] * inv, o[r][dt][1] * inv);
        wv.y = aia::pack_bf16x2(o[r][dt][2] * inv, o[r][dt][3] * inv);
        *reinterpret_cast<uint2*>(op + 16 * dt + 4 * g) = wv;
      }
    }
  } else {
    // Partials in fp16 with a per-row scale: y = O / c, c = max |O| over the
    // row's 512 dims (all 4 waves), so y is in [-1, 1] with 11 mantissa bits
    // relative to the row's largest value -- finer than the bf16 output --
    // and half the bytes of fp32 partials.  The merge multiplies back by c.
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      float mx = 0.f;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int v = 0; v < 4; ++v) mx = fmaxf(mx, fabsf(o[r][dt][v]));
      mx = aia::group4_max(mx);
      if (g == 0) smax[(wid * RB + r) * kRows + n] = mx;
    }
    __syncthreads();
    const int part = part_base + (w - first_wave);
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const float c = fmaxf(fmaxf(smax[r * kRows + n], smax[(RB + r) * kRows + n]),
                            fmaxf(smax[(2 * RB + r) * kRows + n], smax[(3 * RB + r) * kRows + n]));
      if (!rv[r]) continue;
      const float cc = c > 0.f ? c : 1.f, inv = 1.f / cc;
      const int64_t prow = (int64_t)part * seg_rows + r * kRows + n;
      uint16_t* pp = a.part_o + prow * kMlaV + d0;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        uint2 wv;
        wv.x = pack_f16x2(o[r][dt][0] * inv, o[r][dt][1] * inv);
        wv.y = pack_f16x2(o[r][dt][2] * inv, o[r][dt][3] * inv);
        *reinterpret_cast<uint2*>(pp + 16 * dt + 4 * g) = wv;
      }
      // the scale goes into the weights: (m + log2 c, l / c), so the merge
      // folds y = O / c exactly as it folds O
      if (g == 0 && wid == 0) a.part_ml[prow] = make_float2(m[r] + __log2f(cc), lsum[r] * inv);
    }
  }
}

// Three work-groups per CU (the register budget of 3 waves per SIMD fits a
// 3-deep pipeline without spills); the default 768 ranges fill the chip once.
#ifndef AIA_MLA_WAVES_PER_EU
#define AIA_MLA_WAVES_PER_EU 3
#endif
// The two-row-block instantiation (verify / prefill steps) needs more
// registers: two waves per SIMD.
template <int RB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(RB == 1 ? AIA_MLA_WAVES_PER_EU : 2)))
void mla_attn_kernel(MlaArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t vt_all[4][kTile * kVStride];
  __shared__ __attribute__((aligned(16))) float sx[2 * 4 * RB * 256];
  __shared__ float smax[4 * RB * kRows];
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int w = blockIdx.x;   // one tile range per work-group
  if (w >= a.waves) return;
  const int* wr = a.wave_rec + (int64_t)w * kRecInts;
  const int pre = wr[16 + (lane & (kRecBlocks - 1))];
  const int nseg = a.hdr[0], total_tiles = a.hdr[1];
  const int nhb = (a.group + a.hb - 1) / a.hb;
  int s = wr[0];
  int t = wr[1];
  const int t_end = wr[2], tpw = wr[3], s_last = wr[13];
  if (s < 0 || s >= nseg || t < 0 || t >= t_end || t_end > total_tiles || tpw < 1 ||
      s_last < s || s_last >= nseg)
    return;
  int rec[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) rec[i] = wr[4 + i];
  bool first = true;
  while (true) {
    if (!rec_ok(rec, total_tiles, a.batch, a.tokens, 1, nhb)) return;
    if (rec[6] > t) {
      const int chunk_end = min(t_end, rec[6]);
      mla_segment<RB>(a, rec, t - rec[5], chunk_end - rec[5], w, tpw, wr[14], wr[15], vt_all[wid],
                      sx, smax, lane, wid, first, pre);
      first = false;
      t = chunk_end;
      if (t >= t_end) break;
    }
    if (++s > s_last) return;
    const int* r = a.seg + (int64_t)s * 8;
#pragma unroll
    for (int i = 0; i < 8; ++i) rec[i] = r[i];
  }
}

// ---------------------------------------------------------------- absorbed-MLA prefill units
//
// Prefill items of the absorbed-MLA path (one latent head of 576 values, V =
// its first 512, Hq query heads), planned as the GQA units are (128-row items
// of one request's (token, head) rows, cut into key chunks when they are
// few, chunk partials folded by the merge kernel).  A work-group of 4 waves,
// one per SIMD, takes its unit's rows in two passes of 64, 16 rows per wave:
//   Q (16 rows x 576) as MFMA operands in registers (72 VGPRs) and O (16 x
//   512 fp32, 128 registers); 32 rows per wave would need about 400;
//   keys go through LDS in 32-key sub-tiles, a ring of four buffers filled by
//   direct loads three sub-tiles ahead (at one wave per SIMD no other wave
//   covers a load's latency), one barrier per sub-tile;
//   per sub-tile: QK^T over 576 dims (four accumulation chains per 16 keys),
//   softmax, PV over the first 512 dims (V^T through transposing reads).
// The cache slots of a sub-tile's keys are computed by wave 0 four
// sub-tiles ahead from the unit's block ids, which it stages in LDS (2048
// at a time) so that no load the compiler tracks sits behind the direct
// loads in the loop (its wait would drain them).
// LDS sub-tile: the 512 latent values of key r (1 KB, one direct load) at
// row r of stride 1040 bytes -- the 16-byte pad puts the 16 keys of a K
// fragment read, and the keys of a V^T read group, on different banks --
// then the 64 rope values of every key, 128 bytes per key, its eight 16-byte
// chunks swizzled (chunk c at c ^ (r mod 8)) since eight keys' rope share
// one direct load.
constexpr int kMlaSub = 32;                                       // keys per sub-tile
constexpr int kMlaRing = 4;                                       // sub-tile buffers
constexpr int kMlaAhead = kMlaRing - 1;                           // loads ahead
constexpr int kMlaPfRow = 520;                                    // latent row stride (elements)
constexpr int kMlaPfRope = kMlaSub * kMlaPfRow;                   // rope region offset
constexpr int kMlaPfBuf = kMlaPfRope + kMlaSub * (kMlaK - kMlaV);   // elements per buffer
constexpr int kMlaLoads = kMlaSub / kPfWaves + 1;                 // direct loads per wave
constexpr int kMlaBtl = 2048;                                     // staged block ids
constexpr int kMlaKJ = kMlaK / 32;                                // 18 QK k-steps
constexpr int kMlaDT = kMlaV / 16;                                // 32 output tiles
constexpr int kMlaPassRows = kPfWaves * kRows;                    // 64 rows per pass
constexpr float kMlaPfSpan = 64.f;   // log2 growth allowed over a row's reference max
// s_waitcnt immediate: vmcnt(n) only (vmcnt bits 3:0 and 15:14)
constexpr int wait_vmcnt(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }
static_assert(wait_vmcnt(0) == kWaitVmcnt0, "s_waitcnt encoding");
static_assert(kPfWaves == 4 && kPfKeys == 2 * kMlaSub && kPfRows % kMlaPassRows == 0 &&
              kMlaV == 512 && kMlaK - kMlaV == 64 && kMlaSub == 8 * kPfWaves,
              "MLA prefill unit shape");

__global__ __launch_bounds__(kPfWaves * 64) __attribute__((amdgpu_waves_per_eu(1, 1)))
void mla_prefill_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t ring[kMlaRing * kMlaPfBuf];
  __shared__ int slots[kMlaRing][kMlaSub];
  __shared__ int btl[kMlaBtl];
  __shared__ int rerun_flag;
  const int wg = blockIdx.x;
  // this work-group's unit, as the GQA units take theirs (one kv head)
  int4 w0 = make_int4(0, 0, 0, 0), w1 = w0, w2 = w0;
  if (wg < kPfTargetWgs) {
    w0 = a.dealt[3 * wg];
    w1 = a.dealt[3 * wg + 1];
    w2 = a.dealt[3 * wg + 2];
  }
  const int count = a.hdr[6];
  if (wg >= count) return;
  int unit;
  int4 it, iq;
  if (a.hdr[9] == count) {
    it = w0;
    iq = w1;
    unit = w2.x;
    if (unit < 0 || unit >= count) return;
  } else {
    unit = xcd_range(wg, count);
    it = a.units[2 * unit];
    iq = a.units[2 * unit + 1];
  }
  const int b = it.x, row0 = it.y, t0 = it.z, t1 = it.w;
  if (b < 0 || b >= a.batch) return;
  const int q_begin = iq.x, lq = iq.y, lk = iq.z;
  const int G = a.group;
  const int nrows = lq * G;
  if (row0 < 0 || row0 >= nrows || q_begin < 0 || q_begin + lq > a.tokens) return;
  const int ctx0 = lk - lq;
  const int row_end = min(nrows, row0 + kPfRows);
  const int kend = max(0, min(lk, ctx0 + (row_end - 1) / G + 1));   // the item's keys
  const int ntiles = (kend + kPfKeys - 1) / kPfKeys;
  if (t0 < 0 || t1 < t0 || t1 > ntiles) return;
  const bool whole = t0 == 0 && t1 == ntiles;
  if (!whole && unit >= a.part_units) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int32_t* btrow = a.bt + (int64_t)b * a.bt_stride;
  const int bs = a.bs;

  // Wave 0: stage block ids [wb, wb + kMlaBtl) of the row (those below nbk)
  int wb = -1;
  auto stage_ids = [&](int first, int nbk) __attribute__((always_inline)) {
    wb = first;
    for (int e = lane; e < kMlaBtl && first + e < nbk; e += 64)
      btl[e] = min(max(btrow[first + e], 0), a.nb - 1);
  };
  // Wave 0, lanes 0..31: cache slots of sub-tile v's keys (keys past the
  // pass's last visible one re-read it)
  auto make_slots = [&](int v, int kendp, int nbk) __attribute__((always_inline)) {
    const int p = min(v * kMlaSub + lane, kendp - 1);
    const int bi = p / bs;
    if (__builtin_amdgcn_readfirstlane((v * kMlaSub) / bs) < wb ||
        __builtin_amdgcn_readfirstlane(min(v * kMlaSub + kMlaSub, kendp) - 1) / bs >= wb + kMlaBtl)
      stage_ids((v * kMlaSub) / bs, nbk);       // rare: a unit spanning more than kMlaBtl blocks
    if (lane < kMlaSub) slots[v % kMlaRing][lane] = btl[bi - wb] * bs + (p - bi * bs);
  };
  // Direct loads of sub-tile v into its ring buffer: wave w loads the latent
  // of keys 8 w .. 8 w + 7 (one key per load, lane l its chunk l) and their
  // rope (lane l chunk (l % 8) ^ (key % 8) of key 8 w + l / 8).
  auto issue = [&](int v) __attribute__((always_inline)) {
    uint16_t* dst = ring + (v % kMlaRing) * kMlaPfBuf;
    const int* sl = slots[v % kMlaRing];
#pragma unroll
    for (int i = 0; i < kMlaSub / kPfWaves; ++i) {
      const int r = wid * (kMlaSub / kPfWaves) + i;
      const int slot = __builtin_amdgcn_readfirstlane(sl[r]);
      lds_load16(a.kc + (int64_t)slot * kMlaK + 8 * lane, dst + r * kMlaPfRow);
    }
    const int r = wid * (kMlaSub / kPfWaves) + (lane >> 3);
    lds_load16(a.kc + (int64_t)sl[r] * kMlaK + kMlaV + 8 * ((lane & 7) ^ (r & 7)),
               dst + kMlaPfRope + wid * (kMlaSub / kPfWaves) * 64);
  };

  for (int pass = 0; pass < kPfRows / kMlaPassRows; ++pass) {
    const int prow0 = row0 + pass * kMlaPassRows;
    if (prow0 >= row_end) break;                      // uniform over the work-group
    const int prow_end = min(row_end, prow0 + kMlaPassRows);
    // keys this pass's last row sees, and its share of the unit's sub-tiles
    const int kendp = max(0, min(lk, ctx0 + (prow_end - 1) / G + 1));
    const int u0 = 2 * t0;
    const int u1 = min(2 * t1, (kendp + kMlaSub - 1) / kMlaSub);
    const int nbk = (kendp + bs - 1) / bs;            // blocks the pass may touch

    const int row = prow0 + wid * kRows + n;
    const bool rv = row < prow_end;
    const int tokr = row / G, headr = row - tokr * G;
    const int lim = rv ? min(ctx0 + tokr, lk - 1) : -1;
    int wlim_lo = rv ? lim : 0x7fffffff, wlim_hi = lim;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      wlim_lo = min(wlim_lo, __shfl_xor(wlim_lo, d));
      wlim_hi = max(wlim_hi, __shfl_xor(wlim_hi, d));
    }
    uint4 qf[kMlaKJ];
    if (rv) {
      const uint4* qp = reinterpret_cast<const uint4*>(
          a.q + (int64_t)(q_begin + tokr) * a.q_ts + (int64_t)headr * a.q_hs);
#pragma unroll
      for (int j = 0; j < kMlaKJ; ++j) qf[j] = qp[4 * j + g];
    } else {
#pragma unroll
      for (int j = 0; j < kMlaKJ; ++j) qf[j] = make_uint4(0, 0, 0, 0);
    }
    // Softmax without rescaling O: a row's reference m is its max over its
    // first visible sub-tile, and later scores may exceed it by up to
    // 2^kMlaPfSpan (P then stays a finite bf16, O and l finite fp32), so the
    // loop holds no rescale branch (one would keep O's 128 registers moving
    // between register files every sub-tile).  A row whose scores climb
    // further sets `ovf`, and the work-group then runs its sub-tiles again
    // with every row's exact max as m (rmax, tracked on the way).
    float4_t o[kMlaDT];
    float m = -INFINITY, lsum = 0.f, rmax = -INFINITY;
    bool ovf = false;

#pragma clang loop unroll(disable)
    for (int attempt = 0; attempt < 2; ++attempt) {
      // O lives in the accumulation registers throughout (the empty asm
      // pins it there; left to itself the compiler copied all 128 values
      // between register files every sub-tile)
#pragma unroll
      for (int dt = 0; dt < kMlaDT; ++dt) {
        o[dt] = float4_t{0.f, 0.f, 0.f, 0.f};
        asm volatile("" : "+a"(o[dt]));
      }
      lsum = 0.f;
      if (attempt > 0) { m = rmax; ovf = false; }   // every row's exact max
      if (u1 > u0) {
        // prologue: Q has arrived; slots of the first four sub-tiles, then
        // the loads of the first three
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        __syncthreads();                              // the ring is free
        if (wid == 0) {
          wb = -1;
          stage_ids((u0 * kMlaSub) / bs, nbk);
          __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
          for (int v = u0; v < min(u1, u0 + kMlaRing); ++v) make_slots(v, kendp, nbk);
        }
        __syncthreads();
        for (int v = u0; v < min(u1, u0 + kMlaAhead); ++v) issue(v);
#pragma clang loop unroll(disable)
        for (int u = u0; u < u1; ++u) {
          // sub-tile u's loads are the oldest of up to three in flight
          const int younger = min(kMlaAhead - 1, u1 - 1 - u);
          if (younger >= 2) __builtin_amdgcn_s_waitcnt(wait_vmcnt(2 * kMlaLoads));
          else if (younger == 1) __builtin_amdgcn_s_waitcnt(wait_vmcnt(kMlaLoads));
          else __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
          __syncthreads();
          const uint16_t* kt = ring + (u % kMlaRing) * kMlaPfBuf;
          const int kb = u * kMlaSub;
          if (kb <= wlim_hi) {                        // some row of this wave sees the keys
            float4_t acc[2];
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
              const int r = 16 * s2 + n;
              const uint16_t* kl = kt + r * kMlaPfRow + 8 * g;
              float4_t part[4];
#pragma unroll
              for (int c4 = 0; c4 < 4; ++c4) part[c4] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
              for (int j = 0; j < kMlaKJ - 2; ++j)
                part[j & 3] = qk_step(*reinterpret_cast<const uint4*>(kl + 32 * j), qf[j], part[j & 3]);
#pragma unroll
              for (int j = kMlaKJ - 2; j < kMlaKJ; ++j) {
                const int c = (4 * (j - (kMlaKJ - 2)) + g) ^ (r & 7);
                part[j & 3] = qk_step(*reinterpret_cast<const uint4*>(kt + kMlaPfRope + r * 64 + 8 * c),
                                      qf[j], part[j & 3]);
              }
              acc[s2] = (part[0] + part[1]) + (part[2] + part[3]);
            }
            if (u + kMlaAhead < u1) issue(u + kMlaAhead);
            const bool mask = kb + kMlaSub - 1 > wlim_lo;
            float sv[2][4];
            float tmax = -INFINITY;
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
              for (int v = 0; v < 4; ++v) {
                sv[s2][v] = (mask && kb + 16 * s2 + 4 * g + v > lim) ? -INFINITY : acc[s2][v];
                tmax = fmaxf(tmax, sv[s2][v]);
              }
            tmax = aia::group4_max(tmax);
            const float tm = tmax * a.scale_log2;
            rmax = fmaxf(rmax, tm);
            if (m == -INFINITY) m = tm;               // O and l are still zero
            ovf = ovf || tm > m + kMlaPfSpan;
            const float msub = m == -INFINITY ? 0.f : m;
            float p[2][4];
            float psum = 0.f;
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
              for (int v = 0; v < 4; ++v) {
                p[s2][v] = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[s2][v], a.scale_log2, -msub));
                psum += p[s2][v];
              }
            lsum += psum;
            uint4 pb;
            pb.x = aia::pack_bf16x2(p[0][0], p[0][1]);
            pb.y = aia::pack_bf16x2(p[0][2], p[0][3]);
            pb.z = aia::pack_bf16x2(p[1][0], p[1][1]);
            pb.w = aia::pack_bf16x2(p[1][2], p[1][3]);
            // PV: lane (n, g) addresses key 4 g + n / 4 (and + 16), dims
            // 16 dt + 4 (n % 4)
            const uint16_t* v0p = kt + (4 * g + (n >> 2)) * kMlaPfRow + 4 * (n & 3);
            const uint16_t* v1p = v0p + 16 * kMlaPfRow;
#pragma unroll
            for (int dt = 0; dt < kMlaDT; ++dt) {
              const short4_t x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)(v0p + 16 * dt));
              const short4_t x1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)(v1p + 16 * dt));
              const bf16x8_t va = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7));
              o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, as_b8(pb), o[dt], 0, 0, 0);
            }
#pragma unroll
            for (int dt = 0; dt < kMlaDT; ++dt) asm volatile("" : "+a"(o[dt]));
          } else if (u + kMlaAhead < u1) {
            issue(u + kMlaAhead);
          }
          // slots of sub-tile u + 4 into the ring slot sub-tile u's loads used
          if (wid == 0 && u + kMlaRing < u1) make_slots(u + kMlaRing, kendp, nbk);
        }
      }
      // a row past its reference span: the work-group runs its sub-tiles again
      if (tid == 0) rerun_flag = 0;
      __syncthreads();
      if (__any(ovf) && lane == 0) rerun_flag = 1;
      __syncthreads();
      const int rerun = rerun_flag;
      __syncthreads();
      if (!rerun) break;
    }

    lsum = aia::group4_sum(lsum);
    float cmax = 0.f;
    if (!whole) {
#pragma unroll
      for (int dt = 0; dt < kMlaDT; ++dt)
#pragma unroll
        for (int v = 0; v < 4; ++v) cmax = fmaxf(cmax, fabsf(o[dt][v]));
      cmax = aia::group4_max(cmax);
    }
    if (!rv) continue;
    if (!whole) {      // partial: y = O / c in fp16, (m + log2 c, l / c)
      const float c = cmax > 0.f ? cmax : 1.f, ic = 1.f / c;
      const int64_t prow = (int64_t)unit * kPfRows + (row - row0);
      uint16_t* pp = a.part_o + prow * kMlaV;
#pragma unroll
      for (int dt = 0; dt < kMlaDT; ++dt) {
        uint2 hv;
        hv.x = pack_f16x2(o[dt][0] * ic, o[dt][1] * ic);
        hv.y = pack_f16x2(o[dt][2] * ic, o[dt][3] * ic);
        *reinterpret_cast<uint2*>(pp + 16 * dt + 4 * g) = hv;
      }
      if (g == 0) a.part_ml[prow] = make_float2(m + __log2f(c), lsum * ic);
      continue;
    }
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
    uint16_t* op = a.out + (int64_t)(q_begin + tokr) * a.o_ts + (int64_t)headr * a.o_hs;
#pragma unroll
    for (int dt = 0; dt < kMlaDT; ++dt) {
      uint2 wv;
      wv.x = aia::pack_bf16x2(o[dt][0] * inv, o[dt][1] * inv);
      wv.y = aia::pack_bf16x2(o[dt][2] * inv, o[dt][3] * inv);
      *reinterpret_cast<uint2*>(op + 16 * dt + 4 * g) = wv;
    }
  }
}

int launch_merge(char* ws, const Layout& L, const Geometry& g, int32_t nw, int32_t dv, int32_t batch,
                 int32_t tokens, int32_t waves,
                 const uint16_t* part_o,
                 const float2* part_ml, const int32_t* seg, uint16_t* out, int64_t o_ts,
                 int64_t o_hs, hipStream_t s) {
  MergeArgs mg;
  mg.hdr = reinterpret_cast<const int32_t*>(ws + L.hdr);
  mg.seg = seg; mg.part_o = part_o; mg.part_ml = part_ml;
  mg.out = out; mg.o_ts = o_ts; mg.o_hs = o_hs; mg.group = g.group; mg.hb = g.hb; mg.dv = dv;
  mg.nw = nw; mg.hkv = g.hkv; mg.rb = g.rb; mg.tokens = tokens;
  mg.mrg = reinterpret_cast<const int32_t*>(ws + L.mrg); mg.mrg_cap = L.mrg_cap;
  const bool pf = L.pf_mrg_cap > 0;
  mg.pf_mrg = pf ? reinterpret_cast<const int4*>(ws + L.pfm) : nullptr;
  // wide: 64-element slices (MLA, or 8+ rows per segment) and about 8 or
  // more ranges per segment, i.e. a dozen partials per item
  const bool wide = AIA_MERGE_WIDE && L.pf_mrg_cap == 0 &&
                    (dv == kMlaV || (int64_t)g.hb * ((tokens + batch - 1) / batch) >= 8) &&
                    (int64_t)waves >= 8LL * batch * g.nkvg * g.nhb;
  const int threads = wide ? 512 : 256;
  const int64_t pf_slices = (int64_t)kPfRows * dv / (8 * threads);   // see merge_kernel
  mg.pf_items_cap = L.pf_mrg_cap * g.hkv * pf_slices;
  mg.pf_o = reinterpret_cast<const uint16_t*>(ws + L.pf_o);
  mg.pf_ml = reinterpret_cast<const float2*>(ws + L.pf_ml);
  const int64_t pitems = pf ? L.pf_mrg_cap * g.hkv * pf_slices : 0;
  const int64_t items = L.mrg_cap > pitems ? L.mrg_cap : pitems;
  int64_t mgrid = items < 2048 ? items : 2048;
  if (mgrid < 1) mgrid = 1;
  // Fixed-slot merges for small steps (kFixParts): one work-group per
  // (segment, kv head) when a segment's row span holds at most 16 elements
  // (rows x dv / 16, rows bounded by the query tokens a request can hold),
  // each thread of its kFixWaves waves loading kFixParts / (4 kFixWaves)
  // slots.  (configs[3]'s verify
  // segments, 64-128 elements, keep the records: in passes of 16 elements
  // the call went 40.6 -> 54 us, and with one wave per 16 elements and 8 slot
  // loads per thread 40.6 -> 42 us, config 1 then 21.9 -> 22.75.)
  mg.fixed_slots = 0;
  mg.part_cap = L.part_cap;
  if (small_geometry(g, dv, batch, L.seg_cap) && L.part_cap >= kFixParts * L.seg_cap) {
    const int64_t nq_max = std::min<int64_t>(g.qs, (int64_t)tokens - batch + 1);
    const int64_t rows_max = std::min<int64_t>(
        (int64_t)kRows * g.rb, nq_max <= g.qb ? nq_max * g.hb : (int64_t)kRows * ((nq_max + g.qb - 1) / g.qb));
    if (nq_max >= 1 && rows_max * (dv / kMergeDims) <= 16) {
      mg.fixed_slots = 1;
      mgrid = L.seg_cap * nw;
    }
  }
  if (mg.fixed_slots && !wide) {
    // kFixWaves waves of kFixParts / (4 kFixWaves) slot loads per thread (config 1,
    // us per layer: 2 waves 21.62-21.66, 1 wave 21.87-21.91, 4 waves 21.86-21.89)
    merge_kernel<kFixWaves, kFixParts / (4 * kFixWaves)><<<(unsigned)mgrid, 64 * kFixWaves, 0, s>>>(mg);
    return aia::check_hip(hipGetLastError(), "merge_kernel launch");
  }
  if (wide) merge_kernel<8, 0><<<(unsigned)mgrid, threads, 0, s>>>(mg);
  else merge_kernel<4, 0><<<(unsigned)mgrid, threads, 0, s>>>(mg);
  return aia::check_hip(hipGetLastError(), "merge_kernel launch");
}

// The small planner takes GQA steps without prefill routing whose segments
// fit one wave (AIA_PLANNER=large in the environment, read once, sends every
// step to plan_kernel: for comparisons).
bool small_plan(const Geometry& g, int32_t dv, int32_t batch, const Layout& L) {
  static const bool force_large = [] {
    const char* e = getenv("AIA_PLANNER");
    return e && strcmp(e, "large") == 0;
  }();
  return !force_large && small_geometry(g, dv, batch, L.seg_cap);
}

// The attention launches of one call, for one cache layout.
template <bool NZ>
int launch_gqa(const AttnArgs& a, const PrefillArgs& pa, const Layout& L, const Geometry& g,
               int32_t head_dim, int32_t waves, bool one_block, hipStream_t s) {
  using aia::check_hip;
  if (AIA_MIXED && L.pf_cap > 0 && g.nw == kPfWaves && g.rb == 1 && head_dim == kHeadDim) {
    const int npf = (int)(L.pf_unit_cap * g.hkv);
    const dim3 grid((unsigned)(npf + waves));
    if (one_block && pa.kn) gqa_mixed_kernel<true, true, NZ><<<grid, kPfWaves * 64, 0, s>>>(a, pa, npf);
    else if (one_block) gqa_mixed_kernel<true, false, NZ><<<grid, kPfWaves * 64, 0, s>>>(a, pa, npf);
    else if (pa.kn) gqa_mixed_kernel<false, true, NZ><<<grid, kPfWaves * 64, 0, s>>>(a, pa, npf);
    else gqa_mixed_kernel<false, false, NZ><<<grid, kPfWaves * 64, 0, s>>>(a, pa, npf);
    if (int rc = check_hip(hipGetLastError(), "gqa_mixed_kernel launch")) return rc;
  } else {
#define AIA_GQA_LAUNCH_D(NW, D)                                                   \
  (g.rb == 2 ? gqa_attn_kernel<NW, 2, D, NZ><<<waves, 64 * NW, 0, s>>>(a)            \
             : gqa_attn_kernel<NW, 1, D, NZ><<<waves, 64 * NW, 0, s>>>(a))
#define AIA_GQA_LAUNCH(NW)                                                        \
  (head_dim == 64 ? AIA_GQA_LAUNCH_D(NW, 64) : AIA_GQA_LAUNCH_D(NW, kHeadDim))
    switch (g.nw) {
      case 1: AIA_GQA_LAUNCH(1); break;
      case 2: AIA_GQA_LAUNCH(2); break;
      case 3: AIA_GQA_LAUNCH(3); break;
      case 4: AIA_GQA_LAUNCH(4); break;
      case 5: AIA_GQA_LAUNCH(5); break;
      case 6: AIA_GQA_LAUNCH(6); break;
      case 7: AIA_GQA_LAUNCH(7); break;
      default: AIA_GQA_LAUNCH(8); break;
    }
#undef AIA_GQA_LAUNCH
#undef AIA_GQA_LAUNCH_D
    if (int rc = check_hip(hipGetLastError(), "gqa_attn_kernel launch")) return rc;
    if (L.pf_cap > 0) {
      const dim3 grid((unsigned)(L.pf_unit_cap * g.hkv));
#define AIA_PF_LAUNCH(D)                                                                   \
  (one_block && pa.kn ? gqa_prefill_kernel<true, true, D, NZ><<<grid, kPfWaves * 64, 0, s>>>(pa)   \
   : one_block        ? gqa_prefill_kernel<true, false, D, NZ><<<grid, kPfWaves * 64, 0, s>>>(pa)  \
   : pa.kn            ? gqa_prefill_kernel<false, true, D, NZ><<<grid, kPfWaves * 64, 0, s>>>(pa)  \
                      : gqa_prefill_kernel<false, false, D, NZ><<<grid, kPfWaves * 64, 0, s>>>(pa))
      if (head_dim == 64) AIA_PF_LAUNCH(64);
      else AIA_PF_LAUNCH(kHeadDim);
#undef AIA_PF_LAUNCH
      if (int rc = check_hip(hipGetLastError(), "gqa_prefill_kernel launch")) return rc;
    }
  }
  return AIA_OK;
}

int check_heads(const char* fn, int32_t hq, int32_t hkv) {
  if (hq <= 0 || hkv <= 0 || hq % hkv != 0)
    return aia::fail(AIA_ERR_INVALID, "%s: num_q_heads %d must be a positive multiple of num_kv_heads %d",
                     fn, hq, hkv);
  return AIA_OK;
}

}  // namespace

extern "C" int aia_attn_workspace_bytes(int32_t batch, int32_t num_tokens, int32_t num_q_heads,
                                        int32_t num_kv_heads, int32_t head_dim_v,
                                        int32_t num_waves, int64_t* bytes) {
  if (int rc = check_heads("aia_attn_workspace_bytes", num_q_heads, num_kv_heads)) return rc;
  if (batch < 0 || num_tokens < 0 || head_dim_v <= 0 || !bytes)
    return aia::fail(AIA_ERR_INVALID, "aia_attn_workspace_bytes: bad arguments");
  const Geometry g = geometry(num_q_heads, num_kv_heads, batch, num_tokens, head_dim_v);
  *bytes = layout(batch, num_tokens, g, head_dim_v, resolve_waves(num_waves, g, head_dim_v)).total;
  return AIA_OK;
}

extern "C" int aia_attn_workspace_layout(int32_t batch, int32_t num_tokens, int32_t num_q_heads,
                                         int32_t num_kv_heads, int32_t head_dim_v,
                                         int32_t num_waves, int64_t* offsets, int32_t count) {
  if (int rc = check_heads("aia_attn_workspace_layout", num_q_heads, num_kv_heads)) return rc;
  if (batch < 0 || num_tokens < 0 || head_dim_v <= 0 || !offsets || count < 1)
    return aia::fail(AIA_ERR_INVALID, "aia_attn_workspace_layout: bad arguments");
  const Geometry g = geometry(num_q_heads, num_kv_heads, batch, num_tokens, head_dim_v);
  const int32_t waves = resolve_waves(num_waves, g, head_dim_v);
  const Layout L = layout(batch, num_tokens, g, head_dim_v, waves);
  const int64_t v[] = {L.hdr, L.seg, L.wave, L.part_ml, L.part_o, L.req, L.mrg, L.pf, L.pfm,
                       L.pfw, L.pf_ml, L.pf_o, L.total, L.seg_cap, L.mrg_cap, L.pf_cap,
                       L.pf_unit_cap, L.pf_mrg_cap, waves, kPfRows, kPfKeys};
  const int n = (int)(sizeof(v) / sizeof(v[0]));
  for (int i = 0; i < count; ++i) offsets[i] = i < n ? v[i] : -1;
  return AIA_OK;
}

extern "C" int aia_attn_plan(const int32_t* cu_seqlens_q, const int32_t* seqlens_kv,
                             const int32_t* block_table, int32_t block_table_stride,
                             int32_t block_size, int32_t batch,
                             int32_t num_tokens, int32_t num_q_heads, int32_t num_kv_heads,
                             int32_t head_dim_v, int32_t num_waves, void* workspace,
                             int64_t workspace_bytes, void* stream) {
  using namespace aia;
  if (int rc = check_heads("aia_attn_plan", num_q_heads, num_kv_heads)) return rc;
  if (batch < 0 || batch > kMaxBatch)
    return fail(AIA_ERR_CAPACITY, "aia_attn_plan: batch %d exceeds planner limit %d", batch, kMaxBatch);
  if (batch > 0 && (!cu_seqlens_q || !seqlens_kv || !block_table))
    return fail(AIA_ERR_INVALID, "aia_attn_plan: null metadata");
  if (block_size <= 0) return fail(AIA_ERR_INVALID, "aia_attn_plan: block_size %d", block_size);
  if (!workspace) return fail(AIA_ERR_INVALID, "aia_attn_plan: null workspace");
  if ((uintptr_t)workspace & 255)
    return fail(AIA_ERR_INVALID, "aia_attn_plan: workspace must be 256-byte aligned");
  const Geometry g = geometry(num_q_heads, num_kv_heads, batch, num_tokens, head_dim_v);
  const int32_t waves = resolve_waves(num_waves, g, head_dim_v);
  const Layout L = layout(batch, num_tokens, g, head_dim_v, waves);
  if (workspace_bytes < L.total)
    return fail(AIA_ERR_CAPACITY, "aia_attn_plan: workspace %lld bytes < %lld needed",
                (long long)workspace_bytes, (long long)L.total);
  char* ws = static_cast<char*>(workspace);
  if (small_plan(g, head_dim_v, batch, L)) {
    plan_small_kernel<<<1, kSmallPlanThreads, 0, (hipStream_t)stream>>>(
        cu_seqlens_q, seqlens_kv, block_table, block_table_stride, block_size, batch, g, waves,
        head_dim_v, reinterpret_cast<int32_t*>(ws + L.hdr),
        reinterpret_cast<int32_t*>(ws + L.seg), reinterpret_cast<int32_t*>(ws + L.wave),
        reinterpret_cast<int32_t*>(ws + L.mrg), (int32_t)L.seg_cap, (int32_t)L.part_cap);
    return check_hip(hipGetLastError(), "aia_attn_plan launch");
  }
  plan_kernel<<<1, kPlanThreads, 0, (hipStream_t)stream>>>(
      cu_seqlens_q, seqlens_kv, block_table, block_table_stride, block_size, batch, g, waves,
      head_dim_v, reinterpret_cast<int32_t*>(ws + L.hdr),
      reinterpret_cast<int32_t*>(ws + L.seg), reinterpret_cast<int32_t*>(ws + L.wave),
      reinterpret_cast<int32_t*>(ws + L.req),
      reinterpret_cast<int32_t*>(ws + L.mrg), reinterpret_cast<int4*>(ws + L.pf),
      reinterpret_cast<int4*>(ws + L.pfm), reinterpret_cast<int4*>(ws + L.pfw),
      (int32_t)L.pf_cap, (int32_t)L.pf_unit_cap,
      (int32_t)L.pf_mrg_cap, (int32_t)L.seg_cap,
      small_geometry(g, head_dim_v, batch, L.seg_cap) ? (int32_t)L.part_cap : 0);
  return check_hip(hipGetLastError(), "aia_attn_plan launch");
}

extern "C" int aia_paged_attention_gqa(
    const void* query, int64_t q_token_stride, int64_t q_head_stride, const void* key_cache,
    const void* value_cache, const int32_t* block_table, int32_t block_table_stride,
    const int32_t* cu_seqlens_q, const int32_t* seqlens_kv, int32_t batch, int32_t num_tokens,
    int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
    int32_t num_blocks, float scale, void* out, int64_t out_token_stride, int64_t out_head_stride,
    const void* key_new, const void* value_new, int64_t new_key_token_stride,
    int64_t new_value_token_stride, int32_t num_waves, int32_t flags, void* workspace,
    int64_t workspace_bytes, void* stream) {
  using namespace aia;
  if (int rc = check_heads("aia_paged_attention_gqa", num_q_heads, num_kv_heads)) return rc;
  if (head_dim != kHeadDim && head_dim != 64)
    return fail(AIA_ERR_UNSUPPORTED, "aia_paged_attention_gqa: head_dim %d (128 or 64)", head_dim);
  if (!(scale > 0.f))
    return fail(AIA_ERR_INVALID, "aia_paged_attention_gqa: scale %g must be positive", (double)scale);
  if (block_size <= 0 || num_blocks <= 0)
    return fail(AIA_ERR_INVALID, "aia_paged_attention_gqa: block_size %d / num_blocks %d",
                block_size, num_blocks);
  if ((int64_t)num_blocks * block_size > INT32_MAX)
    return fail(AIA_ERR_INVALID, "aia_paged_attention_gqa: %d blocks of %d slots exceed the int32 slot range",
                num_blocks, block_size);
  if (flags & ~AIA_ATTN_KV_NZ)
    return fail(AIA_ERR_INVALID, "aia_paged_attention_gqa: unknown flags 0x%x", flags);
  if (num_tokens == 0 || batch == 0) return AIA_OK;    // empty step (zero-size tensors)
  if (!query || !key_cache || !value_cache || !block_table || !out || !workspace || !cu_seqlens_q ||
      !seqlens_kv)
    return fail(AIA_ERR_INVALID, "aia_paged_attention_gqa: null pointer argument");
  if ((uintptr_t)workspace & 255)
    return fail(AIA_ERR_INVALID, "aia_paged_attention_gqa: workspace must be 256-byte aligned");
  if (q_token_stride % 8 || q_head_stride % 8 || out_token_stride % 4 || out_head_stride % 8 ||
      ((uintptr_t)query & 15) || ((uintptr_t)key_cache & 15) || ((uintptr_t)value_cache & 15) ||
      ((uintptr_t)out & 15))
    return fail(AIA_ERR_INVALID, "aia_paged_attention_gqa: query/out/cache must be 16-byte aligned "
                "with strides a multiple of 8 elements");
  if ((key_new == nullptr) != (value_new == nullptr))
    return fail(AIA_ERR_INVALID, "aia_paged_attention_gqa: key_new and value_new go together");
  if (key_new && (new_key_token_stride % 8 || new_value_token_stride % 8 ||
                  ((uintptr_t)key_new & 15) || ((uintptr_t)value_new & 15)))
    return fail(AIA_ERR_INVALID, "aia_paged_attention_gqa: new K/V rows must be 16-byte aligned "
                "with token strides a multiple of 8 elements");
  const Geometry g = geometry(num_q_heads, num_kv_heads, batch, num_tokens, head_dim);
  const int32_t waves = resolve_waves(num_waves, g, head_dim);
  const Layout L = layout(batch, num_tokens, g, head_dim, waves);
  if (workspace_bytes < L.total)
    return fail(AIA_ERR_CAPACITY, "aia_paged_attention_gqa: workspace %lld bytes < %lld needed",
                (long long)workspace_bytes, (long long)L.total);
  char* ws = static_cast<char*>(workspace);
  AttnArgs a;
  a.q = static_cast<const uint16_t*>(query);
  a.q_ts = q_token_stride; a.q_hs = q_head_stride;
  a.kc = static_cast<uint16_t*>(const_cast<void*>(key_cache));
  a.vc = static_cast<uint16_t*>(const_cast<void*>(value_cache));
  a.kn = static_cast<const uint16_t*>(key_new);
  a.vn = static_cast<const uint16_t*>(value_new);
  a.kn_ts = new_key_token_stride; a.vn_ts = new_value_token_stride;
  a.bt = block_table; a.bt_stride = block_table_stride;
  a.hkv = g.hkv; a.group = g.group; a.hb = g.hb; a.bs = block_size; a.nb = num_blocks;
  a.nw = g.nw;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.seg = reinterpret_cast<const int32_t*>(ws + L.seg);
  a.wave_rec = reinterpret_cast<const int32_t*>(ws + L.wave);
  a.part_o = reinterpret_cast<uint16_t*>(ws + L.part_o);
  a.part_ml = reinterpret_cast<float2*>(ws + L.part_ml);
  a.out = static_cast<uint16_t*>(out);
  a.o_ts = out_token_stride; a.o_hs = out_head_stride;
  a.waves = waves;
  a.hdr = reinterpret_cast<const int32_t*>(ws + L.hdr);
  a.batch = batch; a.tokens = num_tokens;
  hipStream_t s = (hipStream_t)stream;
  PrefillArgs pa = {};
  if (L.pf_cap > 0) {
    pa.q = a.q; pa.q_ts = a.q_ts; pa.q_hs = a.q_hs;
    pa.kc = a.kc; pa.vc = a.vc; pa.kn = a.kn; pa.vn = a.vn; pa.kn_ts = a.kn_ts; pa.vn_ts = a.vn_ts;
    pa.bt = block_table; pa.bt_stride = block_table_stride;
    pa.cu_q = cu_seqlens_q; pa.kvlen = seqlens_kv;
    pa.hkv = g.hkv; pa.group = g.group; pa.bs = block_size; pa.nb = num_blocks;
    pa.batch = batch; pa.tokens = num_tokens;
    pa.scale_log2 = a.scale_log2;
    pa.out = a.out; pa.o_ts = a.o_ts; pa.o_hs = a.o_hs;
    pa.units = reinterpret_cast<const int4*>(ws + L.pf);
    pa.dealt = reinterpret_cast<const int4*>(ws + L.pfw);
    pa.hdr = a.hdr;
    pa.part_o = reinterpret_cast<uint16_t*>(ws + L.pf_o);
    pa.part_ml = reinterpret_cast<float2*>(ws + L.pf_ml);
    pa.part_units = (int32_t)(L.pf_slots / g.hkv);
  }
  const bool one_block = block_size % kPfKeys == 0;
  if (int rc = (flags & AIA_ATTN_KV_NZ) ? launch_gqa<true>(a, pa, L, g, head_dim, waves, one_block, s)
                                        : launch_gqa<false>(a, pa, L, g, head_dim, waves, one_block, s))
    return rc;
  return launch_merge(ws, L, g, g.nw, head_dim, batch, num_tokens, waves, a.part_o, a.part_ml, a.seg, a.out, a.o_ts, a.o_hs,
                      s);
}

extern "C" int aia_paged_attention_mla(
    const void* q_latent, int64_t q_token_stride, int64_t q_head_stride, const void* latent_cache,
    const int32_t* block_table, int32_t block_table_stride, const int32_t* cu_seqlens_q,
    const int32_t* seqlens_kv, int32_t batch, int32_t num_tokens, int32_t num_heads,
    int32_t kv_lora_rank, int32_t rope_dim, int32_t block_size, int32_t num_blocks, float scale,
    void* out, int64_t out_token_stride, int64_t out_head_stride, int32_t num_waves, int32_t flags,
    void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace aia;
  if (flags != 0) return fail(AIA_ERR_INVALID, "aia_paged_attention_mla: flags must be 0");
  if (kv_lora_rank != kMlaV || rope_dim != kMlaK - kMlaV)
    return fail(AIA_ERR_UNSUPPORTED, "aia_paged_attention_mla: latent %d + rope %d (only 512 + 64)",
                kv_lora_rank, rope_dim);
  if (int rc = check_heads("aia_paged_attention_mla", num_heads, 1)) return rc;
  if (block_size <= 0 || num_blocks <= 0)
    return fail(AIA_ERR_INVALID, "aia_paged_attention_mla: block_size %d / num_blocks %d",
                block_size, num_blocks);
  if ((int64_t)num_blocks * block_size > INT32_MAX)
    return fail(AIA_ERR_INVALID, "aia_paged_attention_mla: %d blocks of %d slots exceed the int32 slot range",
                num_blocks, block_size);
  if (num_tokens == 0 || batch == 0) return AIA_OK;    // empty step (zero-size tensors)
  if (!q_latent || !latent_cache || !block_table || !out || !workspace)
    return fail(AIA_ERR_INVALID, "aia_paged_attention_mla: null pointer argument");
  if ((uintptr_t)workspace & 255)
    return fail(AIA_ERR_INVALID, "aia_paged_attention_mla: workspace must be 256-byte aligned");
  if (q_token_stride % 8 || q_head_stride % 8 || out_token_stride % 8 || out_head_stride % 8 ||
      ((uintptr_t)q_latent & 15) || ((uintptr_t)latent_cache & 15) || ((uintptr_t)out & 15))
    return fail(AIA_ERR_INVALID, "aia_paged_attention_mla: tensors must be 16-byte aligned with "
                "strides a multiple of 8 elements");
  const Geometry g = geometry(num_heads, 1, batch, num_tokens, kMlaV);
  const int32_t waves = resolve_waves(num_waves, g, kMlaV);
  const Layout L = layout(batch, num_tokens, g, kMlaV, waves);
  if (workspace_bytes < L.total)
    return fail(AIA_ERR_CAPACITY, "aia_paged_attention_mla: workspace %lld bytes < %lld needed",
                (long long)workspace_bytes, (long long)L.total);
  char* ws = static_cast<char*>(workspace);
  MlaArgs a;
  a.q = static_cast<const uint16_t*>(q_latent);
  a.q_ts = q_token_stride; a.q_hs = q_head_stride;
  a.cache = static_cast<const uint16_t*>(latent_cache);
  a.bt = block_table; a.bt_stride = block_table_stride;
  a.group = g.group; a.hb = g.hb; a.bs = block_size; a.nb = num_blocks;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.seg = reinterpret_cast<const int32_t*>(ws + L.seg);
  a.wave_rec = reinterpret_cast<const int32_t*>(ws + L.wave);
  a.part_o = reinterpret_cast<uint16_t*>(ws + L.part_o);
  a.part_ml = reinterpret_cast<float2*>(ws + L.part_ml);
  a.out = static_cast<uint16_t*>(out);
  a.o_ts = out_token_stride; a.o_hs = out_head_stride;
  a.waves = waves;
  a.hdr = reinterpret_cast<const int32_t*>(ws + L.hdr);
  a.batch = batch; a.tokens = num_tokens;
  hipStream_t s = (hipStream_t)stream;
  if (g.rb == 2) mla_attn_kernel<2><<<waves, 256, 0, s>>>(a);
  else mla_attn_kernel<1><<<waves, 256, 0, s>>>(a);
  if (int rc = check_hip(hipGetLastError(), "mla_attn_kernel launch")) return rc;
  if (L.pf_cap > 0) {     // prefill items (requests of 128+ rows)
    PrefillArgs pa = {};
    pa.q = a.q; pa.q_ts = a.q_ts; pa.q_hs = a.q_hs;
    pa.kc = const_cast<uint16_t*>(a.cache);
    pa.bt = block_table; pa.bt_stride = block_table_stride;
    pa.cu_q = cu_seqlens_q; pa.kvlen = seqlens_kv;
    pa.hkv = 1; pa.group = g.group; pa.bs = block_size; pa.nb = num_blocks;
    pa.batch = batch; pa.tokens = num_tokens;
    pa.scale_log2 = a.scale_log2;
    pa.out = a.out; pa.o_ts = a.o_ts; pa.o_hs = a.o_hs;
    pa.units = reinterpret_cast<const int4*>(ws + L.pf);
    pa.dealt = reinterpret_cast<const int4*>(ws + L.pfw);
    pa.hdr = a.hdr;
    pa.part_o = reinterpret_cast<uint16_t*>(ws + L.pf_o);
    pa.part_ml = reinterpret_cast<float2*>(ws + L.pf_ml);
    pa.part_units = (int32_t)L.pf_slots;
    mla_prefill_kernel<<<(unsigned)L.pf_unit_cap, kPfWaves * 64, 0, s>>>(pa);
    if (int rc = check_hip(hipGetLastError(), "mla_prefill_kernel launch")) return rc;
  }
  return launch_merge(ws, L, g, 1, kMlaV, batch, num_tokens, waves, a.part_o, a.part_ml, a.seg, a.out, a.o_ts, a.o_hs,
                      s);
}
