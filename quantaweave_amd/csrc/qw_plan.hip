// Capacity plan: per-expert histogram, prefix scans, and capacity slots.
//
// Reference: TopKMoE._plan, src/quantweave_moe_model.py:166-188.  The reference
// orders routes with two stable argsorts (weight descending, then expert), i.e.
// by the key (expert asc, weight desc, route id asc), keeps the first
// `capacity` routes of each expert and lists the rest as dropped.  Here the
// position of a route inside its expert is its rank under that key, counted
// directly: rank(r) = #{r' in expert(r) : key(r') < key(r)}.  Keys are unique
// (they contain r), so ranks are a permutation and no sort is needed; the
// result is independent of scheduling.
#include "qw_common.h"

namespace qw {

constexpr int kPlanThreads = 1024;

// Order-preserving map of a float onto uint32 (NaN largest, like torch.sort).
__device__ __forceinline__ uint32_t weight_key(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Block-wide exclusive scan of one int per thread (1024 threads).
__device__ int block_exclusive_scan(int v, int* warp_tot, int* total) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  int incl = v;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int n = __shfl_up(incl, o, kWave);
    if (lane >= o) incl += n;
  }
  if (lane == kWave - 1) warp_tot[wave] = incl;
  __syncthreads();
  if (wave == 0) {
    const int nw = blockDim.x / kWave;
    int w = lane < nw ? warp_tot[lane] : 0;
    int wi = w;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int n = __shfl_up(wi, o, kWave);
      if (lane >= o) wi += n;
    }
    if (lane < nw) warp_tot[lane] = wi - w;  // exclusive wave offsets
    if (lane == nw - 1) *total = wi;
  }
  __syncthreads();
  const int r = warp_tot[wave] + incl - v;
  __syncthreads();
  return r;
}

// Histogram of routes per expert and the scans derived from it.  One block.
__global__ __launch_bounds__(kPlanThreads) void plan_count_kernel(
    const int32_t* __restrict__ top_idx, int R, int E, int capacity, int32_t* __restrict__ counts,
    int32_t* __restrict__ kept_counts, int32_t* __restrict__ kept_offsets, int32_t* __restrict__ totals,
    int32_t* __restrict__ route_off, int32_t* __restrict__ cursor, int32_t* __restrict__ drop_off) {
  __shared__ int hist[1024];
  __shared__ int warp_tot[kPlanThreads / kWave];
  __shared__ int tot_kept, tot_drop, tot_routes;
  for (int e = threadIdx.x; e < E; e += blockDim.x) hist[e] = 0;
  __syncthreads();
  for (int r = threadIdx.x; r < R; r += blockDim.x) {
    const int e = top_idx[r];
    if (e >= 0 && e < E) atomicAdd(&hist[e], 1);
  }
  __syncthreads();
  const int e = threadIdx.x;  // E <= 1024 == blockDim.x
  const int c = e < E ? hist[e] : 0;
  const int kc = c < capacity ? c : capacity;
  const int dc = c - kc;
  const int ro = block_exclusive_scan(c, warp_tot, &tot_routes);
  const int ko = block_exclusive_scan(kc, warp_tot, &tot_kept);
  const int dof = block_exclusive_scan(dc, warp_tot, &tot_drop);
  if (e < E) {
    counts[e] = c;
    kept_counts[e] = kc;
    kept_offsets[e] = ko;
    route_off[e] = ro;
    cursor[e] = ro;
    drop_off[e] = dof;
  }
  if (e == 0) {
    kept_offsets[E] = tot_kept;
    totals[0] = tot_kept;
    totals[1] = tot_drop;
  }
}

// Scatter route ids into per-expert buckets (order inside a bucket is
// irrelevant: the rank kernel orders by key).  Keys: high word ~weight_key(w)
// so larger weights come first, low word the route id.
__global__ void plan_bucket_kernel(const int32_t* __restrict__ top_idx, const float* __restrict__ top_w, int R,
                                   int E, int32_t* __restrict__ cursor, uint64_t* __restrict__ bucket_key,
                                   int32_t* __restrict__ bucket_expert) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= R) return;
  const int e = top_idx[r];
  if (e < 0 || e >= E) return;
  const int pos = atomicAdd(&cursor[e], 1);
  bucket_key[pos] = (static_cast<uint64_t>(~weight_key(top_w[r])) << 32) | static_cast<uint32_t>(r);
  bucket_expert[pos] = e;
}

// Rank every bucketed route inside its expert and emit slots / drops.
// Keys of the block's experts are streamed through LDS in tiles.
__global__ __launch_bounds__(256) void plan_rank_kernel(
    const uint64_t* __restrict__ bucket_key, const int32_t* __restrict__ bucket_expert,
    const int32_t* __restrict__ route_off, const int32_t* __restrict__ counts,
    const int32_t* __restrict__ kept_offsets, const int32_t* __restrict__ drop_off,
    const int32_t* __restrict__ totals_routes, const float* __restrict__ top_w, int R, int K, int capacity,
    int32_t* __restrict__ slot_token, float* __restrict__ slot_weight, int32_t* __restrict__ route_slot,
    int32_t* __restrict__ dropped_token, int32_t* __restrict__ dropped_expert) {
  (void)totals_routes;
  __shared__ uint64_t tile[256];
  const int pos = blockIdx.x * 256 + threadIdx.x;
  const int nvalid = *totals_routes;  // routes with a valid expert id
  const bool active = pos < nvalid;
  uint64_t my_key = 0;
  int e = -1, lo = 0, hi = 0;
  if (active) {
    my_key = bucket_key[pos];
    e = bucket_expert[pos];
    lo = route_off[e];
    hi = lo + counts[e];
  }
  // The block covers bucket positions [b0, b0+256): the experts spanned are a
  // contiguous range, so the union of their key ranges is [first_lo, last_hi).
  __shared__ int s_lo, s_hi;
  const int b0 = blockIdx.x * 256;
  const int last = min(b0 + 255, nvalid - 1);
  if (threadIdx.x == 0) {
    s_lo = (b0 < nvalid) ? route_off[bucket_expert[b0]] : 0;
    s_hi = (b0 < nvalid) ? route_off[bucket_expert[last]] + counts[bucket_expert[last]] : 0;
  }
  __syncthreads();
  const int span_lo = s_lo, span_hi = s_hi;
  int rank = 0;
  for (int base = span_lo; base < span_hi; base += 256) {
    const int i = base + threadIdx.x;
    tile[threadIdx.x] = (i < span_hi) ? bucket_key[i] : 0;
    __syncthreads();
    if (active) {
      const int j0 = max(lo - base, 0), j1 = min(hi - base, 256);
      for (int j = j0; j < j1; ++j) rank += (tile[j] < my_key) ? 1 : 0;
    }
    __syncthreads();
  }
  if (!active) return;
  const int r = static_cast<int>(my_key & 0xffffffffu);
  if (rank < capacity) {
    const int s = kept_offsets[e] + rank;
    slot_token[s] = r / K;
    slot_weight[s] = top_w[r];
    route_slot[r] = s;
  } else {
    const int q = drop_off[e] + (rank - capacity);
    dropped_token[q] = r / K;
    dropped_expert[q] = e;
    route_slot[r] = -1;
  }
}

// Routes whose expert id is out of range are marked as not kept.
__global__ void plan_mark_invalid_kernel(const int32_t* __restrict__ top_idx, int R, int E,
                                         int32_t* __restrict__ route_slot) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= R) return;
  const int e = top_idx[r];
  if (e < 0 || e >= E) route_slot[r] = -1;
}

// Number of routes with a valid expert id = route_off[E-1] + counts[E-1].
__global__ void plan_valid_total_kernel(const int32_t* __restrict__ route_off, const int32_t* __restrict__ counts,
                                        int E, int32_t* __restrict__ out) {
  if (threadIdx.x == 0 && blockIdx.x == 0) *out = route_off[E - 1] + counts[E - 1];
}

size_t plan_workspace_bytes(int64_t T, int64_t K, int64_t E) {
  Carver c(nullptr);
  const size_t R = static_cast<size_t>(T * K);
  c.take<int32_t>(E);   // route_off
  c.take<int32_t>(E);   // cursor
  c.take<int32_t>(E);   // drop_off
  c.take<int32_t>(4);   // valid total
  c.take<uint64_t>(R);  // bucket keys
  c.take<int32_t>(R);   // bucket experts
  return c.used + 256;
}

int plan(const int32_t* top_idx, const float* top_w, int64_t T, int64_t K, int64_t E, int64_t capacity,
         int32_t* counts, int32_t* kept_counts, int32_t* kept_offsets, int32_t* slot_token, float* slot_weight,
         int32_t* route_slot, int32_t* dropped_token, int32_t* dropped_expert, int32_t* totals, void* ws,
         size_t ws_bytes, hipStream_t stream) {
  QW_REQUIRE(E >= 1 && E <= 1024, "experts must be in [1, 1024], got %lld", (long long)E);
  QW_REQUIRE(K >= 1 && K <= E, "top_k must be between 1 and num_experts");
  QW_REQUIRE(T >= 0 && T * K <= INT32_MAX, "tokens*top_k exceeds int32");
  QW_REQUIRE(capacity >= 0, "capacity must be >= 0");
  QW_REQUIRE(counts && kept_counts && kept_offsets && totals, "counts, kept_counts, kept_offsets, totals required");
  const int R = static_cast<int>(T * K);
  QW_REQUIRE(R == 0 || (top_idx && top_w && slot_token && slot_weight && route_slot && dropped_token &&
                        dropped_expert),
             "route arrays are required");
  const size_t need = plan_workspace_bytes(T, K, E);
  if (ws_bytes < need || (need && !ws))
    return set_error(QW_ERR_WORKSPACE, "plan workspace needs %zu bytes, got %zu", need, ws_bytes);
  const int cap = capacity > INT32_MAX ? INT32_MAX : static_cast<int>(capacity);
  Carver c(ws);
  int32_t* route_off = c.take<int32_t>(E);
  int32_t* cursor = c.take<int32_t>(E);
  int32_t* drop_off = c.take<int32_t>(E);
  int32_t* valid = c.take<int32_t>(4);
  uint64_t* bkey = c.take<uint64_t>(R);
  int32_t* bexp = c.take<int32_t>(R);
  const int e = static_cast<int>(E);
  plan_count_kernel<<<1, kPlanThreads, 0, stream>>>(top_idx, R, e, cap, counts, kept_counts, kept_offsets, totals,
                                                    route_off, cursor, drop_off);
  QW_LAUNCH_CHECK("plan_count_kernel");
  if (R == 0) return QW_OK;
  plan_valid_total_kernel<<<1, 64, 0, stream>>>(route_off, counts, e, valid);
  QW_LAUNCH_CHECK("plan_valid_total_kernel");
  const unsigned nb = static_cast<unsigned>(ceil_div(R, 256));
  plan_bucket_kernel<<<nb, 256, 0, stream>>>(top_idx, top_w, R, e, cursor, bkey, bexp);
  QW_LAUNCH_CHECK("plan_bucket_kernel");
  plan_mark_invalid_kernel<<<nb, 256, 0, stream>>>(top_idx, R, e, route_slot);
  QW_LAUNCH_CHECK("plan_mark_invalid_kernel");
  plan_rank_kernel<<<nb, 256, 0, stream>>>(bkey, bexp, route_off, counts, kept_offsets, drop_off, valid, top_w, R,
                                           static_cast<int>(K), cap, slot_token, slot_weight, route_slot,
                                           dropped_token, dropped_expert);
  QW_LAUNCH_CHECK("plan_rank_kernel");
  return QW_OK;
}

}  // namespace qw
