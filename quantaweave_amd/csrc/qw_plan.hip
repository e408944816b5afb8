// Capacity plan: per-expert route counts, prefix scans and capacity slots.
//
// Reference: TopKMoE._plan, src/quantweave_moe_model.py:166-188.  The reference
// orders routes with two stable argsorts (weight descending, then expert), i.e.
// by the key (expert asc, weight desc, route id asc), keeps the first
// `capacity` routes of each expert and lists the rest as dropped.
//
// One kernel, one workgroup per expert.  Every workgroup reads all routes once
// (16 expert ids and weights per thread, loads issued together), builds the
// histogram of all experts in LDS (per-wave copies, summed afterwards) and
// gathers its own expert's route keys
//   key = (~order(weight)) << 32 | route id        (unique per route)
// into LDS (a wave finds its matches with one ballot per route column and
// claims their positions with a single LDS atomic).  From the histogram it
// derives every offset itself (one scan of the packed kept and dropped
// counts), sorts its keys and writes kept slots and dropped routes at their
// plan positions.  The sort ranks each 64-key chunk by counting (one wave per
// chunk), then merges sorted runs pairwise: a key's place in the merged run is
// its index in its own run plus the number of smaller keys in the partner
// run (a binary search).  Keys are unique, so these places form a
// permutation, the order inside the gather does not matter and the result
// does not depend on scheduling.  An expert with more routes than the LDS
// holds gathers its keys into its own slice of the workspace and sorts them
// there with a bitonic network (same result, slower: one global-memory pass
// per network stage).
#include "qw_common.h"

namespace qw {

constexpr int kPlanThreads = 1024;
constexpr int kSortCap = 8192;  // keys an expert sorts in LDS (two buffers of 64 KiB)
constexpr int kChunkLog = 6;
constexpr int kChunk = 1 << kChunkLog;  // keys one wave ranks by counting before the merges
constexpr int kKeysPerThread = kSortCap / kPlanThreads;
constexpr int kMaxExperts = 1024;
constexpr int kRoutesPerThread = 16;

// Order-preserving map of a float onto uint32 (NaN largest, like torch.sort).
__device__ __forceinline__ uint32_t weight_key(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// The weight a key was made from (weight_key inverted, exact for every bit pattern).
__device__ __forceinline__ float key_weight(uint64_t key) {
  const uint32_t k = ~static_cast<uint32_t>(key >> 32);
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

__device__ __forceinline__ uint64_t route_key(const float* top_w, int r) {
  return (static_cast<uint64_t>(~weight_key(top_w[r])) << 32) | static_cast<uint32_t>(r);
}

// One merge round over n keys in LDS: run r (keys [r*run, (r+1)*run)) pairs
// with run r ^ 1, and a key moves to (start of the pair) + (its index in its
// run) + (keys of the partner run below it), found by binary lifting over the
// powers of two <= run.  Thread t holds keys t + u*kPlanThreads, u < NU; their
// searches step together, so their LDS reads are in flight together.  A wave
// with no key skips the search.
template <int NU>
__device__ __forceinline__ void merge_round(const uint64_t* __restrict__ src, uint64_t* __restrict__ dst, int n,
                                            int lg, int tid) {
  const int run = 1 << lg;
  if ((tid & ~(kWave - 1)) >= n) return;  // the wave's first key is past n (and so are its later ones)
  uint64_t k[NU];
  int pb[NU], len[NU], cnt[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int i = tid + u * kPlanThreads;
    pb[u] = ((i >> lg) ^ 1) << lg;
    const int pe = pb[u] + run < n ? pb[u] + run : n;
    len[u] = i < n && pb[u] < n ? pe - pb[u] : 0;
    k[u] = src[i < n ? i : 0];
    cnt[u] = 0;
  }
  for (int step = run; step >= 1; step >>= 1) {
    uint64_t v[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int j = cnt[u] + step - 1;
      v[u] = src[j < len[u] ? pb[u] + j : 0];  // past the partner's length: element 0, ignored
    }
#pragma unroll
    for (int u = 0; u < NU; ++u)
      if (cnt[u] + step <= len[u] && v[u] < k[u]) cnt[u] += step;
  }
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int i = tid + u * kPlanThreads;
    if (i < n) dst[((i >> lg) & ~1) * run + (i & (run - 1)) + cnt[u]] = k[u];
  }
}

// Merge rounds from sorted runs of kChunk keys in buf[1] up to one run of n keys;
// returns the buffer that holds the result.
template <int NU>
__device__ __forceinline__ int merge_all(uint64_t (*buf)[kSortCap], int n, int tid) {
  int cur = 1;
  for (int lg = kChunkLog; (1 << lg) < n; ++lg) {
    merge_round<NU>(buf[cur], buf[cur ^ 1], n, lg, tid);
    __syncthreads();
    cur ^= 1;
  }
  return cur;
}

// Offsets, per-expert ranking and placement.
__global__ __launch_bounds__(kPlanThreads) void plan_kernel(
    const int32_t* __restrict__ top_idx, const float* __restrict__ top_w, int R, int E, int K, int capacity,
    int32_t* __restrict__ counts, int32_t* __restrict__ kept_counts, int32_t* __restrict__ kept_offsets,
    int32_t* __restrict__ totals, int32_t* __restrict__ slot_token, float* __restrict__ slot_weight,
    int32_t* __restrict__ route_slot, int32_t* __restrict__ dropped_token, int32_t* __restrict__ dropped_expert,
    uint64_t* __restrict__ spill) {
  constexpr int kWaves = kPlanThreads / kWave;
  // Two key buffers; the second holds the per-wave histograms until the
  // offsets are known.
  __shared__ uint64_t buf[2][kSortCap];
  static_assert(sizeof(int) * kWaves * kMaxExperts <= sizeof(buf[1]), "histograms must fit a key buffer");
  uint64_t* const keys = buf[0];
  int (*const hist)[kMaxExperts] = reinterpret_cast<int (*)[kMaxExperts]>(&buf[1][0]);
  __shared__ uint64_t warp_tot[kWaves];
  __shared__ uint64_t s_tot;
  __shared__ int s_kept_off, s_drop_off, s_route_off, s_fill, s_fill_big;
  const int e = blockIdx.x;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  for (int i = tid; i < kWaves * E; i += kPlanThreads) hist[i / E][i % E] = 0;
  if (tid == 0) {
    s_fill = 0;
    s_fill_big = 0;
  }
  __syncthreads();

  // ---- one pass over the routes: histogram of all experts, keys of expert e ----
  // (the keys go to LDS when they fit; the count decides afterwards)
  for (int base = 0; base < R; base += kPlanThreads * kRoutesPerThread) {
    // expert ids and weights of 16 routes per thread, all loads issued before any use
    int v[kRoutesPerThread];
    float wv[kRoutesPerThread];
#pragma unroll
    for (int i = 0; i < kRoutesPerThread; ++i) {
      const int r = base + i * kPlanThreads + tid;
      v[i] = r < R ? top_idx[r] : -1;
      wv[i] = r < R ? top_w[r] : 0.0f;
    }
    uint64_t mask[kRoutesPerThread];
    int wave_n = 0;
#pragma unroll
    for (int i = 0; i < kRoutesPerThread; ++i) {
      const int r = base + i * kPlanThreads + tid;
      const bool valid = r < R && v[i] >= 0 && v[i] < E;
      if (valid) atomicAdd(&hist[wave][v[i]], 1);
      if (r < R && !valid && e == 0) route_slot[r] = -1;  // out-of-range expert id: never kept
      mask[i] = __ballot(valid && v[i] == e);
      wave_n += __popcll(mask[i]);
    }
    if (wave_n != 0) {
      // this expert's routes of the wave: one LDS atomic, then consecutive positions
      int first = 0;
      if (lane == 0) first = atomicAdd(&s_fill, wave_n);
      first = __shfl(first, 0, kWave);
      const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
      for (int i = 0; i < kRoutesPerThread; ++i) {
        const int r = base + i * kPlanThreads + tid;
        if ((mask[i] >> lane) & 1ull) {
          const int p = first + __popcll(mask[i] & below);
          if (p < kSortCap) keys[p] = (static_cast<uint64_t>(~weight_key(wv[i])) << 32) | static_cast<uint32_t>(r);
        }
        first += __popcll(mask[i]);
      }
    }
  }
  __syncthreads();

  // ---- counts and offsets of every expert (E <= blockDim) ----
  int c = 0;
  if (tid < E) {
#pragma unroll 4
    for (int w = 0; w < kWaves; ++w) c += hist[w][tid];
  }
  const int kc = c < capacity ? c : capacity;
  // kept count in the low word, dropped count in the high word: every prefix
  // sum of either is at most R < 2^31, so the words never carry into each other
  const uint64_t packed = (static_cast<uint64_t>(c - kc) << 32) | static_cast<uint32_t>(kc);
  auto publish = [&](uint64_t excl, uint64_t tot) {
    const int ko = static_cast<int>(excl & 0xffffffffu), dof = static_cast<int>(excl >> 32);
    if (tid == e) {
      s_kept_off = ko;
      s_drop_off = dof;
      s_route_off = ko + dof;
    }
    if (e == 0 && tid < E) {
      counts[tid] = c;
      kept_counts[tid] = kc;
      kept_offsets[tid] = ko;
    }
    if (e == 0 && tid == 0) {
      kept_offsets[E] = static_cast<int>(tot & 0xffffffffu);
      totals[0] = static_cast<int>(tot & 0xffffffffu);
      totals[1] = static_cast<int>(tot >> 32);
    }
  };
  if (E <= kWave) {
    // every expert in wave 0: a wave scan, no workgroup barrier
    if (wave == 0) {
      uint64_t incl = packed;
#pragma unroll
      for (int o = 1; o < kWave; o <<= 1) {
        const uint64_t v = __shfl_up(incl, o, kWave);
        if (lane >= o) incl += v;
      }
      publish(incl - packed, __shfl(incl, kWave - 1, kWave));
    }
  } else {
    const uint64_t excl = block_exclusive_scan(packed, warp_tot, &s_tot);
    publish(excl, s_tot);
  }
  __syncthreads();
  const int n = __builtin_amdgcn_readfirstlane(s_fill);  // the same in every lane
  if (n == 0) return;
  const int kept_off = s_kept_off, drop_off = s_drop_off;

  auto place = [&](uint64_t key, int rank) {
    const int r = static_cast<int>(key & 0xffffffffu);
    if (rank < capacity) {
      const int s = kept_off + rank;
      slot_token[s] = r / K;
      slot_weight[s] = key_weight(key);
      route_slot[r] = s;
    } else {
      const int q = drop_off + (rank - capacity);
      dropped_token[q] = r / K;
      dropped_expert[q] = e;
      route_slot[r] = -1;
    }
  };

  if (n <= kSortCap) {
    // ---- sort in LDS: rank each 64-key chunk by counting (all lanes of the
    //      wave read the same key: broadcast), sorted chunks to buf[1] ----
    for (int q = wave; q * kChunk < n; q += kWaves) {
      const int base = q * kChunk, m = n - base < kChunk ? n - base : kChunk;
      const int i = base + lane;
      const uint64_t k = i < n ? keys[i] : 0ull;
      int rank = 0;
#pragma unroll 16
      for (int j = 0; j < m; ++j) rank += keys[base + j] < k ? 1 : 0;
      if (i < n) buf[1][base + rank] = k;
    }
    __syncthreads();
    // ---- merge sorted runs pairwise up to one sorted run ----
    const int nu = (n + kPlanThreads - 1) / kPlanThreads;  // keys per thread
    const int cur = nu == 1   ? merge_all<1>(buf, n, tid)
                    : nu == 2 ? merge_all<2>(buf, n, tid)
                    : nu <= 4 ? merge_all<4>(buf, n, tid)
                              : merge_all<kKeysPerThread>(buf, n, tid);
    const uint64_t* src = buf[cur];
    for (int i = tid; i < n; i += kPlanThreads) place(src[i], i);
  } else {
    // ---- large expert: its n keys in its own slice of the workspace (n routes
    //      of expert e start at s_route_off), sorted there ----
    uint64_t* mine = spill + s_route_off;
    for (int r = tid; r < R; r += blockDim.x) {
      if (top_idx[r] == e) {
        const int p = atomicAdd(&s_fill_big, 1);  // its own counter: s_fill is still read above
        mine[p] = route_key(top_w, r);
      }
    }
    __threadfence();
    __syncthreads();
    // Bitonic network in the form whose compare-exchanges all put the smaller
    // key first: the first stage of each merge pairs i with the mirror index
    // (size - 1 - i within the block), the later ones i with i + stride.
    // Positions n .. p2-1 stand for +infinity keys: such a key never moves, so
    // a pair whose upper index is past n is skipped and nothing is padded.
    // Loads bypass the L1 (the keys were just written by other waves).
    auto cmpx = [&](int lo, int hi) {
      if (hi >= n) return;
      const uint64_t a = __hip_atomic_load(&mine[lo], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint64_t b = __hip_atomic_load(&mine[hi], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (a > b) {
        mine[lo] = b;
        mine[hi] = a;
      }
    };
    int p2 = 1;
    while (p2 < n) p2 <<= 1;
    for (int size = 2; size <= p2; size <<= 1) {
      const int half = size >> 1;
      for (int i = tid; i < p2 / 2; i += blockDim.x) {
        const int blk = i / half, j = i % half;
        cmpx(blk * size + j, blk * size + size - 1 - j);
      }
      __threadfence();
      __syncthreads();
      for (int stride = half >> 1; stride > 0; stride >>= 1) {
        for (int i = tid; i < p2 / 2; i += blockDim.x) {
          const int lo = 2 * i - (i & (stride - 1));
          cmpx(lo, lo + stride);
        }
        __threadfence();
        __syncthreads();
      }
    }
    for (int i = tid; i < n; i += blockDim.x)
      place(__hip_atomic_load(&mine[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), i);
  }
}

size_t plan_workspace_bytes(int64_t T, int64_t K, int64_t E) {
  (void)E;
  Carver c(nullptr);
  c.take<uint64_t>(static_cast<size_t>(T * K));  // keys of experts too large for LDS
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
  if (ws_bytes < need || !ws)
    return set_error(QW_ERR_WORKSPACE, "plan workspace needs %zu bytes, got %zu", need, ws_bytes);
  const int cap = capacity > INT32_MAX ? INT32_MAX : static_cast<int>(capacity);
  Carver c(ws);
  uint64_t* spill = c.take<uint64_t>(static_cast<size_t>(R));
  const int e = static_cast<int>(E);
  plan_kernel<<<e, kPlanThreads, 0, stream>>>(top_idx, top_w, R, e, static_cast<int>(K), cap, counts, kept_counts,
                                              kept_offsets, totals, slot_token, slot_weight, route_slot, dropped_token,
                                              dropped_expert, spill);
  QW_LAUNCH_CHECK("plan_kernel");
  return QW_OK;
}

}  // namespace qw
