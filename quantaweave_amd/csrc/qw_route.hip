// Router logits, softmax, top-k and renormalisation on gfx950.
//
// Reference: src/quantweave_moe_model.py:124-137 (TopKMoE.forward, fp32 routing
// with autocast disabled).  The reference routes with torch's own kernels, so
// the routing here is torch's arithmetic step for step: the softmax is the
// one-wave softmax PyTorch runs for rows of up to 1024 fp32 values
// (softmax_warp_forward in aten/src/ATen/native/cuda/PersistentSoftmax.cuh:
// the maximum, e = exp(l - max) with the device library's expf, per-lane sums
// over the lane's values in index order, an xor butterfly over lane offsets
// 32, 16, ..., 1, then e / sum), the selection is torch.topk's order and the
// renormalisation is w / w.sum(-1).  This file is compiled with
// -ffp-contract=off so each of those operations stays the single IEEE-754
// operation written.
#include <type_traits>

#include "qw_common.h"

namespace qw {

// e^x as torch's softmax computes it: the device math library's expf (what
// the float overload of ::exp calls in device code).
__device__ __forceinline__ float softmax_expf(float x) { return expf(x); }

// Total order on floats as unsigned keys: -inf < ... < -0 < +0 < ... < +inf < NaN.
__device__ __forceinline__ uint32_t sortable_key(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// torch.topk's comparison: NaN above every number, otherwise a > b.
__device__ __forceinline__ bool topk_greater(float a, float b) { return (a != a && b == b) || a > b; }

// torch.topk's order of the K <= 64 chosen values (lane j < K holds choice j
// as (key value kv, expert e, probability p); the choices arrive sorted by
// sortable_key(kv) descending, equal keys by ascending expert, which is the set
// torch.topk chooses).  torch's selection writes the chosen values above the
// k-th value in expert order, then those equal to the k-th value in expert
// order (compared as its radix-select keys: sortable_key's order, -0 below
// +0), and then sorts them by their float value (-0 equal to +0):
//   K <= 32: a 32-wide bitonic network that is not stable (bitonicSort and
//            bitonicSwap in aten/src/ATen/native/cuda/SortUtils.cuh with GTOp,
//            invalid entries last); lane i of the first 32 plays element i,
//            exchanging with lane i ^ stride;
//   K > 32:  a stable sort, which differs from the arrival order only where
//            -0 and +0 are both chosen next to each other.
// Without equal float values among the choices both give the arrival order, so
// the common case returns after one wave vote.
__device__ __forceinline__ void topk_tie_order(int K, float& kv, int& e, float& p) {
  const int lane = threadIdx.x % kWave;
  const float prev = __shfl_up(kv, 1, kWave);
  const bool tie = lane >= 1 && lane < K && prev == kv;
  if (K > 32 ? !__any(tie && sortable_key(prev) != sortable_key(kv)) : !__any(tie)) return;
  const uint32_t kth = sortable_key(__shfl(kv, K - 1, kWave));
  const int grp = (lane < K && sortable_key(kv) > kth) ? 0 : 1;
  int pos = 0;  // place in the order torch's selection writes
  for (int i = 0; i < K; ++i) {
    const int gi = __builtin_amdgcn_readlane(grp, i), ei = __builtin_amdgcn_readlane(e, i);
    pos += (gi < grp || (gi == grp && ei < e)) ? 1 : 0;
  }
  if (K > 32) {
    int rank = 0;  // stable descending sort of that order
    for (int i = 0; i < K; ++i) {
      const float ki = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(kv), i));
      const int pi = __builtin_amdgcn_readlane(pos, i);
      rank += (topk_greater(ki, kv) || (!topk_greater(kv, ki) && pi < pos)) ? 1 : 0;
    }
    pos = rank;
  }
  const int dst = (lane < K ? pos : lane) * 4;  // a permutation of the lanes: choice j moves to lane pos
  kv = __int_as_float(__builtin_amdgcn_ds_permute(dst, __float_as_int(kv)));
  e = __builtin_amdgcn_ds_permute(dst, e);
  p = __int_as_float(__builtin_amdgcn_ds_permute(dst, __float_as_int(p)));
  if (K > 32) return;
  int valid = lane < K ? 1 : 0;
#pragma unroll
  for (int size = 2; size <= 32; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const float okv = __shfl_xor(kv, stride, kWave);
      const int oe = __shfl_xor(e, stride, kWave);
      const float op = __shfl_xor(p, stride, kWave);
      const int ovalid = __shfl_xor(valid, stride, kWave);
      const bool lower = (lane & stride) == 0;
      const float ka = lower ? kv : okv, kb = lower ? okv : kv;
      const int va = lower ? valid : ovalid, vb = lower ? ovalid : valid;
      const bool swap = (topk_greater(ka, kb) && va) || !vb;
      const bool dir = size < 32 && (lane & size) != 0;  // the last merge runs in one direction
      if (swap == dir) {
        kv = okv;
        e = oe;
        p = op;
        valid = ovalid;
      }
    }
  }
}

// w.sum(-1) of a row of K < 128 chosen weights as torch reduces it (the
// thread reduction of aten/src/ATen/native/cuda/Reduce.cuh for a contiguous
// last dimension of K values): with B = 2^floor(log2 K) (at most 64) threads,
// thread i adds w_i + w_{i+B} (just w_i when i + B >= K), then the B partial
// sums meet in a shuffle-down tree (offsets 1, 2, 4, ...).  Lane j holds w_j in
// lo and, for K > 64, w_{j+64} in hi.  Every lane gets the sum.
__device__ __forceinline__ float topk_weight_sum(float lo, float hi, int K) {
  const int lane = threadIdx.x % kWave;
  const int B = K >= kWave ? kWave : (1 << (31 - __builtin_clz(static_cast<unsigned>(K))));
  const float up = K > kWave ? hi : __shfl_down(lo, B < kWave ? B : 0, kWave);
  float v = lane < B ? (lane + B < K ? lo + up : lo) : 0.0f;
  for (int o = 1; o < B; o <<= 1) v = v + __shfl_down(v, o, kWave);
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}

// ---------------------------------------------------------------------------
// Router GEMM, split over K: partial[s, t, e] = sum over the s-th K range of
// x[t, k] * W[e, k] (fp32 accumulation).  The top-k kernel adds the partials
// in ascending s, so the logits do not depend on scheduling.
//
// General kernel (any dtype pair, any d): 64x64 output tile per 256-thread
// block, K staged through LDS in slices of 16 (the next slice loaded into
// registers during the current one's multiplies), fp32 FMA.
// ---------------------------------------------------------------------------
template <int XDT, int WDT>
__global__ __launch_bounds__(256) void router_logits_kernel(const void* __restrict__ x, int64_t x_stride,
                                                            const void* __restrict__ w, int T, int D, int E,
                                                            int k_len, float* __restrict__ partial) {
  constexpr int TM = 64, TN = 64, TK = 16;
  __shared__ float xs[TK][TM + 4];
  __shared__ float ws[TK][TN + 4];
  const int tid = threadIdx.x;
  const int t0 = blockIdx.x * TM, e0 = blockIdx.z * TN;
  const int k_begin = blockIdx.y * k_len, k_end = min(D, k_begin + k_len);
  float* out = partial + static_cast<int64_t>(blockIdx.y) * T * E;
  const int ty = tid / 16, tx = tid % 16;
  float acc[4][4] = {};
  // the next slice's values are loaded into registers while this one is
  // multiplied, so only the first slice waits for memory
  constexpr int PER = TM * TK / 256;
  float xr[PER], wr[PER];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int i = tid + q * 256;
      const int m = i / TK, kk = i % TK;
      const int t = t0 + m, k = k0 + kk, e = e0 + m;
      xr[q] = (t < T && k < k_end) ? load_act<XDT>(x, static_cast<int64_t>(t) * x_stride + k) : 0.0f;
      wr[q] = (e < E && k < k_end) ? load_act<WDT>(w, static_cast<int64_t>(e) * D + k) : 0.0f;
    }
  };
  if (k_begin < k_end) fetch(k_begin);
  for (int k0 = k_begin; k0 < k_end; k0 += TK) {
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int i = tid + q * 256;
      xs[i % TK][i / TK] = xr[q];
      ws[i % TK][i / TK] = wr[q];
    }
    __syncthreads();
    if (k0 + TK < k_end) fetch(k0 + TK);
#pragma unroll
    for (int kk = 0; kk < TK; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = xs[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = ws[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = t0 + ty * 4 + i;
    if (t >= T) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = e0 + tx * 4 + j;
      if (e < E) out[static_cast<int64_t>(t) * E + e] = acc[i][j];
    }
  }
}

// Router for a few tokens (decode): the GEMM is a GEMV per token, bound by
// reading the router weight once.  Block (e, b): expert e, tokens
// [b*TT, b*TT + TT); thread i accumulates x[t, d] * w[e, d] for d = VEC*i + 256*VEC*j (+ 0..VEC-1) with
// fma (rows past the last token repeat it, so every load is issued at once);
// the TT per-thread sums are reduced across
// the wave (reduce_scatter) and then across the 4 waves in wave order, and
//   logits[t, e] = sum / temperature
// is written directly (no split-K partials).  With cast_out (fp32 x only) the
// expert-0 blocks also write x rounded to bf16 or fp16 (the decode step's
// expert input), so no other kernel reads x again for it.
constexpr int kGemvMaxTokens = 64;  // the GEMV router serves up to this many tokens

template <int XDT, int WDT, int VEC, int TT>
__global__ __launch_bounds__(256) void router_gemv_kernel(const void* __restrict__ x, int64_t x_stride,
                                                          const void* __restrict__ w, int T, int D, int E,
                                                          float temperature, float* __restrict__ logits,
                                                          uint16_t* __restrict__ cast_out, int cast_f16) {
  constexpr int L = log2i<TT>();
  __shared__ float red[4][TT];
  const int e = blockIdx.x;
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int64_t wrow = static_cast<int64_t>(e) * D;
  const int t0 = blockIdx.y * TT;
  {
    const int nt = min(TT, T - t0);
    float acc[TT];
#pragma unroll
    for (int i = 0; i < TT; ++i) acc[i] = 0.0f;
    for (int d = tid * VEC; d < D; d += 256 * VEC) {
      float wv[VEC];
      load_vec<WDT, VEC>(w, wrow + d, wv);
      float xv[TT][VEC];
#pragma unroll
      for (int i = 0; i < TT; ++i)
        load_vec<XDT, VEC>(x, static_cast<int64_t>(t0 + min(i, nt - 1)) * x_stride + d, xv[i]);
      if (XDT == QW_F32 && cast_out != nullptr && e == 0) {
        // the expert-0 blocks also write the rows rounded to bf16 (fp16): contiguous x, x_stride == D
#pragma unroll
        for (int i = 0; i < TT; ++i)
          if (i < nt)
#pragma unroll
            for (int u = 0; u < VEC; ++u)
              cast_out[static_cast<int64_t>(t0 + i) * D + d + u] = cast_f16 ? f32_to_f16(xv[i][u]) : f32_to_bf16(xv[i][u]);
      }
#pragma unroll
      for (int i = 0; i < TT; ++i)
#pragma unroll
        for (int u = 0; u < VEC; ++u) acc[i] = __builtin_fmaf(xv[i][u], wv[u], acc[i]);
    }
    const float r = reduce_scatter<TT>(acc, lane);  // the wave's sum of token lane >> (6 - L)
    if ((lane & ((1 << (6 - L)) - 1)) == 0) red[wave][lane >> (6 - L)] = r;
    __syncthreads();
    if (tid < nt) {
      const float s = ((red[0][tid] + red[1][tid]) + red[2][tid]) + red[3][tid];
      logits[static_cast<int64_t>(t0 + tid) * E + e] = s / temperature;
    }
  }
}

// bf16 x bf16 (or fp16 x fp16) router GEMM on MFMA (products of bf16 or fp16
// values are exact in fp32, so this is the same fp32 dot product up to
// accumulation order).  Tile: 64 tokens x 64 experts per 256-thread block;
// wave w owns tokens w*16..w*16+15.
typedef __bf16 rbf16x8 __attribute__((ext_vector_type(8)));  // 16-bit operands (bf16 or fp16 bits)
typedef _Float16 rf16x8 __attribute__((ext_vector_type(8)));
typedef float rf32x4 __attribute__((ext_vector_type(4)));

// One 16x16x32 MFMA step on operands of the 16-bit type DT.
template <int DT>
__device__ __forceinline__ rf32x4 rmfma(rbf16x8 a, rbf16x8 b, rf32x4 c) {
  if constexpr (DT == QW_F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(rf16x8, a), __builtin_bit_cast(rf16x8, b), c, 0,
                                                   0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

template <int DT>
__global__ __launch_bounds__(256) void router_mfma_kernel(const uint16_t* __restrict__ x, int64_t x_stride,
                                                          const uint16_t* __restrict__ w, int T, int D, int E,
                                                          int k_len, float* __restrict__ partial) {
  constexpr int BK = 64, LROW = BK + 8;
  __shared__ __attribute__((aligned(16))) uint16_t As[64 * LROW];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[64 * LROW];
  const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  const int t0 = blockIdx.x * 64, e0 = blockIdx.z * 64;
  const int k_begin = blockIdx.y * k_len, k_end = min(D, k_begin + k_len);
  float* out = partial + static_cast<int64_t>(blockIdx.y) * T * E;
  // 64 rows x 8 pieces of 16 bytes per slice and operand: 2 pieces per thread
  const uint16_t* a_src[2];
  const uint16_t* b_src[2];
  int dst[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = tid + i * 256, row = c / 8, ch = c % 8;
    dst[i] = row * LROW + ch * 8;
    a_src[i] = (t0 + row < T) ? x + static_cast<int64_t>(t0 + row) * x_stride + ch * 8 : nullptr;
    b_src[i] = (e0 + row < E) ? w + static_cast<int64_t>(e0 + row) * D + ch * 8 : nullptr;
  }
  uint4 ra[2], rb[2];
  auto load = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      ra[i] = a_src[i] ? *reinterpret_cast<const uint4*>(a_src[i] + k0) : make_uint4(0, 0, 0, 0);
      rb[i] = b_src[i] ? *reinterpret_cast<const uint4*>(b_src[i] + k0) : make_uint4(0, 0, 0, 0);
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      *reinterpret_cast<uint4*>(&As[dst[i]]) = ra[i];
      *reinterpret_cast<uint4*>(&Bs[dst[i]]) = rb[i];
    }
  };
  rf32x4 acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = rf32x4{0.f, 0.f, 0.f, 0.f};
  const int l16 = lane % 16, kq = (lane / 16) * 8;
  if (k_begin < k_end) {  // an empty split still writes its (zero) partial
    load(k_begin);
    stash();
  }
  __syncthreads();
  for (int k0 = k_begin; k0 < k_end; k0 += BK) {
    const bool more = k0 + BK < k_end;
    if (more) load(k0 + BK);
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      const rbf16x8 afr = *reinterpret_cast<const rbf16x8*>(&As[(wave * 16 + l16) * LROW + ks * 32 + kq]);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const rbf16x8 bfr = *reinterpret_cast<const rbf16x8*>(&Bs[(t * 16 + l16) * LROW + ks * 32 + kq]);
        acc[t] = rmfma<DT>(afr, bfr, acc[t]);
      }
    }
    __syncthreads();
    if (more) {
      stash();
      __syncthreads();
    }
  }
  const int rq = (lane / 16) * 4;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int e = e0 + t * 16 + l16;
    if (e >= E) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tok = t0 + wave * 16 + rq + r;
      if (tok < T) out[static_cast<int64_t>(tok) * E + e] = acc[t][r];
    }
  }
}

// ---------------------------------------------------------------------------
// One wavefront per token.  Lane l owns experts l, l+64, ..., l+64*(EPL-1).
//   m = max_e L_e;  q_e = softmax_expf(L_e - m)
//   S = (per-lane sequential sum over its experts in index order) reduced by
//       the xor butterfly with lane offsets 32, 16, 8, 4, 2, 1
//   p_e = q_e / S
//   top-k: k rounds of a wave argmax on (key desc, expert asc), key = p_e,
//          or L_e + bias_e when a bias is given, or L_e when `select_logits`
//          is set and there is no bias (the decode step's selection); equal
//          keys then take torch.topk's order (topk_tie_order)
//   w_j = p_{idx_j} / S_w, S_w = torch's sum of the k weights (topk_weight_sum)
// ---------------------------------------------------------------------------
//
// The per-token part: softmax and top-k of one token's logits l (lane l owns
// experts l + 64*c) by one wave.  probs are stored here.  With K <= 64 the
// choices are returned, lane j holding choice j's expert and renormalised
// weight in *out_e / *out_w (lanes >= K: unspecified), and the caller stores
// them; with more choices lane 0 stores each expert to top_idx and every lane
// stores its renormalised weights.
template <int EPL>
__device__ __forceinline__ void select_token(float (&l)[EPL], int t, int E, int K, const float* __restrict__ bias,
                                             int select_logits, float* __restrict__ probs,
                                             int32_t* __restrict__ top_idx, float* __restrict__ top_w, int* out_e,
                                             float* out_w) {
  const int lane = threadIdx.x % kWave;
  float p[EPL];
  float m = -__builtin_inff();
#pragma unroll
  for (int c = 0; c < EPL; ++c) m = fmaxf(m, l[c]);
  // fmaxf drops NaN; a NaN logit must poison the row as it does in torch.
  bool has_nan = false;
#pragma unroll
  for (int c = 0; c < EPL; ++c) has_nan |= (l[c] != l[c]);
  m = wave_max(m);
  if (__any(has_nan)) m = __builtin_nanf("");
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < EPL; ++c) {
    const int e = lane + c * kWave;
    p[c] = (e < E) ? softmax_expf(l[c] - m) : 0.0f;
    s += p[c];
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, kWave);
#pragma unroll
  for (int c = 0; c < EPL; ++c) {
    const int e = lane + c * kWave;
    p[c] = p[c] / s;
    if (probs != nullptr && e < E) probs[static_cast<int64_t>(t) * E + e] = p[c];
  }
  // selection keys
  uint32_t key[EPL];
  float kval[EPL];
#pragma unroll
  for (int c = 0; c < EPL; ++c) {
    const int e = lane + c * kWave;
    kval[c] = (bias != nullptr && e < E) ? l[c] + bias[e] : (select_logits ? l[c] : p[c]);
    key[c] = (e < E) ? sortable_key(kval[c]) : 0u;
  }
  uint32_t taken = 0;
  int my_e = 0;
  float my_p = 0.0f, my_p_hi = 0.0f, my_k = 0.0f, seq_sum = 0.0f;
  for (int j = 0; j < K; ++j) {
    uint64_t best = 0;
#pragma unroll
    for (int c = 0; c < EPL; ++c) {
      const int e = lane + c * kWave;
      if (e < E && !((taken >> c) & 1u)) {
        const uint64_t cand = (static_cast<uint64_t>(key[c]) << 32) | (0xffffffffu - static_cast<uint32_t>(e));
        best = cand > best ? cand : best;
      }
    }
    best = wave_max_u64(best);
    const int e_sel = __builtin_amdgcn_readfirstlane(
        static_cast<int>(0xffffffffu - static_cast<uint32_t>(best & 0xffffffffu)));  // the same in every lane
    const int owner = e_sel % kWave, slot = e_sel / kWave;
    float p_sel = 0.0f, k_sel = 0.0f;
#pragma unroll
    for (int c = 0; c < EPL; ++c)
      if (c == slot) {
        p_sel = p[c];
        k_sel = kval[c];
      }
    p_sel = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p_sel), owner));
    k_sel = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(k_sel), owner));
    if (lane == owner) taken |= 1u << slot;
    if (lane == j) {
      my_e = e_sel;
      my_p = p_sel;
      my_k = k_sel;
    }
    if (lane == j - kWave) my_p_hi = p_sel;
    if (K > kWave && lane == 0) {
      top_idx[static_cast<int64_t>(t) * K + j] = e_sel;
      if (K > 2 * kWave) top_w[static_cast<int64_t>(t) * K + j] = p_sel;
    }
    seq_sum = (j == 0) ? p_sel : seq_sum + p_sel;
  }
  if (K > 2 * kWave) {
    // more than 128 choices: renormalised by the plain sum in choice order
    // (torch reduces rows this long in vectors; not restated here)
    if (lane == 0)
      for (int j = 0; j < K; ++j) top_w[static_cast<int64_t>(t) * K + j] /= seq_sum;
    return;
  }
  if (K <= kWave) topk_tie_order(K, my_k, my_e, my_p);
  const float sum = topk_weight_sum(my_p, my_p_hi, K);
  if (K <= kWave) {
    *out_e = my_e;
    *out_w = my_p / sum;
  } else {
    float* w = top_w + static_cast<int64_t>(t) * K;
    w[lane] = my_p / sum;
    if (lane + kWave < K) w[lane + kWave] = my_p_hi / sum;
  }
}

// select_token for E <= 64 (lane l owns expert l) on TT tokens of one wave at
// once: each token goes through exactly the operations select_token applies
// (same reduction trees, same order), and the TT independent chains of
// cross-lane exchanges overlap instead of running one after another.  Tokens
// with valid[i] false are computed on their (finite) inputs and not stored.
// Lane j < K returns round j's expert and renormalised weight of token i in
// out_e[i] / out_w[i].
template <int TT>
__device__ __forceinline__ void select_tokens(float (&l)[TT], const int (&t)[TT], const bool (&valid)[TT], int E,
                                              int K, const float* __restrict__ bias, int select_logits,
                                              float* __restrict__ probs, int (&out_e)[TT], float (&out_w)[TT]) {
  const int lane = threadIdx.x % kWave;
  const bool live = lane < E;
  float m[TT], p[TT], s[TT];
#pragma unroll
  for (int i = 0; i < TT; ++i) m[i] = wave_max(l[i]);
#pragma unroll
  for (int i = 0; i < TT; ++i) {
    if (__any(l[i] != l[i])) m[i] = __builtin_nanf("");  // fmaxf drops NaN; torch's softmax does not
    p[i] = live ? softmax_expf(l[i] - m[i]) : 0.0f;
    s[i] = 0.0f + p[i];  // select_token's per-lane sum starts at 0 (0 + -0 is +0)
    out_e[i] = 0;
    out_w[i] = 0.0f;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1)
#pragma unroll
    for (int i = 0; i < TT; ++i) s[i] += __shfl_xor(s[i], o, kWave);
  uint64_t key[TT];
  float kval[TT], out_k[TT];
  const float b = (bias != nullptr && live) ? bias[lane] : 0.0f;
#pragma unroll
  for (int i = 0; i < TT; ++i) {
    p[i] = p[i] / s[i];
    if (probs != nullptr && live && valid[i]) probs[static_cast<int64_t>(t[i]) * E + lane] = p[i];
    kval[i] = (bias != nullptr && live) ? l[i] + b : (select_logits ? l[i] : p[i]);
    key[i] = live ? (static_cast<uint64_t>(sortable_key(kval[i])) << 32) | (0xffffffffu - static_cast<uint32_t>(lane))
                  : 0;
    out_k[i] = 0.0f;
  }
  for (int j = 0; j < K; ++j) {
    uint64_t best[TT];
#pragma unroll
    for (int i = 0; i < TT; ++i) best[i] = wave_max_u64(key[i]);
#pragma unroll
    for (int i = 0; i < TT; ++i) {
      const int e_sel = __builtin_amdgcn_readfirstlane(
          static_cast<int>(0xffffffffu - static_cast<uint32_t>(best[i] & 0xffffffffu)));  // the same in every lane
      const float p_sel = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p[i]), e_sel));
      const float k_sel = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(kval[i]), e_sel));
      if (lane == e_sel) key[i] = 0;  // taken
      if (lane == j) {
        out_e[i] = e_sel;
        out_w[i] = p_sel;
        out_k[i] = k_sel;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < TT; ++i) {
    topk_tie_order(K, out_k[i], out_e[i], out_w[i]);
    out_w[i] = out_w[i] / topk_weight_sum(out_w[i], 0.0f, K);
  }
}

// With `partial` != NULL the logits are first assembled from the router GEMM's
// split-K partials: L = ((p_0 + p_1) + ... + p_{S-1}) / temperature, and
// written to `logits`.
template <int EPL>
__global__ __launch_bounds__(256) void route_topk_kernel(const float* __restrict__ partial, int splits,
                                                         float temperature, float* __restrict__ logits, int T, int E,
                                                         int K, const float* __restrict__ bias,
                                                         int select_logits, float* __restrict__ probs,
                                                         int32_t* __restrict__ top_idx,
                                                         float* __restrict__ top_w) {
  const int lane = threadIdx.x % kWave;
  const int t = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (t >= T) return;
  float l[EPL];
#pragma unroll
  for (int c = 0; c < EPL; ++c) {
    const int e = lane + c * kWave;
    if (e < E) {
      const int64_t i = static_cast<int64_t>(t) * E + e;
      if (partial != nullptr) {
        float v = partial[i];
        for (int sp = 1; sp < splits; ++sp) v += partial[static_cast<int64_t>(sp) * T * E + i];
        v = v / temperature;
        logits[i] = v;
        l[c] = v;
      } else {
        l[c] = logits[i];
      }
    } else {
      l[c] = -__builtin_inff();
    }
  }
  int me = 0;
  float mw = 0.0f;
  select_token<EPL>(l, t, E, K, bias, select_logits, probs, top_idx, top_w, &me, &mw);
  if (K <= kWave && lane < K) {
    top_idx[static_cast<int64_t>(t) * K + lane] = me;
    top_w[static_cast<int64_t>(t) * K + lane] = mw;
  }
}

// ---------------------------------------------------------------------------
// Router logits and routing in one kernel (bf16, or fp16, x and weights, E <= 64,
// D % 64 == 0): 32 tokens per 512-thread block.  Wave w multiplies the
// block's token rows by the E router rows over the 64-wide k chunks
// w, w + 8, w + 16, ... with bf16 (fp16) MFMA (fp32 accumulation; operands go from
// global memory straight into registers, up to four chunks requested together
// before their multiplies), the eight partial sums meet in LDS and are added in
// wave order, L = (((p_0 + p_1) + ...) + p_7) / temperature, and wave w then
// routes tokens 4w..4w+3 together (select_tokens), writing logits, probs and
// choices exactly as route_topk_kernel does from the same logits.
// ---------------------------------------------------------------------------
constexpr int kFuseTokens = 32, kFuseWaves = 8, kFuseChunk = 64, kFuseSteps = kFuseChunk / 32;
constexpr int kFusePitch = 68;  // LDS row pitch in floats: the partial stores of a wave hit 64 distinct banks

template <int DT>
__global__ __launch_bounds__(kFuseWaves * kWave) void router_topk_kernel(
    const uint16_t* __restrict__ x, int64_t x_stride, const uint16_t* __restrict__ w, int T, int D, int E, int K,
    float temperature, const float* __restrict__ bias, int select_logits, float* __restrict__ logits,
    float* __restrict__ probs, int32_t* __restrict__ top_idx, float* __restrict__ top_w) {
  __shared__ float part[kFuseWaves][kFuseTokens][kFusePitch];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int t0 = blockIdx.x * kFuseTokens;
  const int l16 = lane % 16, kq = (lane / 16) * 8;
  // a-operand rows: tokens t0 + 16m + l16; b-operand rows: experts 16n + l16.
  // Rows past T or E read row 0 instead: an output row (column) depends only on
  // its own a (b) row, and those rows and columns are never read back.
  const uint16_t* arow0 = x + static_cast<int64_t>(t0 + l16 < T ? t0 + l16 : 0) * x_stride + kq;
  const uint16_t* arow1 = x + static_cast<int64_t>(t0 + 16 + l16 < T ? t0 + 16 + l16 : 0) * x_stride + kq;
  const uint16_t* brow[4];
#pragma unroll
  for (int n = 0; n < 4; ++n) brow[n] = w + static_cast<int64_t>(16 * n + l16 < E ? 16 * n + l16 : 0) * D + kq;
  rf32x4 acc[2][4];
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[m][n] = rf32x4{0.f, 0.f, 0.f, 0.f};
  // one chunk: k-steps of 32, lane (l16, kq) holding elements k0 + 32s + kq .. +7 of its rows
#define QW_RT_LOAD(A, B, C)                                                                  \
  {                                                                                          \
    const int k0_ = (C) * kFuseChunk;                                                        \
    _Pragma("unroll") for (int s = 0; s < kFuseSteps; ++s) {                                          \
      A[0][s] = *reinterpret_cast<const uint4*>(arow0 + k0_ + 32 * s);                       \
      A[1][s] = *reinterpret_cast<const uint4*>(arow1 + k0_ + 32 * s);                       \
      _Pragma("unroll") for (int n = 0; n < 4; ++n) B[n][s] =                                \
          *reinterpret_cast<const uint4*>(brow[n] + k0_ + 32 * s);                           \
    }                                                                                        \
  }
#define QW_RT_MUL(A, B)                                                                      \
  {                                                                                          \
    _Pragma("unroll") for (int s = 0; s < kFuseSteps; ++s) {                                          \
      _Pragma("unroll") for (int m = 0; m < 2; ++m) {                                        \
        const rbf16x8 af = __builtin_bit_cast(rbf16x8, A[m][s]);                             \
        _Pragma("unroll") for (int n = 0; n < 4; ++n) acc[m][n] =                            \
            rmfma<DT>(af, __builtin_bit_cast(rbf16x8, B[n][s]), acc[m][n]);                  \
      }                                                                                      \
    }                                                                                        \
  }
  // The wave's chunks go in batches of up to four: all loads of a batch are
  // issued before its first multiply (one memory round trip per batch).
  const int nc = D / kFuseChunk;
  const int mine = wave < nc ? (nc - 1 - wave) / kFuseWaves + 1 : 0;  // chunks of this wave
  auto batch = [&](auto n_c, int c0) {
    constexpr int N = decltype(n_c)::value;
    uint4 a[N][2][kFuseSteps], b[N][4][kFuseSteps];
#pragma unroll
    for (int i = 0; i < N; ++i) QW_RT_LOAD(a[i], b[i], c0 + i * kFuseWaves);
    __builtin_amdgcn_sched_barrier(0);  // every load of the batch before the first multiply
#pragma unroll
    for (int i = 0; i < N; ++i) QW_RT_MUL(a[i], b[i]);
  };
  for (int i0 = 0; i0 < mine; i0 += 4) {
    const int c0 = wave + i0 * kFuseWaves;
    const int n = mine - i0;
    if (n >= 4) batch(std::integral_constant<int, 4>{}, c0);
    else if (n == 3) batch(std::integral_constant<int, 3>{}, c0);
    else if (n == 2) batch(std::integral_constant<int, 2>{}, c0);
    else batch(std::integral_constant<int, 1>{}, c0);
  }
#undef QW_RT_LOAD
#undef QW_RT_MUL
  // lane holds C[token 16m + 4(lane/16) + r][expert 16n + l16]
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
      for (int r = 0; r < 4; ++r) part[wave][16 * m + 4 * (lane / 16) + r][16 * n + l16] = acc[m][n][r];
  __syncthreads();
  constexpr int TPW = kFuseTokens / kFuseWaves;  // tokens each wave routes
  float l[TPW];
  int tok[TPW];
  bool ok[TPW];
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int tl = wave * TPW + i;
    tok[i] = t0 + tl;
    ok[i] = tok[i] < T;
    if (lane < E) {
      float v = part[0][tl][lane];
#pragma unroll
      for (int p = 1; p < kFuseWaves; ++p) v += part[p][tl][lane];
      v = v / temperature;
      if (ok[i]) logits[static_cast<int64_t>(tok[i]) * E + lane] = v;
      l[i] = v;
    } else {
      l[i] = -__builtin_inff();
    }
  }
  int me[TPW];
  float mw[TPW];
  select_tokens<TPW>(l, tok, ok, E, K, bias, select_logits, probs, me, mw);
#pragma unroll
  for (int i = 0; i < TPW; ++i)
    if (ok[i] && lane < K) {
      top_idx[static_cast<int64_t>(tok[i]) * K + lane] = me[i];
      top_w[static_cast<int64_t>(tok[i]) * K + lane] = mw[i];
    }
}

static bool router_topk_fits(int xdt, int wdt, const void* x, int64_t x_stride, const void* w, int64_t T,
                             int64_t D, int64_t E) {
  return is_half(xdt) && wdt == xdt && T > kGemvMaxTokens && E <= kWave && D % kFuseChunk == 0 &&
         x_stride % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0;
}

static int launch_topk(const float* partial, int splits, float temperature, float* logits, int T, int E, int K,
                       const float* bias, int select_logits, float* probs, int32_t* top_idx, float* top_w,
                       hipStream_t stream) {
  const int waves_per_block = 4;
  const dim3 grid(static_cast<unsigned>(ceil_div(T, waves_per_block)));
  const dim3 block(waves_per_block * kWave);
  const int epl = static_cast<int>(ceil_div(E, kWave));
#define QW_TK(N)                                                                                               \
  route_topk_kernel<N><<<grid, block, 0, stream>>>(partial, splits, temperature, logits, T, E, K, bias, \
                                                   select_logits, probs, top_idx, top_w)
  if (epl <= 1) QW_TK(1);
  else if (epl <= 2) QW_TK(2);
  else if (epl <= 4) QW_TK(4);
  else if (epl <= 8) QW_TK(8);
  else QW_TK(16);
#undef QW_TK
  QW_LAUNCH_CHECK("route_topk_kernel");
  return QW_OK;
}

// ---------------------------------------------------------------------------
// Routing and capacity plan of a small batch in one workgroup (decode sizes:
// R = T*K <= kSmallRoutes, K <= 64), replacing the plan kernel, and for up to
// 16 tokens (`routed` = 0) the top-k kernel too:
//   1. wave w routes token w exactly as route_topk_kernel does, the choices
//      also going to LDS (`routed` = 1: the choices are read from top_idx and
//      top_w, written by route_topk_kernel);
//   2. thread r < R counts route r into an LDS histogram; counts, kept counts
//      min(count, capacity) and their exclusive scans give every expert's
//      kept and dropped offsets (as plan_kernel does);
//   3. thread r ranks route r among the routes of its expert by the plan key
//      (weight descending, then route id: src/quantweave_moe_model.py:174-175)
//      and writes its slot, or its dropped entry.
// Optionally the same workgroup writes cast_out = bf16(cast_x) (or fp16 with
// cast_f16; n values), the decode step's expert input.  THREADS is 1024, or 64
// (one wave: its barriers cost next to nothing) for one or two tokens with
// at most 64 routes and 64 experts, whose cast the router GEMV writes instead.
// ---------------------------------------------------------------------------
constexpr int kSmallThreads = 1024;
constexpr int kSmallTokens = 64;       // tokens of the one-workgroup plan
constexpr int kSmallRouteTokens = 16;  // tokens it also routes (one per wave)
constexpr int kSmallRoutes = 256;
constexpr int kSmallLogits = 8192;  // T*E logits staged in LDS

template <int EPL, int THREADS>
__global__ __launch_bounds__(THREADS) void route_plan_small_kernel(
    int routed, const float* __restrict__ partial, int splits, float temperature, float* __restrict__ logits, int T,
    int E, int K, const float* __restrict__ bias, int select_logits,
    float* __restrict__ probs, int32_t* __restrict__ top_idx, float* __restrict__ top_w, int capacity,
    int32_t* __restrict__ counts, int32_t* __restrict__ kept_counts, int32_t* __restrict__ kept_offsets,
    int32_t* __restrict__ totals, int32_t* __restrict__ slot_token, float* __restrict__ slot_weight,
    int32_t* __restrict__ route_slot, int32_t* __restrict__ dropped_token, int32_t* __restrict__ dropped_expert,
    const float* __restrict__ cast_x, int cast_n, uint16_t* __restrict__ cast_out, int cast_f16) {
  constexpr int kWaves = THREADS / kWave;
  __shared__ float s_logit[kSmallLogits];
  __shared__ int s_e[kSmallRoutes];
  __shared__ float s_w[kSmallRoutes];
  __shared__ uint64_t s_key[kSmallRoutes];
  __shared__ int hist[1024], s_ko[1024], s_do[1024];
  __shared__ uint64_t warp_tot[kWaves];
  __shared__ uint64_t s_tot;
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int R = T * K;
  for (int i = tid; i < E; i += THREADS) hist[i] = 0;
  if (cast_out != nullptr) {
    for (int i = tid * 4; i < cast_n; i += THREADS * 4) {
      if (i + 4 <= cast_n && (cast_n & 3) == 0) {
        const float4 v = *reinterpret_cast<const float4*>(cast_x + i);
        uint2 o;
        if (cast_f16) {
          o.x = pack_half2<QW_F16>(v.x, v.y);
          o.y = pack_half2<QW_F16>(v.z, v.w);
        } else {
          o.x = pack_half2<QW_BF16>(v.x, v.y);
          o.y = pack_half2<QW_BF16>(v.z, v.w);
        }
        *reinterpret_cast<uint2*>(cast_out + i) = o;
      } else {
        for (int j = i; j < i + 4 && j < cast_n; ++j)
          cast_out[j] = cast_f16 ? f32_to_f16(cast_x[j]) : f32_to_bf16(cast_x[j]);
      }
    }
  }
  if (routed) {
    // ---- the routing was done by route_topk_kernel: its choices into LDS ----
    for (int r = tid; r < R; r += THREADS) {
      const int me = top_idx[r];
      const float mw = top_w[r];
      s_e[r] = me;
      s_w[r] = mw;
      s_key[r] = (static_cast<uint64_t>(~sortable_key(mw)) << 32) | static_cast<uint32_t>(r);
    }
  }
  // ---- 0. all logits into LDS at once (summing split-K partials if given) ----
  for (int i = tid; i < (routed ? 0 : T * E); i += THREADS) {
    float v;
    if (partial != nullptr) {
      v = partial[i];
#pragma unroll 4
      for (int sp = 1; sp < splits; ++sp) v += partial[static_cast<int64_t>(sp) * T * E + i];
      v = v / temperature;
      logits[i] = v;
    } else {
      v = logits[i];
    }
    s_logit[i] = v;
  }
  __syncthreads();
  // ---- 1. routing, one wave per token ----
  for (int t = wave; t < (routed ? 0 : T); t += kWaves) {
    float l[EPL];
#pragma unroll
    for (int c = 0; c < EPL; ++c) {
      const int e = lane + c * kWave;
      l[c] = e < E ? s_logit[t * E + e] : -__builtin_inff();
    }
    int me = 0;
    float mw = 0.0f;
    select_token<EPL>(l, t, E, K, bias, select_logits, probs, top_idx, top_w, &me, &mw);
    if (lane < K) {
      const int r = t * K + lane;
      top_idx[r] = me;
      top_w[r] = mw;
      s_e[r] = me;
      s_w[r] = mw;
      s_key[r] = (static_cast<uint64_t>(~sortable_key(mw)) << 32) | static_cast<uint32_t>(r);
    }
  }
  __syncthreads();
  // ---- 2. counts and offsets ----
  int my_e = -1;
  if (tid < R) {
    my_e = s_e[tid];
    atomicAdd(&hist[my_e], 1);
  }
  __syncthreads();
  const int c = tid < E ? hist[tid] : 0;
  const int kc = c < capacity ? c : capacity;
  // kept count in the low word, dropped count in the high word (every prefix
  // sum is at most R, so the words never carry into each other): one scan
  const uint64_t excl =
      block_exclusive_scan((static_cast<uint64_t>(c - kc) << 32) | static_cast<uint32_t>(kc), warp_tot, &s_tot);
  const int ko = static_cast<int>(excl & 0xffffffffu), dof = static_cast<int>(excl >> 32);
  if (tid < E) {
    s_ko[tid] = ko;
    s_do[tid] = dof;
    counts[tid] = c;
    kept_counts[tid] = kc;
    kept_offsets[tid] = ko;
  }
  if (tid == 0) {
    kept_offsets[E] = static_cast<int>(s_tot & 0xffffffffu);
    totals[0] = static_cast<int>(s_tot & 0xffffffffu);
    totals[1] = static_cast<int>(s_tot >> 32);
  }
  __syncthreads();
  // ---- 3. rank within the expert and place ----
  if (tid < R) {
    const uint64_t key = s_key[tid];
    int pos = 0;
    for (int j = 0; j < R; ++j) pos += (s_e[j] == my_e && s_key[j] < key) ? 1 : 0;
    const int token = tid / K;
    if (pos < capacity) {
      const int s = s_ko[my_e] + pos;
      slot_token[s] = token;
      slot_weight[s] = s_w[tid];
      route_slot[tid] = s;
    } else {
      const int q = s_do[my_e] + (pos - capacity);
      dropped_token[q] = token;
      dropped_expert[q] = my_e;
      route_slot[tid] = -1;
    }
  }
}

template <int XD, int WD, int VEC>
static void launch_router_gemv_tt(const void* x, int64_t x_stride, const void* w, int t, int d, int e,
                                  float temperature, float* logits, uint16_t* cast_out, int cast_f16,
                                  hipStream_t stream) {
  const dim3 g16(e, static_cast<unsigned>(ceil_div(t, 16)));
  if (t <= 1)
    router_gemv_kernel<XD, WD, VEC, 1><<<e, 256, 0, stream>>>(x, x_stride, w, t, d, e, temperature, logits, cast_out,
                                                              cast_f16);
  else if (t <= 4)
    router_gemv_kernel<XD, WD, VEC, 4><<<e, 256, 0, stream>>>(x, x_stride, w, t, d, e, temperature, logits, cast_out,
                                                              cast_f16);
  else
    router_gemv_kernel<XD, WD, VEC, 16><<<g16, 256, 0, stream>>>(x, x_stride, w, t, d, e, temperature, logits,
                                                                 cast_out, cast_f16);
}

template <int XD, int WD>
static void launch_router_gemv_vec(bool vec, const void* x, int64_t x_stride, const void* w, int t, int d, int e,
                                   float temperature, float* logits, uint16_t* cast_out, int cast_f16,
                                   hipStream_t stream) {
  if (vec) launch_router_gemv_tt<XD, WD, 4>(x, x_stride, w, t, d, e, temperature, logits, cast_out, cast_f16, stream);
  else launch_router_gemv_tt<XD, WD, 1>(x, x_stride, w, t, d, e, temperature, logits, cast_out, cast_f16, stream);
}

// Calls f(XD, WD) with the dtype codes of the router input and weights as
// compile-time constants (fp32, bf16 or fp16 each).
template <typename Fn>
static void with_router_dtypes(int xdt, int wdt, Fn&& f) {
  auto inner = [&](auto xd) {
    if (wdt == QW_F32) f(xd, std::integral_constant<int, QW_F32>{});
    else if (wdt == QW_F16) f(xd, std::integral_constant<int, QW_F16>{});
    else f(xd, std::integral_constant<int, QW_BF16>{});
  };
  if (xdt == QW_F32) inner(std::integral_constant<int, QW_F32>{});
  else if (xdt == QW_F16) inner(std::integral_constant<int, QW_F16>{});
  else inner(std::integral_constant<int, QW_BF16>{});
}

static int launch_router_gemv(const void* x, int xdt, int64_t x_stride, const void* w, int wdt, int t, int d,
                              int e, float temperature, float* logits, hipStream_t stream,
                              uint16_t* cast_out = nullptr, int cast_f16 = 0) {
  const bool vec = d % 4 == 0 && x_stride % 4 == 0 && (reinterpret_cast<uintptr_t>(x) % 16) == 0 &&
                   (reinterpret_cast<uintptr_t>(w) % 16) == 0;
  with_router_dtypes(xdt, wdt, [&](auto xd, auto wd) {
    launch_router_gemv_vec<decltype(xd)::value, decltype(wd)::value>(vec, x, x_stride, w, t, d, e, temperature,
                                                                       logits, cast_out, cast_f16, stream);
  });
  QW_LAUNCH_CHECK("router_gemv_kernel");
  return QW_OK;
}

int route_validate(int64_t T, int64_t E, int64_t K) {
  QW_REQUIRE(T >= 0 && T <= INT32_MAX / 64, "tokens out of range: %lld", (long long)T);
  QW_REQUIRE(E >= 1 && E <= 1024, "experts must be in [1, 1024], got %lld", (long long)E);
  QW_REQUIRE(K >= 1 && K <= E, "top_k must be between 1 and num_experts (got %lld, %lld)", (long long)K,
             (long long)E);
  QW_REQUIRE(T * K <= INT32_MAX, "tokens*top_k exceeds int32");
  return QW_OK;
}

int route_from_logits(const float* logits, int64_t T, int64_t E, int64_t K, const float* bias, float* probs,
                      int32_t* top_idx, float* top_w, hipStream_t stream) {
  int st = route_validate(T, E, K);
  if (st) return st;
  if (T == 0) return QW_OK;
  QW_REQUIRE(logits && top_idx && top_w, "logits, top_idx and top_w are required");
  return launch_topk(nullptr, 0, 1.0f, const_cast<float*>(logits), static_cast<int>(T), static_cast<int>(E),
                     static_cast<int>(K), bias, 0, probs, top_idx, top_w, stream);
}

// Split count for the router GEMM: enough blocks to cover the chip, each
// split a multiple of 64 long and at least 256 deep.
int router_splits(int64_t T, int64_t D, int64_t E) {
  const int64_t tiles = ceil_div(T, 64) * ceil_div(E, 64);
  int64_t s = 1;
  while (tiles * s < 512 && D / (s * 2) >= 256) s *= 2;
  return static_cast<int>(s);
}

size_t route_workspace_bytes(int64_t T, int64_t D, int64_t E) {
  return static_cast<size_t>(router_splits(T, D, E)) * T * E * sizeof(float);
}

// Router logits: up to kGemvMaxTokens tokens (or a small layer) by the GEMV
// kernel straight into `logits` (*splits = 0); more by the tiled GEMM into
// split-K partials (*splits > 0) that the next kernel sums and divides by the
// temperature.
static int launch_router_cast(const void* x, int xdt, int64_t x_stride, const void* w, int wdt, int64_t T,
                              int64_t D, int64_t E, float temperature, float* logits, float* partial,
                              size_t partial_bytes, int* splits_out, hipStream_t stream, uint16_t* cast_out,
                              int cast_f16) {
  const int t = static_cast<int>(T), d = static_cast<int>(D), e = static_cast<int>(E);
  // The GEMV kernel issues all its loads at once but reads x once per expert:
  // it serves a few tokens, and any batch whose x re-reads stay within 16 MiB
  // (small layers, where the tiled kernel's K loop would wait on every slice).
  if (T <= kGemvMaxTokens || T * E * D * (xdt == QW_F32 ? 4 : 2) <= (int64_t{16} << 20)) {
    *splits_out = 0;
    return launch_router_gemv(x, xdt, x_stride, w, wdt, t, d, e, temperature, logits, stream, cast_out, cast_f16);
  }
  QW_REQUIRE(cast_out == nullptr, "the cast rides on the GEMV router only");
  const int splits = router_splits(T, D, E);
  if (partial_bytes < static_cast<size_t>(splits) * T * E * sizeof(float) || !partial)
    return set_error(QW_ERR_WORKSPACE, "router needs %zu bytes of partial sums", route_workspace_bytes(T, D, E));
  *splits_out = splits;
  int64_t k_len = ceil_div(D, splits);
  k_len = ceil_div(k_len, 64) * 64;
  const dim3 grid(static_cast<unsigned>(ceil_div(T, 64)), static_cast<unsigned>(splits),
                  static_cast<unsigned>(ceil_div(E, 64)));
  const int kl = static_cast<int>(k_len);
  if (is_half(xdt) && wdt == xdt && D % 64 == 0) {
    if (xdt == QW_F16)
      router_mfma_kernel<QW_F16><<<grid, 256, 0, stream>>>(static_cast<const uint16_t*>(x), x_stride,
                                                           static_cast<const uint16_t*>(w), t, d, e, kl, partial);
    else
      router_mfma_kernel<QW_BF16><<<grid, 256, 0, stream>>>(static_cast<const uint16_t*>(x), x_stride,
                                                            static_cast<const uint16_t*>(w), t, d, e, kl, partial);
    QW_LAUNCH_CHECK("router_mfma_kernel");
  } else {
    with_router_dtypes(xdt, wdt, [&](auto xd, auto wd) {
      router_logits_kernel<decltype(xd)::value, decltype(wd)::value>
          <<<grid, 256, 0, stream>>>(x, x_stride, w, t, d, e, kl, partial);
    });
    QW_LAUNCH_CHECK("router_logits_kernel");
  }
  return QW_OK;
}

static int launch_router(const void* x, int xdt, int64_t x_stride, const void* w, int wdt, int64_t T, int64_t D,
                         int64_t E, float temperature, float* logits, float* partial, size_t partial_bytes,
                         int* splits_out, hipStream_t stream) {
  return launch_router_cast(x, xdt, x_stride, w, wdt, T, D, E, temperature, logits, partial, partial_bytes,
                            splits_out, stream, nullptr, 0);
}

int route(const void* x, int xdt, int64_t x_stride, const void* w, int wdt, int64_t T, int64_t D, int64_t E,
          int64_t K, float temperature, const float* bias, float* logits, float* probs, int32_t* top_idx,
          float* top_w, float* partial, size_t partial_bytes, hipStream_t stream, bool select_logits) {
  int st = route_validate(T, E, K);
  if (st) return st;
  QW_REQUIRE(xdt == QW_F32 || xdt == QW_BF16 || xdt == QW_F16, "router input dtype must be f32, bf16 or f16");
  QW_REQUIRE(wdt == QW_F32 || wdt == QW_BF16 || wdt == QW_F16, "router weight dtype must be f32, bf16 or f16");
  QW_REQUIRE(D >= 1 && D <= INT32_MAX, "d_model out of range");
  QW_REQUIRE(x_stride >= D, "x row stride %lld smaller than d_model %lld", (long long)x_stride, (long long)D);
  QW_REQUIRE(temperature > 0.0f, "router_temperature must be positive");
  if (T == 0) return QW_OK;
  QW_REQUIRE(x && w && logits && top_idx && top_w, "x, router_w, logits, top_idx and top_w are required");
  const int t = static_cast<int>(T), e = static_cast<int>(E), k = static_cast<int>(K);
  if (router_topk_fits(xdt, wdt, x, x_stride, w, T, D, E)) {
    const unsigned g = static_cast<unsigned>(ceil_div(T, kFuseTokens));
    if (xdt == QW_F16)
      router_topk_kernel<QW_F16><<<g, kFuseWaves * kWave, 0, stream>>>(
          static_cast<const uint16_t*>(x), x_stride, static_cast<const uint16_t*>(w), t, static_cast<int>(D), e, k,
          temperature, bias, select_logits ? 1 : 0, logits, probs, top_idx, top_w);
    else
      router_topk_kernel<QW_BF16><<<g, kFuseWaves * kWave, 0, stream>>>(
          static_cast<const uint16_t*>(x), x_stride, static_cast<const uint16_t*>(w), t, static_cast<int>(D), e, k,
          temperature, bias, select_logits ? 1 : 0, logits, probs, top_idx, top_w);
    QW_LAUNCH_CHECK("router_topk_kernel");
    return QW_OK;
  }
  int splits = 0;
  st = launch_router(x, xdt, x_stride, w, wdt, T, D, E, temperature, logits, partial, partial_bytes, &splits, stream);
  if (st) return st;
  return launch_topk(splits ? partial : nullptr, splits, temperature, logits, t, e, k, bias, select_logits ? 1 : 0,
                     probs, top_idx, top_w, stream);
}

// Small batches: router logits, then routing + plan (+ cast) in one workgroup.
// The caller checks route_plan_small_fits first.
bool route_plan_small_fits(int64_t T, int64_t E, int64_t K) {
  return T >= 1 && T <= kSmallTokens && K >= 1 && K <= kWave && K <= E && E <= 1024 && T * K <= kSmallRoutes &&
         (T > kSmallRouteTokens || T * E <= kSmallLogits);
}

int route_plan_small(const void* x, int xdt, int64_t x_stride, const void* w, int wdt, int64_t T, int64_t D,
                     int64_t E, int64_t K, float temperature, const float* bias, bool select_logits, float* logits,
                     float* probs, int32_t* top_idx, float* top_w, int64_t capacity, int32_t* counts,
                     int32_t* kept_counts, int32_t* kept_offsets, int32_t* totals, int32_t* slot_token,
                     float* slot_weight, int32_t* route_slot, int32_t* dropped_token, int32_t* dropped_expert,
                     const float* cast_x, uint16_t* cast_out, int cast_dtype, float* partial,
                     size_t partial_bytes, hipStream_t stream) {
  int st = route_validate(T, E, K);
  if (st) return st;
  QW_REQUIRE(route_plan_small_fits(T, E, K), "batch too large for the one-workgroup plan");
  QW_REQUIRE(xdt == QW_F32 || xdt == QW_BF16 || xdt == QW_F16, "router input dtype must be f32, bf16 or f16");
  QW_REQUIRE(wdt == QW_F32 || wdt == QW_BF16 || wdt == QW_F16, "router weight dtype must be f32, bf16 or f16");
  QW_REQUIRE(D >= 1 && D <= INT32_MAX / kSmallTokens && x_stride >= D, "bad router sizes");
  QW_REQUIRE(temperature > 0.0f, "router_temperature must be positive");
  QW_REQUIRE(capacity >= 0, "capacity must be >= 0");
  QW_REQUIRE(x && w && logits && top_idx && top_w && counts && kept_counts && kept_offsets && totals && slot_token &&
                 slot_weight && route_slot && dropped_token && dropped_expert,
             "routing and plan arrays are required");
  QW_REQUIRE(cast_out == nullptr || (cast_x != nullptr && x_stride == D), "cast needs contiguous fp32 rows");
  QW_REQUIRE(cast_out == nullptr || is_half(cast_dtype), "the cast is to bf16 or f16");
  const int t = static_cast<int>(T), d = static_cast<int>(D), e = static_cast<int>(E), k = static_cast<int>(K);
  int splits = 0;
  const int routed = T > kSmallRouteTokens ? 1 : 0;
  if (routed) {
    st = route(x, xdt, x_stride, w, wdt, T, D, E, K, temperature, bias, logits, probs, top_idx, top_w, partial,
               partial_bytes, stream, select_logits);
  }
  // one or two tokens: the GEMV router writes the cast and one wave plans
  const bool tiny = !routed && T <= 2 && T * K <= kWave && E <= kWave && T <= kGemvMaxTokens &&
                    (cast_out == nullptr || (cast_x == x && xdt == QW_F32));
  if (!routed) {
    st = launch_router_cast(x, xdt, x_stride, w, wdt, T, D, E, temperature, logits, partial, partial_bytes, &splits,
                            stream, tiny ? cast_out : nullptr, cast_dtype == QW_F16 ? 1 : 0);
  }
  if (st) return st;
  const float* part = splits ? partial : nullptr;
  const int cap = capacity > INT32_MAX ? INT32_MAX : static_cast<int>(capacity);
  const int n = cast_out && !tiny ? t * d : 0;
  const int epl = static_cast<int>(ceil_div(E, kWave));
#define QW_RP(N, TH)                                                                                          \
  route_plan_small_kernel<N, TH><<<1, TH, 0, stream>>>(routed, part, splits, temperature, logits, t, e, k, bias, \
                                                       select_logits ? 1 : 0, probs, top_idx, top_w, cap, counts, \
                                                       kept_counts, kept_offsets, totals, slot_token, slot_weight, \
                                                       route_slot, dropped_token, dropped_expert, cast_x, n,       \
                                                       n ? cast_out : nullptr, cast_dtype == QW_F16 ? 1 : 0)
  if (tiny) QW_RP(1, kWave);
  else if (epl <= 1) QW_RP(1, kSmallThreads);
  else if (epl <= 2) QW_RP(2, kSmallThreads);
  else if (epl <= 4) QW_RP(4, kSmallThreads);
  else if (epl <= 8) QW_RP(8, kSmallThreads);
  else QW_RP(16, kSmallThreads);
#undef QW_RP
  QW_LAUNCH_CHECK("route_plan_small_kernel");
  return QW_OK;
}

}  // namespace qw
