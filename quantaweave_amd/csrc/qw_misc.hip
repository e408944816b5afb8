// Permute, combine, balance loss, weight quantisation and the plain grouped
// matmul.
#include "qw_weights.h"
#include "qw_ffn.h"

namespace qw {

// ---------------------------------------------------------------------------
// Permute: out[s] = x[slot_token[s]] (src/quantweave_moe_model.py:195).
// One block per row; 16-byte vectors when the row is 16-byte aligned.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void permute_kernel(const char* __restrict__ x, int64_t row_bytes,
                                                      const int32_t* __restrict__ slot_token,
                                                      const int32_t* __restrict__ totals, int max_rows,
                                                      char* __restrict__ out) {
  const int s = blockIdx.x;
  const int n = min(*totals, max_rows);
  if (s >= n) return;
  const char* src = x + static_cast<int64_t>(slot_token[s]) * row_bytes;
  char* dst = out + static_cast<int64_t>(s) * row_bytes;
  if ((row_bytes & 15) == 0) {
    const int64_t nv = row_bytes / 16;
    for (int64_t i = threadIdx.x; i < nv; i += blockDim.x)
      reinterpret_cast<uint4*>(dst)[i] = reinterpret_cast<const uint4*>(src)[i];
  } else {
    for (int64_t i = threadIdx.x; i < row_bytes; i += blockDim.x) dst[i] = src[i];
  }
}

int permute(const void* x, int dtype, int64_t D, const int32_t* slot_token, const int32_t* totals, int64_t max_rows,
            void* out, hipStream_t stream) {
  QW_REQUIRE(dtype == QW_F32 || dtype == QW_BF16 || dtype == QW_F16, "permute dtype must be f32, bf16 or f16");
  QW_REQUIRE(D >= 1 && max_rows >= 0 && max_rows <= INT32_MAX, "bad permute sizes");
  if (max_rows == 0) return QW_OK;
  QW_REQUIRE(x && slot_token && totals && out, "permute pointers are required");
  const int64_t row_bytes = D * (dtype == QW_F32 ? 4 : 2);
  permute_kernel<<<static_cast<unsigned>(max_rows), 256, 0, stream>>>(
      static_cast<const char*>(x), row_bytes, slot_token, totals, static_cast<int>(max_rows), static_cast<char*>(out));
  QW_LAUNCH_CHECK("permute_kernel");
  return QW_OK;
}

// ---------------------------------------------------------------------------
// Combine: out[t] = the kept routes of t added in ascending expert order (the
// plan order of `tokens`) in fp32, starting from zero, and rounded to the
// output dtype once — the arithmetic of torch's
// `zeros_like(flat).index_add_(0, tokens, y)` (src/quantweave_moe_model.py:192,
// :201, :211), which for a bf16 output accumulates in fp32 in index order and
// rounds at the end.  One block per token.
// WEIGHTED: each row enters as (y * w).to(out dtype), w the route's router
// weight — `expert_output * weights[:, None]` (:201) with unweighted rows.
// The same kernel with weights off and OUT = fp32 is the backward of the row
// gather flat[tokens] (:192): index_add of the rows' gradients.
// ---------------------------------------------------------------------------
// STATIC: the accumulation of the capacity-free static dispatch
// (TopKMoE._static_output, src/quantweave_moe_model.py:235-245): the route
// weight is cast to the output dtype before the product
// (`dense_weights[:, e].to(flat_hidden.dtype)`), and `output = output + term`
// rounds after every add, expert by expert in ascending order (the experts
// with weight zero add exact zeros and are skipped).
// KMAX >= K bounds the routes per token; the token's kept routes are put in
// ascending expert order in registers (a static ranking network, no indexed
// private memory).
template <int ACT, int OUT, int VEC, int KMAX, bool WEIGHTED, bool STATIC = false>
__global__ __launch_bounds__(256) void combine_kernel(const void* __restrict__ y, const int32_t* __restrict__ route_slot,
                                                      const int32_t* __restrict__ top_idx,
                                                      const float* __restrict__ top_w, int K, int D,
                                                      void* __restrict__ out) {
  // products and sums rounded one by one (no fused multiply-add): the weighted
  // term is the reference's y * w, rounded to the output dtype before its
  // index_add; the sum is rounded when it is stored
#pragma clang fp contract(off)
  const int t = blockIdx.x;
  int sl[KMAX], ex[KMAX];
  float wt[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    sl[j] = j < K ? route_slot[static_cast<int64_t>(t) * K + j] : -1;
    ex[j] = j < K ? top_idx[static_cast<int64_t>(t) * K + j] : 0;
    wt[j] = (WEIGHTED && j < K) ? top_w[static_cast<int64_t>(t) * K + j] : 1.0f;
    if (STATIC) wt[j] = round_act<OUT>(wt[j]);
  }
  // rank of each kept route among the kept routes by expert id (experts of a token are distinct)
  int rk[KMAX];
  int nk = 0;
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    int r = 0;
#pragma unroll
    for (int i = 0; i < KMAX; ++i) r += (sl[i] >= 0 && ex[i] < ex[j]) ? 1 : 0;
    rk[j] = sl[j] >= 0 ? r : KMAX;
    nk += sl[j] >= 0 ? 1 : 0;
  }
  int slot[KMAX];
  float wsl[KMAX];
#pragma unroll
  for (int p = 0; p < KMAX; ++p) {
    int s = 0;
    float w = 1.0f;
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
      s = rk[j] == p ? sl[j] : s;
      w = rk[j] == p ? wt[j] : w;
    }
    slot[p] = s;
    wsl[p] = w;
  }
  const int64_t row = static_cast<int64_t>(t) * D;
  // the rows of up to G routes are requested together, then added in order
  // (a route past the kept ones reads the first kept route's row and adds
  // nothing; the empty volatile asm keeps each load ahead of the additions
  // instead of sunk into its route's branch)
  constexpr int G = KMAX < 4 ? KMAX : 4;
  static_assert(KMAX % G == 0, "whole groups of routes");
  for (int c = threadIdx.x * VEC; c < D; c += blockDim.x * VEC) {
    float acc[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) acc[v] = 0.0f;
    auto add = [&](const float (&yr)[VEC], float w) {
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        const float term = WEIGHTED ? round_act<OUT>(yr[v] * w) : yr[v];
        acc[v] = STATIC ? round_act<OUT>(acc[v] + term) : acc[v] + term;
      }
    };
    if constexpr (KMAX <= 16) {
#pragma unroll
      for (int j0 = 0; j0 < KMAX; j0 += G) {
        if (j0 >= nk) break;
        float yv[G][VEC];
#pragma unroll
        for (int g = 0; g < G; ++g)
          load_vec<ACT, VEC>(y, static_cast<int64_t>(j0 + g < nk ? slot[j0 + g] : slot[0]) * D + c, yv[g]);
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int v = 0; v < VEC; ++v) asm volatile("" : "+v"(yv[g][v]));
#pragma unroll
        for (int g = 0; g < G; ++g)
          if (j0 + g < nk) add(yv[g], wsl[j0 + g]);
      }
    } else {  // one route at a time
#pragma unroll
      for (int j = 0; j < KMAX; ++j) {
        if (j < nk) {
          float yv[VEC];
          load_vec<ACT, VEC>(y, static_cast<int64_t>(slot[j]) * D + c, yv);
          add(yv, wsl[j]);
        }
      }
    }
    store_vec<OUT, VEC>(out, row + c, acc);
  }
}

template <int ACT, int OUT, int KMAX, bool WEIGHTED, bool STATIC>
void launch_combine_vec(const void* y, const int32_t* route_slot, const int32_t* top_idx, const float* top_w,
                        unsigned g, int k, int d, void* out, hipStream_t stream) {
  constexpr int V = (ACT != QW_F32 || OUT != QW_F32) ? 8 : 4;
  if (d % V == 0)
    combine_kernel<ACT, OUT, V, KMAX, WEIGHTED, STATIC>
        <<<g, 256, 0, stream>>>(y, route_slot, top_idx, top_w, k, d, out);
  else
    combine_kernel<ACT, OUT, 1, KMAX, WEIGHTED, STATIC>
        <<<g, 256, 0, stream>>>(y, route_slot, top_idx, top_w, k, d, out);
}

template <int KMAX, bool WEIGHTED, bool STATIC>
int launch_combine(const void* y, int dtype, const int32_t* route_slot, const int32_t* top_idx, const float* top_w,
                   unsigned g, int k, int d, void* out, int out_dtype, hipStream_t stream) {
#define QW_CB(A, O)                                                                                             \
  if (dtype == A && out_dtype == O)                                                                             \
    launch_combine_vec<A, O, KMAX, WEIGHTED, STATIC>(y, route_slot, top_idx, top_w, g, k, d, out, stream);   \
  else
  QW_CB(QW_F32, QW_F32)
  QW_CB(QW_F32, QW_BF16)
  QW_CB(QW_BF16, QW_F32)
  QW_CB(QW_BF16, QW_BF16)
  QW_CB(QW_F16, QW_F16)
  QW_CB(QW_F16, QW_F32)
  QW_CB(QW_F32, QW_F16)
  return set_error(QW_ERR_INVALID, "combine does not take rows of dtype %d into an output of dtype %d", dtype,
                   out_dtype);
#undef QW_CB
  QW_LAUNCH_CHECK("combine_kernel");
  return QW_OK;
}

template <bool WEIGHTED, bool STATIC = false>
int combine_k(const void* y, int dtype, const int32_t* route_slot, const int32_t* top_idx, const float* top_w,
              int64_t T, int64_t K, int64_t D, void* out, int out_dtype, hipStream_t stream) {
  const unsigned g = static_cast<unsigned>(T);
  const int k = static_cast<int>(K), d = static_cast<int>(D);
#define QW_CK(N)                                                                                                 \
  if (K <= N)                                                                                                    \
    return launch_combine<N, WEIGHTED, STATIC>(y, dtype, route_slot, top_idx, top_w, g, k, d, out, out_dtype, stream);
  QW_CK(2)
  QW_CK(4)
  QW_CK(8)
  QW_CK(16)
#undef QW_CK
  return launch_combine<64, WEIGHTED, STATIC>(y, dtype, route_slot, top_idx, top_w, g, k, d, out, out_dtype, stream);
}

static int combine_check(const void* y, int dtype, const int32_t* route_slot, const int32_t* top_idx, int64_t T,
                         int64_t K, int64_t D, void* out, int out_dtype) {
  QW_REQUIRE((dtype == QW_F32 || dtype == QW_BF16 || dtype == QW_F16) &&
                 (out_dtype == QW_F32 || out_dtype == QW_BF16 || out_dtype == QW_F16),
             "combine dtypes must be f32, bf16 or f16");
  QW_REQUIRE(!(is_half(dtype) && is_half(out_dtype) && dtype != out_dtype),
             "combine does not mix bf16 and f16 (rows %d, output %d)", dtype, out_dtype);
  QW_REQUIRE(K >= 1 && K <= 64, "combine supports top_k in [1, 64], got %lld", (long long)K);
  QW_REQUIRE(T >= 0 && T <= INT32_MAX && D >= 1 && D <= INT32_MAX, "bad combine sizes");
  QW_REQUIRE(T == 0 || (y && route_slot && top_idx && out), "combine pointers are required");
  return QW_OK;
}

int combine_weighted(const void* y, int dtype, const int32_t* route_slot, const int32_t* top_idx, const float* top_w,
                     int64_t T, int64_t K, int64_t D, void* out, int out_dtype, hipStream_t stream) {
  if (const int st = combine_check(y, dtype, route_slot, top_idx, T, K, D, out, out_dtype)) return st;
  if (T == 0) return QW_OK;
  if (top_w) return combine_k<true>(y, dtype, route_slot, top_idx, top_w, T, K, D, out, out_dtype, stream);
  return combine_k<false>(y, dtype, route_slot, top_idx, nullptr, T, K, D, out, out_dtype, stream);
}

int combine_static(const void* y, int dtype, const int32_t* route_slot, const int32_t* top_idx, const float* top_w,
                   int64_t T, int64_t K, int64_t D, void* out, int out_dtype, hipStream_t stream) {
  if (const int st = combine_check(y, dtype, route_slot, top_idx, T, K, D, out, out_dtype)) return st;
  QW_REQUIRE(T == 0 || top_w, "the static combine needs the route weights");
  if (T == 0) return QW_OK;
  return combine_k<true, true>(y, dtype, route_slot, top_idx, top_w, T, K, D, out, out_dtype, stream);
}

int combine(const void* y, int dtype, const int32_t* route_slot, const int32_t* top_idx, int64_t T, int64_t K,
            int64_t D, void* out, hipStream_t stream) {
  return combine_weighted(y, dtype, route_slot, top_idx, nullptr, T, K, D, out, dtype, stream);
}

// ---------------------------------------------------------------------------
// Decode-step combine, the last line of the one-token MoE step
// (src/fast_decode.py:177):
//   out[t] = residual[t] + ((y_0 * w_0 + y_1 * w_1) + ...)
// with y_j the expert output row of route j of token t (activation dtype,
// widened to fp32), w_j its renormalised router weight, products and sums
// rounded in fp32 in top-k order, and no rounding to the activation dtype.
// Routes without a slot (route_slot < 0) add nothing.  One block per token;
// `out` may be `residual` (each element is read, then written, by one thread).
// ---------------------------------------------------------------------------
template <int ACT, int VEC, int KMAX>
__global__ __launch_bounds__(256) void decode_combine_kernel(const void* __restrict__ y,
                                                             const int32_t* __restrict__ route_slot,
                                                             const float* __restrict__ top_w, const float* residual,
                                                             int K, int D, float* out) {
  const int t = blockIdx.x;
  const int64_t row = static_cast<int64_t>(t) * D;
  const int64_t first = static_cast<int64_t>(t) * K;
  if constexpr (KMAX > 0) {
    // K <= KMAX: the token's slots and weights are read once, the rows of up
    // to G routes and the residual are requested together, then added in
    // top-k order (a route without a slot reads the row of the token's first
    // slotted route and adds nothing; the empty volatile asm keeps each row's
    // load ahead of the additions instead of sunk into its route's branch)
    int sl[KMAX];
    float wt[KMAX];
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
      sl[j] = j < K ? route_slot[first + j] : -1;
      wt[j] = j < K ? top_w[first + j] : 0.0f;
    }
    int any = -1;
#pragma unroll
    for (int j = KMAX - 1; j >= 0; --j) any = sl[j] >= 0 ? sl[j] : any;
    constexpr int G = KMAX < 4 ? KMAX : 4;
    static_assert(KMAX % G == 0, "whole groups of routes");
    for (int c = threadIdx.x * VEC; c < D; c += blockDim.x * VEC) {
      float rv[VEC];
      if (residual != nullptr) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) rv[v] = residual[row + c + v];
      }
      float acc[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[v] = 0.0f;
#pragma unroll
      for (int j0 = 0; j0 < KMAX; j0 += G) {
        if (j0 >= K || any < 0) break;
        float yv[G][VEC];
#pragma unroll
        for (int g = 0; g < G; ++g)
          load_vec<ACT, VEC>(y, static_cast<int64_t>(sl[j0 + g] >= 0 ? sl[j0 + g] : any) * D + c, yv[g]);
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int v = 0; v < VEC; ++v) asm volatile("" : "+v"(yv[g][v]));
#pragma unroll
        for (int g = 0; g < G; ++g) {
          if (sl[j0 + g] < 0) continue;
#pragma unroll
          for (int v = 0; v < VEC; ++v) acc[v] = __fadd_rn(acc[v], __fmul_rn(yv[g][v], wt[j0 + g]));
        }
      }
      if (residual != nullptr) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[v] = __fadd_rn(rv[v], acc[v]);
      }
#pragma unroll
      for (int v = 0; v < VEC; ++v) out[row + c + v] = acc[v];
    }
  } else {
    for (int c = threadIdx.x * VEC; c < D; c += blockDim.x * VEC) {
      float acc[VEC];
#pragma unroll
      for (int v = 0; v < VEC; ++v) acc[v] = 0.0f;
      for (int j = 0; j < K; ++j) {
        const int s = route_slot[first + j];
        if (s < 0) continue;
        const float w = top_w[first + j];
        float yv[VEC];
        load_vec<ACT, VEC>(y, static_cast<int64_t>(s) * D + c, yv);
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[v] = __fadd_rn(acc[v], __fmul_rn(yv[v], w));
      }
      if (residual != nullptr) {
#pragma unroll
        for (int v = 0; v < VEC; ++v) acc[v] = __fadd_rn(residual[row + c + v], acc[v]);
      }
#pragma unroll
      for (int v = 0; v < VEC; ++v) out[row + c + v] = acc[v];
    }
  }
}

template <int ACT, int VEC>
void launch_decode_combine(const void* y, const int32_t* route_slot, const float* top_w, const float* residual,
                           unsigned g, int k, int d, float* out, hipStream_t stream) {
  if (k <= 2)
    decode_combine_kernel<ACT, VEC, 2><<<g, 256, 0, stream>>>(y, route_slot, top_w, residual, k, d, out);
  else if (k <= 4)
    decode_combine_kernel<ACT, VEC, 4><<<g, 256, 0, stream>>>(y, route_slot, top_w, residual, k, d, out);
  else if (k <= 8)
    decode_combine_kernel<ACT, VEC, 8><<<g, 256, 0, stream>>>(y, route_slot, top_w, residual, k, d, out);
  else
    decode_combine_kernel<ACT, VEC, 0><<<g, 256, 0, stream>>>(y, route_slot, top_w, residual, k, d, out);
}

int decode_combine(const void* y, int dtype, const int32_t* route_slot, const float* top_w, const float* residual,
                   int64_t T, int64_t K, int64_t D, float* out, hipStream_t stream) {
  QW_REQUIRE(dtype == QW_F32 || dtype == QW_BF16 || dtype == QW_F16, "decode combine dtype must be f32, bf16 or f16");
  QW_REQUIRE(T >= 0 && T <= INT32_MAX && K >= 1 && D >= 1 && D <= INT32_MAX, "bad decode combine sizes");
  if (T == 0) return QW_OK;
  QW_REQUIRE(y && route_slot && top_w && out, "decode combine pointers are required");
  const unsigned g = static_cast<unsigned>(T);
  const int k = static_cast<int>(K), d = static_cast<int>(D);
  if (dtype == QW_F16 && d % 8 == 0)
    launch_decode_combine<QW_F16, 8>(y, route_slot, top_w, residual, g, k, d, out, stream);
  else if (dtype == QW_F16)
    launch_decode_combine<QW_F16, 1>(y, route_slot, top_w, residual, g, k, d, out, stream);
  else if (dtype == QW_BF16 && d % 8 == 0)
    launch_decode_combine<QW_BF16, 8>(y, route_slot, top_w, residual, g, k, d, out, stream);
  else if (dtype == QW_BF16)
    launch_decode_combine<QW_BF16, 1>(y, route_slot, top_w, residual, g, k, d, out, stream);
  else if (d % 4 == 0)
    launch_decode_combine<QW_F32, 4>(y, route_slot, top_w, residual, g, k, d, out, stream);
  else
    launch_decode_combine<QW_F32, 1>(y, route_slot, top_w, residual, g, k, d, out, stream);
  QW_LAUNCH_CHECK("decode_combine_kernel");
  return QW_OK;
}

// fp32 -> bf16 or fp16, round to nearest even (`normed.to(dtype)`,
// src/fast_decode.py:174).  Four elements per thread when n % 4 == 0.
template <int DT>
__global__ __launch_bounds__(256) void cast_half_kernel(const float* __restrict__ x, int64_t n,
                                                        uint16_t* __restrict__ out) {
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
  if (i >= n) return;
  if ((n & 3) == 0) {
    const float4 v = *reinterpret_cast<const float4*>(x + i);
    uint2 o;
    o.x = pack_half2<DT>(v.x, v.y);
    o.y = pack_half2<DT>(v.z, v.w);
    *reinterpret_cast<uint2*>(out + i) = o;
  } else {
    for (int64_t j = i; j < i + 4 && j < n; ++j) out[j] = f32_to_half<DT>(x[j]);
  }
}

int cast_half(const float* x, int64_t n, uint16_t* out, int dtype, hipStream_t stream) {
  QW_REQUIRE(n >= 0, "bad cast size");
  QW_REQUIRE(is_half(dtype), "the cast is to bf16 or f16");
  if (n == 0) return QW_OK;
  QW_REQUIRE(x && out, "cast pointers are required");
  const unsigned g = static_cast<unsigned>(ceil_div(ceil_div(n, 4), 256));
  if (dtype == QW_F16) cast_half_kernel<QW_F16><<<g, 256, 0, stream>>>(x, n, out);
  else cast_half_kernel<QW_BF16><<<g, 256, 0, stream>>>(x, n, out);
  QW_LAUNCH_CHECK("cast_half_kernel");
  return QW_OK;
}

// ---------------------------------------------------------------------------
// QW_BF16T packing: one thread per 16-byte piece of the tiled output, which is
// written in order (the reads are 16-byte pieces of the plain rows).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void pack_bf16_tiles_kernel(const uint16_t* __restrict__ w, int64_t pieces,
                                                              int64_t rows, int64_t cols,
                                                              uint16_t* __restrict__ out) {
  const int64_t o = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (o >= pieces) return;
  const int64_t per_expert = rows * cols / 8;
  const int64_t e = o / per_expert, rem = o % per_expert;
  const int64_t tile = rem / 64, i = rem % 64;
  const int64_t kt = cols / 64;
  const int64_t rb = tile / kt, kb = tile % kt;
  const int64_t row = 8 * rb + i / 8;
  const int64_t p = (i % 8) ^ ((row >> 1) & 7);
  const uint4 v = *reinterpret_cast<const uint4*>(w + e * rows * cols + row * cols + kb * 64 + p * 8);
  *reinterpret_cast<uint4*>(out + o * 8) = v;
}

int pack_bf16_tiles(const void* w, int64_t E, int64_t rows, int64_t cols, void* out, hipStream_t stream) {
  QW_REQUIRE(E >= 1 && rows >= 1 && cols >= 1, "bad tile packing sizes");
  QW_REQUIRE(rows % 8 == 0 && cols % 64 == 0,
             "tiled bf16 weights need out_features %% 8 == 0 and in_features %% 64 == 0 (got %lld, %lld)",
             (long long)rows, (long long)cols);
  QW_REQUIRE(w && out, "packing pointers are required");
  QW_REQUIRE(w != out, "packing cannot run in place");
  QW_REQUIRE((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(out)) % 16 == 0,
             "packing needs 16-byte aligned buffers");
  const int64_t pieces = E * rows * cols / 8;
  pack_bf16_tiles_kernel<<<static_cast<unsigned>(ceil_div(pieces, 256)), 256, 0, stream>>>(
      static_cast<const uint16_t*>(w), pieces, rows, cols, static_cast<uint16_t*>(out));
  QW_LAUNCH_CHECK("pack_bf16_tiles_kernel");
  return QW_OK;
}

// ---------------------------------------------------------------------------
// Balance loss (src/quantweave_moe_model.py:152-154).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void importance_kernel(const float* __restrict__ probs, int T, int E,
                                                         float* __restrict__ importance) {
  __shared__ float red[256];
  const int e = blockIdx.x;
  float s = 0.0f;
  for (int t = threadIdx.x; t < T; t += 256) s += probs[static_cast<int64_t>(t) * E + e];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int o = 128; o >= 1; o >>= 1) {
    if (threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) importance[e] = red[0] / static_cast<float>(T);
}

__global__ void balance_kernel(const float* __restrict__ importance, const int32_t* __restrict__ counts, int T, int K,
                               int E, float* __restrict__ balance) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  const float routes = static_cast<float>(static_cast<int64_t>(T) * K);
  float s = 0.0f;
  for (int e = 0; e < E; ++e) s += importance[e] * (static_cast<float>(counts[e]) / routes);
  *balance = static_cast<float>(E) * s;
}

// The same with per-workgroup partial sums (coalesced row reads over token
// chunks) summed afterwards in a fixed order: deterministic, and the probs
// matrix is read by many CUs instead of one workgroup per strided column.
constexpr int kImpRows = 64;  // tokens per partial-sum workgroup

__global__ __launch_bounds__(256) void importance_partial_kernel(const float* __restrict__ probs, int T, int E,
                                                                 float* __restrict__ partial) {
  __shared__ float red[4][64];
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  const int e = blockIdx.y * 64 + lane;
  const int t0 = blockIdx.x * kImpRows, t1 = min(T, t0 + kImpRows);
  // all of the thread's loads in flight at once, then added in token order
  // (a token past the end adds +0, which leaves the non-negative sum as it is)
  float v[kImpRows / 4];
#pragma unroll
  for (int i = 0; i < kImpRows / 4; ++i) {
    const int t = t0 + wave + 4 * i;
    v[i] = (e < E && t < t1) ? probs[static_cast<int64_t>(t) * E + e] : 0.0f;
  }
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < kImpRows / 4; ++i) s += v[i];
  red[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && e < E)
    partial[static_cast<int64_t>(blockIdx.x) * E + e] = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
}

// One workgroup of 16 waves; lane l holds expert e0 + l of each 64-expert
// block.  Wave w adds the partial rows w, w + 16, ... in order (whole rows:
// coalesced loads, all of a wave's rows in flight together), the 16 wave sums
// are added in wave order, so importance[e] = sum / T does not depend on
// scheduling.  The balance term is then summed over experts in ascending order
// by one thread.
__global__ __launch_bounds__(1024) void importance_final_kernel(const float* __restrict__ partial, int nb, int T,
                                                                int K, int E, const int32_t* __restrict__ counts,
                                                                float* __restrict__ importance,
                                                                float* __restrict__ balance) {
  constexpr int kW = 16, kRowsPerLoad = 8;
  __shared__ float term[1024];
  __shared__ float red[kW][kWave];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const float routes = static_cast<float>(static_cast<int64_t>(T) * K);
  for (int e0 = 0; e0 < E; e0 += kWave) {
    const int e = e0 + lane;
    float s = 0.0f;
    for (int b0 = wave; b0 < nb; b0 += kW * kRowsPerLoad) {
      float v[kRowsPerLoad];
#pragma unroll
      for (int i = 0; i < kRowsPerLoad; ++i) {
        const int b = b0 + kW * i;
        v[i] = (b < nb && e < E) ? partial[static_cast<int64_t>(b) * E + e] : 0.0f;
      }
#pragma unroll
      for (int i = 0; i < kRowsPerLoad; ++i) s += v[i];  // rows in order; +0 past the end (sums are >= 0)
    }
    red[wave][lane] = s;
    __syncthreads();
    if (wave == 0 && e < E) {
      float t = 0.0f;
#pragma unroll
      for (int w = 0; w < kW; ++w) t += red[w][lane];
      const float imp = t / static_cast<float>(T);
      importance[e] = imp;
      term[e] = imp * (static_cast<float>(counts[e]) / routes);
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    // ascending order; 16 reads in flight at a time (the terms are >= 0, so
    // the +0 past E changes nothing)
    float s = 0.0f;
    for (int e0 = 0; e0 < E; e0 += 16) {
      float v[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) v[i] = e0 + i < E ? term[e0 + i] : 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) s += v[i];
    }
    *balance = static_cast<float>(E) * s;
  }
}

size_t balance_workspace_bytes(int64_t T, int64_t E) {
  return static_cast<size_t>(ceil_div(T, kImpRows)) * static_cast<size_t>(E) * sizeof(float) + 256;
}

int balance_ws(const float* probs, const int32_t* counts, int64_t T, int64_t K, int64_t E, float* importance,
               float* bal, void* ws, size_t ws_bytes, hipStream_t stream) {
  QW_REQUIRE(T >= 1 && T <= INT32_MAX && E >= 1 && E <= 1024 && K >= 1, "bad balance sizes");
  QW_REQUIRE(probs && counts && bal && importance, "balance pointers are required");
  const size_t need = balance_workspace_bytes(T, E);
  if (!ws || ws_bytes < need)
    return set_error(QW_ERR_WORKSPACE, "balance workspace needs %zu bytes, got %zu", need, ws_bytes);
  const int nb = static_cast<int>(ceil_div(T, kImpRows));
  float* partial = static_cast<float*>(ws);
  const dim3 g(static_cast<unsigned>(nb), static_cast<unsigned>(ceil_div(E, 64)));
  importance_partial_kernel<<<g, 256, 0, stream>>>(probs, static_cast<int>(T), static_cast<int>(E), partial);
  QW_LAUNCH_CHECK("importance_partial_kernel");
  importance_final_kernel<<<1, 1024, 0, stream>>>(partial, nb, static_cast<int>(T), static_cast<int>(K),
                                                   static_cast<int>(E), counts, importance, bal);
  QW_LAUNCH_CHECK("importance_final_kernel");
  return QW_OK;
}

int balance(const float* probs, const int32_t* counts, int64_t T, int64_t K, int64_t E, float* importance,
            float* bal, hipStream_t stream, float* scratch_importance) {
  QW_REQUIRE(T >= 1 && T <= INT32_MAX && E >= 1 && E <= 1024 && K >= 1, "bad balance sizes");
  QW_REQUIRE(probs && counts && bal, "balance pointers are required");
  float* imp = importance ? importance : scratch_importance;
  QW_REQUIRE(imp != nullptr, "balance needs an importance buffer");
  importance_kernel<<<static_cast<unsigned>(E), 256, 0, stream>>>(probs, static_cast<int>(T), static_cast<int>(E), imp);
  QW_LAUNCH_CHECK("importance_kernel");
  balance_kernel<<<1, 64, 0, stream>>>(imp, counts, static_cast<int>(T), static_cast<int>(K), static_cast<int>(E), bal);
  QW_LAUNCH_CHECK("balance_kernel");
  return QW_OK;
}

// ---------------------------------------------------------------------------
// Quantisation, QuantizedLinear.from_linear (src/quantization.py:43-59).
// One thread per (row, group).
// ---------------------------------------------------------------------------
template <int WDT, int BITS>
__global__ void quantize_kernel(const void* __restrict__ w, int64_t rows, int64_t cols, int64_t group,
                                int64_t groups, void* __restrict__ qweight, float* __restrict__ scales) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= rows * groups) return;
  const int64_t row = i / groups, g = i % groups;
  const int64_t c0 = g * group;
  const float limit = BITS == 8 ? 127.0f : 7.0f;
  const float lo = BITS == 8 ? -127.0f : -8.0f;
  float amax = 0.0f;
  for (int64_t c = c0; c < c0 + group; ++c) {
    const float v = c < cols ? load_act<WDT>(w, row * cols + c) : 0.0f;
    amax = fmaxf(amax, fabsf(v));
  }
  const float s = fmaxf(amax / limit, 1e-8f);
  scales[row * groups + g] = s;
  if (BITS == 8) {
    int8_t* q = static_cast<int8_t*>(qweight) + row * groups * group;
    for (int64_t c = c0; c < c0 + group; ++c) {
      const float v = c < cols ? load_act<WDT>(w, row * cols + c) : 0.0f;
      const float r = fminf(fmaxf(__builtin_rintf(v / s), lo), limit);
      q[c] = static_cast<int8_t>(r);
    }
  } else {
    uint8_t* q = static_cast<uint8_t*>(qweight) + row * (groups * group / 2);
    for (int64_t c = c0; c < c0 + group; c += 2) {
      const float v0 = c < cols ? load_act<WDT>(w, row * cols + c) : 0.0f;
      const float v1 = c + 1 < cols ? load_act<WDT>(w, row * cols + c + 1) : 0.0f;
      const int q0 = static_cast<int>(fminf(fmaxf(__builtin_rintf(v0 / s), lo), limit)) + 8;
      const int q1 = static_cast<int>(fminf(fmaxf(__builtin_rintf(v1 / s), lo), limit)) + 8;
      q[c / 2] = static_cast<uint8_t>(q0 | (q1 << 4));
    }
  }
}

int quantize(const void* w, int wdt, int64_t rows, int64_t cols, int bits, int64_t group, void* qweight, float* scales,
             hipStream_t stream) {
  QW_REQUIRE(bits == 4 || bits == 8, "bits must be 4 or 8");
  QW_REQUIRE(wdt == QW_F32 || wdt == QW_BF16 || wdt == QW_F16, "weight dtype must be f32, bf16 or f16");
  QW_REQUIRE(group >= 1, "group_size must be positive");
  QW_REQUIRE(!(bits == 4 && (group % 2)), "group_size must be even for 4-bit weights");
  QW_REQUIRE(rows >= 0 && cols >= 1, "bad quantize sizes");
  if (rows == 0) return QW_OK;
  QW_REQUIRE(w && qweight && scales, "quantize pointers are required");
  const int64_t groups = ceil_div(cols, group);
  const int64_t n = rows * groups;
  const unsigned g = static_cast<unsigned>(ceil_div(n, 256));
  if (wdt == QW_F32 && bits == 8) quantize_kernel<QW_F32, 8><<<g, 256, 0, stream>>>(w, rows, cols, group, groups, qweight, scales);
  else if (wdt == QW_F32) quantize_kernel<QW_F32, 4><<<g, 256, 0, stream>>>(w, rows, cols, group, groups, qweight, scales);
  else if (wdt == QW_F16 && bits == 8) quantize_kernel<QW_F16, 8><<<g, 256, 0, stream>>>(w, rows, cols, group, groups, qweight, scales);
  else if (wdt == QW_F16) quantize_kernel<QW_F16, 4><<<g, 256, 0, stream>>>(w, rows, cols, group, groups, qweight, scales);
  else if (bits == 8) quantize_kernel<QW_BF16, 8><<<g, 256, 0, stream>>>(w, rows, cols, group, groups, qweight, scales);
  else quantize_kernel<QW_BF16, 4><<<g, 256, 0, stream>>>(w, rows, cols, group, groups, qweight, scales);
  QW_LAUNCH_CHECK("quantize_kernel");
  return QW_OK;
}

template <int WF>
__global__ void dequantize_kernel(WView v, float* __restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= v.rows * v.cols) return;
  const int64_t row = i / v.cols, col = i % v.cols;
  out[i] = load_weight<WF>(v, 0, row, col);
}

int dequantize(const void* qweight, const float* scales, int bits, int64_t rows, int64_t cols, int64_t group,
               float* out, hipStream_t stream) {
  QW_REQUIRE(bits == 4 || bits == 8, "bits must be 4 or 8");
  QW_REQUIRE(group >= 1 && !(bits == 4 && (group % 2)), "bad group_size");
  QW_REQUIRE(rows >= 0 && cols >= 1, "bad dequantize sizes");
  if (rows == 0) return QW_OK;
  QW_REQUIRE(qweight && scales && out, "dequantize pointers are required");
  const WView v = make_wview(bits == 8 ? QW_I8 : QW_U4, qweight, scales, rows, cols, group);
  const unsigned g = static_cast<unsigned>(ceil_div(rows * cols, 256));
  if (bits == 8) dequantize_kernel<QW_I8><<<g, 256, 0, stream>>>(v, out);
  else dequantize_kernel<QW_U4><<<g, 256, 0, stream>>>(v, out);
  QW_LAUNCH_CHECK("dequantize_kernel");
  return QW_OK;
}

}  // namespace qw
