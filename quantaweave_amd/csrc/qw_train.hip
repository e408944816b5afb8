// Elementwise and per-token pieces of the MoE layer's backward pass.
//
// Reference: the autograd graph of TopKMoE.forward (src/quantweave_moe_model.py:
// 113-164) around the grouped expert kernels:
//   * swiglu / swiglu_backward: `F.silu(gate) * up` of grouped_swiglu
//     (src/moe_kernels.py:194) and its derivative;
//   * combine_backward: `expert_output * weights[:, None]` scattered with
//     index_add_ (src/quantweave_moe_model.py:201-202), differentiated with
//     respect to the expert rows and the router weights;
//   * route_backward: the router weights' chain top-k gather -> renormalise
//     (:128-135), the load-balance loss (:152-154) and the softmax over
//     logits / temperature (:126-127), down to d(x . W_router^T).
// bf16 tensors follow torch's bf16 arithmetic: every torch op rounds its
// result to bf16, so the kernels round where the reference's ops do.
#include "qw_common.h"

namespace qw {

namespace {

__device__ __forceinline__ float sigmoid_f32(float g) { return 1.0f / (1.0f + __expf(-g)); }

// h = silu(g) * u; bf16: silu rounded, then the product rounded.
template <int DT, int VEC>
__global__ __launch_bounds__(256) void swiglu_kernel(const void* __restrict__ g, const void* __restrict__ u, int64_t n,
                                                     void* __restrict__ h) {
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * VEC;
  if (i >= n) return;
  float gv[VEC], uv[VEC], hv[VEC];
  load_vec<DT, VEC>(g, i, gv);
  load_vec<DT, VEC>(u, i, uv);
#pragma unroll
  for (int v = 0; v < VEC; ++v) hv[v] = round_act<DT>(gv[v] * sigmoid_f32(gv[v])) * uv[v];
  store_vec<DT, VEC>(h, i, hv);
}

// d_u = dh * silu(g); d_g = (dh * u) * sigmoid(g) * (1 + g * (1 - sigmoid(g)))
// (torch's silu_backward), each product rounded where torch rounds it.
template <int DT, int VEC>
__global__ __launch_bounds__(256) void swiglu_backward_kernel(const void* __restrict__ dh, const void* __restrict__ g,
                                                              const void* __restrict__ u, int64_t n,
                                                              void* __restrict__ dg, void* __restrict__ du) {
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * VEC;
  if (i >= n) return;
  float dhv[VEC], gv[VEC], uv[VEC], dgv[VEC], duv[VEC];
  load_vec<DT, VEC>(dh, i, dhv);
  load_vec<DT, VEC>(g, i, gv);
  load_vec<DT, VEC>(u, i, uv);
#pragma unroll
  for (int v = 0; v < VEC; ++v) {
    const float sg = sigmoid_f32(gv[v]);
    const float s = round_act<DT>(gv[v] * sg);
    duv[v] = dhv[v] * s;
    const float ds = round_act<DT>(dhv[v] * uv[v]);
    dgv[v] = ds * (sg * (1.0f + gv[v] * (1.0f - sg)));
  }
  store_vec<DT, VEC>(dg, i, dgv);
  store_vec<DT, VEC>(du, i, duv);
}

// One block per token.  For every kept route j of token t (slot s):
//   grad_y[s]     = (grad_out[t] * w_j) in y's dtype
//   grad_top_w[j] = sum_c grad_out[t, c] * y[s, c]   (fp32, fixed order)
// Dropped routes get grad_top_w = 0 and no row.
template <int OUT, int ACT, int VEC>
__global__ __launch_bounds__(256) void combine_backward_kernel(const void* __restrict__ grad_out,
                                                               const void* __restrict__ y,
                                                               const int32_t* __restrict__ route_slot,
                                                               const float* __restrict__ top_w, int K, int D,
                                                               void* __restrict__ grad_y,
                                                               float* __restrict__ grad_top_w) {
  __shared__ float red[4];
  const int t = blockIdx.x;
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  const int64_t row = static_cast<int64_t>(t) * D;
  for (int j = 0; j < K; ++j) {
    const int64_t r = static_cast<int64_t>(t) * K + j;
    const int s = route_slot[r];
    if (s < 0) {
      if (tid == 0) grad_top_w[r] = 0.0f;
      continue;
    }
    const float w = top_w[r];
    const int64_t srow = static_cast<int64_t>(s) * D;
    float dot = 0.0f;
    for (int c = tid * VEC; c < D; c += 256 * VEC) {
      float gv[VEC], yv[VEC], dy[VEC];
      load_vec<OUT, VEC>(grad_out, row + c, gv);
      load_vec<ACT, VEC>(y, srow + c, yv);
#pragma unroll
      for (int v = 0; v < VEC; ++v) {
        dy[v] = gv[v] * w;
        dot = __builtin_fmaf(gv[v], yv[v], dot);
      }
      store_vec<ACT, VEC>(grad_y, srow + c, dy);
    }
    dot = wave_sum_f(dot);
    if (lane == 0) red[wave] = dot;
    __syncthreads();
    if (tid == 0) grad_top_w[r] = ((red[0] + red[1]) + red[2]) + red[3];
    __syncthreads();
  }
}

// One wave per token (4 per block).  With p = probs[t], idx/w = the token's
// top-k experts and renormalised weights, g = grad_top_w[t]:
//   S      = sum_j p[idx_j]
//   dp_j   = (g_j - sum_k g_k w_k) / S                      (w_j = p[idx_j] / S)
//   dP[e]  = grad_probs[t, e] + grad_balance * E * counts[e] / (T * K * T) + sum_{idx_j = e} dp_j
//   out[e] = p[e] * (dP[e] - sum_e' dP[e'] p[e']) / temperature
// dP is staged in `out` by the lane that later overwrites it.
__global__ __launch_bounds__(256) void route_backward_kernel(const float* __restrict__ probs,
                                                             const int32_t* __restrict__ top_idx,
                                                             const float* __restrict__ top_w,
                                                             const float* __restrict__ grad_top_w,
                                                             const float* __restrict__ grad_probs,
                                                             const float* __restrict__ grad_balance,
                                                             const int32_t* __restrict__ counts, int T, int E, int K,
                                                             float temperature, float* __restrict__ out) {
  const int lane = threadIdx.x % kWave;
  const int t = blockIdx.x * 4 + threadIdx.x / kWave;
  if (t >= T) return;
  const int64_t prow = static_cast<int64_t>(t) * E, krow = static_cast<int64_t>(t) * K;
  int idx = 0;
  float pj = 0.0f, gj = 0.0f, wj = 0.0f;
  if (lane < K) {
    idx = top_idx[krow + lane];
    pj = probs[prow + idx];
    gj = grad_top_w[krow + lane];
    wj = top_w[krow + lane];
  }
  const float S = wave_sum_f(pj);
  const float A = wave_sum_f(gj * wj);
  const float dpj = (gj - A) / S;
  const float bal = grad_balance ? grad_balance[0] * static_cast<float>(E) /
                                       (static_cast<float>(T) * static_cast<float>(K) * static_cast<float>(T))
                                 : 0.0f;
  float dot = 0.0f;
  for (int e0 = 0; e0 < E; e0 += kWave) {
    const int e = e0 + lane;
    float dP = 0.0f;
    for (int j = 0; j < K; ++j) {
      const int ij = __shfl(idx, j, kWave);
      const float dj = __shfl(dpj, j, kWave);
      if (ij == e) dP += dj;
    }
    if (e < E) {
      if (grad_probs) dP += grad_probs[prow + e];
      if (grad_balance) dP += bal * static_cast<float>(counts[e]);
      out[prow + e] = dP;
      dot = __builtin_fmaf(dP, probs[prow + e], dot);
    }
  }
  dot = wave_sum_f(dot);
  for (int e = lane; e < E; e += kWave) {
    const float p = probs[prow + e];
    out[prow + e] = p * (out[prow + e] - dot) / temperature;
  }
}

template <int DT>
void launch_swiglu(const void* g, const void* u, int64_t n, void* h, void* dh, void* dg, void* du, bool backward,
                   hipStream_t stream) {
  const bool v8 = n % 8 == 0;
  const int64_t per = v8 ? 8 : 1;
  const unsigned blocks = static_cast<unsigned>(ceil_div(ceil_div(n, per), 256));
  if (backward) {
    if (v8) swiglu_backward_kernel<DT, 8><<<blocks, 256, 0, stream>>>(dh, g, u, n, dg, du);
    else swiglu_backward_kernel<DT, 1><<<blocks, 256, 0, stream>>>(dh, g, u, n, dg, du);
  } else {
    if (v8) swiglu_kernel<DT, 8><<<blocks, 256, 0, stream>>>(g, u, n, h);
    else swiglu_kernel<DT, 1><<<blocks, 256, 0, stream>>>(g, u, n, h);
  }
}

template <int OUT, int ACT>
void launch_combine_backward(const void* grad_out, const void* y, const int32_t* route_slot, const float* top_w,
                             int T, int K, int D, void* grad_y, float* grad_top_w, hipStream_t stream) {
  if (D % 8 == 0)
    combine_backward_kernel<OUT, ACT, 8><<<T, 256, 0, stream>>>(grad_out, y, route_slot, top_w, K, D, grad_y,
                                                                grad_top_w);
  else
    combine_backward_kernel<OUT, ACT, 1><<<T, 256, 0, stream>>>(grad_out, y, route_slot, top_w, K, D, grad_y,
                                                                grad_top_w);
}

}  // namespace

int swiglu(const void* g, const void* u, int dtype, int64_t n, void* h, hipStream_t stream) {
  QW_REQUIRE(dtype == QW_F32 || dtype == QW_BF16 || dtype == QW_F16, "swiglu dtype must be f32, bf16 or f16");
  QW_REQUIRE(n >= 0, "bad swiglu size");
  if (n == 0) return QW_OK;
  QW_REQUIRE(g && u && h, "swiglu pointers are required");
  QW_REQUIRE(ceil_div(n, 256) <= INT32_MAX, "swiglu size out of range");
  if (dtype == QW_F32) launch_swiglu<QW_F32>(g, u, n, h, nullptr, nullptr, nullptr, false, stream);
  else if (dtype == QW_F16) launch_swiglu<QW_F16>(g, u, n, h, nullptr, nullptr, nullptr, false, stream);
  else launch_swiglu<QW_BF16>(g, u, n, h, nullptr, nullptr, nullptr, false, stream);
  QW_LAUNCH_CHECK("swiglu_kernel");
  return QW_OK;
}

int swiglu_backward(const void* dh, const void* g, const void* u, int dtype, int64_t n, void* dg, void* du,
                    hipStream_t stream) {
  QW_REQUIRE(dtype == QW_F32 || dtype == QW_BF16 || dtype == QW_F16, "swiglu dtype must be f32, bf16 or f16");
  QW_REQUIRE(n >= 0, "bad swiglu size");
  if (n == 0) return QW_OK;
  QW_REQUIRE(dh && g && u && dg && du, "swiglu backward pointers are required");
  QW_REQUIRE(ceil_div(n, 256) <= INT32_MAX, "swiglu size out of range");
  if (dtype == QW_F32) launch_swiglu<QW_F32>(g, u, n, nullptr, const_cast<void*>(dh), dg, du, true, stream);
  else if (dtype == QW_F16) launch_swiglu<QW_F16>(g, u, n, nullptr, const_cast<void*>(dh), dg, du, true, stream);
  else launch_swiglu<QW_BF16>(g, u, n, nullptr, const_cast<void*>(dh), dg, du, true, stream);
  QW_LAUNCH_CHECK("swiglu_backward_kernel");
  return QW_OK;
}

int combine_backward(const void* grad_out, int out_dtype, const void* y, int y_dtype, const int32_t* route_slot,
                     const float* top_w, int64_t T, int64_t K, int64_t D, void* grad_y, float* grad_top_w,
                     hipStream_t stream) {
  QW_REQUIRE((out_dtype == QW_F32 || out_dtype == QW_BF16 || out_dtype == QW_F16) &&
                 (y_dtype == QW_F32 || y_dtype == QW_BF16 || y_dtype == QW_F16) &&
                 !(is_half(out_dtype) && is_half(y_dtype) && out_dtype != y_dtype),
             "combine backward dtypes must be f32, bf16 or f16 (bf16 and f16 not mixed)");
  QW_REQUIRE(T >= 0 && T <= INT32_MAX && K >= 1 && K <= 64 && D >= 1 && D <= INT32_MAX,
             "bad combine backward sizes");
  if (T == 0) return QW_OK;
  QW_REQUIRE(grad_out && y && route_slot && top_w && grad_y && grad_top_w, "combine backward pointers are required");
  const int t = static_cast<int>(T), k = static_cast<int>(K), d = static_cast<int>(D);
  if (out_dtype == QW_F16 && y_dtype == QW_F16)
    launch_combine_backward<QW_F16, QW_F16>(grad_out, y, route_slot, top_w, t, k, d, grad_y, grad_top_w, stream);
  else if (out_dtype == QW_F32 && y_dtype == QW_F16)
    launch_combine_backward<QW_F32, QW_F16>(grad_out, y, route_slot, top_w, t, k, d, grad_y, grad_top_w, stream);
  else if (out_dtype == QW_F16 && y_dtype == QW_F32)
    launch_combine_backward<QW_F16, QW_F32>(grad_out, y, route_slot, top_w, t, k, d, grad_y, grad_top_w, stream);
  else if (out_dtype == QW_F32 && y_dtype == QW_F32)
    launch_combine_backward<QW_F32, QW_F32>(grad_out, y, route_slot, top_w, t, k, d, grad_y, grad_top_w, stream);
  else if (out_dtype == QW_F32)
    launch_combine_backward<QW_F32, QW_BF16>(grad_out, y, route_slot, top_w, t, k, d, grad_y, grad_top_w, stream);
  else if (y_dtype == QW_F32)
    launch_combine_backward<QW_BF16, QW_F32>(grad_out, y, route_slot, top_w, t, k, d, grad_y, grad_top_w, stream);
  else
    launch_combine_backward<QW_BF16, QW_BF16>(grad_out, y, route_slot, top_w, t, k, d, grad_y, grad_top_w, stream);
  QW_LAUNCH_CHECK("combine_backward_kernel");
  return QW_OK;
}

int route_backward(const float* probs, const int32_t* top_idx, const float* top_w, const float* grad_top_w,
                   const float* grad_probs, const float* grad_balance, const int32_t* counts, int64_t T, int64_t E,
                   int64_t K, float temperature, float* out, hipStream_t stream) {
  QW_REQUIRE(T >= 0 && T <= INT32_MAX && E >= 1 && E <= INT32_MAX && K >= 1 && K <= 64 && K <= E,
             "bad route backward sizes (top_k must be in [1, min(64, experts)])");
  QW_REQUIRE(temperature > 0.0f, "temperature must be positive");
  if (T == 0) return QW_OK;
  QW_REQUIRE(probs && top_idx && top_w && grad_top_w && out, "route backward pointers are required");
  QW_REQUIRE(!grad_balance || counts, "the balance gradient needs the per-expert route counts");
  const unsigned blocks = static_cast<unsigned>(ceil_div(T, 4));
  route_backward_kernel<<<blocks, 256, 0, stream>>>(probs, top_idx, top_w, grad_top_w, grad_probs, grad_balance,
                                                    counts, static_cast<int>(T), static_cast<int>(E),
                                                    static_cast<int>(K), temperature, out);
  QW_LAUNCH_CHECK("route_backward_kernel");
  return QW_OK;
}

}  // namespace qw
