// Grouped SwiGLU expert FFN — general kernel for every weight format.
//
// Reference: SparseSwiGLU.forward (src/quantweave_moe_model.py:59-60) applied
// per expert over its contiguous block of plan-ordered rows
// (src/quantweave_moe_model.py:203-211, src/moe_kernels.py:186-195), and
// QuantizedLinear.forward (src/quantization.py:71-72) for quantised experts.
//
// This kernel is the exact-semantics path for any (activation dtype, weight
// format, shape): weights are dequantised into LDS (rounded to the activation
// dtype as the reference's `.to(x.dtype)` does) and multiplied with fp32
// accumulation on the vector ALUs.  The MFMA prefill kernel and the decode
// GEMV kernels specialise the shapes that matter for throughput.
//
// Stage 1 (GATEUP): h[s, c] = silu(x_s . G_e[c]) * (x_s . U_e[c])
// Stage 2 (DOWN):   y[s, c] = (h_s . D_e[c]) * row_weight[s]
#include <algorithm>

#include "qw_weights.h"
#include "qw_ffn.h"

namespace qw {

namespace {

constexpr int GB_N = 64;   // weight rows per tile
constexpr int GB_M = 16;   // activation rows per chunk
constexpr int GB_K = 64;   // reduction slice

template <int ACT, int WF, bool GATEUP>
__global__ __launch_bounds__(256) void ffn_generic_kernel(const void* __restrict__ x,
                                                          const int32_t* __restrict__ row_index,
                                                          const int32_t* __restrict__ offsets, WView wa, WView wb,
                                                          int K, int N_out, int max_rows,
                                                          const float* __restrict__ row_weight,
                                                          void* __restrict__ out, void* __restrict__ save_a,
                                                          void* __restrict__ save_b) {
  __shared__ float ws[GB_N][GB_K + 1];
  __shared__ float xs[GB_M][GB_K + 1];
  __shared__ float os[GB_M][GB_N + 1];
  const int e = blockIdx.y;
  // rows of expert e, clamped to the caller's buffers
  const int r0 = max(offsets[e], 0), r1 = min(offsets[e + 1], max_rows);
  if (r1 <= r0) return;
  const int tid = threadIdx.x;
  // GATEUP: tile covers 32 output columns: weight rows 0..31 gate, 32..63 up.
  // DOWN:   tile covers 64 output columns.
  constexpr int COLS = GATEUP ? GB_N / 2 : GB_N;
  const int c0 = blockIdx.x * COLS;
  if (c0 >= N_out) return;
  const int n = tid % GB_N;        // weight row in tile
  const int mg = tid / GB_N;       // 0..3 -> rows mg*4 .. mg*4+3
  // 16-row chunks of the expert, dealt over the grid's z extent
  for (int m0 = r0 + static_cast<int>(blockIdx.z) * GB_M; m0 < r1; m0 += static_cast<int>(gridDim.z) * GB_M) {
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < K; k0 += GB_K) {
      for (int i = tid; i < GB_N * GB_K; i += 256) {
        const int wr = i / GB_K, kk = i % GB_K;
        const int k = k0 + kk;
        float v = 0.0f;
        if (GATEUP) {
          const int c = c0 + (wr % COLS);
          if (c < N_out && k < K) v = load_weight<WF>(wr < COLS ? wa : wb, e, c, k);
        } else {
          const int c = c0 + wr;
          if (c < N_out && k < K) v = load_weight<WF>(wa, e, c, k);
        }
        ws[wr][kk] = round_act<ACT>(v);
      }
      for (int i = tid; i < GB_M * GB_K; i += 256) {
        const int m = i / GB_K, kk = i % GB_K;
        const int s = m0 + m, k = k0 + kk;
        float v = 0.0f;
        if (s < r1 && k < K) {
          const int64_t src = row_index ? row_index[s] : s;
          v = load_act<ACT>(x, src * K + k);
        }
        xs[m][kk] = v;
      }
      __syncthreads();
#pragma unroll 8
      for (int kk = 0; kk < GB_K; ++kk) {
        const float wv = ws[n][kk];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = __builtin_fmaf(wv, xs[mg * 4 + i][kk], acc[i]);
      }
      __syncthreads();
    }
    if (GATEUP) {
#pragma unroll
      for (int i = 0; i < 4; ++i) os[mg * 4 + i][n] = acc[i];
      __syncthreads();
      for (int i = tid; i < GB_M * COLS; i += 256) {
        const int m = i / COLS, c = i % COLS;
        const int s = m0 + m;
        if (s < r1 && c0 + c < N_out) {
          const float g = round_act<ACT>(os[m][c]);
          const float u = round_act<ACT>(os[m][c + COLS]);
          const int64_t o = static_cast<int64_t>(s) * N_out + c0 + c;
          store_act<ACT>(out, o, swiglu_act<ACT>(g, u));
          if (save_a) {  // gate and up projections, for the backward pass
            store_act<ACT>(save_a, o, g);
            store_act<ACT>(save_b, o, u);
          }
        }
      }
      __syncthreads();
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int s = m0 + mg * 4 + i;
        if (s < r1 && c0 + n < N_out) {
          const float wgt = row_weight ? row_weight[s] : 1.0f;
          const int64_t o = static_cast<int64_t>(s) * N_out + c0 + n;
          store_act<ACT>(out, o, round_act<ACT>(acc[i]) * wgt);
          if (save_a) store_act<ACT>(save_a, o, acc[i]);  // the row before its weight
        }
      }
    }
  }
}

// Workgroups per (column tile, expert): one per 16-row chunk of an expert of
// the expected size, at most 32 (each loops over its share of the chunks).
unsigned row_splits(int64_t avg_rows) {
  return static_cast<unsigned>(std::min<int64_t>(std::max<int64_t>(ceil_div(avg_rows, GB_M), 1), 32));
}

template <int ACT, int WF>
int launch_generic_t(const FfnArgs& a, hipStream_t stream) {
  const dim3 blk(256);
  const unsigned z = row_splits(a.avg_rows > 0 ? a.avg_rows : ceil_div(a.max_rows, a.experts));
  const dim3 g1(static_cast<unsigned>(ceil_div(a.d_ff, GB_N / 2)), static_cast<unsigned>(a.experts), z);
  ffn_generic_kernel<ACT, WF, true><<<g1, blk, 0, stream>>>(a.x, a.row_index, a.offsets, a.gate, a.up,
                                                            static_cast<int>(a.d_model), static_cast<int>(a.d_ff),
                                                            static_cast<int>(a.max_rows), nullptr, a.hidden,
                                                            a.save_gate, a.save_up);
  QW_LAUNCH_CHECK("ffn_generic_kernel<gateup>");
  const dim3 g2(static_cast<unsigned>(ceil_div(a.d_model, GB_N)), static_cast<unsigned>(a.experts), z);
  ffn_generic_kernel<ACT, WF, false><<<g2, blk, 0, stream>>>(a.hidden, nullptr, a.offsets, a.down, a.down,
                                                             static_cast<int>(a.d_ff), static_cast<int>(a.d_model),
                                                             static_cast<int>(a.max_rows), a.row_weight, a.y,
                                                             a.save_y, nullptr);
  QW_LAUNCH_CHECK("ffn_generic_kernel<down>");
  return QW_OK;
}

}  // namespace

int launch_ffn_generic(const FfnArgs& a, hipStream_t stream) {
#define QW_GEN(ACT, WF) \
  if (a.act == ACT && a.wfmt == WF) return launch_generic_t<ACT, WF>(a, stream);
  QW_GEN(QW_F32, QW_F32)
  QW_GEN(QW_F32, QW_BF16)
  QW_GEN(QW_F32, QW_I8)
  QW_GEN(QW_F32, QW_U4)
  QW_GEN(QW_BF16, QW_F32)
  QW_GEN(QW_BF16, QW_BF16)
  QW_GEN(QW_BF16, QW_I8)
  QW_GEN(QW_BF16, QW_U4)
  QW_GEN(QW_F32, QW_BF16T)
  QW_GEN(QW_BF16, QW_BF16T)
  QW_GEN(QW_F16, QW_F16)
  QW_GEN(QW_F16, QW_F16T)
  QW_GEN(QW_F16, QW_F32)
  QW_GEN(QW_F16, QW_BF16)
  QW_GEN(QW_F16, QW_I8)
  QW_GEN(QW_F16, QW_U4)
  QW_GEN(QW_F32, QW_F16)
  QW_GEN(QW_F32, QW_F16T)
  QW_GEN(QW_BF16, QW_F16)
#undef QW_GEN
  return set_error(QW_ERR_INVALID, "unsupported activation/weight format pair (%d, %d)", a.act, a.wfmt);
}

int grouped_matmul_generic(const void* x, int act, const WView& w, int wfmt, int64_t E, const int32_t* offsets,
                           int64_t rows, void* out, hipStream_t stream) {
  const dim3 g(static_cast<unsigned>(ceil_div(w.rows, GB_N)), static_cast<unsigned>(E), row_splits(ceil_div(rows, E)));
  const int K = static_cast<int>(w.cols), N = static_cast<int>(w.rows), nrows = static_cast<int>(rows);
#define QW_GM(ACT, WF)                                                                                         \
  if (act == ACT && wfmt == WF) {                                                                              \
    ffn_generic_kernel<ACT, WF, false><<<g, 256, 0, stream>>>(x, nullptr, offsets, w, w, K, N, nrows, nullptr, out, \
                                                              nullptr, nullptr);                                \
    QW_LAUNCH_CHECK("ffn_generic_kernel<matmul>");                                                            \
    return QW_OK;                                                                                              \
  }
  QW_GM(QW_F32, QW_F32)
  QW_GM(QW_F32, QW_BF16)
  QW_GM(QW_F32, QW_I8)
  QW_GM(QW_F32, QW_U4)
  QW_GM(QW_BF16, QW_F32)
  QW_GM(QW_BF16, QW_BF16)
  QW_GM(QW_BF16, QW_I8)
  QW_GM(QW_BF16, QW_U4)
  QW_GM(QW_F32, QW_BF16T)
  QW_GM(QW_BF16, QW_BF16T)
  QW_GM(QW_F16, QW_F16)
  QW_GM(QW_F16, QW_F16T)
  QW_GM(QW_F16, QW_F32)
  QW_GM(QW_F16, QW_BF16)
  QW_GM(QW_F16, QW_I8)
  QW_GM(QW_F16, QW_U4)
  QW_GM(QW_F32, QW_F16)
  QW_GM(QW_F32, QW_F16T)
  QW_GM(QW_BF16, QW_F16)
#undef QW_GM
  return set_error(QW_ERR_INVALID, "unsupported activation/weight format pair (%d, %d)", act, wfmt);
}

}  // namespace qw
