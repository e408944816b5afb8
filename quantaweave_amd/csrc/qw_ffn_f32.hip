// Grouped SwiGLU expert FFN in fp32 on the matrix cores
// (v_mfma_f32_16x16x4_f32, gfx950): fp32 activations with fp32 weights.
//
// Reference: SparseSwiGLU.forward (src/quantweave_moe_model.py:59-60) over
// each expert's block of plan-ordered rows, the fp32 grouped GEMM of
// src/moe_kernels.py:41-64 (`tl.dot` with IEEE fp32 inputs, :114-115) and the
// fp32 default of its benchmark() (:198-227).
//
// A workgroup of 4 waves (2 x 2) owns a tile of 64 rows of one expert by 64
// weight rows: GATEUP 32 gate rows and the matching 32 up rows (32 hidden
// columns, SiLU(g)*u formed in registers), DOWN 64 output columns.  Each wave
// computes 32 rows x 32 weight rows as 2 x 2 MFMA tiles.  Operands go through
// LDS in K slices of 64, double-buffered, with two slices in flight in
// registers: slice s is loaded while slice s-2 is multiplied.
//
// The 16x16x4 instruction takes one fp32 per lane and operand: lane l holds
// row l%16 of its operand and one of 4 reduction indices.  The reduction
// indices may be assigned to (lane group, instruction) pairs in any order, as
// long as both operands agree, so lane group q of the four instructions j of a
// 16-wide K step takes index 4q + j: each lane reads its 4 values of a step
// with one 16-byte LDS read per operand.  The weights are the A operand, so a
// lane ends up holding 4 consecutive output columns of one row.
#include <algorithm>

#include "qw_ffn.h"

namespace qw {

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int F32_THREADS = 256;
constexpr int F32_M = 64;      // rows per tile
constexpr int F32_N = 64;      // weight rows per tile
constexpr int F32_BK = 64;     // K slice
constexpr int F32_LD = F32_BK + 4;  // LDS row stride (floats): padding spreads the 16-byte reads over banks
constexpr int F32_PT = F32_BK / 4 / 8;  // 16-byte pieces per thread, tile row and operand

template <bool GATEUP>
__global__ __launch_bounds__(F32_THREADS) void ffn_f32_mfma_kernel(
    const float* __restrict__ x, const int32_t* __restrict__ row_index, const int32_t* __restrict__ offsets,
    const float* __restrict__ wa, const float* __restrict__ wb, int64_t w_expert_stride, int n_w, int K, int n_out,
    int max_rows, const float* __restrict__ row_weight, float* __restrict__ out, float* __restrict__ save_a,
    float* __restrict__ save_b, const XcdGrid grid) {
  __shared__ __attribute__((aligned(16))) float xs[2][F32_M * F32_LD];
  __shared__ __attribute__((aligned(16))) float ws[2][F32_N * F32_LD];
  int tx, e, tz;
  if (!xcd_tile(grid, blockIdx.x, &tx, &e, &tz)) return;
  const int r0 = max(offsets[e], 0), r1 = min(offsets[e + 1], max_rows);
  if (r1 <= r0) return;
  constexpr int COLS = GATEUP ? F32_N / 2 : F32_N;  // output columns per tile
  const int c0 = tx * COLS;
  if (c0 >= n_out) return;
  const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  const int wm = wave / 2, wn = wave % 2;
  const int l16 = lane % 16, lq = lane / 16;
  const float* wa_e = wa + static_cast<int64_t>(e) * w_expert_stride;
  const float* wb_e = wb + static_cast<int64_t>(e) * w_expert_stride;
  // LDS weight row of tile row n: GATEUP rows 0..31 gate, 32..63 up
  auto w_row = [&](int n) -> const float* {
    int row;
    const float* base;
    if (GATEUP) {
      row = c0 + (n % (F32_N / 2));
      base = n < F32_N / 2 ? wa_e : wb_e;
    } else {
      row = c0 + n;
      base = wa_e;
    }
    return base + static_cast<int64_t>(min(row, n_w - 1)) * K;  // rows past the end: loaded, not stored
  };
  // this thread's 16-byte pieces of each slice: tile rows tid/8 and tid/8 + 32,
  // columns 4*(tid%8) + 32*p .. +3
  const int lr = tid / 8, lc = (tid % 8) * 4;
  const float* wsrc[2] = {w_row(lr), w_row(lr + 32)};

  for (int m0 = r0 + tz * F32_M; m0 < r1; m0 += grid.zs * F32_M) {
    const float* xsrc[2];
    bool xok[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int s = m0 + lr + 32 * h;
      xok[h] = s < r1;
      const int64_t src = row_index ? row_index[min(s, r1 - 1)] : min(s, r1 - 1);
      xsrc[h] = x + src * K;
    }
    // registers of one slice: [row half][piece] for x and for w
    struct Slice {
      f32x4 x[2][F32_PT], w[2][F32_PT];
    };
    auto load = [&](int k0, Slice& r) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int p = 0; p < F32_PT; ++p) {
          const int k = k0 + lc + 32 * p;
          const bool in_k = k + 3 < K;  // K % 4 == 0: a piece is wholly inside K or wholly past it
          r.x[h][p] = (xok[h] && in_k) ? *reinterpret_cast<const f32x4*>(xsrc[h] + k) : f32x4{0.f, 0.f, 0.f, 0.f};
          r.w[h][p] = in_k ? *reinterpret_cast<const f32x4*>(wsrc[h] + k) : f32x4{0.f, 0.f, 0.f, 0.f};
        }
    };
    auto store = [&](int buf, const Slice& r) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int p = 0; p < F32_PT; ++p) {
          *reinterpret_cast<f32x4*>(&xs[buf][(lr + 32 * h) * F32_LD + lc + 32 * p]) = r.x[h][p];
          *reinterpret_cast<f32x4*>(&ws[buf][(lr + 32 * h) * F32_LD + lc + 32 * p]) = r.w[h][p];
        }
    };
    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int t = 0; t < 2; ++t) acc[i][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    // B (activations) row blocks of this wave: rows wm*32 + 16i; A (weights): tile rows
    // GATEUP t = 0 gate wn*16.., t = 1 up 32 + wn*16..; DOWN wn*32 + 16t
    int arow[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) arow[t] = GATEUP ? (t * 32 + wn * 16) : (wn * 32 + t * 16);
    auto compute = [&](int buf) {
#pragma unroll
      for (int kk = 0; kk < F32_BK; kk += 16) {
        f32x4 a[2], b[2];
#pragma unroll
        for (int t = 0; t < 2; ++t)
          a[t] = *reinterpret_cast<const f32x4*>(&ws[buf][(arow[t] + l16) * F32_LD + kk + 4 * lq]);
#pragma unroll
        for (int i = 0; i < 2; ++i)
          b[i] = *reinterpret_cast<const f32x4*>(&xs[buf][(wm * 32 + 16 * i + l16) * F32_LD + kk + 4 * lq]);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int t = 0; t < 2; ++t)
              acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t][j], b[i][j], acc[i][t], 0, 0, 0);
      }
    };

    // Two slices in flight in registers: slice s is loaded two slices before
    // it is multiplied and stored to LDS one slice before (register sets
    // alternate, so the loop is unrolled by two).
    const int KS = (K + F32_BK - 1) / F32_BK;
    Slice ra, rb;
    load(0, ra);
    if (KS > 1) load(F32_BK, rb);
    store(0, ra);
    __syncthreads();
    for (int ks = 0; ks < KS; ks += 2) {
      if (ks + 2 < KS) load((ks + 2) * F32_BK, ra);
      compute(0);
      if (ks + 1 < KS) store(1, rb);
      __syncthreads();
      if (ks + 1 >= KS) break;
      if (ks + 3 < KS) load((ks + 3) * F32_BK, rb);
      compute(1);
      if (ks + 2 < KS) store(0, ra);
      __syncthreads();
    }
    // epilogue: lane holds, for row block i, row l16 and 4 consecutive weight rows 4*lq .. of tile t
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int s = m0 + wm * 32 + 16 * i + l16;
      if (s >= r1) continue;
      const int64_t orow = static_cast<int64_t>(s) * n_out;
      if constexpr (GATEUP) {
        const int col = c0 + wn * 16 + 4 * lq;
        f32x4 h;
#pragma unroll
        for (int v = 0; v < 4; ++v) h[v] = swiglu_act<QW_F32>(acc[i][0][v], acc[i][1][v]);
        if (col + 3 < n_out) {
          *reinterpret_cast<f32x4*>(out + orow + col) = h;
          if (save_a) {
            *reinterpret_cast<f32x4*>(save_a + orow + col) = acc[i][0];
            *reinterpret_cast<f32x4*>(save_b + orow + col) = acc[i][1];
          }
        } else {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            if (col + v >= n_out) continue;
            out[orow + col + v] = h[v];
            if (save_a) {
              save_a[orow + col + v] = acc[i][0][v];
              save_b[orow + col + v] = acc[i][1][v];
            }
          }
        }
      } else {
        const float wgt = row_weight ? row_weight[s] : 1.0f;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int col = c0 + wn * 32 + 16 * t + 4 * lq;
          f32x4 y;
#pragma unroll
          for (int v = 0; v < 4; ++v) y[v] = acc[i][t][v] * wgt;
          if (col + 3 < n_out) {
            *reinterpret_cast<f32x4*>(out + orow + col) = y;
            if (save_a) *reinterpret_cast<f32x4*>(save_a + orow + col) = acc[i][t];
          } else {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              if (col + v >= n_out) continue;
              out[orow + col + v] = y[v];
              if (save_a) save_a[orow + col + v] = acc[i][t][v];
            }
          }
        }
      }
    }
  }
}

// Small problems (too few 64 x 64 tiles to fill the GPU): a workgroup of 4
// waves owns a 32-row by 32-weight-row tile (GATEUP: 16 gate rows and the
// matching 16 up rows) and its waves split K: wave w takes the 32-wide K
// slices w, w + 4, ...  Each wave reads its MFMA operands straight from
// global memory into registers (lane (l16, q) of a 16-wide K step loads the 4
// consecutive values 4q .. 4q+3 of its row, the same index order as the LDS
// kernel above), with the next slice's loads in flight during the current
// slice's MFMAs; there is no LDS ring and no barrier in the K loop.  The four
// partial tiles meet in LDS and are added in wave order ((w0 + w1) + w2) + w3,
// then the epilogue is the one above.
constexpr int F32S_M = 32, F32S_N = 32, F32S_BK = 32, F32S_ST = F32S_BK / 16;

template <bool GATEUP>
__global__ __launch_bounds__(F32_THREADS) void ffn_f32_small_kernel(
    const float* __restrict__ x, const int32_t* __restrict__ row_index, const int32_t* __restrict__ offsets,
    const float* __restrict__ wa, const float* __restrict__ wb, int64_t w_expert_stride, int n_w, int K, int n_out,
    int max_rows, const float* __restrict__ row_weight, float* __restrict__ out, float* __restrict__ save_a,
    float* __restrict__ save_b, const XcdGrid grid) {
  __shared__ __attribute__((aligned(16))) f32x4 red[4][4][64];  // [wave][tile (i, t)][lane]
  int tx, e, tz;
  if (!xcd_tile(grid, blockIdx.x, &tx, &e, &tz)) return;
  const int r0 = max(offsets[e], 0), r1 = min(offsets[e + 1], max_rows);
  if (r1 <= r0) return;
  constexpr int COLS = GATEUP ? F32S_N / 2 : F32S_N;  // output columns per tile
  const int c0 = tx * COLS;
  if (c0 >= n_out) return;
  const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  const int l16 = lane % 16, lq = lane / 16;
  // weight rows of the two 16-row A tiles: GATEUP t = 0 gate, t = 1 up; DOWN t = 0, 1 consecutive
  const float* wsrc[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int row = GATEUP ? c0 + l16 : c0 + 16 * t + l16;
    const float* base = (GATEUP && t == 1 ? wb : wa) + static_cast<int64_t>(e) * w_expert_stride;
    wsrc[t] = base + static_cast<int64_t>(min(row, n_w - 1)) * K + 4 * lq;  // rows past the end: loaded, not stored
  }
  const int KS = (K + F32S_BK - 1) / F32S_BK;
  for (int m0 = r0 + tz * F32S_M; m0 < r1; m0 += grid.zs * F32S_M) {
    const float* xsrc[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int s = min(m0 + 16 * i + l16, r1 - 1);  // rows past the end: a valid row, not stored
      const int64_t src = row_index ? row_index[s] : s;
      xsrc[i] = x + src * K + 4 * lq;
    }
    // one slice: K steps of 16, per step the lane's 4 values of each operand tile
    struct Slice {
      f32x4 a[F32S_ST][2], b[F32S_ST][2];
    };
    auto load = [&](int ks, Slice& r) {
#pragma unroll
      for (int st = 0; st < F32S_ST; ++st) {
        const int k = ks * F32S_BK + 16 * st;  // + 4 * lq inside the sources
        const bool in_k = k + 4 * lq + 3 < K;  // K % 4 == 0: a piece is wholly inside K or wholly past it
#pragma unroll
        for (int t = 0; t < 2; ++t)
          r.a[st][t] = in_k ? *reinterpret_cast<const f32x4*>(wsrc[t] + k) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 2; ++i)
          r.b[st][i] = in_k ? *reinterpret_cast<const f32x4*>(xsrc[i] + k) : f32x4{0.f, 0.f, 0.f, 0.f};
      }
    };
    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int t = 0; t < 2; ++t) acc[i][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](const Slice& r) {
#pragma unroll
      for (int st = 0; st < F32S_ST; ++st)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int t = 0; t < 2; ++t)
              acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(r.a[st][t][j], r.b[st][i][j], acc[i][t], 0, 0, 0);
    };
    // this wave's slices: wave, wave + 4, ... (the next one loaded during the current one's MFMAs)
    Slice ra, rb;
    int ks = wave;
    if (ks < KS) load(ks, ra);
    while (ks < KS) {
      if (ks + 4 < KS) load(ks + 4, rb);
      compute(ra);
      ks += 4;
      if (ks >= KS) break;
      if (ks + 4 < KS) load(ks + 4, ra);
      compute(rb);
      ks += 4;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int t = 0; t < 2; ++t) red[wave][2 * i + t][lane] = acc[i][t];
    __syncthreads();
    // tile (i, t) summed in wave order; GATEUP: wave i < 2 takes row block i (gate and up), DOWN: wave w tile w
    auto total = [&](int tile) {
      return ((red[0][tile][lane] + red[1][tile][lane]) + red[2][tile][lane]) + red[3][tile][lane];
    };
    if (GATEUP ? wave < 2 : true) {
      const int i = GATEUP ? wave : wave / 2;
      const int s = m0 + 16 * i + l16;
      if (s < r1) {
        const int64_t orow = static_cast<int64_t>(s) * n_out;
        if constexpr (GATEUP) {
          const f32x4 g = total(2 * i), u = total(2 * i + 1);
          const int col = c0 + 4 * lq;
          f32x4 h;
#pragma unroll
          for (int v = 0; v < 4; ++v) h[v] = swiglu_act<QW_F32>(g[v], u[v]);
          if (col + 3 < n_out) {
            *reinterpret_cast<f32x4*>(out + orow + col) = h;
            if (save_a) {
              *reinterpret_cast<f32x4*>(save_a + orow + col) = g;
              *reinterpret_cast<f32x4*>(save_b + orow + col) = u;
            }
          } else {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              if (col + v >= n_out) continue;
              out[orow + col + v] = h[v];
              if (save_a) {
                save_a[orow + col + v] = g[v];
                save_b[orow + col + v] = u[v];
              }
            }
          }
        } else {
          const int t = wave % 2;
          const f32x4 a = total(2 * i + t);
          const float wgt = row_weight ? row_weight[s] : 1.0f;
          const int col = c0 + 16 * t + 4 * lq;
          f32x4 y;
#pragma unroll
          for (int v = 0; v < 4; ++v) y[v] = a[v] * wgt;
          if (col + 3 < n_out) {
            *reinterpret_cast<f32x4*>(out + orow + col) = y;
            if (save_a) *reinterpret_cast<f32x4*>(save_a + orow + col) = a;
          } else {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              if (col + v >= n_out) continue;
              out[orow + col + v] = y[v];
              if (save_a) save_a[orow + col + v] = a[v];
            }
          }
        }
      }
    }
    __syncthreads();  // red is reused by the next row chunk
  }
}

// Workgroups per (column tile, expert) over the grid's z extent: one per
// 64-row chunk of an expert of the expected size, at most 16 (each then loops
// over its share of the chunks).
unsigned f32_row_splits(int64_t avg_rows) {
  return static_cast<unsigned>(std::min<int64_t>(std::max<int64_t>(ceil_div(avg_rows, F32_M), 1), 16));
}

}  // namespace

// fp32 activations and fp32 weights with K a multiple of 4 (16-byte rows);
// *handled stays false for anything else.
int launch_ffn_f32(const FfnArgs& a, hipStream_t stream, bool* handled) {
  *handled = false;
  if (a.act != QW_F32 || a.wfmt != QW_F32) return QW_OK;
  if (a.d_model % 4 || a.d_ff % 4) return QW_OK;
  // every operand the kernels read or write in 16-byte vectors (rows of d_model
  // or d_ff floats, so each row start is aligned when the base is)
  if ((reinterpret_cast<uintptr_t>(a.x) | reinterpret_cast<uintptr_t>(a.gate.w) | reinterpret_cast<uintptr_t>(a.up.w) |
       reinterpret_cast<uintptr_t>(a.down.w) | reinterpret_cast<uintptr_t>(a.y) | reinterpret_cast<uintptr_t>(a.hidden) |
       reinterpret_cast<uintptr_t>(a.save_gate) | reinterpret_cast<uintptr_t>(a.save_up) |
       reinterpret_cast<uintptr_t>(a.save_y)) % 16)
    return QW_OK;
  const int D = static_cast<int>(a.d_model), F = static_cast<int>(a.d_ff), mr = static_cast<int>(a.max_rows);
  const int64_t avg = a.avg_rows > 0 ? a.avg_rows : ceil_div(a.max_rows, a.experts);
  const unsigned z = f32_row_splits(avg);
  if (static_cast<int64_t>(ceil_div(D, F32_N)) * a.experts * z < 512) {
    // too few 64 x 64 down tiles to fill the GPU: 32 x 32 tiles with K split over the
    // waves, one workgroup per 32-row chunk up to the capacity bound (so no
    // workgroup takes two chunks of a full expert one after the other)
    const int64_t cap_rows = a.row_cap > 0 ? std::min<int64_t>(a.row_cap, a.max_rows) : 2 * avg;
    const unsigned zs = static_cast<unsigned>(std::min<int64_t>(std::max<int64_t>(ceil_div(cap_rows, F32S_M), 1), 64));
    const XcdGrid s1 = xcd_grid(ceil_div(F, F32S_N / 2), a.experts, zs);
    if (s1.blocks == 0) return set_error(QW_ERR_UNSUPPORTED, "fp32 expert grid too large");
    ffn_f32_small_kernel<true><<<s1.blocks, F32_THREADS, 0, stream>>>(
        static_cast<const float*>(a.x), a.row_index, a.offsets, static_cast<const float*>(a.gate.w),
        static_cast<const float*>(a.up.w), a.gate.expert_elems, F, D, F, mr, nullptr, static_cast<float*>(a.hidden),
        static_cast<float*>(a.save_gate), static_cast<float*>(a.save_up), s1);
    QW_LAUNCH_CHECK("ffn_f32_small_kernel<gateup>");
    const XcdGrid s2 = xcd_grid(ceil_div(D, F32S_N), a.experts, zs);
    if (s2.blocks == 0) return set_error(QW_ERR_UNSUPPORTED, "fp32 expert grid too large");
    ffn_f32_small_kernel<false><<<s2.blocks, F32_THREADS, 0, stream>>>(
        static_cast<const float*>(a.hidden), nullptr, a.offsets, static_cast<const float*>(a.down.w),
        static_cast<const float*>(a.down.w), a.down.expert_elems, D, F, D, mr, a.row_weight, static_cast<float*>(a.y),
        static_cast<float*>(a.save_y), nullptr, s2);
    QW_LAUNCH_CHECK("ffn_f32_small_kernel<down>");
    *handled = true;
    return QW_OK;
  }
  const XcdGrid g1 = xcd_grid(ceil_div(F, F32_N / 2), a.experts, z);
  if (g1.blocks == 0) return set_error(QW_ERR_UNSUPPORTED, "fp32 expert grid too large");
  ffn_f32_mfma_kernel<true><<<g1.blocks, F32_THREADS, 0, stream>>>(
      static_cast<const float*>(a.x), a.row_index, a.offsets, static_cast<const float*>(a.gate.w),
      static_cast<const float*>(a.up.w), a.gate.expert_elems, F, D, F, mr, nullptr, static_cast<float*>(a.hidden),
      static_cast<float*>(a.save_gate), static_cast<float*>(a.save_up), g1);
  QW_LAUNCH_CHECK("ffn_f32_mfma_kernel<gateup>");
  const XcdGrid g2 = xcd_grid(ceil_div(D, F32_N), a.experts, z);
  if (g2.blocks == 0) return set_error(QW_ERR_UNSUPPORTED, "fp32 expert grid too large");
  ffn_f32_mfma_kernel<false><<<g2.blocks, F32_THREADS, 0, stream>>>(
      static_cast<const float*>(a.hidden), nullptr, a.offsets, static_cast<const float*>(a.down.w),
      static_cast<const float*>(a.down.w), a.down.expert_elems, D, F, D, mr, a.row_weight, static_cast<float*>(a.y),
      static_cast<float*>(a.save_y), nullptr, g2);
  QW_LAUNCH_CHECK("ffn_f32_mfma_kernel<down>");
  *handled = true;
  return QW_OK;
}

// The plain grouped matmul out[rows of e] = x[rows of e] @ w[e]^T in fp32
// (qw_grouped_matmul with fp32 activations and weights).
int grouped_matmul_f32(const float* x, const float* w, int64_t E, int64_t N, int64_t K, const int32_t* offsets,
                       int64_t rows, float* out, hipStream_t stream, bool* handled) {
  *handled = false;
  // 16-byte vectors: x and w rows of K floats, out rows of N floats
  if (K % 4 || N % 4 ||
      (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(out)) % 16)
    return QW_OK;
  const unsigned z = f32_row_splits(ceil_div(rows, E));
  const XcdGrid g = xcd_grid(ceil_div(N, F32_N), E, z);
  if (g.blocks == 0) return set_error(QW_ERR_UNSUPPORTED, "fp32 expert grid too large");
  ffn_f32_mfma_kernel<false><<<g.blocks, F32_THREADS, 0, stream>>>(x, nullptr, offsets, w, w, N * K,
                                                                 static_cast<int>(N), static_cast<int>(K),
                                                                 static_cast<int>(N), static_cast<int>(rows), nullptr,
                                                                 out, nullptr, nullptr, g);
  QW_LAUNCH_CHECK("ffn_f32_mfma_kernel<matmul>");
  *handled = true;
  return QW_OK;
}

}  // namespace qw
