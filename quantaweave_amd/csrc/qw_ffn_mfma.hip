// Grouped SwiGLU expert FFN on bf16 MFMA (v_mfma_f32_16x16x32_bf16, gfx950)
// for prefill-sized rows per expert.
//
// Reference: src/moe_kernels.py:41-64, :186-195 (grouped GEMM over
// expert-sorted rows, fp32 accumulation) and src/quantweave_moe_model.py:59-60.
//
// One workgroup (8 waves) owns one (expert, row chunk, column tile):
//   row chunk   : up to 32*SUBT plan rows of the expert (the whole expert at the
//                 prefill capacities), so each weight tile is fetched once per
//                 expert rather than once per small row tile;
//   column tile : 256 weight rows — GATEUP: 128 gate + 128 up rows (128 hidden
//                 columns), DOWN: 256 output columns.
// K is staged through LDS in slices of 64 with the next slice prefetched into
// registers while the MFMAs consume the current one.  Waves form a 2 x 4 grid:
// wave (wm, wn) computes row sub-tiles wm, wm+2, ... (16 rows each, skipped
// when past the expert's row count) against its 64 weight rows (GATEUP: 32 gate
// rows and the matching 32 up rows, so SiLU(g)*u is formed in registers).
//
// Workgroup -> tile order is XCD-aware: workgroups are dispatched round-robin
// over the 8 XCDs, so block b runs on XCD b%8; all tiles of one expert are
// given to one XCD and enumerated column-fastest, which keeps the expert's
// activation rows resident in that XCD's L2 while its weight tiles stream.
#include "qw_ffn.h"

namespace qw {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int MF_BK = 64;             // K slice
constexpr int MF_LDS_ROW = MF_BK + 8;  // bf16 per LDS row (16-byte pad: conflict-free 128-bit reads)
constexpr int MF_NB = 256;            // weight rows per column tile
constexpr int MF_THREADS = 512;
constexpr int kXcds = 8;

template <bool GATEUP, int SUBT>
__global__ __launch_bounds__(MF_THREADS) void ffn_mfma_kernel(
    const uint16_t* __restrict__ x, const int32_t* __restrict__ row_index, const int32_t* __restrict__ offsets,
    int max_rows, const uint16_t* __restrict__ wa, const uint16_t* __restrict__ wb, int64_t w_expert_stride,
    int n_w, int K, const float* __restrict__ row_weight, uint16_t* __restrict__ out, int n_out, int n_tiles,
    int m_chunks, int experts) {
  constexpr int MCH = 32 * SUBT;                       // rows per chunk
  constexpr int A_CHUNKS = MCH * (MF_BK / 8);          // 16-byte pieces of the A slice
  constexpr int A_PER = (A_CHUNKS + MF_THREADS - 1) / MF_THREADS;
  constexpr int B_CHUNKS = MF_NB * (MF_BK / 8);
  constexpr int B_PER = B_CHUNKS / MF_THREADS;
  __shared__ __attribute__((aligned(16))) uint16_t As[MCH * MF_LDS_ROW];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[MF_NB * MF_LDS_ROW];

  // ---- tile of this workgroup (XCD-aware enumeration) ----
  const int b = blockIdx.x;
  const int xcd = b % kXcds, j = b / kXcds;
  const int per_expert = m_chunks * n_tiles;
  const int e = xcd + kXcds * (j / per_expert);
  if (e >= experts) return;
  const int rem = j % per_expert;
  const int mc = rem / n_tiles, nt = rem % n_tiles;
  const int e_lo = max(offsets[e], 0);
  const int r0 = e_lo + mc * MCH;
  const int r1 = min(min(offsets[e + 1], r0 + MCH), max_rows);
  const int count = r1 - r0;
  if (count <= 0) return;

  const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  const int wm = wave / 4, wn = wave % 4;
  // weight rows of this column tile
  const int n0 = nt * (GATEUP ? MF_NB / 2 : MF_NB);
  const uint16_t* wa_e = wa + static_cast<int64_t>(e) * w_expert_stride;
  const uint16_t* wb_e = wb + static_cast<int64_t>(e) * w_expert_stride;

  // ---- per-thread global source pointers (constant over K) ----
  const uint16_t* a_src[A_PER];
  int a_dst[A_PER];
#pragma unroll
  for (int i = 0; i < A_PER; ++i) {
    const int c = tid + i * MF_THREADS;
    const int row = c / (MF_BK / 8), ch = c % (MF_BK / 8);
    a_src[i] = nullptr;
    a_dst[i] = -1;
    if (c < A_CHUNKS) {
      a_dst[i] = row * MF_LDS_ROW + ch * 8;
      if (row < count) {
        const int64_t src = row_index ? row_index[r0 + row] : (r0 + row);
        a_src[i] = x + src * K + ch * 8;
      }
    }
  }
  const uint16_t* b_src[B_PER];
  int b_dst[B_PER];
#pragma unroll
  for (int i = 0; i < B_PER; ++i) {
    const int c = tid + i * MF_THREADS;
    const int row = c / (MF_BK / 8), ch = c % (MF_BK / 8);
    b_dst[i] = row * MF_LDS_ROW + ch * 8;
    int wrow;
    const uint16_t* base;
    if (GATEUP) {
      wrow = n0 + (row % (MF_NB / 2));
      base = row < MF_NB / 2 ? wa_e : wb_e;
    } else {
      wrow = n0 + row;
      base = wa_e;
    }
    b_src[i] = wrow < n_w ? base + static_cast<int64_t>(wrow) * K + ch * 8 : nullptr;
  }

  uint4 ra[A_PER], rb[B_PER];
  auto load = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_PER; ++i)
      ra[i] = a_src[i] ? *reinterpret_cast<const uint4*>(a_src[i] + k0) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < B_PER; ++i)
      rb[i] = b_src[i] ? *reinterpret_cast<const uint4*>(b_src[i] + k0) : make_uint4(0, 0, 0, 0);
  };
  auto stash = [&]() {
#pragma unroll
    for (int i = 0; i < A_PER; ++i)
      if (a_dst[i] >= 0) *reinterpret_cast<uint4*>(&As[a_dst[i]]) = ra[i];
#pragma unroll
    for (int i = 0; i < B_PER; ++i) *reinterpret_cast<uint4*>(&Bs[b_dst[i]]) = rb[i];
  };

  f32x4 acc[SUBT][4];
#pragma unroll
  for (int i = 0; i < SUBT; ++i)
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[i][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  // B rows (in the LDS tile) of this wave's 4 MFMA column tiles
  int brow[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    if (GATEUP) brow[t] = (t < 2 ? 0 : MF_NB / 2) + wn * 32 + (t % 2) * 16;
    else brow[t] = wn * 64 + t * 16;
  }
  const int l16 = lane % 16, kq = (lane / 16) * 8;
  // row sub-tiles active in this chunk (wave-uniform)
  const int active_sub = (count + 15) / 16;

  load(0);
  stash();
  __syncthreads();
  const int KT = K / MF_BK;
  for (int kt = 0; kt < KT; ++kt) {
    if (kt + 1 < KT) load((kt + 1) * MF_BK);
#pragma unroll
    for (int ks = 0; ks < MF_BK / 32; ++ks) {
      bf16x8 bfr[4];
#pragma unroll
      for (int t = 0; t < 4; ++t)
        bfr[t] = *reinterpret_cast<const bf16x8*>(&Bs[(brow[t] + l16) * MF_LDS_ROW + ks * 32 + kq]);
#pragma unroll
      for (int i = 0; i < SUBT; ++i) {
        const int s = wm + 2 * i;
        if (s < active_sub) {
          const bf16x8 afr = *reinterpret_cast<const bf16x8*>(&As[(s * 16 + l16) * MF_LDS_ROW + ks * 32 + kq]);
#pragma unroll
          for (int t = 0; t < 4; ++t) acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(afr, bfr[t], acc[i][t], 0, 0, 0);
        }
      }
    }
    __syncthreads();
    if (kt + 1 < KT) {
      stash();
      __syncthreads();
    }
  }

  // ---- epilogue: lane holds rows 4*(lane/16)+r of column lane%16 of each tile ----
  const int rq = (lane / 16) * 4;
#pragma unroll
  for (int i = 0; i < SUBT; ++i) {
    const int s = wm + 2 * i;
    if (s >= active_sub) continue;
    if (GATEUP) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int col = n0 + wn * 32 + t * 16 + l16;
        if (col >= n_out) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = s * 16 + rq + r;
          if (row < count) {
            const float g = acc[i][t][r], u = acc[i][t + 2][r];
            out[static_cast<int64_t>(r0 + row) * n_out + col] = f32_to_bf16(silu_f32(g) * u);
          }
        }
      }
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int col = n0 + wn * 64 + t * 16 + l16;
        if (col >= n_out) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = s * 16 + rq + r;
          if (row < count) {
            const float wgt = row_weight ? row_weight[r0 + row] : 1.0f;
            out[static_cast<int64_t>(r0 + row) * n_out + col] = f32_to_bf16(round_to_bf16(acc[i][t][r]) * wgt);
          }
        }
      }
    }
  }
}

template <bool GATEUP, int SUBT>
int launch_t(const void* x, const int32_t* row_index, const int32_t* offsets, int max_rows, const void* wa,
             const void* wb, int64_t w_stride, int n_w, int K, const float* row_weight, void* out, int n_out,
             int experts, int64_t rows_cap, hipStream_t stream) {
  const int n_tiles = static_cast<int>(ceil_div(GATEUP ? n_w : n_out, GATEUP ? MF_NB / 2 : MF_NB));
  const int m_chunks = static_cast<int>(ceil_div(rows_cap, 32 * SUBT));
  const int64_t grid = static_cast<int64_t>(ceil_div(experts, kXcds)) * kXcds * m_chunks * n_tiles;
  if (grid > INT32_MAX) return set_error(QW_ERR_UNSUPPORTED, "MFMA grid too large");
  ffn_mfma_kernel<GATEUP, SUBT><<<static_cast<unsigned>(grid), MF_THREADS, 0, stream>>>(
      static_cast<const uint16_t*>(x), row_index, offsets, max_rows, static_cast<const uint16_t*>(wa),
      static_cast<const uint16_t*>(wb), w_stride, n_w, K, row_weight, static_cast<uint16_t*>(out), n_out, n_tiles,
      m_chunks, experts);
  QW_LAUNCH_CHECK(GATEUP ? "ffn_mfma_kernel<gateup>" : "ffn_mfma_kernel<down>");
  return QW_OK;
}

// rows_cap: most rows any expert can hold (the capacity bound).
template <bool GATEUP>
int launch_sel(int subt, const void* x, const int32_t* row_index, const int32_t* offsets, int max_rows,
               const void* wa, const void* wb, int64_t w_stride, int n_w, int K, const float* row_weight, void* out,
               int n_out, int experts, int64_t rows_cap, hipStream_t stream) {
#define QW_MF(S)                                                                                                \
  if (subt == S)                                                                                               \
    return launch_t<GATEUP, S>(x, row_index, offsets, max_rows, wa, wb, w_stride, n_w, K, row_weight, out, n_out, \
                               experts, rows_cap, stream);
  QW_MF(2)
  QW_MF(4)
  QW_MF(6)
  QW_MF(8)
  QW_MF(10)
#undef QW_MF
  return set_error(QW_ERR_UNSUPPORTED, "no MFMA variant for %d row sub-tiles", subt);
}

int pick_subt(int64_t rows_cap) {
  // smallest chunk holding the whole expert, up to 320 rows
  for (int s : {2, 4, 6, 8, 10})
    if (rows_cap <= 32 * s) return s;
  return 10;
}

}  // namespace

int launch_ffn_mfma(const FfnArgs& a, hipStream_t stream, bool* handled) {
  *handled = false;
  if (a.act != QW_BF16 || a.wfmt != QW_BF16) return QW_OK;
  if (a.d_model % MF_BK || a.d_ff % MF_BK) return QW_OK;
  if (a.avg_rows < 16) return QW_OK;  // decode-sized: weight streaming kernels
  const int64_t rows_cap = a.row_cap > 0 ? a.row_cap : a.max_rows;
  const int subt = pick_subt(rows_cap);
  const int D = static_cast<int>(a.d_model), F = static_cast<int>(a.d_ff), E = static_cast<int>(a.experts);
  const int mr = static_cast<int>(a.max_rows);
  int st = launch_sel<true>(subt, a.x, a.row_index, a.offsets, mr, a.gate.w, a.up.w, a.gate.expert_elems, F, D,
                            nullptr, a.hidden, F, E, rows_cap, stream);
  if (st) return st;
  st = launch_sel<false>(subt, a.hidden, nullptr, a.offsets, mr, a.down.w, a.down.w, a.down.expert_elems, D, F,
                         a.row_weight, a.y, D, E, rows_cap, stream);
  if (st) return st;
  *handled = true;
  return QW_OK;
}

}  // namespace qw
