// Internal interface of the grouped expert-FFN kernels.
#pragma once
#include "qw_weights.h"

namespace qw {

// One grouped SwiGLU evaluation over plan-ordered rows.
struct FfnArgs {
  const void* x;             // activations [*, d_model] (act dtype)
  const int32_t* row_index;  // row s reads x[row_index[s]]; NULL: x[s]
  const int32_t* offsets;    // [experts+1] row blocks per expert (device)
  int64_t experts, d_model, d_ff, max_rows;
  int act, wfmt;
  WView gate, up, down;
  const float* row_weight;   // per-row combine weight or NULL
  void* hidden;              // [max_rows, d_ff] act dtype (workspace)
  void* y;                   // [max_rows, d_model] act dtype
  float* partial;            // split-K partial sums (workspace), may be NULL
  int64_t avg_rows;          // expected rows per expert (host-side estimate)
  int64_t row_cap;           // most rows any one expert can hold (capacity bound)
  // Optional saved activations for a backward pass (act dtype, plan-ordered
  // rows): gate and up projections [max_rows, d_ff] before the SiLU, and the
  // expert output rows [max_rows, d_model] before the row weight.  The GEMV
  // path does not save; the MFMA and general kernels do.
  void* save_gate = nullptr;
  void* save_up = nullptr;
  void* save_y = nullptr;
};

// Workgroup order of the grouped kernels whose work items are (column tile x,
// expert e, row chunk z).  Workgroups are dispatched round-robin over the
// chip's 8 XCDs (block b on XCD b % 8), each XCD with its own L2.  Every tile
// of an expert reads the expert's rows or its weights, so all of an expert's
// tiles go to one XCD (experts e, e + 8, ... on XCD e % 8) and each byte is
// fetched from HBM by one L2 only.  With fewer than 8 experts an expert takes
// xpe = 8 / E XCDs, which share its row chunks (z = sub, sub + xpe, ...), so
// the whole chip still works.  The order is a performance choice only: every
// (x, e, z) is visited by exactly one workgroup whatever the placement.
constexpr int kXcds = 8;

struct XcdGrid {
  int gx, experts, zs, xpe;  // column tiles, experts, row chunks, XCDs per expert
  unsigned blocks;  // 0 when the grid would not fit a launch
};

inline XcdGrid xcd_grid(int64_t gx, int64_t experts, int64_t zs) {
  XcdGrid g;
  g.gx = static_cast<int>(gx);
  g.experts = static_cast<int>(experts);
  g.zs = static_cast<int>(zs);
  g.xpe = experts >= kXcds ? 1 : kXcds / static_cast<int>(experts);
  const int64_t per_xcd = g.xpe == 1 ? (experts + kXcds - 1) / kXcds * gx * zs : gx * ((zs + g.xpe - 1) / g.xpe);
  g.blocks = kXcds * per_xcd > INT32_MAX ? 0u : static_cast<unsigned>(kXcds * per_xcd);
  return g;
}

// Work item of block b; false for the blocks past the work (an expert index
// past E, or a row chunk past zs).
__device__ __forceinline__ bool xcd_tile(const XcdGrid& g, int b, int* x, int* e, int* z) {
  const int xcd = b % kXcds, j = b / kXcds;
  if (g.xpe == 1) {
    const int per = g.gx * g.zs;
    *e = xcd + kXcds * (j / per);
    *x = (j % per) % g.gx;
    *z = (j % per) / g.gx;
  } else {
    *e = xcd / g.xpe;
    *x = j % g.gx;
    *z = xcd % g.xpe + g.xpe * (j / g.gx);
  }
  return *e < g.experts && *z < g.zs;
}

int launch_ffn_generic(const FfnArgs& a, hipStream_t stream);
int launch_ffn_mfma(const FfnArgs& a, hipStream_t stream, bool* handled);
int launch_ffn_f32(const FfnArgs& a, hipStream_t stream, bool* handled);
int grouped_matmul_f32(const float* x, const float* w, int64_t E, int64_t N, int64_t K, const int32_t* offsets,
                       int64_t rows, float* out, hipStream_t stream, bool* handled);
int launch_ffn_gemv(const FfnArgs& a, hipStream_t stream, bool* handled);

}  // namespace qw
