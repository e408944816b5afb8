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

int launch_ffn_generic(const FfnArgs& a, hipStream_t stream);
int launch_ffn_mfma(const FfnArgs& a, hipStream_t stream, bool* handled);
int launch_ffn_f32(const FfnArgs& a, hipStream_t stream, bool* handled);
int grouped_matmul_f32(const float* x, const float* w, int64_t E, int64_t N, int64_t K, const int32_t* offsets,
                       int64_t rows, float* out, hipStream_t stream, bool* handled);
int launch_ffn_gemv(const FfnArgs& a, hipStream_t stream, bool* handled);

}  // namespace qw
