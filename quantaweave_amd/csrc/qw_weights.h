// Expert weight formats: element access with in-register dequantisation.
//
// Reference layouts: src/quantization.py:36-40 (buffers), :53-58 (packing),
// :61-69 (dequantize).  A quantised nn.Linear [out, in] is stored as
//   QW_I8: qweight int8  [out, padded]      scales fp32 [out, padded/group]
//   QW_U4: qweight uint8 [out, padded/2]    scales fp32 [out, padded/group]
// with padded = ceil(in/group)*group.  int4 byte b of a row holds input columns
// 2b (low nibble) and 2b+1 (high nibble), each as q + 8.  The dequantised
// weight is q * scale in fp32, which the reference then casts to the
// activation dtype (`self.dequantize().to(x.dtype)`, src/quantization.py:72).
#pragma once
#include "qw_common.h"

namespace qw {

// Geometry of one stacked projection (all experts) in a given format.
struct WView {
  const void* w;         // base of expert 0
  const float* scales;   // QW_I8 / QW_U4 only
  int64_t rows;          // out_features
  int64_t cols;          // in_features
  int64_t row_stride;    // elements (F32/BF16/I8) or bytes (U4) per stored row
  int64_t group;         // quantisation group size (columns)
  int64_t groups;        // scale columns per row
  int64_t expert_elems;  // stored elements (or bytes) per expert
  int64_t expert_scales; // scale entries per expert
};

inline WView make_wview(int fmt, const void* w, const float* scales, int64_t rows, int64_t cols, int64_t group) {
  WView v{};
  v.w = w;
  v.scales = scales;
  v.rows = rows;
  v.cols = cols;
  v.group = group;
  if (fmt == QW_F32 || fmt == QW_BF16 || fmt == QW_BF16T || fmt == QW_F16 || fmt == QW_F16T) {
    v.row_stride = cols;
    v.groups = 0;
  } else {
    const int64_t padded = ceil_div(cols, group) * group;
    v.groups = padded / group;
    v.row_stride = (fmt == QW_I8) ? padded : padded / 2;
  }
  v.expert_elems = rows * v.row_stride;
  v.expert_scales = rows * v.groups;
  return v;
}

// Element offset of W[row][col] in the QW_BF16T tiles of a [rows, cols] matrix:
// tile (row/8, col/64) of 512 elements; in it, 16-byte piece
// 8*(row%8) + (p ^ ((row/2) % 8)) with p = (col%64) / 8, then col%8.
__host__ __device__ __forceinline__ int64_t bf16t_index(int64_t row, int64_t col, int64_t cols) {
  const int64_t tile = (row >> 3) * (cols >> 6) + (col >> 6);
  const int piece = 8 * static_cast<int>(row & 7) + (static_cast<int>((col >> 3) & 7) ^ static_cast<int>((row >> 1) & 7));
  return tile * 512 + piece * 8 + (col & 7);
}

// Dequantised fp32 value of element (row, col) of expert e, before the cast to
// the activation dtype.
template <int WF>
__device__ __forceinline__ float load_weight(const WView& v, int64_t e, int64_t row, int64_t col) {
  if constexpr (WF == QW_F32) {
    return static_cast<const float*>(v.w)[e * v.expert_elems + row * v.row_stride + col];
  } else if constexpr (WF == QW_BF16) {
    return bf16_to_f32(static_cast<const uint16_t*>(v.w)[e * v.expert_elems + row * v.row_stride + col]);
  } else if constexpr (WF == QW_BF16T) {
    return bf16_to_f32(static_cast<const uint16_t*>(v.w)[e * v.expert_elems + bf16t_index(row, col, v.cols)]);
  } else if constexpr (WF == QW_F16) {
    return f16_to_f32(static_cast<const uint16_t*>(v.w)[e * v.expert_elems + row * v.row_stride + col]);
  } else if constexpr (WF == QW_F16T) {
    return f16_to_f32(static_cast<const uint16_t*>(v.w)[e * v.expert_elems + bf16t_index(row, col, v.cols)]);
  } else if constexpr (WF == QW_I8) {
    const int8_t q = static_cast<const int8_t*>(v.w)[e * v.expert_elems + row * v.row_stride + col];
    const float s = v.scales[e * v.expert_scales + row * v.groups + col / v.group];
    return static_cast<float>(q) * s;
  } else {
    const uint8_t b = static_cast<const uint8_t*>(v.w)[e * v.expert_elems + row * v.row_stride + (col >> 1)];
    const int q = ((col & 1) ? (b >> 4) : (b & 0xF)) - 8;
    const float s = v.scales[e * v.expert_scales + row * v.groups + col / v.group];
    return static_cast<float>(q) * s;
  }
}

}  // namespace qw
