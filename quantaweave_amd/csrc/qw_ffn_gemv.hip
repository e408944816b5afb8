// Grouped SwiGLU expert FFN for decode-sized rows per expert: weight streaming.
//
// Reference: src/quantweave_moe_model.py:59-60, :203-211 and, for quantised
// experts, QuantizedLinear.forward (src/quantization.py:61-72), whose layouts
// (src/quantization.py:36-58) are read here as they are stored.
//
// With a handful of routes per expert the FFN is a set of GEMVs whose cost is
// reading each touched expert's weights once.  A workgroup of 4 independent
// waves owns an (expert, column tile); untouched experts exit at once.  Each
// lane streams the 16-byte weight chunks of its wave's rows (all issued before
// any math) and dequantises in registers without materialising a bf16 weight:
//
//  QW_U4 : a chunk is 32 int4 codes u = q + 8, one quantisation group.  Nibbles
//          become bf16 pairs with one v_perm each: bf16 bits 0x43nn = 128 + n.
//          v_dot2_f32_bf16 accumulates sum x*(128+u); the group's exact value
//          is scale * (acc - 136 * sum x) (136 = 128 + the +8 storage bias).
//  QW_I8 : a chunk is 16 int8 codes; u = q ^ 0x80 = q + 128 becomes the fp16
//          1024 + u by the same v_perm trick and v_dot2_f32_f16 accumulates
//          against activations scaled by a power of two into fp16 range
//          (exact for bf16 values); value = scale * (acc - 1152 * sum x) / 2^s.
//  QW_BF16: a chunk is 8 bf16 weights, used directly by v_dot2_f32_bf16.
//
// The activation pieces matching a lane's chunks come straight from L2 (every
// wave of the expert reads the same few rows), are put in the pair order of
// the conversion once per chunk and reused for every row of the wave.  There
// is no LDS and no barrier, so the waves of a CU overlap freely.  Per-row
// partial sums are reduced across the wave with butterflies.
#include "qw_ffn.h"

namespace qw {

namespace {

typedef __bf16 gbf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 gf16x2 __attribute__((ext_vector_type(2)));

constexpr int GV_WAVES = 4;

template <int WF>
struct Fmt;
template <>
struct Fmt<QW_U4> {
  static constexpr int CW = 32;     // weights per 16-byte chunk
  static constexpr float BIAS = 136.0f;
};
template <>
struct Fmt<QW_I8> {
  static constexpr int CW = 16;
  static constexpr float BIAS = 1152.0f;
};
template <>
struct Fmt<QW_BF16> {
  static constexpr int CW = 8;
  static constexpr float BIAS = 0.0f;
};

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(gbf16x2, a), __builtin_bit_cast(gbf16x2, b), c, false);
}
__device__ __forceinline__ float dot2_f16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(gf16x2, a), __builtin_bit_cast(gf16x2, b), c, false);
}

// Converts one 16-byte weight chunk into the operand pairs of the dot products.
template <int WF>
__device__ __forceinline__ void chunk_pairs(const uint4 w, uint32_t* cw) {
  const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
  if constexpr (WF == QW_U4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = wd[i] & 0x0F0F0F0Fu;
      const uint32_t hi = (wd[i] >> 4) & 0x0F0F0F0Fu;
      // bytes [n, 0x43, n', 0x43]: selector picks from {0x43434343 (bytes 4-7), src (bytes 0-3)}
      cw[4 * i + 0] = __builtin_amdgcn_perm(0x43434343u, lo, 0x04010400u);
      cw[4 * i + 1] = __builtin_amdgcn_perm(0x43434343u, lo, 0x04030402u);
      cw[4 * i + 2] = __builtin_amdgcn_perm(0x43434343u, hi, 0x04010400u);
      cw[4 * i + 3] = __builtin_amdgcn_perm(0x43434343u, hi, 0x04030402u);
    }
  } else if constexpr (WF == QW_I8) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t u = wd[i] ^ 0x80808080u;
      cw[2 * i + 0] = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
      cw[2 * i + 1] = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) cw[i] = wd[i];
  }
}

// Activation pieces of one chunk for one route, prepared for the dot products:
// U4: bf16 pairs in the order the nibble conversion emits them, plus the sum
//     of the chunk's 32 values (the bias correction);
// I8: fp16 pairs of x * 2^s (s per route, brings max|x| into [2^14, 2^15));
// BF16: the bf16 pairs as stored.
template <int WF>
__device__ __forceinline__ void prep_chunk(const uint4* raw, float scale, uint32_t* xq, float* xsum) {
  if constexpr (WF == QW_U4) {
    float sm = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {  // piece q: cols 8q..8q+7; v[t] = cols (2t, 2t+1)
      const uint32_t v[4] = {raw[q].x, raw[q].y, raw[q].z, raw[q].w};
      xq[4 * q + 0] = __builtin_amdgcn_perm(v[1], v[0], 0x05040100u);  // (0, 2)
      xq[4 * q + 1] = __builtin_amdgcn_perm(v[3], v[2], 0x05040100u);  // (4, 6)
      xq[4 * q + 2] = __builtin_amdgcn_perm(v[1], v[0], 0x07060302u);  // (1, 3)
      xq[4 * q + 3] = __builtin_amdgcn_perm(v[3], v[2], 0x07060302u);  // (5, 7)
#pragma unroll
      for (int t = 0; t < 4; ++t) sm = dot2_bf16(v[t], 0x3f803f80u, sm);  // + x[2t] + x[2t+1]
    }
    *xsum = sm;
  } else if constexpr (WF == QW_I8) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint32_t v[4] = {raw[q].x, raw[q].y, raw[q].z, raw[q].w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const _Float16 a = static_cast<_Float16>(__uint_as_float(v[t] << 16) * scale);
        const _Float16 b = static_cast<_Float16>(__uint_as_float(v[t] & 0xffff0000u) * scale);
        xq[4 * q + t] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, a)) |
                        (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, b)) << 16);
      }
    }
    float sm = 0.0f;
#pragma unroll
    for (int p = 0; p < 8; ++p) sm = dot2_f16(xq[p], 0x3c003c00u, sm);  // + x'[2p] + x'[2p+1]
    *xsum = sm;
  } else {
    xq[0] = raw[0].x;
    xq[1] = raw[0].y;
    xq[2] = raw[0].z;
    xq[3] = raw[0].w;
    *xsum = 0.0f;
  }
}

// Waves work independently (no LDS, no barriers): wave w of block (tile, e)
// owns units [(tile*GV_WAVES + w)*UNITS, +UNITS) of expert e.  GATEUP: a unit
// is a hidden column (gate row + up row); DOWN: a unit is an output row.  Each
// lane streams its 16-byte weight chunks c = lane + 64*j once, then for every
// pass of up to GV_MAXM routes (2 for int4, 4 otherwise) loads the routes' activation pieces of the same
// chunks from L2, prepares them once and reuses them for all its rows.
template <int WF, bool GATEUP, int UNITS, int CPL, int GV_MAXM>
__global__ __launch_bounds__(GV_WAVES * 64) void ffn_gemv_kernel(
    const uint16_t* __restrict__ x, const int32_t* __restrict__ row_index, const int32_t* __restrict__ offsets,
    int max_rows, WView wa, WView wb, int K, int n_out, const float* __restrict__ row_weight,
    uint16_t* __restrict__ out) {
  constexpr int CW = Fmt<WF>::CW;
  constexpr int DW = CW / 2;   // activation pairs per chunk
  constexpr int XP = CW / 8;   // 16-byte activation pieces per chunk
  constexpr int ROWS = GATEUP ? 2 : 1;
  const int e = blockIdx.y;
  const int r_lo = max(offsets[e], 0), r_hi = min(offsets[e + 1], max_rows);
  if (r_hi <= r_lo) return;
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  const int unit0 = (blockIdx.x * GV_WAVES + wave) * UNITS;
  if (unit0 >= n_out) return;
  const int KC = K / CW;
  const int cpg = wa.group / CW;  // chunks per quantisation group

  // ---- this wave's weight chunks (unconditional loads, indices clamped) ----
  uint4 wv[UNITS][ROWS][CPL];
  float sv[UNITS][ROWS][CPL];
#pragma unroll
  for (int u = 0; u < UNITS; ++u)
#pragma unroll
    for (int rr = 0; rr < ROWS; ++rr) {
      const WView& v = rr == 0 ? wa : wb;
      const int n = min(unit0 + u, n_out - 1);  // rows past the end: loaded, never written
      const int64_t esz = WF == QW_BF16 ? 2 : 1;
      const uint8_t* wrow = static_cast<const uint8_t*>(v.w) + (e * v.expert_elems + n * v.row_stride) * esz;
      const float* srow = WF != QW_BF16 ? v.scales + e * v.expert_scales + n * v.groups : nullptr;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int c = min(lane + 64 * j, KC - 1);  // chunks past the row end are skipped in the math
        wv[u][rr][j] = *reinterpret_cast<const uint4*>(wrow + 16 * c);
        if constexpr (WF != QW_BF16) sv[u][rr][j] = srow[cpg == 1 ? c : c / cpg];
      }
    }

  for (int m0 = r_lo; m0 < r_hi; m0 += GV_MAXM) {
    const int M = min(GV_MAXM, r_hi - m0);
    const uint16_t* xrow[GV_MAXM];
#pragma unroll
    for (int m = 0; m < GV_MAXM; ++m) {
      const int s = m0 + min(m, M - 1);
      xrow[m] = x + static_cast<int64_t>(row_index ? row_index[s] : s) * K;
    }
    // activation pieces of this pass (unconditional loads, clamped)
    uint4 raw[CPL][GV_MAXM][XP];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = min(lane + 64 * j, KC - 1);
#pragma unroll
      for (int m = 0; m < GV_MAXM; ++m)
#pragma unroll
        for (int q = 0; q < XP; ++q) raw[j][m][q] = reinterpret_cast<const uint4*>(xrow[m] + c * CW)[q];
    }
    float scale[GV_MAXM], inv[GV_MAXM];
#pragma unroll
    for (int m = 0; m < GV_MAXM; ++m) scale[m] = inv[m] = 1.0f;
    if constexpr (WF == QW_I8) {
      // per-route power of two bringing max|x| into [2^14, 2^15): fp16 then holds the bf16 values exactly
#pragma unroll
      for (int m = 0; m < GV_MAXM; ++m) {
        float a = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
          if (lane + 64 * j >= KC) continue;
#pragma unroll
          for (int q = 0; q < XP; ++q) {
            const uint32_t v[4] = {raw[j][m][q].x, raw[j][m][q].y, raw[j][m][q].z, raw[j][m][q].w};
#pragma unroll
            for (int t = 0; t < 4; ++t)
              a = fmaxf(a, fmaxf(fabsf(__uint_as_float(v[t] << 16)), fabsf(__uint_as_float(v[t] & 0xffff0000u))));
          }
        }
        a = wave_max(a);
        int ex = 0;
        frexpf(a, &ex);  // a in [2^(ex-1), 2^ex)
        scale[m] = a > 0.0f ? ldexpf(1.0f, 15 - ex) : 1.0f;
        inv[m] = 1.0f / scale[m];
      }
    }
    float part[UNITS][ROWS][GV_MAXM];
#pragma unroll
    for (int u = 0; u < UNITS; ++u)
#pragma unroll
      for (int rr = 0; rr < ROWS; ++rr)
#pragma unroll
        for (int m = 0; m < GV_MAXM; ++m) part[u][rr][m] = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      if (lane + 64 * j >= KC) continue;
      uint32_t xq[GV_MAXM][DW];
      float xs[GV_MAXM];
#pragma unroll
      for (int m = 0; m < GV_MAXM; ++m) {
        if (m >= M) break;
        prep_chunk<WF>(raw[j][m], scale[m], xq[m], &xs[m]);
      }
#pragma unroll
      for (int u = 0; u < UNITS; ++u)
#pragma unroll
        for (int rr = 0; rr < ROWS; ++rr) {
          uint32_t cw[DW];
          chunk_pairs<WF>(wv[u][rr][j], cw);
#pragma unroll
          for (int m = 0; m < GV_MAXM; ++m) {
            if (m >= M) break;
            float d = 0.0f;
#pragma unroll
            for (int p = 0; p < DW; ++p) d = WF == QW_I8 ? dot2_f16(cw[p], xq[m][p], d) : dot2_bf16(cw[p], xq[m][p], d);
            if constexpr (WF == QW_BF16) part[u][rr][m] += d;
            else part[u][rr][m] = __builtin_fmaf(sv[u][rr][j], d - Fmt<WF>::BIAS * xs[m], part[u][rr][m]);
          }
        }
    }
    // ---- reduce over the wave and write ----
#pragma unroll
    for (int u = 0; u < UNITS; ++u) {
      const int n = unit0 + u;
#pragma unroll
      for (int m = 0; m < GV_MAXM; ++m) {
        if (m >= M) break;
        const float g = wave_sum_f(part[u][0][m]) * inv[m];
        const float up = GATEUP ? wave_sum_f(part[u][ROWS - 1][m]) * inv[m] : 0.0f;
        if (lane == 0 && n < n_out) {
          const int s = m0 + m;
          if (GATEUP) {
            out[static_cast<int64_t>(s) * n_out + n] = f32_to_bf16(silu_f32(g) * up);
          } else {
            const float wgt = row_weight ? row_weight[s] : 1.0f;
            out[static_cast<int64_t>(s) * n_out + n] = f32_to_bf16(round_to_bf16(g) * wgt);
          }
        }
      }
    }
  }
}

template <int WF, bool GATEUP, int UNITS, int CPL>
int launch_one(const FfnArgs& a, const WView& wa, const WView& wb, const void* x, const int32_t* row_index, int K,
               int n_out, const float* row_weight, void* out, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(ceil_div(n_out, UNITS * GV_WAVES)), static_cast<unsigned>(a.experts));
  // routes per pass: int4 activation pieces are 4x larger per chunk than bf16 ones
  constexpr int MAXM = WF == QW_U4 ? 2 : 4;
  ffn_gemv_kernel<WF, GATEUP, UNITS, CPL, MAXM><<<grid, GV_WAVES * 64, 0, stream>>>(
      static_cast<const uint16_t*>(x), row_index, a.offsets, static_cast<int>(a.max_rows), wa, wb, K, n_out,
      row_weight, static_cast<uint16_t*>(out));
  QW_LAUNCH_CHECK(GATEUP ? "ffn_gemv_kernel<gateup>" : "ffn_gemv_kernel<down>");
  return QW_OK;
}

// Units per wave for a row of CPL chunks per lane: 8 weight chunks (16-byte
// loads) in flight per lane, whatever the row length.
template <int WF, bool GATEUP>
int launch_cpl(const FfnArgs& a, const WView& wa, const WView& wb, const void* x, const int32_t* row_index, int K,
               int n_out, const float* row_weight, void* out, hipStream_t stream) {
  const int KC = K / Fmt<WF>::CW;
  const int cpl = static_cast<int>(ceil_div(KC, 64));
  constexpr int U1 = GATEUP ? 4 : 8;
  if (cpl <= 1) return launch_one<WF, GATEUP, U1, 1>(a, wa, wb, x, row_index, K, n_out, row_weight, out, stream);
  if (cpl <= 2) return launch_one<WF, GATEUP, U1 / 2, 2>(a, wa, wb, x, row_index, K, n_out, row_weight, out, stream);
  if (cpl <= 4) return launch_one<WF, GATEUP, U1 / 4, 4>(a, wa, wb, x, row_index, K, n_out, row_weight, out, stream);
  return set_error(QW_ERR_UNSUPPORTED, "row of %d chunks is too long for the decode kernel", KC);
}

template <int WF>
int launch_fmt(const FfnArgs& a, hipStream_t stream) {
  const int D = static_cast<int>(a.d_model), F = static_cast<int>(a.d_ff);
  int st = launch_cpl<WF, true>(a, a.gate, a.up, a.x, a.row_index, D, F, nullptr, a.hidden, stream);
  if (st) return st;
  return launch_cpl<WF, false>(a, a.down, a.down, a.hidden, nullptr, F, D, a.row_weight, a.y, stream);
}

}  // namespace

int launch_ffn_gemv(const FfnArgs& a, hipStream_t stream, bool* handled) {
  *handled = false;
  if (a.act != QW_BF16 || a.avg_rows >= 16) return QW_OK;
  int cw = 0;
  if (a.wfmt == QW_U4) {
    if (a.gate.group % 32 || a.down.group % 32) return QW_OK;
    cw = 32;
  } else if (a.wfmt == QW_I8) {
    if (a.gate.group % 16 || a.down.group % 16) return QW_OK;
    cw = 16;
  } else if (a.wfmt == QW_BF16) {
    cw = 8;
  } else {
    return QW_OK;
  }
  if (a.d_model % cw || a.d_ff % cw) return QW_OK;
  if (ceil_div(a.d_model / cw, 64) > 4 || ceil_div(a.d_ff / cw, 64) > 4) return QW_OK;
  // the padded int4/int8 row must equal the logical row (true when K is a multiple of the group)
  if (a.wfmt != QW_BF16 && (a.gate.row_stride * (a.wfmt == QW_U4 ? 2 : 1) != a.d_model ||
                            a.down.row_stride * (a.wfmt == QW_U4 ? 2 : 1) != a.d_ff))
    return QW_OK;
  int st;
  if (a.wfmt == QW_U4) st = launch_fmt<QW_U4>(a, stream);
  else if (a.wfmt == QW_I8) st = launch_fmt<QW_I8>(a, stream);
  else st = launch_fmt<QW_BF16>(a, stream);
  if (st) return st;
  *handled = true;
  return QW_OK;
}

}  // namespace qw
