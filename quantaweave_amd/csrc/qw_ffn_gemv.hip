// Grouped SwiGLU expert FFN for decode-sized rows per expert: weight streaming.
//
// Reference: src/quantweave_moe_model.py:59-60, :203-211 and, for quantised
// experts, QuantizedLinear.forward (src/quantization.py:61-72), whose layouts
// (src/quantization.py:36-58) are read here as they are stored.
//
// With a handful of routes per expert the FFN is a set of GEMVs whose cost is
// reading each touched expert's weights once.  A workgroup (4 waves) owns an
// (expert, column tile); untouched experts exit at once.  Each lane streams
// 16-byte weight chunks of its rows (all loads issued before any math) and
// dequantises in registers without materialising a bf16 weight:
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
// Activation rows of the expert (up to 4 per pass) are staged once per pass in
// LDS in the pair order the conversion produces, with per-chunk sums for the
// bias correction.  Per-row partial sums are reduced across the wave with
// butterflies.
#include "qw_ffn.h"

namespace qw {

namespace {

typedef __bf16 gbf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 gf16x2 __attribute__((ext_vector_type(2)));

constexpr int GV_WAVES = 4;
constexpr int GV_MAXM = 4;  // routes per pass

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

// Makes the compiler treat v as produced here: keeps the weight conversion from
// being hoisted above the activation staging (which would make the staging
// wait for the whole weight stream).
__device__ __forceinline__ void opaque(uint4& v) {
  asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w));
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

// Dot product of converted weight pairs with one staged activation chunk.
template <int WF, int DW>
__device__ __forceinline__ float chunk_dot(const uint32_t* cw, const uint32_t* xs) {
  float acc = 0.0f;
#pragma unroll
  for (int q = 0; q < DW / 4; ++q) {
    const uint4 t = reinterpret_cast<const uint4*>(xs)[q];
    const uint32_t xv[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (WF == QW_I8) acc = dot2_f16(cw[4 * q + i], xv[i], acc);
      else acc = dot2_bf16(cw[4 * q + i], xv[i], acc);
    }
  }
  return acc;
}

// GATEUP: unit = hidden column (gate row + up row); DOWN: unit = output row.
template <int WF, bool GATEUP, int UNITS, int CPL, int XPIECES_MAX>
__global__ __launch_bounds__(GV_WAVES * 64) void ffn_gemv_kernel(
    const uint16_t* __restrict__ x, const int32_t* __restrict__ row_index, const int32_t* __restrict__ offsets,
    int max_rows, WView wa, WView wb, int K, int n_out, const float* __restrict__ row_weight,
    uint16_t* __restrict__ out) {
  constexpr int CW = Fmt<WF>::CW;
  constexpr int DW = CW / 2;  // staged dwords (activation pairs) per chunk
  constexpr int ROWS = GATEUP ? 2 : 1;
  extern __shared__ __attribute__((aligned(16))) uint32_t smem[];
  const int e = blockIdx.y;
  const int r_lo = max(offsets[e], 0), r_hi = min(offsets[e + 1], max_rows);
  if (r_hi <= r_lo) return;
  const int KC = K / CW;                  // chunks per weight row
  uint32_t* xs = smem;                    // [GV_MAXM][KC][DW]
  float* xsum = reinterpret_cast<float*>(smem + GV_MAXM * KC * DW);  // [GV_MAXM][KC]
  float* xscale = xsum + GV_MAXM * KC;    // [GV_MAXM] multiplier applied to x (I8 path)
  const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  const int unit0 = (blockIdx.x * GV_WAVES + wave) * UNITS;

  // weight row pointers of this wave's units; rows past the end are clamped to
  // the last row (loaded, never written) so that every load is unconditional
  const uint8_t* wrow[UNITS][ROWS];
  const float* srow[UNITS][ROWS];
#pragma unroll
  for (int u = 0; u < UNITS; ++u)
#pragma unroll
    for (int rr = 0; rr < ROWS; ++rr) {
      const WView& v = rr == 0 ? wa : wb;
      const int n = min(unit0 + u, n_out - 1);
      const int64_t esz = WF == QW_BF16 ? 2 : 1;
      wrow[u][rr] = static_cast<const uint8_t*>(v.w) + (e * v.expert_elems + n * v.row_stride) * esz;
      srow[u][rr] = WF != QW_BF16 ? v.scales + e * v.expert_scales + n * v.groups : nullptr;
    }
  const int cpg = wa.group / CW;  // chunks per quantisation group

  // Activation pieces (8 columns = 16 bytes) of one pass, loaded into
  // registers before the weight stream is issued so that waiting for them does
  // not wait for the weights (loads complete in issue order).
  constexpr int XPT = (GV_MAXM * XPIECES_MAX + GV_WAVES * 64 - 1) / (GV_WAVES * 64);
  const int KP = K / 8;  // pieces per activation row
  uint4 xr[XPT];
  auto load_x = [&](int m0, int M) {
    // source rows of the pass first (uniform loads, one wait), then the pieces
    int64_t src[GV_MAXM];
#pragma unroll
    for (int m = 0; m < GV_MAXM; ++m) src[m] = m < M ? (row_index ? row_index[m0 + m] : (m0 + m)) : 0;
    // unconditional loads (indices clamped into the pass): a load under a branch
    // makes the compiler wait for it inside the branch
#pragma unroll
    for (int j = 0; j < XPT; ++j) {
      const int i = min(tid + j * GV_WAVES * 64, M * KP - 1);
      const int m = i / KP, q = i % KP;
      int64_t row = src[0];
#pragma unroll
      for (int t = 1; t < GV_MAXM; ++t) row = (m == t) ? src[t] : row;
      xr[j] = reinterpret_cast<const uint4*>(x + row * K)[q];
    }
  };
  load_x(r_lo, min(GV_MAXM, r_hi - r_lo));

  // ---- this wave's weight rows, streamed once for all passes ----
  uint4 wv[UNITS][ROWS][CPL];
  float sv[UNITS][ROWS][CPL];
#pragma unroll
  for (int u = 0; u < UNITS; ++u)
#pragma unroll
    for (int rr = 0; rr < ROWS; ++rr)
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int c = min(lane + 64 * j, KC - 1);  // chunks past the row end are skipped in the math
        wv[u][rr][j] = *reinterpret_cast<const uint4*>(wrow[u][rr] + 16 * c);
        if constexpr (WF != QW_BF16) sv[u][rr][j] = srow[u][rr][cpg == 1 ? c : c / cpg];
      }

  for (int m0 = r_lo; m0 < r_hi; m0 += GV_MAXM) {
    const int M = min(GV_MAXM, r_hi - m0);
    if (m0 != r_lo) load_x(m0, M);
    if constexpr (WF == QW_I8) {
      // power-of-two scale per route so the largest |x| lands in [2^14, 2^15)
      uint32_t* amax_bits = reinterpret_cast<uint32_t*>(xscale);
      if (tid < GV_MAXM) amax_bits[tid] = 0u;
      lds_barrier();
#pragma unroll
      for (int j = 0; j < XPT; ++j) {
        const int i = tid + j * GV_WAVES * 64;
        if (i < M * KP) {
          const uint32_t v[4] = {xr[j].x, xr[j].y, xr[j].z, xr[j].w};
          float a = 0.0f;
#pragma unroll
          for (int t = 0; t < 4; ++t)
            a = fmaxf(a, fmaxf(fabsf(__uint_as_float(v[t] << 16)), fabsf(__uint_as_float(v[t] & 0xffff0000u))));
          atomicMax(&amax_bits[i / KP], __float_as_uint(a));  // non-negative floats order as integers
        }
      }
      lds_barrier();
      if (tid < M) {
        const float amax = __uint_as_float(amax_bits[tid]);
        int ex = 0;
        frexpf(amax, &ex);  // amax in [2^(ex-1), 2^ex)
        xscale[tid] = amax > 0.0f ? ldexpf(1.0f, 15 - ex) : 1.0f;
      }
      lds_barrier();
    }
    // ---- stage activations in LDS: pairs in the order the conversion emits them ----
#pragma unroll
    for (int j = 0; j < XPT; ++j) {
      const int i = tid + j * GV_WAVES * 64;
      if (i >= M * KP) continue;
      const int m = i / KP;
      const uint32_t v[4] = {xr[j].x, xr[j].y, xr[j].z, xr[j].w};  // v[t] = cols (2t, 2t+1) of the piece
      uint4 o;
      if constexpr (WF == QW_U4) {
        // piece i is dword (i % 4) of a 32-column chunk: pairs (0,2), (4,6), (1,3), (5,7)
        o.x = __builtin_amdgcn_perm(v[1], v[0], 0x05040100u);
        o.y = __builtin_amdgcn_perm(v[3], v[2], 0x05040100u);
        o.z = __builtin_amdgcn_perm(v[1], v[0], 0x07060302u);
        o.w = __builtin_amdgcn_perm(v[3], v[2], 0x07060302u);
      } else if constexpr (WF == QW_I8) {
        const float sc = xscale[m];
        uint32_t h[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const _Float16 a = static_cast<_Float16>(__uint_as_float(v[t] << 16) * sc);
          const _Float16 b = static_cast<_Float16>(__uint_as_float(v[t] & 0xffff0000u) * sc);
          h[t] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, a)) |
                 (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, b)) << 16);
        }
        o = make_uint4(h[0], h[1], h[2], h[3]);
      } else {
        o = xr[j];
      }
      // staged layout [m][chunk][DW dwords]: 8 columns are 4 dwords in every format
      reinterpret_cast<uint4*>(xs)[i] = o;
    }
    lds_barrier();
    if constexpr (WF != QW_BF16) {
      // per-chunk activation sums (of the values as staged) for the bias correction
      for (int i = tid; i < M * KC; i += blockDim.x) {
        const uint32_t* q = xs + i * DW;
        float s = 0.0f;
#pragma unroll
        for (int p = 0; p < DW; ++p) {
          if constexpr (WF == QW_U4) s = dot2_bf16(q[p], 0x3f803f80u, s);  // bf16 pair (1, 1)
          else s = dot2_f16(q[p], 0x3c003c00u, s);                        // fp16 pair (1, 1)
        }
        xsum[i] = s;
      }
      lds_barrier();
    }

    float part[UNITS][ROWS][GV_MAXM];
#pragma unroll
    for (int u = 0; u < UNITS; ++u)
#pragma unroll
      for (int rr = 0; rr < ROWS; ++rr)
#pragma unroll
        for (int m = 0; m < GV_MAXM; ++m) part[u][rr][m] = 0.0f;
#pragma unroll
    for (int u = 0; u < UNITS; ++u)
#pragma unroll
      for (int rr = 0; rr < ROWS; ++rr)
#pragma unroll
        for (int j = 0; j < CPL; ++j) opaque(wv[u][rr][j]);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = lane + 64 * j;
      if (c >= KC) continue;
#pragma unroll
      for (int u = 0; u < UNITS; ++u)
#pragma unroll
        for (int rr = 0; rr < ROWS; ++rr) {
          uint32_t cw[DW];
          chunk_pairs<WF>(wv[u][rr][j], cw);
#pragma unroll
          for (int m = 0; m < GV_MAXM; ++m) {
            if (m >= M) break;
            const float d = chunk_dot<WF, DW>(cw, xs + (m * KC + c) * DW);
            if constexpr (WF == QW_BF16) {
              part[u][rr][m] += d;
            } else {
              const float corr = Fmt<WF>::BIAS * xsum[m * KC + c];
              part[u][rr][m] = __builtin_fmaf(sv[u][rr][j], d - corr, part[u][rr][m]);
            }
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
        float g = wave_sum_f(part[u][0][m]);
        float up = GATEUP ? wave_sum_f(part[u][ROWS - 1][m]) : 0.0f;
        if (WF == QW_I8) {
          const float inv = 1.0f / xscale[m];
          g *= inv;
          up *= inv;
        }
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
    lds_barrier();
  }
}

template <int WF, bool GATEUP, int UNITS, int CPL>
int launch_one(const FfnArgs& a, const WView& wa, const WView& wb, const void* x, const int32_t* row_index, int K,
               int n_out, const float* row_weight, void* out, hipStream_t stream) {
  constexpr int CW = Fmt<WF>::CW;
  const int KC = K / CW;
  const size_t lds = static_cast<size_t>(GV_MAXM) * KC * (CW / 2) * 4 + static_cast<size_t>(GV_MAXM) * KC * 4 +
                     GV_MAXM * 4;
  const dim3 grid(static_cast<unsigned>(ceil_div(n_out, GV_WAVES * UNITS)), static_cast<unsigned>(a.experts));
  // largest activation row the register staging covers: K <= 64*CPL chunks
  ffn_gemv_kernel<WF, GATEUP, UNITS, CPL, 64 * CPL * CW / 8><<<grid, GV_WAVES * 64, lds, stream>>>(
      static_cast<const uint16_t*>(x), row_index, a.offsets, static_cast<int>(a.max_rows), wa, wb, K, n_out,
      row_weight, static_cast<uint16_t*>(out));
  QW_LAUNCH_CHECK(GATEUP ? "ffn_gemv_kernel<gateup>" : "ffn_gemv_kernel<down>");
  return QW_OK;
}

template <int WF, bool GATEUP, int UNITS>
int launch_cpl(const FfnArgs& a, const WView& wa, const WView& wb, const void* x, const int32_t* row_index, int K,
               int n_out, const float* row_weight, void* out, hipStream_t stream) {
  const int KC = K / Fmt<WF>::CW;
  const int cpl = static_cast<int>(ceil_div(KC, 64));
  if (cpl <= 1) return launch_one<WF, GATEUP, UNITS, 1>(a, wa, wb, x, row_index, K, n_out, row_weight, out, stream);
  if (cpl <= 2) return launch_one<WF, GATEUP, UNITS, 2>(a, wa, wb, x, row_index, K, n_out, row_weight, out, stream);
  if (cpl <= 4) return launch_one<WF, GATEUP, UNITS, 4>(a, wa, wb, x, row_index, K, n_out, row_weight, out, stream);
  return set_error(QW_ERR_UNSUPPORTED, "row of %d chunks is too long for the decode kernel", KC);
}

// Units per wave: enough 16-byte loads in flight per lane while keeping the
// register count low enough for several resident workgroups per CU.
template <int WF>
int launch_fmt(const FfnArgs& a, hipStream_t stream) {
  const int D = static_cast<int>(a.d_model), F = static_cast<int>(a.d_ff);
  constexpr int GU = WF == QW_U4 ? 2 : 4;
  constexpr int DN = WF == QW_U4 ? 4 : 8;
  int st = launch_cpl<WF, true, GU>(a, a.gate, a.up, a.x, a.row_index, D, F, nullptr, a.hidden, stream);
  if (st) return st;
  return launch_cpl<WF, false, DN>(a, a.down, a.down, a.hidden, nullptr, F, D, a.row_weight, a.y, stream);
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
