// Grouped SwiGLU expert FFN for decode-sized rows per expert: weight streaming.
//
// Reference: src/quantweave_moe_model.py:59-60, :203-211 and, for quantised
// experts, QuantizedLinear.forward (src/quantization.py:61-72), whose layouts
// (src/quantization.py:36-58) are read here as they are stored.
//
// With a handful of routes per expert the FFN is a set of GEMVs whose cost is
// reading each touched expert's weights once.  A one-wave workgroup owns an
// (expert, column tile); untouched experts exit at once.  Each
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
//  QW_BF16: a chunk is 8 bf16 weights, used directly by v_dot2_f32_bf16 (also
//           from QW_BF16T tiles, which only changes where a chunk is read).
//
// fp16 activations (QW_F16) take QW_F16/QW_F16T weights with v_dot2_f32_f16;
// int4 nibbles then become the fp16 pairs 0x64nn = 1024 + n (bias 1032), and
// int8 codes meet the fp16 activations as they are (no rescaling).
//
// The activation pieces matching a lane's chunks come straight from L2 (every
// wave of the expert reads the same few rows), are put in the pair order of
// the conversion once per chunk and reused for every row of the wave.  There
// is no barrier, so the waves of a CU overlap freely.  Per-row partial sums
// are reduced across the wave with butterflies.
//
// int4 rows of up to 4096 codes and int8 rows of up to 2048 take the second
// kernel of this file (ffn_qmf_kernel), which keeps the same streaming scheme
// but forms the dot products on the 4x4x4 matrix cores; the kernel above serves
// bf16 / fp16 weights and longer quantised rows.
#include <cmath>

#include "qw_ffn.h"

namespace qw {

namespace {

typedef __bf16 gbf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 gf16x2 __attribute__((ext_vector_type(2)));

// One wave per workgroup: the waves are independent (no LDS sharing, no
// barrier), and single-wave workgroups let the dispatcher fill every CU's LDS
// with rings (measured 10-15% faster than four-wave workgroups on the decode
// layers).
constexpr int GV_WAVES = 1;

template <int WF>
struct Fmt;
template <>
struct Fmt<QW_U4> {
  static constexpr int CW = 32;     // weights per 16-byte chunk
  static constexpr float BIAS = 136.0f;       // bf16 activations: nibble pairs 128 + n
  static constexpr float BIAS_F16 = 1032.0f;  // fp16 activations: 1024 + n
};
template <>
struct Fmt<QW_I8> {
  static constexpr int CW = 16;
  static constexpr float BIAS = 1152.0f;
  static constexpr float BIAS_F16 = 1152.0f;
};
template <>
struct Fmt<QW_BF16> {
  static constexpr int CW = 8;
};
template <>
struct Fmt<QW_BF16T> : Fmt<QW_BF16> {};  // the same weights in 1 KiB tiles
template <>
struct Fmt<QW_F16> : Fmt<QW_BF16> {};
template <>
struct Fmt<QW_F16T> : Fmt<QW_BF16> {};

// Format of the arithmetic: tiled weights are plain weights once loaded.
constexpr int math_fmt(int wf) { return wf == QW_BF16T ? QW_BF16 : wf == QW_F16T ? QW_F16 : wf; }
constexpr bool quantized(int wf) { return wf == QW_I8 || wf == QW_U4; }

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(gbf16x2, a), __builtin_bit_cast(gbf16x2, b), c, false);
}
__device__ __forceinline__ float dot2_f16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(gf16x2, a), __builtin_bit_cast(gf16x2, b), c, false);
}

// Converts one 16-byte weight chunk into the operand pairs of the dot products
// with activations of type ACT.
template <int ACT, int WF>
__device__ __forceinline__ void chunk_pairs(const uint4 w, uint32_t* cw) {
  const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
  if constexpr (WF == QW_U4) {
    // high bytes 0x43 (bf16 128 + n) or 0x64 (fp16 1024 + n)
    constexpr uint32_t HB = ACT == QW_F16 ? 0x64646464u : 0x43434343u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = wd[i] & 0x0F0F0F0Fu;
      const uint32_t hi = (wd[i] >> 4) & 0x0F0F0F0Fu;
      // bytes [n, HB, n', HB]: selector picks from {HB (bytes 4-7), src (bytes 0-3)}
      cw[4 * i + 0] = __builtin_amdgcn_perm(HB, lo, 0x04010400u);
      cw[4 * i + 1] = __builtin_amdgcn_perm(HB, lo, 0x04030402u);
      cw[4 * i + 2] = __builtin_amdgcn_perm(HB, hi, 0x04010400u);
      cw[4 * i + 3] = __builtin_amdgcn_perm(HB, hi, 0x04030402u);
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
// BF16 / F16: the pairs as stored.
// fp16 activations (ACT == QW_F16) are used as they are (scale 1).
template <int ACT, int WF>
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
      for (int t = 0; t < 4; ++t)  // + x[2t] + x[2t+1]
        sm = ACT == QW_F16 ? dot2_f16(v[t], 0x3c003c00u, sm) : dot2_bf16(v[t], 0x3f803f80u, sm);
    }
    *xsum = sm;
  } else if constexpr (WF == QW_I8) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint32_t v[4] = {raw[q].x, raw[q].y, raw[q].z, raw[q].w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if constexpr (ACT == QW_F16) {
          xq[4 * q + t] = v[t];
          continue;
        }
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

typedef __attribute__((address_space(3))) void lds_void;

// s_waitcnt immediate waiting for vmcnt <= n only (expcnt, lgkmcnt left at max).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | (((N >> 4) & 3) << 14));
}

// LDS bytes of one wave: a ring of STAGES groups (weight chunks, then the
// chunks' scales) and the staging area of the outputs of one pass.
constexpr int GV_GPW_MAX = 8;  // groups per wave, at most

template <int WF, int UNITS, int ROWS, int CPL, int MAXM, bool SAVE = false>
struct GvLds {
  static constexpr int NCH = UNITS * ROWS * CPL;                 // chunk loads per group
  static_assert(NCH == 4 || NCH == 8, "the ring reads four or eight chunks per group");
  static constexpr bool QUANT = quantized(WF);
  static constexpr int STAGE = NCH * 1024 + (QUANT ? NCH * 256 : 0);
  static constexpr int STAGES = 2;
  static constexpr int NDMA = NCH * (QUANT ? 2 : 1);             // DMA instructions per group
  // staged outputs (fp32): per value one output, or with SAVE on gate/up rows
  // three (the SiLU product, the gate and the up projection)
  static constexpr int OUT = GV_GPW_MAX * UNITS * MAXM * 4 * (SAVE && ROWS == 2 ? 3 : 1);
  static constexpr int WAVE = STAGES * STAGE + OUT;
};

// Reads the 8 weight chunks (and, with SCALES, their 8 scales) of this lane from
// one ring stage and waits for them.  Written as one assembly block: the
// compiler cannot tell these reads from the ring's in-flight DMA writes to other
// stages and would wait for every DMA load before each read; the group's own
// DMA loads are covered by the explicit vmcnt wait before this call.
template <bool SCALES>
__device__ __forceinline__ void ring_read8(uint32_t w_addr, uint32_t s_addr, uint4 (&w)[8], float (&sv)[8]) {
  if constexpr (SCALES) {
    asm volatile(
        "ds_read_b128 %0, %16\n"
        "ds_read_b128 %1, %16 offset:1024\n"
        "ds_read_b128 %2, %16 offset:2048\n"
        "ds_read_b128 %3, %16 offset:3072\n"
        "ds_read_b128 %4, %16 offset:4096\n"
        "ds_read_b128 %5, %16 offset:5120\n"
        "ds_read_b128 %6, %16 offset:6144\n"
        "ds_read_b128 %7, %16 offset:7168\n"
        "ds_read_b32 %8, %17\n"
        "ds_read_b32 %9, %17 offset:256\n"
        "ds_read_b32 %10, %17 offset:512\n"
        "ds_read_b32 %11, %17 offset:768\n"
        "ds_read_b32 %12, %17 offset:1024\n"
        "ds_read_b32 %13, %17 offset:1280\n"
        "ds_read_b32 %14, %17 offset:1536\n"
        "ds_read_b32 %15, %17 offset:1792\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3]), "=&v"(w[4]), "=&v"(w[5]), "=&v"(w[6]), "=&v"(w[7]),
          "=&v"(sv[0]), "=&v"(sv[1]), "=&v"(sv[2]), "=&v"(sv[3]), "=&v"(sv[4]), "=&v"(sv[5]), "=&v"(sv[6]),
          "=&v"(sv[7])
        : "v"(w_addr), "v"(s_addr)
        : "memory");
  } else {
    (void)s_addr;
    asm volatile(
        "ds_read_b128 %0, %8\n"
        "ds_read_b128 %1, %8 offset:1024\n"
        "ds_read_b128 %2, %8 offset:2048\n"
        "ds_read_b128 %3, %8 offset:3072\n"
        "ds_read_b128 %4, %8 offset:4096\n"
        "ds_read_b128 %5, %8 offset:5120\n"
        "ds_read_b128 %6, %8 offset:6144\n"
        "ds_read_b128 %7, %8 offset:7168\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3]), "=&v"(w[4]), "=&v"(w[5]), "=&v"(w[6]), "=&v"(w[7])
        : "v"(w_addr)
        : "memory");
#pragma unroll
    for (int i = 0; i < 8; ++i) sv[i] = 1.0f;
  }
}

template <bool SCALES>
__device__ __forceinline__ void ring_read4(uint32_t w_addr, uint32_t s_addr, uint4 (&w)[4], float (&sv)[4]) {
  if constexpr (SCALES) {
    asm volatile(
        "ds_read_b128 %0, %8\n"
        "ds_read_b128 %1, %8 offset:1024\n"
        "ds_read_b128 %2, %8 offset:2048\n"
        "ds_read_b128 %3, %8 offset:3072\n"
        "ds_read_b32 %4, %9\n"
        "ds_read_b32 %5, %9 offset:256\n"
        "ds_read_b32 %6, %9 offset:512\n"
        "ds_read_b32 %7, %9 offset:768\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3]), "=&v"(sv[0]), "=&v"(sv[1]), "=&v"(sv[2]), "=&v"(sv[3])
        : "v"(w_addr), "v"(s_addr)
        : "memory");
  } else {
    (void)s_addr;
    asm volatile(
        "ds_read_b128 %0, %4\n"
        "ds_read_b128 %1, %4 offset:1024\n"
        "ds_read_b128 %2, %4 offset:2048\n"
        "ds_read_b128 %3, %4 offset:3072\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3])
        : "v"(w_addr)
        : "memory");
#pragma unroll
    for (int i = 0; i < 4; ++i) sv[i] = 1.0f;
  }
}

// Eight chunks and the R scales of a group whose rows have one scale each (R
// row sets of 8 / R slots): the scale of row set r sits at s_addr + 256 r and
// serves every slot of that row set.
template <int R>
__device__ __forceinline__ void ring_read8_rs(uint32_t w_addr, uint32_t s_addr, uint4 (&w)[8], float (&sv)[8]) {
  static_assert(R == 1 || R == 2, "one or two row sets of 8 or 4 slots");
  float s0, s1;
  if constexpr (R == 1) {
    asm volatile(
        "ds_read_b128 %0, %9\n"
        "ds_read_b128 %1, %9 offset:1024\n"
        "ds_read_b128 %2, %9 offset:2048\n"
        "ds_read_b128 %3, %9 offset:3072\n"
        "ds_read_b128 %4, %9 offset:4096\n"
        "ds_read_b128 %5, %9 offset:5120\n"
        "ds_read_b128 %6, %9 offset:6144\n"
        "ds_read_b128 %7, %9 offset:7168\n"
        "ds_read_b32 %8, %10\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3]), "=&v"(w[4]), "=&v"(w[5]), "=&v"(w[6]), "=&v"(w[7]),
          "=&v"(s0)
        : "v"(w_addr), "v"(s_addr)
        : "memory");
    s1 = s0;
  } else {
    asm volatile(
        "ds_read_b128 %0, %10\n"
        "ds_read_b128 %1, %10 offset:1024\n"
        "ds_read_b128 %2, %10 offset:2048\n"
        "ds_read_b128 %3, %10 offset:3072\n"
        "ds_read_b128 %4, %10 offset:4096\n"
        "ds_read_b128 %5, %10 offset:5120\n"
        "ds_read_b128 %6, %10 offset:6144\n"
        "ds_read_b128 %7, %10 offset:7168\n"
        "ds_read_b32 %8, %11\n"
        "ds_read_b32 %9, %11 offset:256\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3]), "=&v"(w[4]), "=&v"(w[5]), "=&v"(w[6]), "=&v"(w[7]),
          "=&v"(s0), "=&v"(s1)
        : "v"(w_addr), "v"(s_addr)
        : "memory");
  }
#pragma unroll
  for (int q = 0; q < 8; ++q) sv[q] = q < 8 / R ? s0 : s1;
}

// Six chunks and their scales (the int4 matrix-core kernel's groups of 6).
__device__ __forceinline__ void ring_read6(uint32_t w_addr, uint32_t s_addr, uint4 (&w)[8], float (&sv)[8]) {
  asm volatile(
      "ds_read_b128 %0, %12\n"
      "ds_read_b128 %1, %12 offset:1024\n"
      "ds_read_b128 %2, %12 offset:2048\n"
      "ds_read_b128 %3, %12 offset:3072\n"
      "ds_read_b128 %4, %12 offset:4096\n"
      "ds_read_b128 %5, %12 offset:5120\n"
      "ds_read_b32 %6, %13\n"
      "ds_read_b32 %7, %13 offset:256\n"
      "ds_read_b32 %8, %13 offset:512\n"
      "ds_read_b32 %9, %13 offset:768\n"
      "ds_read_b32 %10, %13 offset:1024\n"
      "ds_read_b32 %11, %13 offset:1280\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3]), "=&v"(w[4]), "=&v"(w[5]), "=&v"(sv[0]), "=&v"(sv[1]),
        "=&v"(sv[2]), "=&v"(sv[3]), "=&v"(sv[4]), "=&v"(sv[5])
      : "v"(w_addr), "v"(s_addr)
      : "memory");
}

// Eight chunks and their eight scales, the scales at sa[q & 3] + 1024 * (q >> 2)
// (the matrix-core kernel's scales loaded 16 bytes per lane).
__device__ __forceinline__ void ring_read8_sv(uint32_t w_addr, const uint32_t (&sa)[4], uint4 (&w)[8],
                                              float (&sv)[8]) {
  asm volatile(
      "ds_read_b128 %0, %16\n"
      "ds_read_b128 %1, %16 offset:1024\n"
      "ds_read_b128 %2, %16 offset:2048\n"
      "ds_read_b128 %3, %16 offset:3072\n"
      "ds_read_b128 %4, %16 offset:4096\n"
      "ds_read_b128 %5, %16 offset:5120\n"
      "ds_read_b128 %6, %16 offset:6144\n"
      "ds_read_b128 %7, %16 offset:7168\n"
      "ds_read_b32 %8, %17\n"
      "ds_read_b32 %9, %18\n"
      "ds_read_b32 %10, %19\n"
      "ds_read_b32 %11, %20\n"
      "ds_read_b32 %12, %17 offset:1024\n"
      "ds_read_b32 %13, %18 offset:1024\n"
      "ds_read_b32 %14, %19 offset:1024\n"
      "ds_read_b32 %15, %20 offset:1024\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3]), "=&v"(w[4]), "=&v"(w[5]), "=&v"(w[6]), "=&v"(w[7]),
        "=&v"(sv[0]), "=&v"(sv[1]), "=&v"(sv[2]), "=&v"(sv[3]), "=&v"(sv[4]), "=&v"(sv[5]), "=&v"(sv[6]),
        "=&v"(sv[7])
      : "v"(w_addr), "v"(sa[0]), "v"(sa[1]), "v"(sa[2]), "v"(sa[3])
      : "memory");
}

// LDS byte address of a pointer into the kernel's dynamic LDS.
__device__ __forceinline__ uint32_t lds_addr(const char* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)p));
}

// The expert of the j-th non-empty row range, in ascending expert order, and its
// rows [*lo, *hi); -1 when fewer than j + 1 experts have rows.  The grid's y
// extent then only needs to cover the experts that can have rows (at most one
// per row), not all of them.  Wave-uniform result.
__device__ __forceinline__ int nth_active_expert(const int32_t* __restrict__ offsets, int E, int max_rows, int j,
                                                 int* lo, int* hi) {
  const int lane = threadIdx.x % kWave;
  for (int c = 0; c < E; c += kWave) {
    const int e = c + lane;
    int a = 0, b = 0;
    if (e < E) {
      a = min(max(offsets[e], 0), max_rows);
      b = min(offsets[e + 1], max_rows);
    }
    const bool act = b > a;
    const uint64_t m = __ballot(act);
    const int n = __popcll(m);
    if (j < n) {
      const bool hit = act && __popcll(m & ((1ull << lane) - 1ull)) == j;
      const int src = __builtin_ctzll(__ballot(hit));
      *lo = __builtin_amdgcn_readfirstlane(__shfl(a, src, kWave));
      *hi = __builtin_amdgcn_readfirstlane(__shfl(b, src, kWave));
      return c + src;
    }
    j -= n;
  }
  return -1;
}

// Waves work independently (no barriers).  A group is UNITS consecutive units
// of expert e (GATEUP: a unit is a hidden column, i.e. a gate row and an up
// row; DOWN: an output row).  Block (b, j) works on the j-th expert that has
// rows; its wave w owns groups [(b*GV_WAVES + w)*gpw, +gpw).  Lane l streams the 16-byte chunks
// c = l + 64*j (j < CPL) of each row, and their scales, HBM -> LDS with
// global_load_lds into a two-stage ring of the wave's own (one group ahead; a
// deeper ring costs more LDS per wave than the extra waves it displaces), so
// the bytes in flight cost no registers; the loads complete in issue order and
// every group issues the same loads, so a fixed vmcnt wait marks a group as
// landed.  The activation pieces of the same chunks for up to MAXM routes come
// from L2 once per pass, are prepared once and kept in registers while the
// wave walks its groups.  Outputs are staged in the wave's LDS and stored once
// the pass is done (a store between the ring loads would break the counts).
// SAVE (training): gate/up also stores the gate and up projections (save_a,
// save_b); down also stores the rows before their row weight (save_a).
template <int ACT, int WF, bool GATEUP, int UNITS, int CPL, int MAXM, bool SAVE>
__global__ __launch_bounds__(GV_WAVES * 64) void ffn_gemv_kernel(
    const uint16_t* __restrict__ x, const int32_t* __restrict__ row_index, const int32_t* __restrict__ offsets,
    int n_experts, int max_rows, WView wa, WView wb, int K, int n_out, int gpw,
    const float* __restrict__ row_weight, uint16_t* __restrict__ out, uint16_t* __restrict__ save_a,
    uint16_t* __restrict__ save_b) {
  constexpr int MW = math_fmt(WF);
  constexpr bool TILED = WF == QW_BF16T || WF == QW_F16T;
  constexpr int CW = Fmt<WF>::CW;
  constexpr int DW = CW / 2;   // activation pairs per chunk
  constexpr int XP = CW / 8;   // 16-byte activation pieces per chunk
  constexpr int ROWS = GATEUP ? 2 : 1;
  constexpr int V = UNITS * ROWS * MAXM;  // values reduced per group
  constexpr int L = log2i<V>();
  constexpr int OUTS = UNITS * MAXM;      // outputs per group
  using LD = GvLds<WF, UNITS, ROWS, CPL, MAXM, SAVE>;
  constexpr int W_AUX = LD::QUANT ? 0 : kLoadStream;  // cache policy of the weight chunk loads
  constexpr int SLOTS = GV_GPW_MAX * OUTS;  // staged values of one kind per wave
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  int r_lo = 0, r_hi = 0;
  const int e = nth_active_expert(offsets, n_experts, max_rows, blockIdx.y, &r_lo, &r_hi);
  if (e < 0) return;
  const int lane = threadIdx.x % 64;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);  // wave-uniform: keeps the group loop scalar
  const int n_groups = (n_out + UNITS - 1) / UNITS;
  const int g_first = (blockIdx.x * GV_WAVES + wave) * gpw;
  if (g_first >= n_groups) return;
  const int g_end = min(g_first + gpw, n_groups);
  char* const ring = smem + wave * LD::WAVE;
  float* const staged = reinterpret_cast<float*>(ring + LD::STAGES * LD::STAGE);
  const int KC = K / CW;
  const int cpg = wa.group / CW;  // chunks per quantisation group
  const int64_t esz = quantized(MW) ? 1 : 2;
  const uint8_t* wbase[ROWS];
  const float* sbase[ROWS];
#pragma unroll
  for (int rr = 0; rr < ROWS; ++rr) {
    const WView& v = rr == 0 ? wa : wb;
    wbase[rr] = static_cast<const uint8_t*>(v.w) + e * v.expert_elems * esz;
    sbase[rr] = quantized(WF) ? v.scales + e * v.expert_scales : nullptr;
  }
  const int64_t wstride = wa.row_stride * esz;
  const int sstride = wa.groups;
  int cidx[CPL], sidx[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    cidx[j] = min(lane + 64 * j, KC - 1);  // chunks past the row end are loaded, never used
    sidx[j] = cpg == 1 ? cidx[j] : cidx[j] / cpg;
  }

  // DMA of group g (clamped to the wave's last group, so every group issues the same loads)
  auto issue = [&](int g) {
    g = min(g, g_end - 1);
    char* st = ring + ((g - g_first) % LD::STAGES) * LD::STAGE;
#pragma unroll
    for (int u = 0; u < UNITS; ++u) {
      const int n = min(g * UNITS + u, n_out - 1);  // rows past the end: loaded, never written
#pragma unroll
      for (int rr = 0; rr < ROWS; ++rr) {
        // QW_BF16T: chunk c of row n sits in tile (n/8, c/8) at 16-byte piece
        // 8*(n%8) + ((c%8) ^ ((n/2) % 8)); the tiles of rows n&~7 start where
        // those rows start in the plain layout
        const uint8_t* wrow = wbase[rr] + static_cast<int64_t>(TILED ? (n & ~7) : n) * wstride;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
          const int q = (u * ROWS + rr) * CPL + j;
          const int64_t off = TILED ? (static_cast<int64_t>(cidx[j] >> 3) << 10) +
                                          ((8 * (n & 7) + ((cidx[j] & 7) ^ ((n >> 1) & 7))) << 4)
                                    : 16 * static_cast<int64_t>(cidx[j]);
          __builtin_amdgcn_global_load_lds(static_cast<const void*>(wrow + off), (lds_void*)(st + q * 1024), 16, 0,
                                           W_AUX);
          if constexpr (LD::QUANT)
            __builtin_amdgcn_global_load_lds(static_cast<const void*>(sbase[rr] + n * sstride + sidx[j]),
                                             (lds_void*)(st + LD::NCH * 1024 + q * 256), 4, 0, 0);
        }
      }
    }
  };

  for (int m0 = r_lo; m0 < r_hi; m0 += MAXM) {
    const int M = min(MAXM, r_hi - m0);
    // ---- the rows' token indices, the first group of the ring, then the activation
    //      pieces of this pass (plain loads): the weight DMA does not wait for the
    //      index loads the activation loads depend on ----
    int xr[MAXM];
#pragma unroll
    for (int m = 0; m < MAXM; ++m) {
      const int s = m0 + min(m, M - 1);
      xr[m] = row_index ? row_index[s] : s;
    }
#pragma unroll
    for (int i = 0; i < LD::STAGES - 1; ++i) issue(g_first + i);
    uint4 raw[CPL][MAXM][XP];
#pragma unroll
    for (int m = 0; m < MAXM; ++m) {
      const uint16_t* xrow = x + static_cast<int64_t>(xr[m]) * K;
#pragma unroll
      for (int j = 0; j < CPL; ++j)
#pragma unroll
        for (int q = 0; q < XP; ++q) raw[j][m][q] = reinterpret_cast<const uint4*>(xrow + cidx[j] * CW)[q];
    }
    float scale[MAXM], inv[MAXM];
#pragma unroll
    for (int m = 0; m < MAXM; ++m) scale[m] = inv[m] = 1.0f;
    if constexpr (WF == QW_I8 && ACT == QW_BF16) {
      // per-route power of two bringing max|x| into [2^14, 2^15): fp16 then holds the bf16 values exactly
#pragma unroll
      for (int m = 0; m < MAXM; ++m) {
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
        // 2^(15 - ex), at most 2^126 (routes of tiny activations: the scale and
        // its inverse stay finite and normal; such rows are then below 2^14)
        scale[m] = a > 0.0f ? ldexpf(1.0f, min(15 - ex, 126)) : 1.0f;
        inv[m] = 1.0f / scale[m];
      }
    }
    uint32_t xq[CPL][MAXM][DW];
    float xs[CPL][MAXM];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      // chunks past the row end get zero activations, so every chunk is used unconditionally below
      const bool valid = lane + 64 * j < KC;
#pragma unroll
      for (int m = 0; m < MAXM; ++m) {
        prep_chunk<ACT, MW>(raw[j][m], scale[m], xq[j][m], &xs[j][m]);
#pragma unroll
        for (int p = 0; p < DW; ++p) xq[j][m][p] = valid ? xq[j][m][p] : 0u;
        xs[j][m] = valid ? xs[j][m] : 0.0f;
      }
    }

    // ---- the groups: issue g+1 (if the wave has it), wait for g, compute g from the ring ----
    static_assert(LD::STAGES == 2, "the wait below assumes one group in flight ahead");
    for (int g = g_first; g < g_end; ++g) {
      if (g + 1 < g_end) {
        issue(g + 1);
        wait_vmcnt<LD::NDMA>();
      } else {
        wait_vmcnt<0>();
      }
      const char* st = ring + ((g - g_first) % LD::STAGES) * LD::STAGE;
      uint4 wq[LD::NCH];
      float sq[LD::NCH];
      if constexpr (LD::NCH == 8)
        ring_read8<LD::QUANT>(lds_addr(st) + lane * 16, lds_addr(st + LD::NCH * 1024) + lane * 4, wq, sq);
      else
        ring_read4<LD::QUANT>(lds_addr(st) + lane * 16, lds_addr(st + LD::NCH * 1024) + lane * 4, wq, sq);
      float part[V];
#pragma unroll
      for (int i = 0; i < V; ++i) part[i] = 0.0f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
#pragma unroll
        for (int u = 0; u < UNITS; ++u)
#pragma unroll
          for (int rr = 0; rr < ROWS; ++rr) {
            const int q = (u * ROWS + rr) * CPL + j;
            const uint4 wv = wq[q];
            const float sv = sq[q];
            uint32_t cw[DW];
            chunk_pairs<ACT, MW>(wv, cw);
#pragma unroll
            for (int m = 0; m < MAXM; ++m) {
              if (m >= M) break;
              float d = 0.0f;
#pragma unroll
              for (int p = 0; p < DW; ++p)
                d = (WF == QW_I8 || ACT == QW_F16) ? dot2_f16(cw[p], xq[j][m][p], d) : dot2_bf16(cw[p], xq[j][m][p], d);
              float& acc = part[((u * MAXM + m) << (ROWS - 1)) | rr];
              if constexpr (!quantized(MW)) acc += d;
              else acc = __builtin_fmaf(sv, d - (ACT == QW_F16 ? Fmt<MW>::BIAS_F16 : Fmt<MW>::BIAS) * xs[j][m], acc);
            }
          }
      }
      if constexpr (WF == QW_I8 && ACT == QW_BF16) {  // undo the power-of-two activation scaling (exact)
#pragma unroll
        for (int u = 0; u < UNITS; ++u)
#pragma unroll
          for (int m = 0; m < MAXM; ++m)
#pragma unroll
            for (int rr = 0; rr < ROWS; ++rr) part[((u * MAXM + m) << (ROWS - 1)) | rr] *= inv[m];
      }
      float r = reduce_scatter<V>(part, lane);
      const int idx = lane >> (6 - L);  // value index this lane now holds
      const int um = GATEUP ? idx >> 1 : idx;
      float* slot = staged + (g - g_first) * OUTS + um;
      if constexpr (GATEUP) {
        const float up = __shfl_xor(r, 1 << (6 - L), kWave);  // the up row of the same unit and route
        if ((lane & ((2 << (6 - L)) - 1)) == 0) {
          *slot = swiglu_act<ACT>(r, up);
          if constexpr (SAVE) {
            slot[SLOTS] = r;
            slot[2 * SLOTS] = up;
          }
        }
      } else {
        if ((lane & ((1 << (6 - L)) - 1)) == 0) *slot = r;
      }
    }
    wait_vmcnt<0>();  // the ring's trailing (clamped) loads land before the next pass reuses the ring
    // ---- outputs of the pass: value v = (group, unit, route) of this wave's staging area ----
    const int n_vals = (g_end - g_first) * OUTS;
    for (int v = lane; v < n_vals; v += 64) {
      const int gi = v / OUTS, um = v % OUTS;
      const int u = um / MAXM, m = um % MAXM;
      const int n = (g_first + gi) * UNITS + u;
      if (m >= M || n >= n_out) continue;
      const int srow = m0 + m;
      const float val = staged[v];
      const int64_t o = static_cast<int64_t>(srow) * n_out + n;
      if constexpr (GATEUP) {
        out[o] = f32_to_half<ACT>(val);
        if constexpr (SAVE) {
          save_a[o] = f32_to_half<ACT>(staged[SLOTS + v]);
          save_b[o] = f32_to_half<ACT>(staged[2 * SLOTS + v]);
        }
      } else {
        const float wgt = row_weight ? row_weight[srow] : 1.0f;
        out[o] = f32_to_half<ACT>(round_act<ACT>(val) * wgt);
        if constexpr (SAVE) save_a[o] = f32_to_half<ACT>(val);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Quantised (int4 / int8) experts with the dot products on the matrix cores
// (decode rows).
//
// v_mfma_f32_4x4x4_16b (bf16 or f16 operands) forms 16 independent 4x4
// products over 4 k values: in block b = lane / 4, lane 4b + i supplies row i
// of A, lane 4b + j column j of B, and lane 4b + j receives D[i][j] in its
// result register i.  Here lane 4b + t supplies route t's activations (A row t)
// and weight row t of the current row set (B column t), and the 16 blocks work
// on 16 different chunks of the rows; one instruction therefore forms the
// products of 4 routes with 4 weight rows over 4 codes of 16 chunks.  Unlike
// the dot-product kernel above, the VALU work per weight (the code conversion
// and one scale per chunk) does not grow with the number of routes.
//
// int4: a dword of 8 codes (byte j holds codes 2j and 2j + 1, low nibble
// first) becomes the operand pairs (0, 2), (4, 6), (1, 3), (5, 7) as in the
// kernel above: the low and the high nibbles are masked into bytes (an AND, a
// shift and an AND) and v_perm puts each pair under the high byte 0x43 (bf16
// 128 + u) or 0x64 (fp16 1024 + u), u = q + 8.  int8: a dword of 4 codes, u =
// q ^ 0x80 = q + 128, becomes two fp16 pairs 1024 + u by v_perm, against fp16
// activations scaled by a power of two per route as in the kernel above.  The
// activations are put in the operand order once per pass.  A chunk's chain of
// 8 (int4) or 4 (int8) instructions yields sum x * (magic value + u); its
// result times the chunk's group scale is accumulated, and one fp32 4x4x1
// product per chunk adds -(magic value + storage bias) * (the chunk's sum of x)
// * scale for the 4 routes and 4 rows, which removes both offsets without VALU
// work.
//
// Lane (b, t) holds chunks c = 16 s + b (s < S) of every row it streams, so one
// row set of 4 rows takes S chunk loads per lane and a group of R row sets
// S * R loads, through the same two-stage ring of global_load_lds as above.
// GATEUP row sets are (gate u, up u, gate u + 1, up u + 1); DOWN row sets are 4
// consecutive output rows.  The partial sums of the 16 blocks are added with a
// reduce-scatter over lane bits 5..2 (ds_bpermute for 32, ds_swizzle below).

typedef _Float16 gf16x4 __attribute__((ext_vector_type(4)));
typedef short gs16x4 __attribute__((ext_vector_type(4)));
typedef float gf32x4 __attribute__((ext_vector_type(4)));

// One 4x4x4 product of 16 blocks on two packed pairs of A and of B.
template <int ACT>
__device__ __forceinline__ gf32x4 mfma4(uint2 a, uint2 b, gf32x4 c) {
  if constexpr (ACT == QW_F16)
    return __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(gf16x4, a), __builtin_bit_cast(gf16x4, b), c, 0, 0,
                                              0);
  else
    return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(gs16x4, a), __builtin_bit_cast(gs16x4, b), c, 0,
                                                  0, 0);
}

template <int NCH, int UPG, int NST>
struct QmfLds {
  static constexpr int STAGE = NCH * 1024 + NCH * 256;  // chunks, then their scales
  static constexpr int STAGES = NST;
  static constexpr int GPW_MAX = 16;                    // groups per wave, at most
  static constexpr int OUT = GPW_MAX * UPG * 4 * 4;     // fp32, 4 routes per unit
  static constexpr int BYTES = STAGES * STAGE + OUT;
};

// The j-th (expert, pass) of the row ranges in ascending expert order, where a
// pass is up to 4 consecutive rows of one expert (an expert with r rows has
// ceil(r / 4) passes); -1 past the last one.  [*lo, *hi) are the pass's rows.
// A block per pass spreads an expert with many routes over as many blocks as
// it has passes.  Wave-uniform result.
__device__ __forceinline__ int nth_active_pass(const int32_t* __restrict__ offsets, int E, int max_rows, int j,
                                               int* lo, int* hi) {
  const int lane = threadIdx.x % kWave;
  for (int c = 0; c < E; c += kWave) {
    const int e = c + lane;
    int a = 0, b = 0;
    if (e < E) {
      a = min(max(offsets[e], 0), max_rows);
      b = min(offsets[e + 1], max_rows);
    }
    const int np = b > a ? (b - a + 3) / 4 : 0;
    int incl = np;  // inclusive prefix sum of the passes over the lanes
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const int v = __shfl_up(incl, d, kWave);
      if (lane >= d) incl += v;
    }
    const int total = __shfl(incl, kWave - 1, kWave);
    if (j < total) {
      const int src = __builtin_ctzll(__ballot(j < incl && j >= incl - np));
      const int p = j - __shfl(incl - np, src, kWave);  // pass of expert c + src
      const int a0 = __shfl(a, src, kWave), b0 = __shfl(b, src, kWave);
      *lo = __builtin_amdgcn_readfirstlane(a0 + 4 * p);
      *hi = __builtin_amdgcn_readfirstlane(min(a0 + 4 * p + 4, b0));
      return c + src;
    }
    j -= total;
  }
  return -1;
}

// Value of lane (lane ^ O) for O in 4, 8, 16 (ds_swizzle, bit mode) or 32
// (ds_bpermute with the byte address of lane ^ 32 in addr32).
template <int O>
__device__ __forceinline__ float xor_lane(float v, int addr32) {
  if constexpr (O == 32) return __int_as_float(__builtin_amdgcn_ds_bpermute(addr32, __float_as_int(v)));
  else return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), (O << 10) | 0x1F));
}

// Sum over lane bits O..4 of V values per lane: the first log2(V) steps halve
// the values a lane holds (bit O set keeps the upper half), the rest add.  A
// lane ends with value (lane >> (6 - log2 V)) & (V - 1), summed over the 16
// lanes that share lane bits 0 and 1.
template <int V, int N, int O>
__device__ __forceinline__ void rs_blocks(float (&v)[V], int lane, int addr32) {
  if constexpr (O >= 4) {
    if constexpr (N > 1) {
      constexpr int half = N / 2;
      const bool upper = lane & O;
#pragma unroll
      for (int i = 0; i < half; ++i) {
        const float give = upper ? v[i] : v[i + half];
        const float keep = upper ? v[i + half] : v[i];
        v[i] = keep + xor_lane<O>(give, addr32);
      }
      rs_blocks<V, half, O / 2>(v, lane, addr32);
    } else {
      v[0] += xor_lane<O>(v[0], addr32);
      rs_blocks<V, 1, O / 2>(v, lane, addr32);
    }
  }
}

// Broadcast of lane 4 * (lane / 4) + I's value to the 4 lanes of its quad.
template <int I>
__device__ __forceinline__ float quad_bcast(float v) {
  return __uint_as_float(dpp_u32<I * 0x55>(__float_as_uint(v)));
}

// FULL: rows of exactly 16 S chunks with one scale per chunk (group 32), so a
// slot's chunk and scale offsets are a lane constant plus an immediate.
// RS: one scale per row (a group as long as the row, as int8 rows quantised
// without a group size are), loaded once per row set instead of once per slot.
// Block (x, y) streams groups [x gpw, (x + 1) gpw) of the y-th pass (up to 4
// rows of one expert, nth_active_pass), so an expert with more routes has more
// blocks rather than longer ones (int8 decode layer: 102.4 -> 96.1 us against
// a block per expert that walks its passes in turn).
template <int ACT, int WF, bool GATEUP, int S, int R, bool FULL, int NST, bool RS = false>
__global__ __launch_bounds__(64) void ffn_qmf_kernel(
    const uint16_t* __restrict__ x, const int32_t* __restrict__ row_index, const int32_t* __restrict__ offsets,
    int n_experts, int max_rows, WView wa, WView wb, int K, int n_out, int gpw, const float* __restrict__ row_weight,
    uint16_t* __restrict__ out) {
  constexpr bool I8 = WF == QW_I8;
  static_assert(WF == QW_U4 || WF == QW_I8, "int4 or int8 weights");
  constexpr int CW = I8 ? 16 : 32;               // codes per 16-byte chunk
  constexpr int NMF = CW / 4;                    // 4x4x4 products per chunk
  constexpr int MT = (I8 || ACT == QW_F16) ? QW_F16 : QW_BF16;  // operand type of the products
  constexpr int NCH = S * R;                     // chunk loads per lane and group
  constexpr int UPG = GATEUP ? 2 * R : 4 * R;    // units (hidden columns or output rows) per group
  constexpr int V = 4 * R;                       // values per lane reduced per group: (row set, route)
  constexpr int L = log2i<V>();
  static_assert(NCH == 4 || NCH == 6 || NCH == 8, "the ring reads four, six or eight chunks per group");
  static_assert(V <= 16, "at most four row sets per group");
  static_assert(NST >= 2 && NST <= 4, "two to four ring stages");
  using LD = QmfLds<NCH, UPG, NST>;
  // cache policies of the weight chunk and scale loads: the non-temporal policy
  // where it measured faster (int8 chunks: int8 decode layer -3.7%; int4
  // scales: int4 decode layer -1.5%); each measured slower or no faster on the
  // other format (int4 chunks: -0.5% to -2.8% with the last-level cache
  // flushed before each layer, +1.2% to +2.5% without)
  constexpr int W_AUX = I8 ? kLoadStream : 0, S_AUX = I8 ? 0 : kLoadStream;
  // SV: one scale per chunk and 4 or 8 slots, so a row set's scales are blocks of
  // 64 floats per row, loaded 16 bytes per lane (S / 4 loads per row set instead
  // of S); lane 16 t' + j fetches row t', floats 4 (j ^ 4 t') .. + 3 of a block
  constexpr bool SV = FULL && S % 4 == 0 && NCH == 8;
  static_assert(!RS || (!FULL && NCH == 8 && R <= 2), "row scales: eight slots in one or two row sets");
  constexpr int NDMA = NCH + (SV ? NCH / 4 : RS ? R : NCH);  // DMA instructions per group
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  int r_lo = 0, r_hi = 0;
  const int e = nth_active_pass(offsets, n_experts, max_rows, blockIdx.y, &r_lo, &r_hi);  // at most 4 rows
  if (e < 0) return;
  const int lane = threadIdx.x;
  const int blk = lane >> 2, t = lane & 3;
  const int n_groups = (n_out + UPG - 1) / UPG;
  const int g_first = blockIdx.x * gpw;
  if (g_first >= n_groups) return;
  const int g_end = min(g_first + gpw, n_groups);
  char* const ring = smem;
  float* const staged = reinterpret_cast<float*>(smem + LD::STAGES * LD::STAGE);
  const int KC = K / CW;
  const int cpg = static_cast<int>(wa.group / CW);  // chunks per quantisation group
  // Loads are coalesced: lane 16 t' + j fetches row t' of the row set, chunk
  // 16 s + (j ^ 4 t'), so each quad of lanes reads 64 contiguous bytes; the
  // chunk lands at ring slot 16 t' + j, and lane (b, t) reads row t, chunk b
  // from slot 16 t + (b ^ 4 t) (16 lanes in a row cover all 16 slot offsets: no
  // bank conflicts).
  // (with SV, ld_blk is also the loading lane's group of 4 scales in a block)
  const int ld_row = lane >> 4, ld_blk = (lane & 15) ^ (4 * ld_row);
  const int rd_slot = 16 * t + (blk ^ (4 * t));
  // the loading lane's matrix: gate/up row sets alternate gate (even) and up (odd) rows
  const bool up_row = GATEUP && (ld_row & 1);
  const uint8_t* const wbase =
      static_cast<const uint8_t*>(up_row ? wb.w : wa.w) + e * (up_row ? wb.expert_elems : wa.expert_elems);
  const float* const sbase = (up_row ? wb.scales : wa.scales) + e * (up_row ? wb.expert_scales : wa.expert_scales);
  const int64_t wstride = wa.row_stride;  // bytes per stored row
  const int sstride = static_cast<int>(wa.groups);
  // chunk and scale index of slot s for the loading lane (chunks past the row end
  // are loaded, never used); FULL: one scale per chunk and no clamping
  int cidx[FULL ? 1 : S], sidx[FULL ? 1 : S];
  if constexpr (!FULL) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      cidx[s] = min(16 * s + ld_blk, KC - 1);
      sidx[s] = cidx[s] / cpg;
    }
  }
  auto chunk_of = [&](int s) {
    if constexpr (FULL) return 16 * s + ld_blk;
    else return cidx[s];
  };
  auto scale_of = [&](int s) {
    if constexpr (FULL) return 16 * s + ld_blk;
    else return sidx[s];
  };
  const int addr32 = (lane ^ 32) << 2;

  // DMA of group g into its ring stage
  auto issue = [&](int g) {
    char* st = ring + ((g - g_first) % LD::STAGES) * LD::STAGE;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int n = min(GATEUP ? g * UPG + 2 * r + (ld_row >> 1) : g * UPG + 4 * r + ld_row, n_out - 1);
      const uint8_t* wrow = wbase + static_cast<int64_t>(n) * wstride;
      const float* srow = sbase + static_cast<int64_t>(n) * sstride;
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const int q = r * S + s;
        __builtin_amdgcn_global_load_lds(static_cast<const void*>(wrow + 16 * chunk_of(s)),
                                         (lds_void*)(st + q * 1024), 16, 0, W_AUX);
        if constexpr (!SV && !RS)
          __builtin_amdgcn_global_load_lds(static_cast<const void*>(srow + scale_of(s)),
                                           (lds_void*)(st + NCH * 1024 + q * 256), 4, 0, S_AUX);
      }
      if constexpr (RS)  // the loading lane's row scale, once for the row set
        __builtin_amdgcn_global_load_lds(static_cast<const void*>(srow), (lds_void*)(st + NCH * 1024 + r * 256), 4,
                                         0, S_AUX);
      if constexpr (SV) {
#pragma unroll
        for (int ib = 0; ib < S / 4; ++ib)
          __builtin_amdgcn_global_load_lds(static_cast<const void*>(srow + 64 * ib + 4 * ld_blk),
                                           (lds_void*)(st + NCH * 1024 + (r * (S / 4) + ib) * 1024), 16, 0, S_AUX);
      }
    }
  };

  for (int m0 = r_lo; m0 < r_hi; m0 += 4) {
    const int M = min(4, r_hi - m0);
    const bool live = t < M;  // this lane's route exists
    // The pass's row indices are read with uniform addresses through a
    // read-only view (scalar loads, counted apart from the vector memory
    // loads): the ring's first groups are requested while they are in
    // flight, and the activation loads after them need not wait for those
    // groups.  (Read as vector loads, the compiler's wait for the row index
    // after the conditional ring requests was vmcnt(0), which also waited
    // for the first weight groups.)
    typedef __attribute__((address_space(4))) const int32_t* const_i32;
    auto issue_first = [&]() {
#pragma unroll
      for (int i = 0; i < LD::STAGES - 1; ++i)
        if (g_first + i < g_end) issue(g_first + i);
    };
    int xr;
    if (row_index != nullptr) {
      const const_i32 ri = (const_i32)row_index;
      int xr4[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) xr4[i] = ri[__builtin_amdgcn_readfirstlane(min(m0 + i, r_hi - 1))];
      issue_first();
      xr = live ? (t == 0 ? xr4[0] : t == 1 ? xr4[1] : t == 2 ? xr4[2] : xr4[3]) : 0;
    } else {
      issue_first();
      xr = live ? m0 + t : 0;
    }
    // ---- activations of route t for this lane's chunks, in the operand order of the codes ----
    uint2 xa[S][NMF];  // A operands: per chunk NMF instructions of 4 activations
    float cz[S];       // this route's bias term per chunk
    float inv_own = 1.0f;  // int8: 1 / sigma of this lane's route
    if constexpr (!I8) {
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const bool ok = live && 16 * s + blk < KC;
        const int c = min(16 * s + blk, KC - 1);
        const uint4* src = reinterpret_cast<const uint4*>(x + static_cast<int64_t>(xr) * K + 32 * c);
        float z = 0.0f;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const uint4 v = ok ? src[p] : make_uint4(0u, 0u, 0u, 0u);  // pairs (0,1) (2,3) (4,5) (6,7)
          // (0, 2, 4, 6) and (1, 3, 5, 7): the order of the code pairs below
          xa[s][2 * p] =
              make_uint2(__builtin_amdgcn_perm(v.y, v.x, 0x05040100u), __builtin_amdgcn_perm(v.w, v.z, 0x05040100u));
          xa[s][2 * p + 1] =
              make_uint2(__builtin_amdgcn_perm(v.y, v.x, 0x07060302u), __builtin_amdgcn_perm(v.w, v.z, 0x07060302u));
          const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int h = 0; h < 4; ++h)  // + x[2h] + x[2h+1]
            z = ACT == QW_F16 ? dot2_f16(vv[h], 0x3c003c00u, z) : dot2_bf16(vv[h], 0x3f803f80u, z);
        }
        cz[s] = -(ACT == QW_F16 ? 1032.0f : 136.0f) * z;
      }
    } else {
      // int8: fp16 operands; bf16 activations are scaled by sigma, the power of two
      // per route bringing its largest |x| into [2^14, 2^15), where they are exact
      // in fp16 (fp16 activations are used as they are)
      uint4 raw[S][2];
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const bool ok = live && 16 * s + blk < KC;
        const int c = min(16 * s + blk, KC - 1);
        const uint4* src = reinterpret_cast<const uint4*>(x + static_cast<int64_t>(xr) * K + 16 * c);
#pragma unroll
        for (int p = 0; p < 2; ++p) raw[s][p] = ok ? src[p] : make_uint4(0u, 0u, 0u, 0u);
      }
      float sigma = 1.0f;
      if constexpr (ACT == QW_BF16) {
        float amax = 0.0f;
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
          for (int p = 0; p < 2; ++p) {
            const uint32_t v[4] = {raw[s][p].x, raw[s][p].y, raw[s][p].z, raw[s][p].w};
#pragma unroll
            for (int h = 0; h < 4; ++h)
              amax = fmaxf(amax, fmaxf(fabsf(__uint_as_float(v[h] << 16)), fabsf(__uint_as_float(v[h] & 0xffff0000u))));
          }
        // the route's largest |x|: the lanes with the same t hold the same route
        amax = fmaxf(amax, xor_lane<4>(amax, addr32));
        amax = fmaxf(amax, xor_lane<8>(amax, addr32));
        amax = fmaxf(amax, xor_lane<16>(amax, addr32));
        amax = fmaxf(amax, xor_lane<32>(amax, addr32));
        int ex = 0;
        frexpf(amax, &ex);  // amax in [2^(ex-1), 2^ex)
        sigma = amax > 0.0f ? ldexpf(1.0f, min(15 - ex, 126)) : 1.0f;  // at most 2^126, as above
        inv_own = 1.0f / sigma;
      }
#pragma unroll
      for (int s = 0; s < S; ++s) {
        uint32_t h2[8];  // fp16 pairs (0,1) .. (14,15)
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const uint32_t v[4] = {raw[s][p].x, raw[s][p].y, raw[s][p].z, raw[s][p].w};
#pragma unroll
          for (int h = 0; h < 4; ++h) {
            if constexpr (ACT == QW_F16) {
              h2[4 * p + h] = v[h];
            } else {
              const _Float16 lo = static_cast<_Float16>(__uint_as_float(v[h] << 16) * sigma);
              const _Float16 hi = static_cast<_Float16>(__uint_as_float(v[h] & 0xffff0000u) * sigma);
              h2[4 * p + h] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, lo)) |
                              (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, hi)) << 16);
            }
          }
        }
        float z = 0.0f;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          xa[s][p] = make_uint2(h2[2 * p], h2[2 * p + 1]);
          z = dot2_f16(h2[2 * p], 0x3c003c00u, z);
          z = dot2_f16(h2[2 * p + 1], 0x3c003c00u, z);
        }
        cz[s] = -1152.0f * z;  // fp16 codes 1024 + u, u = q + 128
      }
    }
    const int idx = (lane >> (6 - L)) & (V - 1);  // value this lane holds after the reduction
    const int rset = idx >> 2, route = idx & 3;
    const bool lead = ((lane >> 2) & ((1 << (4 - L)) - 1)) == 0;  // first of the lanes holding this value
    // 1 / sigma of the route this lane's value belongs to (1 for int4)
    float inv_mine = 1.0f;
    if constexpr (I8 && ACT == QW_BF16) {
      const float q0 = quad_bcast<0>(inv_own), q1 = quad_bcast<1>(inv_own), q2 = quad_bcast<2>(inv_own),
                  q3 = quad_bcast<3>(inv_own);
      inv_mine = route == 0 ? q0 : route == 1 ? q1 : route == 2 ? q2 : q3;
    }

    // ---- the groups ----
    for (int g = g_first; g < g_end; ++g) {
      // keep STAGES - 1 groups in flight; wait until group g has landed (loads complete in order)
      if (g + LD::STAGES - 1 < g_end) issue(g + LD::STAGES - 1);
      const int after = min(LD::STAGES - 1, g_end - 1 - g);  // groups issued after g
      if (after >= 3) wait_vmcnt<3 * NDMA>();
      else if (after == 2) wait_vmcnt<2 * NDMA>();
      else if (after == 1) wait_vmcnt<NDMA>();
      else wait_vmcnt<0>();
      const char* st = ring + ((g - g_first) % LD::STAGES) * LD::STAGE;
      uint4 wq[8];
      float sq[8];
      const uint32_t wa_l = lds_addr(st) + rd_slot * 16, sa_l = lds_addr(st + NCH * 1024) + rd_slot * 4;
      if constexpr (SV) {
        // scale of chunk 16 s + b of row t: block q >> 2, float group 4 (s & 3) + b / 4, read by
        // lane 16 t + (group ^ 4 t), i.e. at 256 t + 64 ((q & 3) ^ t) + 4 b (no bank conflicts)
        const uint32_t sb = lds_addr(st + NCH * 1024) + 256 * t + 4 * blk;
        const uint32_t sa[4] = {sb + 64 * (0 ^ t), sb + 64 * (1 ^ t), sb + 64 * (2 ^ t), sb + 64 * (3 ^ t)};
        ring_read8_sv(wa_l, sa, wq, sq);
      } else if constexpr (RS) {
        ring_read8_rs<R>(wa_l, sa_l, wq, sq);
      } else if constexpr (NCH == 8) {
        ring_read8<true>(wa_l, sa_l, wq, sq);
      } else if constexpr (NCH == 6) {
        ring_read6(wa_l, sa_l, wq, sq);
      } else {
        uint4 w4[4];
        float s4[4];
        ring_read4<true>(wa_l, sa_l, w4, s4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          wq[i] = w4[i];
          sq[i] = s4[i];
        }
      }
      float acc[V];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        gf32x4 a4 = gf32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < S; ++s) {
          const int q = r * S + s;
          const uint32_t wd[4] = {wq[q].x, wq[q].y, wq[q].z, wq[q].w};
          gf32x4 d = gf32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int p = 0; p < 4; ++p) {
            constexpr uint32_t HB = MT == QW_F16 ? 0x64646464u : 0x43434343u;
            if constexpr (I8) {  // codes 4p..4p+3 as fp16 1024 + u, u = q ^ 0x80
              const uint32_t u = wd[p] ^ 0x80808080u;
              const uint2 b = make_uint2(__builtin_amdgcn_perm(HB, u, 0x04010400u), __builtin_amdgcn_perm(HB, u, 0x04030402u));
              d = mfma4<MT>(xa[s][p], b, d);
            } else {
              const uint32_t lo = wd[p] & 0x0F0F0F0Fu, hi = (wd[p] >> 4) & 0x0F0F0F0Fu;
              const uint2 b0 =
                  make_uint2(__builtin_amdgcn_perm(HB, lo, 0x04010400u), __builtin_amdgcn_perm(HB, lo, 0x04030402u));
              const uint2 b1 =
                  make_uint2(__builtin_amdgcn_perm(HB, hi, 0x04010400u), __builtin_amdgcn_perm(HB, hi, 0x04030402u));
              d = mfma4<MT>(xa[s][2 * p], b0, d);
              d = mfma4<MT>(xa[s][2 * p + 1], b1, d);
            }
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) a4[i] = __builtin_fmaf(sq[q], d[i], a4[i]);
          // bias: D[i][j] += (route i's chunk term) * (row j's scale), the 16 blocks at once
          a4 = __builtin_amdgcn_mfma_f32_4x4x1f32(cz[s], sq[q], a4, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[4 * r + i] = a4[i];
      }
      rs_blocks<V, V, 32>(acc, lane, addr32);
      const float val = acc[0] * inv_mine;
      float* slot = staged + (g - g_first) * (UPG * 4);
      if constexpr (GATEUP) {
        const float up = __uint_as_float(dpp_u32<kDppXor1>(__float_as_uint(val)));  // the up row of the same unit
        if (lead && !(t & 1)) slot[(2 * rset + (t >> 1)) * 4 + route] = swiglu_act<ACT>(val, up);
      } else {
        if (lead) slot[(4 * rset + t) * 4 + route] = val;
      }
    }
    // ---- outputs of the pass: value v = (group, unit, route) of the staging area ----
    const int n_vals = (g_end - g_first) * UPG * 4;
    for (int v = lane; v < n_vals; v += 64) {
      const int gi = v / (UPG * 4), rem = v % (UPG * 4);
      const int u = rem >> 2, m = rem & 3;
      const int n = (g_first + gi) * UPG + u;
      if (m >= M || n >= n_out) continue;
      const int srow = m0 + m;
      const float val = staged[v];
      const int64_t o = static_cast<int64_t>(srow) * n_out + n;
      if constexpr (GATEUP) {
        out[o] = f32_to_half<ACT>(val);
      } else {
        const float wgt = row_weight ? row_weight[srow] : 1.0f;
        out[o] = f32_to_half<ACT>(round_act<ACT>(val) * wgt);
      }
    }
  }
}

// Groups per wave: with 6*4096 groups or more over the touched experts (at
// most one per row), 6 for gate/up and 4 for down (the fastest of 3, 4, 6 and 8
// on the int4 and int8 decode layers); below that fewer, so that about 2048
// waves or more (8 per CU) stream the weights, each with its groups in flight
// at once.
static int groups_per_wave(int64_t touched, int64_t n_groups, bool gateup) {
  const int64_t total = touched * n_groups;
  if (total >= 6 * 4096) return gateup ? 6 : 4;
  if (total >= 8192) return 4;
  if (total >= 4096) return 2;
  return 1;
}

template <int ACT, int WF, bool GATEUP, int UNITS, int CPL, bool SAVE>
int launch_save(const FfnArgs& a, const WView& wa, const WView& wb, const void* x, const int32_t* row_index, int K,
                int n_out, const float* row_weight, void* out, void* save_a, void* save_b, hipStream_t stream) {
  // routes per pass: int4 activation pieces are 4x larger per chunk than bf16 ones
  constexpr int MAXM = WF == QW_U4 ? 2 : 4;
  using LD = GvLds<WF, UNITS, GATEUP ? 2 : 1, CPL, MAXM, SAVE>;
  constexpr size_t lds = static_cast<size_t>(GV_WAVES) * LD::WAVE;
  auto kernel = ffn_gemv_kernel<ACT, WF, GATEUP, UNITS, CPL, MAXM, SAVE>;
  const hipError_t attr =
      reserve_lds<ffn_gemv_kernel<ACT, WF, GATEUP, UNITS, CPL, MAXM, SAVE>>(static_cast<int>(lds));
  if (attr != hipSuccess)
    return set_error(QW_ERR_HIP, "cannot reserve %zu bytes of LDS: %s", lds, hipGetErrorString(attr));
  const int64_t n_groups = ceil_div(n_out, UNITS);
  const int64_t touched = a.max_rows < a.experts ? a.max_rows : a.experts;
  const int gpw = groups_per_wave(touched, n_groups, GATEUP);
  const int64_t waves = ceil_div(n_groups, gpw);
  const dim3 grid(static_cast<unsigned>(ceil_div(waves, GV_WAVES)), static_cast<unsigned>(touched));
  kernel<<<grid, GV_WAVES * 64, lds, stream>>>(static_cast<const uint16_t*>(x), row_index, a.offsets,
                                               static_cast<int>(a.experts), static_cast<int>(a.max_rows), wa, wb, K,
                                               n_out, gpw, row_weight, static_cast<uint16_t*>(out),
                                               static_cast<uint16_t*>(save_a), static_cast<uint16_t*>(save_b));
  QW_LAUNCH_CHECK(GATEUP ? "ffn_gemv_kernel<gateup>" : "ffn_gemv_kernel<down>");
  return QW_OK;
}

// The saving variants exist for 16-bit weights only (quantised experts do not train).
template <int ACT, int WF, bool GATEUP, int UNITS, int CPL>
int launch_one(const FfnArgs& a, const WView& wa, const WView& wb, const void* x, const int32_t* row_index, int K,
               int n_out, const float* row_weight, void* out, void* save_a, void* save_b, hipStream_t stream) {
  if constexpr (!quantized(WF)) {
    if (save_a)
      return launch_save<ACT, WF, GATEUP, UNITS, CPL, true>(a, wa, wb, x, row_index, K, n_out, row_weight, out, save_a,
                                                       save_b, stream);
  }
  return launch_save<ACT, WF, GATEUP, UNITS, CPL, false>(a, wa, wb, x, row_index, K, n_out, row_weight, out, nullptr,
                                                    nullptr, stream);
}

// Passes that uniform routing of m rows over E experts makes on average:
// E * sum_r P(r) ceil(r / 4), r ~ Binomial(m, 1 / E); at least 1.
static double expected_passes(int64_t E, int64_t m) {
  if (E <= 1) return std::max<double>(1.0, static_cast<double>((m + 3) / 4));
  const double p = 1.0 / static_cast<double>(E);
  double pr = std::pow(1.0 - p, static_cast<double>(m));  // P(r = 0)
  double sum = 0.0;
  for (int64_t r = 1; r <= m; ++r) {
    pr *= static_cast<double>(m - r + 1) / static_cast<double>(r) * p / (1.0 - p);
    sum += pr * static_cast<double>((r + 3) / 4);
    if (static_cast<double>(r) > 4.0 * static_cast<double>(m) * p + 64.0 && pr < 1e-15) break;
  }
  return std::max(1.0, static_cast<double>(E) * sum);
}

// The int4 matrix-core kernel for one projection: S chunk slots per lane cover
// rows of up to 16 S chunks; R row sets per group keep 4 to 8 chunk loads per
// lane and group.
// Two ring stages: 3 and 4 stages cost waves per CU and measured slower.
constexpr int kQmfStages = 2;

template <int ACT, int WF, bool GATEUP, int S, bool FULL, bool RS = false, int NST = kQmfStages>
int launch_qmf_s(const FfnArgs& a, const WView& wa, const WView& wb, const void* x, const int32_t* row_index, int K,
                  int n_out, const float* row_weight, void* out, hipStream_t stream) {
  constexpr int R = S <= 2 ? 4 : S <= 4 ? 2 : 1;
  constexpr int UPG = GATEUP ? 2 * R : 4 * R;
  using LD = QmfLds<S * R, UPG, NST>;
  auto kernel = ffn_qmf_kernel<ACT, WF, GATEUP, S, R, FULL, NST, RS>;
  const hipError_t attr = reserve_lds<ffn_qmf_kernel<ACT, WF, GATEUP, S, R, FULL, NST, RS>>(LD::BYTES);
  if (attr != hipSuccess)
    return set_error(QW_ERR_HIP, "cannot reserve %d bytes of LDS: %s", LD::BYTES, hipGetErrorString(attr));
  const int64_t n_groups = ceil_div(n_out, UPG);
  const int64_t touched = a.max_rows < a.experts ? a.max_rows : a.experts;
  // Blocks per pass (up to 4 rows of one expert): at most (max_rows + 3
  // touched) / 4 passes, as an expert with r rows has ceil(r / 4) <= (r + 3) / 4.
  const int64_t passes = (a.max_rows + 3 * touched) / 4;
  // Groups per wave: about one round of waves over the device's slots for this
  // kernel (waves per CU as its LDS and registers allow), for the passes that
  // uniform routing of max_rows rows makes on average; a grid of 1.3 to 1.6
  // rounds left the last round partly empty (int4 decode layer: expert stage
  // 53.9 us against 56.2 us with 6 groups per wave; int8 decode layer, down
  // projection: 84.4 us against 88.1 us).  int8 gate/up keeps 6 (several
  // rounds of shorter waves measured faster on its decode layer: 96.1 us
  // against 101.2 us with one round).  Small layers keep the fewer, shorter
  // waves of groups_per_wave.
  int gpw = groups_per_wave(touched, n_groups, GATEUP);
  if (touched * n_groups >= 8192 && WF == QW_I8 && GATEUP) {
    gpw = 6;
  } else if (touched * n_groups >= 8192) {
    // per instantiation and device: waves of this kernel the device holds at
    // once.  A read-only cache filled on first use; threads that race to fill
    // it compute and store the same value (atomics: no torn or unordered access).
    static std::atomic<int> slot_cache[kMaxDevices];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
      return set_error(QW_ERR_HIP, "cannot query the current device");
    int slots = slot_cache[dev].load(std::memory_order_relaxed);
    if (slots == 0) {
      int cus = 0, per_cu = 0;
      if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
          hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 64, LD::BYTES) != hipSuccess || cus <= 0 ||
          per_cu <= 0)
        return set_error(QW_ERR_HIP, "cannot query the occupancy of ffn_qmf_kernel");
      slots = cus * per_cu;
      slot_cache[dev].store(slots, std::memory_order_relaxed);
    }
    const double active = expected_passes(a.experts, a.max_rows);
    const int64_t want = static_cast<int64_t>(std::ceil(active * static_cast<double>(n_groups) / slots));
    gpw = static_cast<int>(want < 2 ? 2 : want > LD::GPW_MAX ? LD::GPW_MAX : want);
  }
  static_assert(LD::GPW_MAX >= 6, "staging holds the groups of one wave");
  if (passes > 65535)
    return set_error(QW_ERR_UNSUPPORTED, "too many rows for the decode kernel (%lld passes)", static_cast<long long>(passes));
  const dim3 grid(static_cast<unsigned>(ceil_div(n_groups, gpw)), static_cast<unsigned>(passes));
  kernel<<<grid, 64, LD::BYTES, stream>>>(static_cast<const uint16_t*>(x), row_index, a.offsets,
                                          static_cast<int>(a.experts), static_cast<int>(a.max_rows), wa, wb, K, n_out,
                                          gpw, row_weight, static_cast<uint16_t*>(out));
  QW_LAUNCH_CHECK(GATEUP ? "ffn_qmf_kernel<gateup>" : "ffn_qmf_kernel<down>");
  return QW_OK;
}

template <int ACT, int WF, bool GATEUP, int S>
int launch_qmf_full(const FfnArgs& a, const WView& wa, const WView& wb, const void* x, const int32_t* row_index, int K,
                    int n_out, const float* row_weight, void* out, hipStream_t stream) {
  constexpr int CW = WF == QW_I8 ? 16 : 32;
  if (K / CW == 16 * S && wa.group == CW)
    return launch_qmf_s<ACT, WF, GATEUP, S, true>(a, wa, wb, x, row_index, K, n_out, row_weight, out, stream);
  constexpr int R = S <= 2 ? 4 : S <= 4 ? 2 : 1;
  if constexpr (S * R == 8 && R <= 2) {
    if (wa.groups == 1 && wb.groups == 1)  // one scale per row
      return launch_qmf_s<ACT, WF, GATEUP, S, false, true>(a, wa, wb, x, row_index, K, n_out, row_weight, out,
                                                           stream);
  }
  return launch_qmf_s<ACT, WF, GATEUP, S, false>(a, wa, wb, x, row_index, K, n_out, row_weight, out, stream);
}

// Quantised rows of up to 128 chunks (4096 int4 or 2048 int8 codes) on the
// matrix cores.
template <int ACT, int WF, bool GATEUP>
int launch_qmf(const FfnArgs& a, const WView& wa, const WView& wb, const void* x, const int32_t* row_index, int K,
               int n_out, const float* row_weight, void* out, hipStream_t stream) {
  const int KC = K / (WF == QW_I8 ? 16 : 32);
#define QW_QMF(S_) launch_qmf_full<ACT, WF, GATEUP, S_>(a, wa, wb, x, row_index, K, n_out, row_weight, out, stream)
  if (KC <= 16) return QW_QMF(1);
  if (KC <= 32) return QW_QMF(2);
  if (KC <= 48) return QW_QMF(3);
  if (KC <= 64) return QW_QMF(4);
  if (KC <= 96) return QW_QMF(6);
  return QW_QMF(8);
#undef QW_QMF
}

// Units per group for a row of CPL chunks per lane: 4 weight chunks (16-byte
// loads) per lane and group (8 for gate/up rows of more than 128 chunks).
template <int ACT, int WF, bool GATEUP>
int launch_cpl(const FfnArgs& a, const WView& wa, const WView& wb, const void* x, const int32_t* row_index, int K,
               int n_out, const float* row_weight, void* out, void* save_a, void* save_b, hipStream_t stream) {
  const int KC = K / Fmt<WF>::CW;
  const int cpl = static_cast<int>(ceil_div(KC, 64));
  constexpr int U1 = GATEUP ? 2 : 4;
  if (cpl <= 1)
    return launch_one<ACT, WF, GATEUP, U1, 1>(a, wa, wb, x, row_index, K, n_out, row_weight, out, save_a, save_b, stream);
  if (cpl <= 2)
    return launch_one<ACT, WF, GATEUP, U1 / 2, 2>(a, wa, wb, x, row_index, K, n_out, row_weight, out, save_a, save_b,
                                             stream);
  if (cpl <= 4)
    return launch_one<ACT, WF, GATEUP, 1, 4>(a, wa, wb, x, row_index, K, n_out, row_weight, out, save_a, save_b, stream);
  return set_error(QW_ERR_UNSUPPORTED, "row of %d chunks is too long for the decode kernel", KC);
}

template <int ACT, int WF>
int launch_fmt(const FfnArgs& a, hipStream_t stream) {
  const int D = static_cast<int>(a.d_model), F = static_cast<int>(a.d_ff);
  // quantised rows of up to 128 chunks (4096 int4 or 2048 int8 codes) take the matrix-core kernel
  constexpr int KMAX = WF == QW_I8 ? 2048 : WF == QW_U4 ? 4096 : 0;
  int st;
  if constexpr (KMAX > 0) {
    st = D <= KMAX ? launch_qmf<ACT, WF, true>(a, a.gate, a.up, a.x, a.row_index, D, F, nullptr, a.hidden, stream)
                   : launch_cpl<ACT, WF, true>(a, a.gate, a.up, a.x, a.row_index, D, F, nullptr, a.hidden, nullptr,
                                               nullptr, stream);
    if (st) return st;
    return F <= KMAX ? launch_qmf<ACT, WF, false>(a, a.down, a.down, a.hidden, nullptr, F, D, a.row_weight, a.y, stream)
                     : launch_cpl<ACT, WF, false>(a, a.down, a.down, a.hidden, nullptr, F, D, a.row_weight, a.y, nullptr,
                                                  nullptr, stream);
  } else {
    st = launch_cpl<ACT, WF, true>(a, a.gate, a.up, a.x, a.row_index, D, F, nullptr, a.hidden, a.save_gate, a.save_up,
                                   stream);
    if (st) return st;
    return launch_cpl<ACT, WF, false>(a, a.down, a.down, a.hidden, nullptr, F, D, a.row_weight, a.y, a.save_y, nullptr,
                                      stream);
  }
}

}  // namespace

int launch_ffn_gemv(const FfnArgs& a, hipStream_t stream, bool* handled) {
  *handled = false;
  if (!is_half(a.act) || a.avg_rows >= 16) return QW_OK;
  const bool f16 = a.act == QW_F16;
  if ((a.save_gate || a.save_y) && quantized(a.wfmt)) return QW_OK;  // quantised experts do not train
  // the matrix-core decode kernel's grid has a row per pass of up to 4 routes:
  // more than a grid dimension holds go to the other kernel families
  const int64_t touched = a.max_rows < a.experts ? a.max_rows : a.experts;
  if (quantized(a.wfmt) && (a.max_rows + 3 * touched) / 4 > 65535) return QW_OK;
  int cw = 0;
  if (a.wfmt == QW_U4) {
    if (a.gate.group % 32 || a.down.group % 32) return QW_OK;
    cw = 32;
  } else if (a.wfmt == QW_I8) {
    if (a.gate.group % 16 || a.down.group % 16) return QW_OK;
    cw = 16;
  } else if ((!f16 && (a.wfmt == QW_BF16 || a.wfmt == QW_BF16T)) || (f16 && (a.wfmt == QW_F16 || a.wfmt == QW_F16T))) {
    cw = 8;
  } else {
    return QW_OK;
  }
  if (a.d_model % cw || a.d_ff % cw) return QW_OK;
  if (ceil_div(a.d_model / cw, 64) > 4 || ceil_div(a.d_ff / cw, 64) > 4) return QW_OK;
  // the padded int4/int8 row must equal the logical row (true when K is a multiple of the group)
  if (quantized(a.wfmt) && (a.gate.row_stride * (a.wfmt == QW_U4 ? 2 : 1) != a.d_model ||
                            a.down.row_stride * (a.wfmt == QW_U4 ? 2 : 1) != a.d_ff))
    return QW_OK;
  int st;
  if (f16) {
    if (a.wfmt == QW_U4) st = launch_fmt<QW_F16, QW_U4>(a, stream);
    else if (a.wfmt == QW_I8) st = launch_fmt<QW_F16, QW_I8>(a, stream);
    else if (a.wfmt == QW_F16T) st = launch_fmt<QW_F16, QW_F16T>(a, stream);
    else st = launch_fmt<QW_F16, QW_F16>(a, stream);
  } else {
    if (a.wfmt == QW_U4) st = launch_fmt<QW_BF16, QW_U4>(a, stream);
    else if (a.wfmt == QW_I8) st = launch_fmt<QW_BF16, QW_I8>(a, stream);
    else if (a.wfmt == QW_BF16T) st = launch_fmt<QW_BF16, QW_BF16T>(a, stream);
    else st = launch_fmt<QW_BF16, QW_BF16>(a, stream);
  }
  if (st) return st;
  *handled = true;
  return QW_OK;
}

}  // namespace qw
