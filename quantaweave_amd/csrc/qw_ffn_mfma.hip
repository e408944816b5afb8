// Grouped SwiGLU expert FFN on 16-bit MFMA (v_mfma_f32_16x16x32_bf16, or
// v_mfma_f32_16x16x32_f16 for fp16 activations; gfx950) for prefill-sized rows
// per expert.
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
//
// Operands move HBM/L2 -> LDS with global_load_lds_dwordx4 (no register
// staging) in K-slices of 64 (two MFMA K steps) through rings of two or three
// stages (three when the row chunk leaves room in the 160 KiB of LDS), the
// next slices requested right after each slice's barrier so they are in
// flight during the MFMAs.  One LDS barrier per slice.  A load group is eight
// whole 128-byte row segments (one KiB), so every request is full cache lines;
// QW_BF16T weights come pre-arranged in exactly those KiB tiles and stream
// contiguously; 16-bit weights, whose lines each slice consumes whole, are read
// with the non-temporal cache policy (measured: headline layer 278 -> 265 us),
// so they do not push the activation rows out of the caches.  Loads complete in
// issue order and every wave issues the same
// loads per slice (rows past the end are clamped to a valid row, their results
// never stored), so a fixed `s_waitcnt vmcnt(n)` marks a slice as landed.
//
// LDS rows are 128 bytes (64 bf16); the eight 16-byte pieces of row r are
// stored XOR-swizzled by ((r >> 1) & 7) so the 16-row fragment reads of the
// MFMAs hit distinct banks.  Within a slice the fragment reads are pipelined
// behind the MFMAs (two activation pair buffers, weight fragments per K step),
// with the order pinned by scheduling barriers.
//
// Waves form a 2 x 4 grid: wave (wm, wn) computes row sub-tiles wm, wm+2, ...
// (16 rows each) against its 64 weight rows (GATEUP: 32 gate rows and the
// matching 32 up rows, so SiLU(g)*u is formed in registers).  Sub-tiles go in
// pairs; a pair wholly past the expert's row count is not multiplied (the K
// loop is instantiated per number of active pairs), and the rows past the
// count inside a live pair run on clamped copies of a valid row and are not
// stored.  The MFMA takes the weights as its A operand, so a
// lane ends up holding 4 consecutive output columns of one row and stores them
// with one 8-byte write.
//
// Quantised weights (QW_I8, QW_U4; src/quantization.py:61-72) take the same
// path: the slice's stored bytes (64 or 32 per weight row) and its two scales
// per row (one per MFMA K step; the group size is a multiple of 32) stream into
// LDS the same way, and each wave turns its weight fragments into bf16 as it
// reads them: w = bf16(q * scale), the fp32 product rounded once, which is
// exactly the reference's `dequantize().to(bfloat16)`.  The stored value
// u = q + bias (bias 128 after flipping the int8 sign bit, 8 for int4 nibbles)
// is converted to fp32 and fma(u, s, -bias*s) gives q*s with one rounding
// (bias*s is a power-of-two multiple of s, so exact).  No bf16 copy of the
// weights is made.
//
// Workgroup -> tile order is XCD-aware: workgroups are dispatched round-robin
// over the 8 XCDs, so block b runs on XCD b%8; all tiles of one expert are
// given to one XCD and enumerated column-fastest, which keeps the expert's
// activation rows (and a second row chunk's weights) in that XCD's L2.
#include <type_traits>

#include "qw_ffn.h"

namespace qw {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));  // 16-bit operands (bf16 or fp16 bits)
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int MF_BK = 64;       // K slice: two MFMA K steps
constexpr int MF_ROWB = 128;    // bytes per LDS row (64 bf16, no padding: swizzled)
constexpr int MF_GROWS = 8;     // rows per 1 KiB load group (8 lanes per 128-byte row)
constexpr int MF_NB = 256;      // weight rows per column tile
constexpr int MF_THREADS = 512;
constexpr int MF_WAVES = 8;
constexpr int MF_NT = 4;        // 16-column MFMA tiles per wave
constexpr int MF_LDS = 160 * 1024;  // LDS per workgroup

// Weight stage of one K slice per weight format: 256 rows of ROWB bytes (64
// columns), rows XOR-swizzled by 16-byte piece, then (quantised formats) two
// fp32 scales per row.  A 1 KiB load group covers GROWS whole rows.
template <int WF>
struct MfB {
  static constexpr bool Q = WF == QW_I8 || WF == QW_U4;
  static constexpr int ROWB = WF == QW_I8 ? 64 : WF == QW_U4 ? 32 : MF_ROWB;
  static constexpr int W_STAGE = MF_NB * ROWB;
  static constexpr int S_STAGE = Q ? MF_NB * 2 * 4 : 0;
  static constexpr int STAGE = W_STAGE + S_STAGE;
  static constexpr int LPR = ROWB / 16;     // lanes (16-byte pieces) per row
  static constexpr int GROWS = 64 / LPR;    // rows per load group
  static constexpr int BL = W_STAGE / 1024 / MF_WAVES;  // weight load groups per wave
  static constexpr int SL = Q ? 1 : 0;      // scale loads per wave (256 bytes each)
  // physical piece of logical piece p in row r: the 16 rows of a fragment read
  // spread over distinct banks
  static __device__ __forceinline__ int swz(int r, int p) {
    if constexpr (WF == QW_I8) return p ^ ((r >> 2) & 3);
    else if constexpr (WF == QW_U4) return p ^ ((r >> 3) & 1);
    else return p ^ ((r >> 1) & 7);
  }
};

// Ring stages (activation and weight slices together) that fit the LDS, at most
// three; the slices requested ahead are one fewer.
template <int WF>
constexpr int mf_stages(int subt) {
  const int stage = 32 * subt * MF_ROWB + MfB<WF>::STAGE;
  return MF_LDS / stage >= 3 ? 3 : 2;
}

// s_waitcnt immediate waiting for vmcnt <= n only (expcnt, lgkmcnt left at max).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | (((N >> 4) & 3) << 14));
}

// 16-byte piece `piece` (0..7) of LDS row `row` is stored at physical piece
// piece ^ ((row >> 1) & 7): the 16-row fragment reads of an MFMA (one logical
// piece, rows 0..15) then touch 16 distinct bank groups.
__device__ __forceinline__ int swz(int row, int piece) { return piece ^ ((row >> 1) & 7); }

// Barrier for the LDS ring: the slice's loads were already waited for with an
// explicit vmcnt, so no fence is needed (a workgroup fence would wait for every
// load still in flight, including the slices requested ahead).  The empty asm
// statements keep the compiler from moving LDS accesses across the barrier.
__device__ __forceinline__ void ring_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Weights of one projection for the kernel: bytes per expert and per stored
// row; scales (quantised formats) per expert, per row, and the group size.
struct MfW {
  const char* w;
  const float* scales;
  int64_t expert_bytes, row_bytes, expert_scales;
  int groups, group;
};

// One 16x16x32 MFMA step in the activation type: bf16, or fp16 bits carried
// in the same 16-byte operand registers.
template <int ACT>
__device__ __forceinline__ f32x4 mfma_step(bf16x8 a, bf16x8 b, f32x4 c) {
  if constexpr (ACT == QW_F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                   0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Eight fp32 values rounded to the activation type, as 16-bit operand bits.
template <int ACT>
__device__ __forceinline__ bf16x8 pack_act8(const float (&f)[8]) {
  if constexpr (ACT == QW_F16) {
    f16x8 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = static_cast<_Float16>(pin_f32(f[i]));  // fp32 first, then RNE to fp16
    return __builtin_bit_cast(bf16x8, r);
  } else {
    bf16x8 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = static_cast<__bf16>(f[i]);
    return r;
  }
}

// Eight int8 weights (bytes 0..7 = columns c..c+7) -> act(q * s).  The sign
// bit flip stores u = q + 128; fma(u, s, -128 s) = q s rounded once.
template <int ACT>
__device__ __forceinline__ bf16x8 dequant_i8(uint2 raw, float s) {
  const uint32_t u0 = raw.x ^ 0x80808080u, u1 = raw.y ^ 0x80808080u;
  const float c = -128.0f * s;
  float f[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[i] = __builtin_fmaf(static_cast<float>((u0 >> (8 * i)) & 0xffu), s, c);
    f[4 + i] = __builtin_fmaf(static_cast<float>((u1 >> (8 * i)) & 0xffu), s, c);
  }
  return pack_act8<ACT>(f);
}

// Eight int4 weights (byte b: column c+2b in the low nibble, c+2b+1 in the
// high one, each stored as q + 8) -> act(q * s).
template <int ACT>
__device__ __forceinline__ bf16x8 dequant_u4(uint32_t raw, float s) {
  const uint32_t lo = raw & 0x0f0f0f0fu, hi = (raw >> 4) & 0x0f0f0f0fu;
  const float c = -8.0f * s;
  float f[8];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    f[2 * b] = __builtin_fmaf(static_cast<float>((lo >> (8 * b)) & 0xffu), s, c);
    f[2 * b + 1] = __builtin_fmaf(static_cast<float>((hi >> (8 * b)) & 0xffu), s, c);
  }
  return pack_act8<ACT>(f);
}

template <int ACT, bool GATEUP, int SUBT, int WF>
__global__ __launch_bounds__(MF_THREADS) void ffn_mfma_kernel(
    const uint16_t* __restrict__ x, const int32_t* __restrict__ row_index, const int32_t* __restrict__ offsets,
    int max_rows, const MfW wa, const MfW wb, int n_w, int K, const float* __restrict__ row_weight,
    uint16_t* __restrict__ out, int n_out, int n_tiles, int m_chunks, int experts, uint16_t* __restrict__ save_a,
    uint16_t* __restrict__ save_b) {
  using B = MfB<WF>;
  constexpr bool TILED = WF == QW_BF16T || WF == QW_F16T;
  constexpr int MCH = 32 * SUBT;                 // rows per chunk
  constexpr int AG = MCH / MF_GROWS;             // 8-row load groups of the A slice
  constexpr int A_STAGE = MCH * MF_ROWB, B_STAGE = B::STAGE;
  constexpr int AL = AG / MF_WAVES;              // A groups per wave
  constexpr int BL = B::BL, SL = B::SL;          // weight groups and scale loads per wave
  constexpr int BLQ = BL + SL;
  constexpr int ST = mf_stages<WF>(SUBT), AHEAD = ST - 1;
  constexpr int W_AUX = B::Q ? 0 : kLoadStream;  // cache policy of the weight loads
  static_assert(AG % MF_WAVES == 0 && B::W_STAGE % (1024 * MF_WAVES) == 0, "load groups per wave");
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  char* const a_ring = smem;
  char* const b_ring = smem + ST * A_STAGE;

  // ---- tile of this workgroup (XCD-aware enumeration) ----
  const int b = blockIdx.x;
  const int xcd = b % kXcds, j = b / kXcds;
  // XCD x takes the row chunks of experts x, x + 8, ..., each chunk's column
  // tiles back to back.  m_chunks > 0: every expert has m_chunks chunk slots
  // (the capacity bound is tight); m_chunks == 0: the chunks that hold rows
  // are found on the device, so a loose bound (no capacity) costs no launches.
  const int nt = j % n_tiles;
  int mc = 0, e;
  if (m_chunks > 0) {
    e = xcd + kXcds * (j / n_tiles / m_chunks);
    mc = (j / n_tiles) % m_chunks;
    if (e >= experts) return;
  } else {
    e = find_tile(offsets, experts, max_rows, MCH, j / n_tiles, &mc, xcd, kXcds);
    if (e < 0) return;
  }
  const int e_lo = max(offsets[e], 0);
  const int r0 = e_lo + mc * MCH;
  const int r1 = min(min(offsets[e + 1], r0 + MCH), max_rows);
  const int count = r1 - r0;
  if (count <= 0) return;

  const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  const int wm = wave / 4, wn = wave % 4;
  const int n0 = nt * (GATEUP ? MF_NB / 2 : MF_NB);
  const char* wa_e = wa.w + static_cast<int64_t>(e) * wa.expert_bytes;
  const char* wb_e = wb.w + static_cast<int64_t>(e) * wb.expert_bytes;

  // ---- per-lane global sources of this wave's load groups (constant over K) ----
  // lane i of a group writes LDS row (8g + i/8), physical piece i%8, which holds
  // logical piece swz(row, i%8) of that row: each group is 8 whole 128-byte row
  // segments.
  const int lrow = lane / 8, lpiece = lane % 8;
  const uint16_t* a_src[AL];
#pragma unroll
  for (int q = 0; q < AL; ++q) {
    const int g = wave + q * MF_WAVES;
    const int row = MF_GROWS * g + lrow;
    const int rr = min(row, count - 1);  // clamp: rows past the end load a valid row
    const int64_t src = row_index ? row_index[r0 + rr] : (r0 + rr);
    a_src[q] = x + src * K + swz(row, lpiece) * 8;
  }
  // weight row (of the projection) behind LDS weight row `row`
  auto weight_row = [&](int row, bool* second) {
    int wrow;
    if (GATEUP) {
      wrow = n0 + (row % (MF_NB / 2));
      *second = row >= MF_NB / 2;
    } else {
      wrow = n0 + row;
      *second = false;
    }
    return min(wrow, n_w - 1);
  };
  const char* b_src[BL];
#pragma unroll
  for (int q = 0; q < BL; ++q) {
    const int g = wave + q * MF_WAVES;
    const int row = B::GROWS * g + lane / B::LPR;
    bool second;
    const int wrow = weight_row(row, &second);
    const char* base = second ? wb_e : wa_e;
    const int64_t row_bytes = second ? wb.row_bytes : wa.row_bytes;
    // the LDS row's swizzle, (row >> 1) & 7, equals (wrow >> 1) & 7: n0 is a multiple of 128
    if (TILED)  // the group's tile column: tiles [wrow/8][kt], one contiguous KiB each
      b_src[q] = base + static_cast<int64_t>(wrow & ~7) * row_bytes + lane * 16;
    else
      b_src[q] = base + static_cast<int64_t>(wrow) * row_bytes + B::swz(row, lane % B::LPR) * 16;
  }
  // scales: lane i of wave w loads the scale of LDS row (64w + i) / 2 for MFMA
  // K step i % 2 (dword 64w + i of the scale stage)
  const float* s_src = nullptr;
  int s_ks = 0, s_group = 1;
  if constexpr (B::Q) {
    const int idx = wave * 64 + lane;
    bool second;
    const int wrow = weight_row(idx / 2, &second);
    const MfW& v = second ? wb : wa;
    s_src = v.scales + static_cast<int64_t>(e) * v.expert_scales + static_cast<int64_t>(wrow) * v.groups;
    s_ks = idx % 2;
    s_group = v.group;
  }
  auto issue_a = [&](int kt) {
    char* st = a_ring + (kt % ST) * A_STAGE;
    const int k0 = kt * MF_BK;
#pragma unroll
    for (int q = 0; q < AL; ++q) {
      const int g = wave + q * MF_WAVES;
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(a_src[q] + k0), (lds_void*)(st + g * 1024), 16, 0,
                                       0);
    }
  };
  auto issue_b = [&](int kt) {
    char* st = b_ring + (kt % ST) * B_STAGE;
#pragma unroll
    for (int q = 0; q < BL; ++q) {
      const int g = wave + q * MF_WAVES;
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(b_src[q] + kt * (TILED ? 1024 : B::ROWB)),
                                       (lds_void*)(st + g * 1024), 16, 0, W_AUX);
    }
    if constexpr (B::Q)
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(s_src + (kt * MF_BK + 32 * s_ks) / s_group),
                                       (lds_void*)(st + B::W_STAGE + wave * 256), 4, 0, 0);
  };

  f32x4 acc[SUBT][MF_NT];
#pragma unroll
  for (int i = 0; i < SUBT; ++i)
#pragma unroll
    for (int t = 0; t < MF_NT; ++t) acc[i][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  // B rows (in the LDS tile) of this wave's MFMA column tiles; GATEUP: tiles
  // 0..1 gate, 2..3 the matching up rows
  int brow[MF_NT];
#pragma unroll
  for (int t = 0; t < MF_NT; ++t) {
    if (GATEUP) brow[t] = (t < MF_NT / 2 ? 0 : MF_NB / 2) + wn * 32 + (t % (MF_NT / 2)) * 16;
    else brow[t] = wn * 64 + t * 16;
  }
  const int l16 = lane % 16, lq = lane / 16;
  const int active_sub = (count + 15) / 16;  // row sub-tiles holding valid rows (wave-uniform)
  const int KT = K / MF_BK;

  // Iteration kt: wait for slice kt (slices kt+1 .. kt+AHEAD-1 may still be in
  // flight), barrier (slice kt visible; every wave is done with slice kt-1),
  // read the first fragments, request slice kt+AHEAD into the stage of slice
  // kt-1, compute slice kt.
  for (int j = 0; j < AHEAD && j < KT; ++j) {
    issue_a(j);
    issue_b(j);
  }
  static_assert(SUBT % 2 == 0, "sub-tiles come in pairs");
  static_assert(AHEAD >= 1 && AHEAD <= 2 && 2 * (AL + BLQ) < 64, "ring depth");
  constexpr int NP = SUBT / 2;  // pairs of sub-tiles per K step
  // The K loop, for a wave whose first NPA sub-tile pairs hold rows: pairs
  // wholly past the expert's rows are not multiplied (their rows are loaded
  // with the rest and never stored).  Every wave takes part in every load and
  // barrier whatever its NPA.
  auto k_loop = [&](auto npa) {
    constexpr int NPA = decltype(npa)::value;
    for (int kt = 0; kt < KT; ++kt) {
      if (AHEAD == 2 && kt + 1 < KT) wait_vmcnt<AL + BLQ>();
      else wait_vmcnt<0>();
      ring_barrier();
      const char* st_a = a_ring + (kt % ST) * A_STAGE;
      const char* st_b = b_ring + (kt % ST) * B_STAGE;
      auto read_a = [&](int i, int ks) {
        const int row = (wm + 2 * i) * 16 + l16;
        return *reinterpret_cast<const bf16x8*>(st_a + row * MF_ROWB + swz(row, lq + 4 * ks) * 16);
      };
      auto read_b = [&](int t, int ks) -> bf16x8 {
        const int row = brow[t] + l16;
        if constexpr (WF == QW_I8) {  // 8 bytes: columns 32ks + 8lq ..
          const uint2 raw = *reinterpret_cast<const uint2*>(st_b + row * B::ROWB +
                                                            B::swz(row, 2 * ks + lq / 2) * 16 + (lq % 2) * 8);
          return dequant_i8<ACT>(raw, *reinterpret_cast<const float*>(st_b + B::W_STAGE + (row * 2 + ks) * 4));
        } else if constexpr (WF == QW_U4) {  // 4 bytes: columns 32ks + 8lq ..
          const uint32_t raw = *reinterpret_cast<const uint32_t*>(st_b + row * B::ROWB + B::swz(row, ks) * 16 + lq * 4);
          return dequant_u4<ACT>(raw, *reinterpret_cast<const float*>(st_b + B::W_STAGE + (row * 2 + ks) * 4));
        } else {
          return *reinterpret_cast<const bf16x8*>(st_b + row * MF_ROWB + swz(row, lq + 4 * ks) * 16);
        }
      };
      // Units u = 0 .. 2*NP-1 are (K step ks = u / NP, sub-tile pair p = u % NP),
      // with activation fragments in two pair buffers (u & 1) and weight fragments
      // per K step.  The reads of unit u+1 (and, before the second K step, its
      // weight fragments) go out right after the first MFMA of unit u, whose wait
      // covered every earlier read, so seven MFMAs hide them.
      bf16x8 wfr[2][MF_NT];
      bf16x8 xb[2][2];
  #pragma unroll
      for (int t = 0; t < MF_NT; ++t) wfr[0][t] = read_b(t, 0);
      xb[0][0] = read_a(0, 0);
      xb[0][1] = read_a(1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, (B::Q ? 2 : 1) * MF_NT + 2, 0);  // first fragments, then the requests
      if (kt + AHEAD < KT) {
        issue_a(kt + AHEAD);
        issue_b(kt + AHEAD);
      }
  #pragma unroll
      for (int u = 0; u < 2 * NPA; ++u) {
        const int ks = u / NPA, p = u % NPA;
        const bf16x8 x0 = xb[u & 1][0], x1 = xb[u & 1][1];
        acc[2 * p][0] = mfma_step<ACT>(wfr[ks][0], x0, acc[2 * p][0]);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (u + 1 < 2 * NPA) {
          const int ks1 = (u + 1) / NPA, p1 = (u + 1) % NPA;
          if (ks1 != ks) {
  #pragma unroll
            for (int t = 0; t < MF_NT; ++t) wfr[1][t] = read_b(t, 1);
            xb[(u + 1) & 1][0] = read_a(2 * p1, 1);
            xb[(u + 1) & 1][1] = read_a(2 * p1 + 1, 1);
            __builtin_amdgcn_sched_group_barrier(0x100, (B::Q ? 2 : 1) * MF_NT + 2, 0);
          } else {
            xb[(u + 1) & 1][0] = read_a(2 * p1, ks1);
            xb[(u + 1) & 1][1] = read_a(2 * p1 + 1, ks1);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
          }
        }
  #pragma unroll
        for (int t = 1; t < MF_NT; ++t)
          acc[2 * p][t] = mfma_step<ACT>(wfr[ks][t], x0, acc[2 * p][t]);
  #pragma unroll
        for (int t = 0; t < MF_NT; ++t)
          acc[2 * p + 1][t] = mfma_step<ACT>(wfr[ks][t], x1, acc[2 * p + 1][t]);
        __builtin_amdgcn_sched_group_barrier(0x008, 2 * MF_NT - 1, 0);
      }
    }
  };
  // this wave's sub-tiles wm, wm + 2, ...: those below active_sub hold rows
  const int wave_sub = active_sub > wm ? (active_sub - wm + 1) / 2 : 0;
  const int npa = __builtin_amdgcn_readfirstlane((wave_sub + 1) / 2);
  if constexpr (NP >= 4) {  // chunks of 256 and 320 rows
    if (npa >= NP) k_loop(std::integral_constant<int, NP>{});
    else if (npa >= 4) k_loop(std::integral_constant<int, 4>{});
    else if (npa == 3) k_loop(std::integral_constant<int, 3>{});
    else if (npa == 2) k_loop(std::integral_constant<int, 2>{});
    else k_loop(std::integral_constant<int, 1>{});
  } else {
    k_loop(std::integral_constant<int, NP>{});
  }

  // ---- epilogue without route weights or saved copies: the tile goes through
  //      LDS (the ring is free once every wave is past its last slice) and
  //      leaves in whole row segments, 16 bytes per lane (gate/up: 128 columns,
  //      256-byte segments, all rows at once; down: 256 columns, 512-byte
  //      segments, half the rows per pass).  A lane's 8-byte pieces (row l16,
  //      columns 4lq..4lq+3 of each 16-column MFMA tile) land in 16-byte chunk
  //      (col / 8) ^ ((row & 15) << 1) of the row (mod the chunks per row),
  //      so neither the writes nor the row reads repeat a bank more than the
  //      access width requires.  Same values as the direct stores below. ----
  if (row_weight == nullptr && save_a == nullptr && n_out % 8 == 0 &&
      (reinterpret_cast<uintptr_t>(out) & 15) == 0) {
    constexpr int OC = GATEUP ? MF_NB / 2 : MF_NB;  // output columns of the tile
    constexpr int CPR = OC / 8;                     // 16-byte chunks per row
    constexpr int PASSES = GATEUP ? 1 : 2;
    constexpr int PR = MCH / PASSES;                // rows per pass
    static_assert(PR * OC * 2 <= ST * (A_STAGE + B_STAGE), "the staged tile fits the ring");
    static_assert(MCH % (16 * PASSES * 2) == 0, "a pass holds whole sub-tile pairs");
    char* const ot = smem;
    auto chunk_of = [](int row, int col) { return (col / 8) ^ (((row & 15) << 1) & (CPR - 1)); };
#pragma unroll
    for (int pass = 0; pass < PASSES; ++pass) {
      __syncthreads();  // pass 0: every wave is done with the ring; pass 1: the stores of pass 0 read LDS
#pragma unroll
      for (int i = 0; i < SUBT; ++i) {
        const int sub = wm + 2 * i;
        if (sub * 16 < pass * PR || sub * 16 >= (pass + 1) * PR) continue;  // not this pass's rows
        if (sub >= active_sub) continue;
        const int row = sub * 16 + l16, rl = row - pass * PR;
#pragma unroll
        for (int t = 0; t < (GATEUP ? MF_NT / 2 : MF_NT); ++t) {
          const int col = GATEUP ? wn * 32 + t * 16 + 4 * lq : wn * 64 + t * 16 + 4 * lq;
          uint32_t pk[2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            if (GATEUP)
              pk[h] = swiglu_pack2<ACT>(acc[i][t][2 * h], acc[i][t][2 * h + 1], acc[i][t + MF_NT / 2][2 * h],
                                        acc[i][t + MF_NT / 2][2 * h + 1]);
            else
              pk[h] = pack_half2<ACT>(acc[i][t][2 * h], acc[i][t][2 * h + 1]);
          }
          *reinterpret_cast<uint2*>(ot + rl * (OC * 2) + chunk_of(row, col) * 16 + (col % 8) * 2) =
              make_uint2(pk[0], pk[1]);
        }
      }
      __syncthreads();
      // SUBT rounds of 16-byte pieces per thread: every LDS read is issued
      // before the first global store, so the reads' latency is paid once.
      // Pieces of rows past the expert's end are read (inside the staged
      // tile) and not stored.
      constexpr int ROUNDS = PR * CPR / MF_THREADS;
      static_assert(PR * CPR % MF_THREADS == 0, "whole rounds of pieces");
      const int rows = min(count - pass * PR, PR);
      uint4 piece[ROUNDS];
#pragma unroll
      for (int u = 0; u < ROUNDS; ++u) {
        const int c = tid + u * MF_THREADS;
        const int rl = c / CPR, q = c % CPR;
        piece[u] = *reinterpret_cast<const uint4*>(ot + rl * (OC * 2) + chunk_of(pass * PR + rl, q * 8) * 16);
      }
      // the pieces as opaque values: otherwise each read sinks into its
      // store's branch and waits there on its own
#pragma unroll
      for (int u = 0; u < ROUNDS; ++u) asm("" : "+v"(piece[u].x), "+v"(piece[u].y), "+v"(piece[u].z), "+v"(piece[u].w));
#pragma unroll
      for (int u = 0; u < ROUNDS; ++u) {
        const int c = tid + u * MF_THREADS;
        const int rl = c / CPR, q = c % CPR;
        const int col = n0 + q * 8;
        if (rl < rows && col < n_out)
          *reinterpret_cast<uint4*>(out + static_cast<int64_t>(r0 + pass * PR + rl) * n_out + col) = piece[u];
      }
    }
    return;
  }

  // ---- epilogue: lane holds row l16 of the sub-tile, columns 4*lq .. 4*lq+3 of each tile ----
  // DOWN: the route weights of all of this lane's rows are requested together
  // (one memory round trip, not one per sub-tile).
  float row_w[GATEUP ? 1 : SUBT];
  if constexpr (!GATEUP) {
#pragma unroll
    for (int i = 0; i < SUBT; ++i) {
      const int row = min((wm + 2 * i) * 16 + l16, count - 1);
      row_w[i] = row_weight ? row_weight[r0 + row] : 1.0f;
    }
  }
#pragma unroll
  for (int i = 0; i < SUBT; ++i) {
    const int s = wm + 2 * i;
    if (s >= active_sub) continue;
    const int row = s * 16 + l16;
    if (row >= count) continue;
    const int64_t orow = static_cast<int64_t>(r0 + row) * n_out;
    if (GATEUP) {
#pragma unroll
      for (int t = 0; t < MF_NT / 2; ++t) {
        const int col = n0 + wn * 32 + t * 16 + 4 * lq;
        if (col >= n_out) continue;
        uint32_t pk[2];
#pragma unroll
        for (int h = 0; h < 2; ++h)
          // the reference's 16-bit tensors: gate, up and silu(gate) are each
          // rounded to the activation type before the product (src/moe_kernels.py:194)
          pk[h] = swiglu_pack2<ACT>(acc[i][t][2 * h], acc[i][t][2 * h + 1], acc[i][t + MF_NT / 2][2 * h],
                                    acc[i][t + MF_NT / 2][2 * h + 1]);
        *reinterpret_cast<uint2*>(out + orow + col) = make_uint2(pk[0], pk[1]);
        if (save_a) {  // gate and up projections, for the backward pass
          uint32_t g2[2], u2[2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            g2[h] = pack_half2<ACT>(acc[i][t][2 * h], acc[i][t][2 * h + 1]);
            u2[h] = pack_half2<ACT>(acc[i][t + MF_NT / 2][2 * h], acc[i][t + MF_NT / 2][2 * h + 1]);
          }
          *reinterpret_cast<uint2*>(save_a + orow + col) = make_uint2(g2[0], g2[1]);
          *reinterpret_cast<uint2*>(save_b + orow + col) = make_uint2(u2[0], u2[1]);
        }
      }
    } else {
      const float wgt = row_w[i];
#pragma unroll
      for (int t = 0; t < MF_NT; ++t) {
        const int col = n0 + wn * 64 + t * 16 + 4 * lq;
        if (col >= n_out) continue;
        uint32_t pk[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          // without weights act(act(v) * 1) is act(v): one rounding
          const float a = row_weight ? round_act<ACT>(acc[i][t][2 * h]) * wgt : acc[i][t][2 * h];
          const float c = row_weight ? round_act<ACT>(acc[i][t][2 * h + 1]) * wgt : acc[i][t][2 * h + 1];
          pk[h] = pack_half2<ACT>(a, c);
        }
        *reinterpret_cast<uint2*>(out + orow + col) = make_uint2(pk[0], pk[1]);
        if (save_a) {  // the rows before their weight, for the backward pass
          uint32_t un[2];
#pragma unroll
          for (int h = 0; h < 2; ++h)
            un[h] = pack_half2<ACT>(acc[i][t][2 * h], acc[i][t][2 * h + 1]);
          *reinterpret_cast<uint2*>(save_a + orow + col) = make_uint2(un[0], un[1]);
        }
      }
    }
  }
}

// Kernel view of one stacked projection.
MfW mf_view(int wf, const WView& v) {
  const int64_t esize = wf == QW_I8 || wf == QW_U4 ? 1 : 2;  // QW_U4 strides are in bytes already
  MfW m;
  m.w = static_cast<const char*>(v.w);
  m.scales = v.scales;
  m.expert_bytes = v.expert_elems * esize;
  m.row_bytes = v.row_stride * esize;
  m.expert_scales = v.expert_scales;
  m.groups = static_cast<int>(v.groups);
  m.group = static_cast<int>(v.group > 0 ? v.group : 1);
  return m;
}

template <int ACT, bool GATEUP, int SUBT, int WF>
int launch_t(const void* x, const int32_t* row_index, const int32_t* offsets, int max_rows, const MfW& wa,
             const MfW& wb, int n_w, int K, const float* row_weight, void* out, int n_out, int experts,
             int64_t rows_cap, void* save_a, void* save_b, hipStream_t stream) {
  const int n_tiles = static_cast<int>(ceil_div(GATEUP ? n_w : n_out, GATEUP ? MF_NB / 2 : MF_NB));
  // chunks one XCD can own: its experts' chunks at the capacity bound, and at
  // most all rows in chunks plus one partial chunk per expert
  const int64_t per_xcd_experts = ceil_div(experts, kXcds);
  const int64_t slots = per_xcd_experts * ceil_div(rows_cap, 32 * SUBT);
  const int64_t found = ceil_div(max_rows, 32 * SUBT) + per_xcd_experts;
  const int64_t chunks = std::min(slots, found);
  const int m_chunks = slots <= found ? static_cast<int>(ceil_div(rows_cap, 32 * SUBT)) : 0;
  const int64_t grid = static_cast<int64_t>(kXcds) * chunks * n_tiles;
  if (grid > INT32_MAX) return set_error(QW_ERR_UNSUPPORTED, "MFMA grid too large");
  const size_t lds = static_cast<size_t>(mf_stages<WF>(SUBT)) * (32 * SUBT * MF_ROWB + MfB<WF>::STAGE);
  const hipError_t attr = reserve_lds<ffn_mfma_kernel<ACT, GATEUP, SUBT, WF>>(static_cast<int>(lds));
  if (attr != hipSuccess)
    return set_error(QW_ERR_HIP, "cannot reserve %zu bytes of LDS: %s", lds, hipGetErrorString(attr));
  ffn_mfma_kernel<ACT, GATEUP, SUBT, WF><<<static_cast<unsigned>(grid), MF_THREADS, lds, stream>>>(
      static_cast<const uint16_t*>(x), row_index, offsets, max_rows, wa, wb, n_w, K, row_weight,
      static_cast<uint16_t*>(out), n_out, n_tiles, m_chunks, experts, static_cast<uint16_t*>(save_a),
      static_cast<uint16_t*>(save_b));
  QW_LAUNCH_CHECK(GATEUP ? "ffn_mfma_kernel<gateup>" : "ffn_mfma_kernel<down>");
  return QW_OK;
}

// rows_cap: most rows any expert can hold (the capacity bound).
template <int ACT, bool GATEUP, int WF>
int launch_sel(int subt, const void* x, const int32_t* row_index, const int32_t* offsets, int max_rows,
               const MfW& wa, const MfW& wb, int n_w, int K, const float* row_weight, void* out, int n_out,
               int experts, int64_t rows_cap, void* save_a, void* save_b, hipStream_t stream) {
#define QW_MF(S)                                                                                                \
  if (subt == S)                                                                                               \
    return launch_t<ACT, GATEUP, S, WF>(x, row_index, offsets, max_rows, wa, wb, n_w, K, row_weight, out, n_out,     \
                                   experts, rows_cap, save_a, save_b, stream);
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

// The quantised projection suits the LDS stage: groups of whole MFMA K steps,
// 16-byte aligned rows and base.
bool quant_fits(const WView& v, int wf) {
  const int64_t row_bytes = v.row_stride;  // int8: one byte per element; int4: bytes
  return v.group > 0 && v.group % 32 == 0 && row_bytes % 16 == 0 &&
         reinterpret_cast<uintptr_t>(v.w) % 16 == 0 && reinterpret_cast<uintptr_t>(v.scales) % 4 == 0 &&
         (wf == QW_I8 || wf == QW_U4);
}

}  // namespace

int launch_ffn_mfma(const FfnArgs& a, hipStream_t stream, bool* handled) {
  *handled = false;
  const bool quant = a.wfmt == QW_I8 || a.wfmt == QW_U4;
  const bool f16 = a.act == QW_F16;
  if (!is_half(a.act)) return QW_OK;
  if (!quant && (f16 ? (a.wfmt != QW_F16 && a.wfmt != QW_F16T) : (a.wfmt != QW_BF16 && a.wfmt != QW_BF16T)))
    return QW_OK;
  if (a.d_model % 64 || a.d_ff % 64) return QW_OK;
  if (quant && !(quant_fits(a.gate, a.wfmt) && quant_fits(a.up, a.wfmt) && quant_fits(a.down, a.wfmt))) return QW_OK;
  if (a.avg_rows < 16) return QW_OK;  // decode-sized: weight streaming kernels
  const int64_t rows_cap = a.row_cap > 0 ? a.row_cap : a.max_rows;
  const int subt = pick_subt(rows_cap);
  const int D = static_cast<int>(a.d_model), F = static_cast<int>(a.d_ff), E = static_cast<int>(a.experts);
  const int mr = static_cast<int>(a.max_rows);
  const MfW g = mf_view(a.wfmt, a.gate), u = mf_view(a.wfmt, a.up), dn = mf_view(a.wfmt, a.down);
  auto both = [&](auto act, auto wf) -> int {
    constexpr int ACT = decltype(act)::value, WF = decltype(wf)::value;
    int st = launch_sel<ACT, true, WF>(subt, a.x, a.row_index, a.offsets, mr, g, u, F, D, nullptr, a.hidden, F, E,
                                  rows_cap, a.save_gate, a.save_up, stream);
    if (st) return st;
    return launch_sel<ACT, false, WF>(subt, a.hidden, nullptr, a.offsets, mr, dn, dn, D, F, a.row_weight, a.y, D, E,
                                 rows_cap, a.save_y, nullptr, stream);
  };
  using BF = std::integral_constant<int, QW_BF16>;
  using HF = std::integral_constant<int, QW_F16>;
  int st;
  switch (a.wfmt) {
    case QW_BF16T: st = both(BF{}, std::integral_constant<int, QW_BF16T>{}); break;
    case QW_F16T: st = both(HF{}, std::integral_constant<int, QW_F16T>{}); break;
    case QW_F16: st = both(HF{}, HF{}); break;
    case QW_I8:
      st = f16 ? both(HF{}, std::integral_constant<int, QW_I8>{}) : both(BF{}, std::integral_constant<int, QW_I8>{});
      break;
    case QW_U4:
      st = f16 ? both(HF{}, std::integral_constant<int, QW_U4>{}) : both(BF{}, std::integral_constant<int, QW_U4>{});
      break;
    default: st = both(BF{}, BF{}); break;
  }
  if (st) return st;
  *handled = true;
  return QW_OK;
}

}  // namespace qw
