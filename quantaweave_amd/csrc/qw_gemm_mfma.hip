// Grouped bf16 GEMMs on the matrix cores, out = A . B^T per expert, for the
// grouped matmul and its backward:
//
//   rows grouped (MODE_ROWS): expert e owns the rows [offsets[e], offsets[e+1])
//     of A and of the output, and its own B[e]; the reduction length K is
//     shared.  Forward:  y  = x  . W[e]^T               (B = W, as stored)
//                  dX:   dx = dy . W[e]                (B = W read reduction-major and
//                                                       transposed on its way into LDS)
//   reduction grouped (MODE_RED): expert e reduces over its own slice of
//     columns [poff[e], poff[e+1]) of A and B and owns the output matrix e.
//                  dW:   dW[e] = dy_e^T . x_e            (A = dy^T, B = x^T)
// (src/moe_kernels.py:41-64 forward, :66-89 and :146-164 backward).
//
// Workgroup: 256 threads, a 128x128 output tile, 64-deep reduction steps.
// Global loads go to registers (16 bytes per lane, four per operand), then to
// an XOR-swizzled LDS tile (128-byte rows, piece ^ (row & 7), so 8 lanes
// reading 8 rows at one logical piece hit 8 different bank groups); two LDS
// stages, the next tile's global loads in flight while the current one is
// multiplied.  Each wave owns a 64x64 quarter: 4x4 v_mfma_f32_16x16x32_bf16
// tiles, fp32 accumulation, bf16 results.  Rows past the end of a group load
// a valid row and are not stored.  The reduction in MODE_RED runs over
// zero-padded slices (multiples of 64); an expert without rows gets zeros.
#include "qw_common.h"

namespace qw {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));  // 16-bit operands (bf16 or fp16 bits)
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int MODE_ROWS = 0, MODE_RED = 1;
constexpr int GT = 128;                      // output tile edge
constexpr int GK = 64;                       // reduction step
constexpr int G_ROWB = GK * 2;               // bytes per LDS row
constexpr int G_OPER = GT * G_ROWB;          // one operand's stage (16 KiB)
constexpr int G_STAGE = 2 * G_OPER;          // A and B
constexpr int G_LDS = 2 * G_STAGE;           // two stages (64 KiB)
constexpr int G_XCDS = 8;                    // XCDs of the MI355X, workgroups dealt round robin

// LDS piece of logical 16-byte piece `piece` of tile row `row`: the 16 rows a
// quarter-wave reads at one logical piece land on 16 different bank groups.
__device__ __forceinline__ int gswz(int row, int piece) { return piece ^ ((row >> 1) & 7); }

template <int DT, int MODE, bool ACCUM, bool BRED, bool C32>
__global__ __launch_bounds__(256) void gemm_nt_kernel(const uint16_t* __restrict__ A, int64_t lda,
                                                      const uint16_t* __restrict__ B, int64_t ldb,
                                                      int64_t b_expert_stride, void* __restrict__ C, int64_t ldc,
                                                      int64_t c_expert_stride, const int32_t* __restrict__ offsets,
                                                      int rows, int M, int N, int K, int E) {
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  // XCD-aware tile order: workgroup b runs on XCD b % 8, so XCD x takes, in
  // turn, the row tiles (MODE_ROWS) or experts (MODE_RED) x, x + 8, ..., each
  // with all its column tiles back to back: the tiles that share an A block
  // (and an expert's B) run close together in one L2.
  const int b = blockIdx.x, xcd = b % G_XCDS, j = b / G_XCDS;
  const int n_nt = (N + GT - 1) / GT;
  int e, nt, m0, mcount, k_lo, k_len;
  const uint16_t* a_base;
  const uint16_t* b_base;
  int64_t c_off;  // element offset of the block's first output row
  if (MODE == MODE_ROWS) {  // row tiles of all experts, found on the device
    int local = 0;
    nt = j % n_nt;
    e = find_tile(offsets, E, rows, GT, (j / n_nt) * G_XCDS + xcd, &local);
    if (e < 0) return;
    const int lo = min(max(offsets[e], 0), rows), hi = min(offsets[e + 1], rows);
    m0 = lo + local * GT;
    if (m0 >= hi) return;
    mcount = min(GT, hi - m0);
    k_lo = 0;
    k_len = K;
    a_base = A + static_cast<int64_t>(m0) * lda;
    b_base = B + static_cast<int64_t>(e) * b_expert_stride;
    c_off = static_cast<int64_t>(m0) * ldc;
  } else {
    const int per_e = ((M + GT - 1) / GT) * n_nt;
    e = (j / per_e) * G_XCDS + xcd;
    if (e >= E) return;
    const int rem = j % per_e;
    nt = rem % n_nt;
    m0 = (rem / n_nt) * GT;
    mcount = min(GT, M - m0);
    k_lo = offsets[e];  // padded slice offsets
    k_len = offsets[e + 1] - k_lo;
    a_base = A + static_cast<int64_t>(m0) * lda + k_lo;
    b_base = B + k_lo;
    c_off = static_cast<int64_t>(e) * c_expert_stride + static_cast<int64_t>(m0) * ldc;
  }
  const int n0 = nt * GT;
  const int ncount = min(GT, N - n0);
  const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  const int wm = wave >> 1, wn = wave & 1;

  // per-thread global sources: piece p of rows (tid >> 3) + 32 q
  const int p = tid & 7, rb = tid >> 3;
  const uint16_t* a_src[4];
  const uint16_t* b_src[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = rb + 32 * q;
    a_src[q] = a_base + static_cast<int64_t>(min(r, mcount - 1)) * lda + 8 * p;
    b_src[q] = b_base + static_cast<int64_t>(n0 + min(r, ncount - 1)) * ldb + 8 * p;
  }
  // BRED (B stored reduction-major, element (red, col) at b_base[red * ldb + col]):
  // thread (kg = tid % 32, ng = tid / 32) loads columns 4 kg .. 4 kg + 3 of the
  // reduction rows 8 ng .. 8 ng + 7 and writes them transposed, one 16-byte
  // piece (8 reduction values) per column.  Columns past N read column N - 4
  // (in bounds, never stored).
  const int kg = tid % 32, ng = tid / 32;
  const uint16_t* bt_src = b_base + static_cast<int64_t>(8 * ng) * ldb + min(n0 + 4 * kg, N - 4);
  uint4 ra0, ra1, ra2, ra3, rb0, rb1, rb2, rb3;
  uint2 rt0, rt1, rt2, rt3, rt4, rt5, rt6, rt7;
#define QW_G_LOAD(kt)                                                        \
  do {                                                                       \
    const int k0_ = (kt) * GK;                                               \
    ra0 = *reinterpret_cast<const uint4*>(a_src[0] + k0_);                   \
    ra1 = *reinterpret_cast<const uint4*>(a_src[1] + k0_);                   \
    ra2 = *reinterpret_cast<const uint4*>(a_src[2] + k0_);                   \
    ra3 = *reinterpret_cast<const uint4*>(a_src[3] + k0_);                   \
    if (BRED) {                                                              \
      const uint16_t* t_ = bt_src + static_cast<int64_t>(k0_) * ldb;         \
      rt0 = *reinterpret_cast<const uint2*>(t_);                             \
      rt1 = *reinterpret_cast<const uint2*>(t_ + ldb);                       \
      rt2 = *reinterpret_cast<const uint2*>(t_ + 2 * ldb);                   \
      rt3 = *reinterpret_cast<const uint2*>(t_ + 3 * ldb);                   \
      rt4 = *reinterpret_cast<const uint2*>(t_ + 4 * ldb);                   \
      rt5 = *reinterpret_cast<const uint2*>(t_ + 5 * ldb);                   \
      rt6 = *reinterpret_cast<const uint2*>(t_ + 6 * ldb);                   \
      rt7 = *reinterpret_cast<const uint2*>(t_ + 7 * ldb);                   \
    } else {                                                                 \
      rb0 = *reinterpret_cast<const uint4*>(b_src[0] + k0_);                 \
      rb1 = *reinterpret_cast<const uint4*>(b_src[1] + k0_);                 \
      rb2 = *reinterpret_cast<const uint4*>(b_src[2] + k0_);                 \
      rb3 = *reinterpret_cast<const uint4*>(b_src[3] + k0_);                 \
    }                                                                        \
  } while (0)
#define QW_LO2(a, b) (((a) & 0xffffu) | ((b) << 16))
#define QW_HI2(a, b) (((a) >> 16) | ((b) & 0xffff0000u))
#define QW_G_STORE(stage)                                                                    \
  do {                                                                                       \
    char* sa_ = smem + (stage) * G_STAGE;                                                    \
    char* sb_ = sa_ + G_OPER;                                                                \
    *reinterpret_cast<uint4*>(sa_ + w_off[0]) = ra0;                                         \
    *reinterpret_cast<uint4*>(sa_ + w_off[1]) = ra1;                                         \
    *reinterpret_cast<uint4*>(sa_ + w_off[2]) = ra2;                                         \
    *reinterpret_cast<uint4*>(sa_ + w_off[3]) = ra3;                                         \
    if (BRED) {                                                                              \
      *reinterpret_cast<uint4*>(sb_ + t_off[0]) = make_uint4(                                \
          QW_LO2(rt0.x, rt1.x), QW_LO2(rt2.x, rt3.x), QW_LO2(rt4.x, rt5.x), QW_LO2(rt6.x, rt7.x)); \
      *reinterpret_cast<uint4*>(sb_ + t_off[1]) = make_uint4(                                \
          QW_HI2(rt0.x, rt1.x), QW_HI2(rt2.x, rt3.x), QW_HI2(rt4.x, rt5.x), QW_HI2(rt6.x, rt7.x)); \
      *reinterpret_cast<uint4*>(sb_ + t_off[2]) = make_uint4(                                \
          QW_LO2(rt0.y, rt1.y), QW_LO2(rt2.y, rt3.y), QW_LO2(rt4.y, rt5.y), QW_LO2(rt6.y, rt7.y)); \
      *reinterpret_cast<uint4*>(sb_ + t_off[3]) = make_uint4(                                \
          QW_HI2(rt0.y, rt1.y), QW_HI2(rt2.y, rt3.y), QW_HI2(rt4.y, rt5.y), QW_HI2(rt6.y, rt7.y)); \
    } else {                                                                                 \
      *reinterpret_cast<uint4*>(sb_ + w_off[0]) = rb0;                                       \
      *reinterpret_cast<uint4*>(sb_ + w_off[1]) = rb1;                                       \
      *reinterpret_cast<uint4*>(sb_ + w_off[2]) = rb2;                                       \
      *reinterpret_cast<uint4*>(sb_ + w_off[3]) = rb3;                                       \
    }                                                                                        \
  } while (0)
  int w_off[4];  // LDS byte offset of this thread's piece in rows rb + 32 q
  int t_off[4];  // BRED: LDS byte offset of piece ng of rows 4 kg + c
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = rb + 32 * q;
    w_off[q] = r * G_ROWB + gswz(r, p) * 16;
    const int rt = 4 * kg + q;
    t_off[q] = rt * G_ROWB + gswz(rt, ng) * 16;
  }

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nk = k_len / GK;
  if (nk > 0) {
    QW_G_LOAD(0);
    QW_G_STORE(0);
  }
  __syncthreads();
  const int l16 = lane & 15, lq = lane >> 4;
  for (int kt = 0; kt < nk; ++kt) {
    const bool more = kt + 1 < nk;
    if (more) QW_G_LOAD(kt + 1);
    const char* sa = smem + (kt & 1) * G_STAGE;
    const char* sb = sa + G_OPER;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      bf16x8 af[4], bf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = wm * 64 + 16 * i + l16;
        af[i] = *reinterpret_cast<const bf16x8*>(sa + r * G_ROWB + gswz(r, 4 * ks + lq) * 16);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = wn * 64 + 16 * j + l16;
        bf[j] = *reinterpret_cast<const bf16x8*>(sb + r * G_ROWB + gswz(r, 4 * ks + lq) * 16);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if constexpr (DT == QW_F16)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, bf[j]),
                                                               __builtin_bit_cast(f16x8, af[i]), acc[i][j], 0, 0, 0);
          else
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf[j], af[i], acc[i][j], 0, 0, 0);
        }
    }
    if (more) QW_G_STORE((kt + 1) & 1);
    __syncthreads();
  }
#undef QW_G_LOAD
#undef QW_G_STORE
#undef QW_LO2
#undef QW_HI2

  // ---- epilogue through LDS when the output rows are 16-byte aligned: the fp32
  //      tile (the stages are free after the loop's last barrier) leaves in
  //      whole row segments, 16 bytes per lane.  Chunk c (4 fp32) of tile row m
  //      sits at chunk c ^ (m & 15), so the 16 rows of an MFMA tile write 16
  //      different bank groups.  Same sums and roundings as the direct stores
  //      below (the accumulate path adds the old value before rounding). ----
  {
    constexpr int ES = C32 ? 4 : 2;  // output bytes per element
    constexpr int OV = 16 / ES;      // output elements per 16-byte store
    static_assert(GT * GT * 4 <= G_LDS, "the fp32 tile fits the stages");
    const bool aligned = (reinterpret_cast<uintptr_t>(static_cast<char*>(C) + (c_off + n0) * ES) % 16) == 0 &&
                         ((ldc * ES) % 16) == 0;
    if (aligned) {
      float* const t = reinterpret_cast<float*>(smem);  // [GT][GT]
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int m = wm * 64 + 16 * i + l16, n = wn * 64 + 16 * j + 4 * lq;
          *reinterpret_cast<f32x4*>(t + m * GT + 4 * ((n / 4) ^ (m & 15))) = acc[i][j];
        }
      __syncthreads();
      constexpr int CPR = GT / OV;  // 16-byte output chunks per tile row
      for (int c = tid; c < mcount * CPR; c += 256) {
        const int r = c / CPR, n = (c % CPR) * OV;
        if (n >= ncount) continue;
        float v[OV];
#pragma unroll
        for (int h = 0; h < OV / 4; ++h) {
          const f32x4 x = *reinterpret_cast<const f32x4*>(t + r * GT + 4 * ((n / 4 + h) ^ (r & 15)));
#pragma unroll
          for (int u = 0; u < 4; ++u) v[4 * h + u] = x[u];
        }
        const int64_t o = c_off + static_cast<int64_t>(r) * ldc + n0 + n;
        if constexpr (C32) {
          float* co = static_cast<float*>(C) + o;
          if (n + OV <= ncount) {
            if (ACCUM) {
              const float4 old = *reinterpret_cast<const float4*>(co);
              v[0] += old.x;
              v[1] += old.y;
              v[2] += old.z;
              v[3] += old.w;
            }
            *reinterpret_cast<float4*>(co) = make_float4(v[0], v[1], v[2], v[3]);
          } else {
            for (int u = 0; u < OV && n + u < ncount; ++u) co[u] = v[u] + (ACCUM ? co[u] : 0.0f);
          }
        } else {
          uint16_t* co = static_cast<uint16_t*>(C) + o;
          if (n + OV <= ncount) {
            uint32_t w[OV / 2];
            if (ACCUM) {
              const uint4 old = *reinterpret_cast<const uint4*>(co);
              const uint32_t ow[4] = {old.x, old.y, old.z, old.w};
#pragma unroll
              for (int u = 0; u < 4; ++u) {
                v[2 * u] += half_to_f32<DT>(ow[u] & 0xffffu);
                v[2 * u + 1] += half_to_f32<DT>(ow[u] >> 16);
              }
            }
#pragma unroll
            for (int u = 0; u < OV / 2; ++u)
              w[u] = pack_half2<DT>(v[2 * u], v[2 * u + 1]);
            *reinterpret_cast<uint4*>(co) = make_uint4(w[0], w[1], w[2], w[3]);
          } else {
            for (int u = 0; u < OV && n + u < ncount; ++u)
              co[u] = f32_to_half<DT>(v[u] + (ACCUM ? half_to_f32<DT>(co[u]) : 0.0f));
          }
        }
      }
      return;
    }
  }

  // lane holds C[m = 16 i + l16][n = 16 j + 4 lq + v] of its wave's quarter;
  // C32: fp32 output, else the operands' 16-bit type
  const bool vec = (ldc & 3) == 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = wm * 64 + 16 * i + l16;
    if (m >= mcount) continue;
    const int64_t row = c_off + static_cast<int64_t>(m) * ldc + n0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = wn * 64 + 16 * j + 4 * lq;
      f32x4 v = acc[i][j];
      if (C32) {
        float* c = static_cast<float*>(C) + row;
        if (vec && n + 3 < ncount) {
          if (ACCUM) {
            const float4 old = *reinterpret_cast<const float4*>(c + n);
            v[0] += old.x;
            v[1] += old.y;
            v[2] += old.z;
            v[3] += old.w;
          }
          *reinterpret_cast<float4*>(c + n) = make_float4(v[0], v[1], v[2], v[3]);
        } else {
#pragma unroll
          for (int u = 0; u < 4; ++u)
            if (n + u < ncount) c[n + u] = v[u] + (ACCUM ? c[n + u] : 0.0f);
        }
        continue;
      }
      uint16_t* crow = static_cast<uint16_t*>(C) + row;
      if (vec && n + 3 < ncount) {
        if (ACCUM) {
          const uint2 old = *reinterpret_cast<const uint2*>(crow + n);
          v[0] += half_to_f32<DT>(old.x & 0xffffu);
          v[1] += half_to_f32<DT>(old.x >> 16);
          v[2] += half_to_f32<DT>(old.y & 0xffffu);
          v[3] += half_to_f32<DT>(old.y >> 16);
        }
        const uint32_t lo = pack_half2<DT>(v[0], v[1]);
        const uint32_t hi = pack_half2<DT>(v[2], v[3]);
        *reinterpret_cast<uint2*>(crow + n) = make_uint2(lo, hi);
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (n + u < ncount) crow[n + u] = f32_to_half<DT>(v[u] + (ACCUM ? half_to_f32<DT>(crow[n + u]) : 0.0f));
      }
    }
  }
}

// Padded slice offsets: poff[e] = sum over e' < e of len(e') rounded up to 64.
__global__ __launch_bounds__(64) void pad_offsets_kernel(const int32_t* __restrict__ offsets, int E, int rows,
                                                         int32_t* __restrict__ poff) {
  const int lane = threadIdx.x;
  int carry = 0;
  for (int e0 = 0; e0 < E; e0 += 64) {
    const int e = e0 + lane;
    int len = 0;
    if (e < E) {
      const int lo = min(max(offsets[e], 0), rows), hi = min(offsets[e + 1], rows);
      len = max(hi - lo, 0);
    }
    const int padded = (len + 63) & ~63;
    int v = padded;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int t = __shfl_up(v, o, 64);
      if (lane >= o) v += t;
    }
    if (e < E) poff[e] = carry + v - padded;
    carry += __shfl(v, 63, 64);
  }
  if (lane == 0) poff[E] = carry;
}

// Plan-ordered rows src [rows, C] -> dst [C, ld] with expert e's rows at columns
// poff[e] .. poff[e] + len(e) and zeros up to the padded end of its slice.
// blockIdx.y enumerates the 64-row tiles of all experts.
__global__ __launch_bounds__(256) void transpose_pad_kernel(const uint16_t* __restrict__ src, int C,
                                                            const int32_t* __restrict__ offsets,
                                                            const int32_t* __restrict__ poff, int E, int rows,
                                                            int64_t ld, uint16_t* __restrict__ dst) {
  __shared__ uint16_t tile[64][66];
  int local = 0;
  const int e = find_tile(offsets, E, rows, 64, blockIdx.y, &local);
  if (e < 0) return;
  const int lo = min(max(offsets[e], 0), rows), hi = min(offsets[e + 1], rows);
  const int len = max(hi - lo, 0);
  const int r0 = local * 64;
  const int c0 = blockIdx.x * 64;
  const int tx = threadIdx.x % 64, ty = threadIdx.x / 64;
  for (int i = ty; i < 64; i += 4) {
    const int r = r0 + i, c = c0 + tx;
    tile[i][tx] = (r < len && c < C) ? src[static_cast<int64_t>(lo + r) * C + c] : 0;
  }
  __syncthreads();
  const int64_t col0 = poff[e] + r0;
  for (int i = ty; i < 64; i += 4) {
    const int c = c0 + i;
    if (c < C) dst[static_cast<int64_t>(c) * ld + col0 + tx] = tile[tx][i];
  }
}

// The same transpose 16 bytes per access (C % 8 == 0, 16-byte aligned rows):
// a thread loads 8 consecutive columns of a row and stores 8 consecutive rows
// of a column.  The 16-byte chunk j of tile row i sits at chunk j ^ ((i / 8) % 8),
// so the column reads (rows 8j .. 8j+7 for the 8 chunks j of a wave) spread
// over 32 banks.
__global__ __launch_bounds__(256) void transpose_pad_vec_kernel(const uint16_t* __restrict__ src, int C,
                                                                const int32_t* __restrict__ offsets,
                                                                const int32_t* __restrict__ poff, int E, int rows,
                                                                int64_t ld, uint16_t* __restrict__ dst) {
  __shared__ __attribute__((aligned(16))) uint16_t tile[64][72];  // 144-byte rows
  int local = 0;
  const int e = find_tile(offsets, E, rows, 64, blockIdx.y, &local);
  if (e < 0) return;
  const int lo = min(max(offsets[e], 0), rows), hi = min(offsets[e + 1], rows);
  const int len = max(hi - lo, 0);
  const int r0 = local * 64;
  const int c0 = blockIdx.x * 64;
  const int t = threadIdx.x, j = t % 8;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int i = t / 8 + 32 * h;  // tile row
    const int r = r0 + i, c = c0 + 8 * j;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (r < len && c < C) v = *reinterpret_cast<const uint4*>(src + static_cast<int64_t>(lo + r) * C + c);
    *reinterpret_cast<uint4*>(&tile[i][8 * (j ^ ((i / 8) % 8))]) = v;
  }
  __syncthreads();
  const int64_t col0 = poff[e] + r0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int cc = t / 8 + 32 * h;  // tile column = output row
    const int c = c0 + cc;
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t a = tile[8 * j + 2 * q][8 * ((cc / 8) ^ j) + cc % 8];
      const uint32_t b = tile[8 * j + 2 * q + 1][8 * ((cc / 8) ^ j) + cc % 8];
      w[q] = a | (b << 16);
    }
    if (c < C) *reinterpret_cast<uint4*>(dst + static_cast<int64_t>(c) * ld + col0 + 8 * j) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

template <int DT, int MODE, bool ACCUM, bool BRED = false, bool C32 = false>
int launch_gemm(const void* A, int64_t lda, const void* B, int64_t ldb, int64_t b_stride, void* C, int64_t ldc,
                int64_t c_stride, const int32_t* offsets, int rows, int M, int N, int K, int E, int64_t m_extent,
                hipStream_t stream) {
  const hipError_t attr = reserve_lds<gemm_nt_kernel<DT, MODE, ACCUM, BRED, C32>>(G_LDS);
  if (attr != hipSuccess) return set_error(QW_ERR_HIP, "cannot reserve LDS: %s", hipGetErrorString(attr));
  // one grid dimension: MODE_ROWS, the row tiles of all experts (at most
  // rows/128 + E) times the column tiles; MODE_RED, experts times output tiles;
  // rounded up so that every XCD gets the same count of row tiles / experts
  const int64_t n_nt = ceil_div(N, GT);
  const int64_t blocks = MODE == MODE_ROWS ? G_XCDS * n_nt * ceil_div(ceil_div(m_extent, GT) + E, G_XCDS)
                                           : G_XCDS * n_nt * ceil_div(m_extent, GT) * ceil_div(E, G_XCDS);
  if (blocks > INT32_MAX) return set_error(QW_ERR_UNSUPPORTED, "grouped GEMM grid too large");
  gemm_nt_kernel<DT, MODE, ACCUM, BRED, C32><<<static_cast<unsigned>(blocks), 256, G_LDS, stream>>>(
      static_cast<const uint16_t*>(A), lda, static_cast<const uint16_t*>(B), ldb, b_stride, C, ldc, c_stride, offsets,
      rows, M, N, K, E);
  QW_LAUNCH_CHECK("gemm_nt_kernel");
  return QW_OK;
}

}  // namespace

// Pitch of the padded transposed rows: every expert's slice rounded up to 64.
int64_t padded_pitch(int64_t rows, int64_t E) { return align_up(static_cast<size_t>(rows), 64) + 64 * E; }

size_t gemm_backward_workspace_bytes(int64_t E, int64_t N, int64_t K, int64_t rows) {
  Carver c(nullptr);
  const int64_t rp = padded_pitch(rows, E);
  c.take<uint16_t>(static_cast<size_t>(N) * rp);     // dy^T
  c.take<uint16_t>(static_cast<size_t>(K) * rp);     // x^T
  c.take<int32_t>(E + 1);                            // padded offsets
  return c.used + 256;
}

// Grid limits of the matrix-core path: row tiles of all experts in one grid dimension.
bool gemm_rows_fits(int64_t K, int64_t rows, int64_t E) {
  return K % GK == 0 && K <= INT32_MAX && ceil_div(rows, GT) + E <= 65535;
}

bool gemm_backward_fits(int64_t rows, int64_t E) { return ceil_div(rows, 64) + E <= 65535; }

// out[r] = x[r] . w[e]^T over the rows of each expert (bf16 or fp16, w [E, N, K]).
int gemm_grouped_forward(const void* x, const void* w, int dtype, int64_t E, int64_t N, int64_t K,
                         const int32_t* offsets, int64_t rows, int64_t rows_per_expert, void* out, hipStream_t stream) {
  (void)rows_per_expert;
  if (dtype == QW_F16)
    return launch_gemm<QW_F16, MODE_ROWS, false>(x, K, w, K, N * K, out, N, 0, offsets, static_cast<int>(rows), 0,
                                                 static_cast<int>(N), static_cast<int>(K), static_cast<int>(E), rows,
                                                 stream);
  return launch_gemm<QW_BF16, MODE_ROWS, false>(x, K, w, K, N * K, out, N, 0, offsets, static_cast<int>(rows), 0,
                                                static_cast<int>(N), static_cast<int>(K), static_cast<int>(E), rows,
                                                stream);
}

// Backward of gemm_grouped_forward on the matrix cores (bf16 or fp16, DT):
//   gx = gy . w[e] (+ gx when accumulate), gw[e] = gy_e^T . x_e (fp32 when gw_f32).
template <int DT>
int gemm_backward_t(const void* gy, const void* x, const void* w, int64_t E, int64_t N, int64_t K,
                    const int32_t* offsets, int64_t rows, void* gx, int accumulate, void* gw, int gw_f32, void* ws,
                    size_t ws_bytes, hipStream_t stream) {
  const size_t need = gemm_backward_workspace_bytes(E, N, K, rows);
  if (!ws || ws_bytes < need)
    return set_error(QW_ERR_WORKSPACE, "grouped backward workspace needs %zu bytes, got %zu", need, ws_bytes);
  Carver c(ws);
  const int64_t rp = padded_pitch(rows, E);
  uint16_t* gyt = c.take<uint16_t>(static_cast<size_t>(N) * rp);
  uint16_t* xt = c.take<uint16_t>(static_cast<size_t>(K) * rp);
  int32_t* poff = c.take<int32_t>(E + 1);
  const int e = static_cast<int>(E), n = static_cast<int>(N), k = static_cast<int>(K), r = static_cast<int>(rows);
  if (gx != nullptr && rows > 0) {  // B = w read reduction-major: no transposed copy
    const int st = accumulate
                       ? launch_gemm<DT, MODE_ROWS, true, true>(gy, N, w, K, N * K, gx, K, 0, offsets, r, 0, k, n, e,
                                                                rows, stream)
                       : launch_gemm<DT, MODE_ROWS, false, true>(gy, N, w, K, N * K, gx, K, 0, offsets, r, 0, k, n, e,
                                                                 rows, stream);
    if (st) return st;
  }
  if (gw != nullptr) {
    pad_offsets_kernel<<<1, 64, 0, stream>>>(offsets, e, r, poff);
    QW_LAUNCH_CHECK("pad_offsets_kernel");
    if (rows > 0) {
      const int64_t rt = ceil_div(rows, 64) + E;  // 64-row tiles of all experts, at most
      if (rt > 65535) return set_error(QW_ERR_UNSUPPORTED, "too many row tiles for the transpose grid");
      const dim3 g1(static_cast<unsigned>(ceil_div(N, 64)), static_cast<unsigned>(rt));
      const dim3 g2(static_cast<unsigned>(ceil_div(K, 64)), static_cast<unsigned>(rt));
      auto vec_ok = [](const void* p, int64_t cols) { return cols % 8 == 0 && reinterpret_cast<uintptr_t>(p) % 16 == 0; };
      if (vec_ok(gy, N))
        transpose_pad_vec_kernel<<<g1, 256, 0, stream>>>(static_cast<const uint16_t*>(gy), n, offsets, poff, e, r, rp,
                                                         gyt);
      else
        transpose_pad_kernel<<<g1, 256, 0, stream>>>(static_cast<const uint16_t*>(gy), n, offsets, poff, e, r, rp, gyt);
      if (vec_ok(x, K))
        transpose_pad_vec_kernel<<<g2, 256, 0, stream>>>(static_cast<const uint16_t*>(x), k, offsets, poff, e, r, rp,
                                                         xt);
      else
        transpose_pad_kernel<<<g2, 256, 0, stream>>>(static_cast<const uint16_t*>(x), k, offsets, poff, e, r, rp, xt);
      QW_LAUNCH_CHECK("transpose_pad_kernel");
    }
    return gw_f32 ? launch_gemm<DT, MODE_RED, false, false, true>(gyt, rp, xt, rp, 0, gw, K, N * K, poff, r, n, k,
                                                                  0, e, N, stream)
                  : launch_gemm<DT, MODE_RED, false>(gyt, rp, xt, rp, 0, gw, K, N * K, poff, r, n, k, 0, e, N, stream);
  }
  return QW_OK;
}

int gemm_grouped_backward(const void* gy, const void* x, const void* w, int dtype, int64_t E, int64_t N, int64_t K,
                          const int32_t* offsets, int64_t rows, int64_t rows_per_expert, void* gx, int accumulate,
                          void* gw, int gw_f32, void* ws, size_t ws_bytes, hipStream_t stream) {
  (void)rows_per_expert;
  if (dtype == QW_F16)
    return gemm_backward_t<QW_F16>(gy, x, w, E, N, K, offsets, rows, gx, accumulate, gw, gw_f32, ws, ws_bytes,
                                   stream);
  return gemm_backward_t<QW_BF16>(gy, x, w, E, N, K, offsets, rows, gx, accumulate, gw, gw_f32, ws, ws_bytes, stream);
}

}  // namespace qw
