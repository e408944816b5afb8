// Backward of the grouped matmul y[rows of e] = x[rows of e] @ W[e]^T.
//
// Reference: _GroupedMatmul.backward (src/moe_kernels.py:146-164) with its two
// kernels: grad_x through the forward kernel with the weight transposed
// (:118-135, transpose=True), and _grouped_dw_kernel (:66-89):
//   grad_x[r, k]    = sum_n grad_y[r, n] * W[e][n, k]          (r in rows of e)
//   grad_W[e][n, k] = sum_{r in rows of e} grad_y[r, n] * x[r, k]
// An expert without rows gets an exactly zero grad_W.  fp32 accumulation,
// output in the operands' dtype (fp32 or bf16); with `accumulate` grad_x
// receives grad_x + result (one rounding), which sums the gate and up
// projections' input gradients of a SwiGLU expert in place.
//
// bf16 and fp16 with a workspace run on the matrix cores (gemm_grouped_backward,
// qw_gemm_mfma.hip); fp32 runs on the fp32 matrix cores (v_mfma_f32_16x16x4_f32,
// the two kernels below) when rows are 16-byte aligned.  Otherwise two
// vector-ALU kernels compute a 64x64 output tile per 256-thread
// block (4x4 per thread) from 16-deep slices of the reduction staged in LDS;
// the reduction runs in ascending order, so results do not depend on
// scheduling.
#include "qw_common.h"

namespace qw {

namespace {

constexpr int BT = 64;  // output tile edge
constexpr int BR = 16;  // reduction slice

// grad_x: block (k tile, row tile, expert)
template <int DT>
__global__ __launch_bounds__(256) void grouped_dx_kernel(const void* __restrict__ gy, const void* __restrict__ w,
                                                         const int32_t* __restrict__ offsets, int N, int K,
                                                         int rows, int accumulate, void* __restrict__ gx) {
  __shared__ float gs[BR][BT + 4];  // [n][row]
  __shared__ float ws[BR][BT + 4];  // [n][k]
  const int e = blockIdx.z;
  const int lo = min(max(offsets[e], 0), rows), hi = min(offsets[e + 1], rows);
  const int r0 = lo + blockIdx.y * BT;
  if (r0 >= hi) return;
  const int k0 = blockIdx.x * BT;
  const int tid = threadIdx.x, ty = tid / 16, tx = tid % 16;
  const int64_t wbase = static_cast<int64_t>(e) * N * K;
  float acc[4][4] = {};
  for (int n0 = 0; n0 < N; n0 += BR) {
    for (int i = tid; i < BT * BR; i += 256) {
      const int m = i / BR, nn = i % BR;
      const int r = r0 + m, n = n0 + nn;
      gs[nn][m] = (r < hi && n < N) ? load_act<DT>(gy, static_cast<int64_t>(r) * N + n) : 0.0f;
      const int wn = i / BT, kk = i % BT;
      const int n2 = n0 + wn, k = k0 + kk;
      ws[wn][kk] = (n2 < N && k < K) ? load_act<DT>(w, wbase + static_cast<int64_t>(n2) * K + k) : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int nn = 0; nn < BR; ++nn) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = gs[nn][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = ws[nn][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = r0 + ty * 4 + i;
    if (r >= hi) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k = k0 + tx * 4 + j;
      if (k >= K) continue;
      const int64_t o = static_cast<int64_t>(r) * K + k;
      store_act<DT>(gx, o, accumulate ? load_act<DT>(gx, o) + acc[i][j] : acc[i][j]);
    }
  }
}

// grad_W: block (k tile, n tile, expert); ODT the output dtype
template <int DT, int ODT>
__global__ __launch_bounds__(256) void grouped_dw_kernel(const void* __restrict__ gy, const void* __restrict__ x,
                                                         const int32_t* __restrict__ offsets, int N, int K,
                                                         int rows, void* __restrict__ gw) {
  __shared__ float gs[BR][BT + 4];  // [row][n]
  __shared__ float xs[BR][BT + 4];  // [row][k]
  const int e = blockIdx.z;
  const int lo = min(max(offsets[e], 0), rows), hi = min(offsets[e + 1], rows);
  const int n0 = blockIdx.y * BT, k0 = blockIdx.x * BT;
  const int tid = threadIdx.x, ty = tid / 16, tx = tid % 16;
  float acc[4][4] = {};
  for (int m0 = lo; m0 < hi; m0 += BR) {
    for (int i = tid; i < BR * BT; i += 256) {
      const int m = i / BT, c = i % BT;
      const int r = m0 + m;
      const bool ok = r < hi;
      gs[m][c] = (ok && n0 + c < N) ? load_act<DT>(gy, static_cast<int64_t>(r) * N + n0 + c) : 0.0f;
      xs[m][c] = (ok && k0 + c < K) ? load_act<DT>(x, static_cast<int64_t>(r) * K + k0 + c) : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < BR; ++m) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = gs[m][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = xs[m][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
  const int64_t wbase = static_cast<int64_t>(e) * N * K;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int n = n0 + ty * 4 + i;
    if (n >= N) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k = k0 + tx * 4 + j;
      if (k < K) store_act<ODT>(gw, wbase + static_cast<int64_t>(n) * K + k, acc[i][j]);
    }
  }
}

// ---------------------------------------------------------------------------
// fp32 on the matrix cores.  A 256-thread workgroup (2 x 2 waves) computes a
// 64 x 64 output tile from 64-deep reduction slices staged in LDS (two
// buffers; the next slice is loaded into registers while the current one is
// multiplied).  Each LDS tile is [64 tile rows][64 reduction indices] with
// the reduction contiguous, so a lane reads the 4 reduction values of a
// 16-wide step with one 16-byte read; lane group q of the four 16x16x4
// instructions of a step takes reduction index 4q + j (any assignment works
// when both operands agree).  Operands whose reduction index is not the
// contiguous one in memory are transposed on their way into LDS.  The
// reduction runs in ascending order.
// ---------------------------------------------------------------------------
typedef float bf32x4 __attribute__((ext_vector_type(4)));
constexpr int FB_T = 64, FB_R = 64, FB_LD = FB_R + 4;

// Products of one slice: acc[i][t] += A rows (wn*32 + 16t) x B rows (wm*32 + 16i)
__device__ __forceinline__ void fb_compute(const float* As, const float* Bs, int wm, int wn, int l16, int lq,
                                           bf32x4 (&acc)[2][2]) {
#pragma unroll
  for (int kk = 0; kk < FB_R; kk += 16) {
    bf32x4 a[2], b[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) a[t] = *reinterpret_cast<const bf32x4*>(As + (wn * 32 + 16 * t + l16) * FB_LD + kk + 4 * lq);
#pragma unroll
    for (int i = 0; i < 2; ++i) b[i] = *reinterpret_cast<const bf32x4*>(Bs + (wm * 32 + 16 * i + l16) * FB_LD + kk + 4 * lq);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int t = 0; t < 2; ++t) acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t][j], b[i][j], acc[i][t], 0, 0, 0);
  }
}

// grad_x[r, k] (+)= sum_n gy[r, n] W_e[n, k]; block (k tile, row tile, expert).
// A = W_e transposed into LDS ([k][n]), B = gy rows ([r][n]).
__global__ __launch_bounds__(256) void grouped_dx_f32_kernel(const float* __restrict__ gy, const float* __restrict__ w,
                                                             const int32_t* __restrict__ offsets, int N, int K,
                                                             int rows, int accumulate, float* __restrict__ gx) {
  __shared__ __attribute__((aligned(16))) float As[2][FB_T * FB_LD];
  __shared__ __attribute__((aligned(16))) float Bs[2][FB_T * FB_LD];
  const int e = blockIdx.z;
  const int lo = min(max(offsets[e], 0), rows), hi = min(offsets[e + 1], rows);
  const int r0 = lo + blockIdx.y * FB_T;
  if (r0 >= hi) return;
  const int k0 = blockIdx.x * FB_T;
  const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  const int wm = wave / 2, wn = wave % 2, l16 = lane % 16, lq = lane / 16;
  const float* we = w + static_cast<int64_t>(e) * N * K;
  // this thread's 16-byte pieces: tile rows tid/16 + 16h, columns 4*(tid%16)
  const int pr = tid / 16, pc = 4 * (tid % 16);
  bf32x4 ra[4], rb[4];
  auto load = [&](int n0) {
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int n = n0 + pr + 16 * h, k = k0 + pc;  // W row n, columns k..k+3
      ra[h] = (n < N && k < K) ? *reinterpret_cast<const bf32x4*>(we + static_cast<int64_t>(n) * K + k)
                               : bf32x4{0.f, 0.f, 0.f, 0.f};
      const int r = r0 + pr + 16 * h, nn = n0 + pc;  // gy row r, columns nn..nn+3
      rb[h] = (r < hi && nn < N) ? *reinterpret_cast<const bf32x4*>(gy + static_cast<int64_t>(r) * N + nn)
                                 : bf32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int h = 0; h < 4; ++h) {
#pragma unroll
      for (int j = 0; j < 4; ++j) As[buf][(pc + j) * FB_LD + pr + 16 * h] = ra[h][j];  // [k][n]
      *reinterpret_cast<bf32x4*>(&Bs[buf][(pr + 16 * h) * FB_LD + pc]) = rb[h];      // [r][n]
    }
  };
  bf32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int t = 0; t < 2; ++t) acc[i][t] = bf32x4{0.f, 0.f, 0.f, 0.f};
  const int S = (N + FB_R - 1) / FB_R;
  load(0);
  store(0);
  __syncthreads();
  for (int sl = 0; sl < S; ++sl) {
    if (sl + 1 < S) load((sl + 1) * FB_R);
    fb_compute(As[sl & 1], Bs[sl & 1], wm, wn, l16, lq, acc);
    if (sl + 1 < S) store((sl + 1) & 1);
    __syncthreads();
  }
  // lane holds grad_x[row wm*32 + 16i + l16][k wn*32 + 16t + 4lq .. +3]
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = r0 + wm * 32 + 16 * i + l16;
    if (r >= hi) continue;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int k = k0 + wn * 32 + 16 * t + 4 * lq;
      float* o = gx + static_cast<int64_t>(r) * K + k;
      if (k + 3 < K) {
        bf32x4 v = acc[i][t];
        if (accumulate) {
          const bf32x4 old = *reinterpret_cast<const bf32x4*>(o);
#pragma unroll
          for (int j = 0; j < 4; ++j) v[j] = old[j] + v[j];
        }
        *reinterpret_cast<bf32x4*>(o) = v;
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (k + j < K) o[j] = accumulate ? o[j] + acc[i][t][j] : acc[i][t][j];
      }
    }
  }
}

// grad_W_e[n, k] = sum over the rows r of expert e of gy[r, n] x[r, k] (exactly
// zero without rows); block (k tile, n tile, expert).  A = x transposed
// ([k][r]), B = gy transposed ([n][r]).
__global__ __launch_bounds__(256) void grouped_dw_f32_kernel(const float* __restrict__ gy, const float* __restrict__ x,
                                                             const int32_t* __restrict__ offsets, int N, int K,
                                                             int rows, float* __restrict__ gw) {
  __shared__ __attribute__((aligned(16))) float As[2][FB_T * FB_LD];
  __shared__ __attribute__((aligned(16))) float Bs[2][FB_T * FB_LD];
  const int e = blockIdx.z;
  const int lo = min(max(offsets[e], 0), rows), hi = min(offsets[e + 1], rows);
  const int n0 = blockIdx.y * FB_T, k0 = blockIdx.x * FB_T;
  const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  const int wm = wave / 2, wn = wave % 2, l16 = lane % 16, lq = lane / 16;
  const int pr = tid / 16, pc = 4 * (tid % 16);
  bf32x4 ra[4], rb[4];
  auto load = [&](int m0) {
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int r = m0 + pr + 16 * h;
      const bool ok = r < hi;
      ra[h] = (ok && k0 + pc < K) ? *reinterpret_cast<const bf32x4*>(x + static_cast<int64_t>(r) * K + k0 + pc)
                                  : bf32x4{0.f, 0.f, 0.f, 0.f};
      rb[h] = (ok && n0 + pc < N) ? *reinterpret_cast<const bf32x4*>(gy + static_cast<int64_t>(r) * N + n0 + pc)
                                  : bf32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int h = 0; h < 4; ++h)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        As[buf][(pc + j) * FB_LD + pr + 16 * h] = ra[h][j];  // [k][r]
        Bs[buf][(pc + j) * FB_LD + pr + 16 * h] = rb[h][j];  // [n][r]
      }
  };
  bf32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int t = 0; t < 2; ++t) acc[i][t] = bf32x4{0.f, 0.f, 0.f, 0.f};
  const int S = (hi - lo + FB_R - 1) / FB_R;  // 0 for an expert without rows
  if (S > 0) {
    load(lo);
    store(0);
  }
  __syncthreads();
  for (int sl = 0; sl < S; ++sl) {
    if (sl + 1 < S) load(lo + (sl + 1) * FB_R);
    fb_compute(As[sl & 1], Bs[sl & 1], wm, wn, l16, lq, acc);
    if (sl + 1 < S) store((sl + 1) & 1);
    __syncthreads();
  }
  // lane holds grad_W[n wm*32 + 16i + l16][k wn*32 + 16t + 4lq .. +3]
  float* ge = gw + static_cast<int64_t>(e) * N * K;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int n = n0 + wm * 32 + 16 * i + l16;
    if (n >= N) continue;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int k = k0 + wn * 32 + 16 * t + 4 * lq;
      float* o = ge + static_cast<int64_t>(n) * K + k;
      if (k + 3 < K) {
        *reinterpret_cast<bf32x4*>(o) = acc[i][t];
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (k + j < K) o[j] = acc[i][t][j];
      }
    }
  }
}

}  // namespace

size_t gemm_backward_workspace_bytes(int64_t E, int64_t N, int64_t K, int64_t rows);
bool gemm_backward_fits(int64_t rows, int64_t E);
int gemm_grouped_backward(const void* gy, const void* x, const void* w, int dtype, int64_t E, int64_t N, int64_t K,
                          const int32_t* offsets, int64_t rows, int64_t rows_per_expert, void* gx, int accumulate,
                          void* gw, int gw_f32, void* ws, size_t ws_bytes, hipStream_t stream);

size_t grouped_backward_workspace_bytes(int64_t E, int64_t N, int64_t K, int64_t rows, int dtype) {
  return is_half(dtype) ? gemm_backward_workspace_bytes(E, N, K, rows) : 256;
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int grouped_matmul_backward(const void* gy, const void* x, const void* w, int dtype, int64_t E, int64_t N, int64_t K,
                            const int32_t* offsets, int64_t rows, int64_t max_rows_per_expert, void* gx, int accumulate,
                            void* gw, int gw_dtype, void* ws, size_t ws_bytes, hipStream_t stream) {
  QW_REQUIRE(dtype == QW_F32 || dtype == QW_BF16 || dtype == QW_F16, "grouped backward dtype must be f32, bf16 or f16");
  QW_REQUIRE(gw_dtype == dtype || gw_dtype == QW_F32, "grad_w dtype must be the operands' dtype or f32");
  QW_REQUIRE(E >= 1 && E <= 65535 && N >= 1 && K >= 1 && N <= INT32_MAX && K <= INT32_MAX && rows >= 0 &&
                 rows <= INT32_MAX && max_rows_per_expert >= 0,
             "bad grouped backward sizes");
  QW_REQUIRE(offsets != nullptr, "offsets are required");
  if (gx != nullptr && rows > 0) QW_REQUIRE(gy && w, "grad_x needs grad_out and w");
  if (gw != nullptr) QW_REQUIRE(rows == 0 || (gy && x), "grad_w needs grad_out and x");
  const int64_t per = max_rows_per_expert > 0 && max_rows_per_expert < rows ? max_rows_per_expert : rows;
  QW_REQUIRE(ceil_div(per, BT) <= 65535 && ceil_div(N, BT) <= 65535, "grouped backward sizes out of range");
  // matrix-core path (bf16/fp16 with a workspace): dX needs out_features % 64 == 0, dW any shape
  const bool core = is_half(dtype) && ws != nullptr && ws_bytes >= gemm_backward_workspace_bytes(E, N, K, rows) &&
                    aligned16(gy) && aligned16(x) && aligned16(w) && gemm_backward_fits(rows, E);
  const bool core_dx = core && gx != nullptr && aligned16(gx) && N % 64 == 0 && K % 4 == 0;
  const bool core_dw = core && gw != nullptr && aligned16(gw);
  if (core_dx || core_dw) {
    const int st = gemm_grouped_backward(gy, x, w, dtype, E, N, K, offsets, rows, per, core_dx ? gx : nullptr, accumulate,
                                         core_dw ? gw : nullptr, gw_dtype == QW_F32, ws, ws_bytes, stream);
    if (st) return st;
    if (core_dx) gx = nullptr;
    if (core_dw) gw = nullptr;
  }
  const int n = static_cast<int>(N), k = static_cast<int>(K), r = static_cast<int>(rows);
  // fp32 matrix-core path: 16-byte rows and bases
  const bool f32_core = dtype == QW_F32 && N % 4 == 0 && K % 4 == 0 && aligned16(gy) && aligned16(x) &&
                        aligned16(w) && (gx == nullptr || aligned16(gx)) && (gw == nullptr || aligned16(gw));
  if (f32_core && gx != nullptr && rows > 0) {
    const dim3 g(static_cast<unsigned>(ceil_div(K, FB_T)), static_cast<unsigned>(ceil_div(per, FB_T)),
                 static_cast<unsigned>(E));
    grouped_dx_f32_kernel<<<g, 256, 0, stream>>>(static_cast<const float*>(gy), static_cast<const float*>(w), offsets,
                                                 n, k, r, accumulate, static_cast<float*>(gx));
    QW_LAUNCH_CHECK("grouped_dx_f32_kernel");
    gx = nullptr;
  }
  if (f32_core && gw != nullptr && gw_dtype == QW_F32) {
    const dim3 g(static_cast<unsigned>(ceil_div(K, FB_T)), static_cast<unsigned>(ceil_div(N, FB_T)),
                 static_cast<unsigned>(E));
    grouped_dw_f32_kernel<<<g, 256, 0, stream>>>(static_cast<const float*>(gy), static_cast<const float*>(x), offsets,
                                                 n, k, r, static_cast<float*>(gw));
    QW_LAUNCH_CHECK("grouped_dw_f32_kernel");
    gw = nullptr;
  }
  if (gx != nullptr && rows > 0) {
    const dim3 g(static_cast<unsigned>(ceil_div(K, BT)), static_cast<unsigned>(ceil_div(per, BT)),
                 static_cast<unsigned>(E));
    if (dtype == QW_F32) grouped_dx_kernel<QW_F32><<<g, 256, 0, stream>>>(gy, w, offsets, n, k, r, accumulate, gx);
    else if (dtype == QW_F16) grouped_dx_kernel<QW_F16><<<g, 256, 0, stream>>>(gy, w, offsets, n, k, r, accumulate, gx);
    else grouped_dx_kernel<QW_BF16><<<g, 256, 0, stream>>>(gy, w, offsets, n, k, r, accumulate, gx);
    QW_LAUNCH_CHECK("grouped_dx_kernel");
  }
  if (gw != nullptr) {
    const dim3 g(static_cast<unsigned>(ceil_div(K, BT)), static_cast<unsigned>(ceil_div(N, BT)),
                 static_cast<unsigned>(E));
    if (dtype == QW_F32) grouped_dw_kernel<QW_F32, QW_F32><<<g, 256, 0, stream>>>(gy, x, offsets, n, k, r, gw);
    else if (dtype == QW_F16 && gw_dtype == QW_F32)
      grouped_dw_kernel<QW_F16, QW_F32><<<g, 256, 0, stream>>>(gy, x, offsets, n, k, r, gw);
    else if (dtype == QW_F16) grouped_dw_kernel<QW_F16, QW_F16><<<g, 256, 0, stream>>>(gy, x, offsets, n, k, r, gw);
    else if (gw_dtype == QW_F32) grouped_dw_kernel<QW_BF16, QW_F32><<<g, 256, 0, stream>>>(gy, x, offsets, n, k, r, gw);
    else grouped_dw_kernel<QW_BF16, QW_BF16><<<g, 256, 0, stream>>>(gy, x, offsets, n, k, r, gw);
    QW_LAUNCH_CHECK("grouped_dw_kernel");
  }
  return QW_OK;
}

}  // namespace qw
