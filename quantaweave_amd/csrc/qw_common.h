// Shared device/host helpers of the gfx950 MoE expert-FFN library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "qwmoe.h"

// ---------------------------------------------------------------------------
// Errors (host side).  The message buffer is thread-local; entry points return
// a qw_status and never abort.
// ---------------------------------------------------------------------------
namespace qw {

int set_error(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

#define QW_REQUIRE(cond, ...)                                    \
  do {                                                           \
    if (!(cond)) return ::qw::set_error(QW_ERR_INVALID, __VA_ARGS__); \
  } while (0)

#define QW_HIP_CHECK(expr)                                                            \
  do {                                                                                \
    hipError_t qw_e_ = (expr);                                                        \
    if (qw_e_ != hipSuccess)                                                          \
      return ::qw::set_error(QW_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(qw_e_)); \
  } while (0)

// Checked after every launch: reports a launch-configuration failure as a status.
#define QW_LAUNCH_CHECK(name)                                                        \
  do {                                                                               \
    hipError_t qw_e_ = hipGetLastError();                                            \
    if (qw_e_ != hipSuccess)                                                         \
      return ::qw::set_error(QW_ERR_HIP, "launch of %s failed: %s", name, hipGetErrorString(qw_e_)); \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Carves aligned sub-buffers out of a caller workspace.
struct Carver {
  char* base;
  size_t used = 0;
  explicit Carver(void* p) : base(static_cast<char*>(p)) {}
  template <typename T>
  T* take(size_t count) {
    used = align_up(used, 256);
    T* p = base ? reinterpret_cast<T*>(base + used) : nullptr;
    used += count * sizeof(T);
    return p;
  }
};

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------
constexpr int kWave = 64;

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }

// Round-to-nearest-even float -> bf16 (NaN stays NaN), the rounding torch uses
// for `.to(torch.bfloat16)`.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float round_to_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

template <int DT>
__device__ __forceinline__ float load_act(const void* p, int64_t i) {
  if constexpr (DT == QW_F32) return static_cast<const float*>(p)[i];
  else return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
}

template <int DT>
__device__ __forceinline__ void store_act(void* p, int64_t i, float v) {
  if constexpr (DT == QW_F32) static_cast<float*>(p)[i] = v;
  else static_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
}

// Rounds an fp32 value to what storing it in activation dtype DT keeps.
template <int DT>
__device__ __forceinline__ float round_act(float v) {
  if constexpr (DT == QW_F32) return v;
  else return round_to_bf16(v);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + __expf(-g)); }

// Workgroup barrier that orders LDS only.  __syncthreads() also waits for every
// outstanding global load of the wave (vmcnt(0)); this one lets global loads
// stay in flight across the barrier.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

}  // namespace qw
