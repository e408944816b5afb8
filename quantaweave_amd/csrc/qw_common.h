// Shared device/host helpers of the gfx950 MoE expert-FFN library.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
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

// Raises kernel K's dynamic LDS limit to `bytes` on the current device, once
// per device (the attribute is per device; a process may drive several).
template <auto K>
inline hipError_t reserve_lds(int bytes) {
  static std::atomic<uint64_t> done{0};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = dev < 64 ? (1ull << dev) : 0;
  if (bit && (done.load(std::memory_order_acquire) & bit)) return hipSuccess;
  e = hipFuncSetAttribute(reinterpret_cast<const void*>(K), hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_release);
  return e;
}

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------
constexpr int kWave = 64;

// Cache-policy operand of global_load_lds for a stream read once: the
// non-temporal bit (nt), so the lines it brings in are the first to leave the
// caches and the data that is read again (activation rows, hidden rows) stays.
// Used where every line of the stream is consumed by one load instruction
// (16-bit weight tiles and rows, int8 decode chunks); on partial-line streams
// (int4 and int8 rows in the prefill kernel, read a quarter or half line per K
// slice) it evicts lines that the next slice still needs, and is not used.
// (An enumerator, used through a constexpr local: the builtin's operand must be
// a constant that is not an l-value when the host pass parses the kernel.)
enum : int { kLoadStream = 2 };
constexpr int kMaxDevices = 64;  // per-device tables of the library (scratch addresses, occupancy caches)

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }

// Round-to-nearest-even float -> bf16, the rounding torch uses for
// `.to(torch.bfloat16)` on non-NaN values: (bits + 0x7fff + lsb) >> 16; a NaN
// keeps its sign and top payload with the quiet bit set (torch returns one
// canonical NaN).  gfx950's conversion
// instruction (v_cvt_pk_bf16_f32, what the cast compiles to) produces exactly
// these bits for every input, NaNs and denormals included; the bf16 rounding
// test pins it against the formula.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f)); }

__device__ __forceinline__ float round_to_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// IEEE binary16: the conversion rounds to nearest even (v_cvt_f16_f32), as
// torch's `.to(torch.float16)` does; values past 65504 become infinities.
// The fp32 value is pinned first (an empty asm operand): otherwise the
// compiler folds an fp32 fma or multiply feeding the conversion into one
// mixed-precision instruction (v_fma_mix*) that rounds once to fp16, where
// the reference forms the fp32 result and then rounds it to fp16.
__device__ __forceinline__ float f16_to_f32(uint16_t h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }
__device__ __forceinline__ float pin_f32(float f) {
  asm("" : "+v"(f));
  return f;
}
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(pin_f32(f)));
}
__device__ __forceinline__ float round_to_f16(float f) { return f16_to_f32(f32_to_f16(f)); }

// 16-bit activation types (QW_BF16, QW_F16) and their weight formats.
__host__ __device__ constexpr bool is_half(int dt) { return dt == QW_BF16 || dt == QW_F16; }

template <int DT>
__device__ __forceinline__ float half_to_f32(uint16_t h) {
  if constexpr (DT == QW_F16) return f16_to_f32(h);
  else return bf16_to_f32(h);
}
template <int DT>
__device__ __forceinline__ uint16_t f32_to_half(float f) {
  if constexpr (DT == QW_F16) return f32_to_f16(f);
  else return f32_to_bf16(f);
}

// Two values rounded to DT and packed, a in the low half: the bits of
// f32_to_half(a) | f32_to_half(b) << 16.  The pair is one v_cvt_pk_bf16_f32
// or v_cvt_pk_f16_f32 (fp16 inputs pinned first, as in f32_to_f16); the
// scalar form compiles to one conversion per value and an OR to merge them.
template <int DT>
__device__ __forceinline__ uint32_t pack_half2(float a, float b) {
  if constexpr (DT == QW_F16) {
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    const f16x2_t v = {static_cast<_Float16>(pin_f32(a)), static_cast<_Float16>(pin_f32(b))};
    return __builtin_bit_cast(uint32_t, v);
  } else {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
    return __builtin_bit_cast(uint32_t, v);
  }
}

template <int DT>
__device__ __forceinline__ float load_act(const void* p, int64_t i) {
  if constexpr (DT == QW_F32) return static_cast<const float*>(p)[i];
  else return half_to_f32<DT>(static_cast<const uint16_t*>(p)[i]);
}

template <int DT>
__device__ __forceinline__ void store_act(void* p, int64_t i, float v) {
  if constexpr (DT == QW_F32) static_cast<float*>(p)[i] = v;
  else static_cast<uint16_t*>(p)[i] = f32_to_half<DT>(v);
}

// Rounds an fp32 value to what storing it in activation dtype DT keeps.
template <int DT>
__device__ __forceinline__ float round_act(float v) {
  if constexpr (DT == QW_F32) return v;
  else if constexpr (DT == QW_F16) return round_to_f16(v);
  else return round_to_bf16(v);
}

// VEC consecutive activations from element i, widened to fp32, in one load
// (VEC 4 or 8 needs i aligned to VEC).
template <int DT, int VEC>
__device__ __forceinline__ void load_vec(const void* p, int64_t i, float (&v)[VEC]) {
  if constexpr (VEC == 8 && DT == QW_BF16) {
    const uint4 q = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + i);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      v[2 * u] = __uint_as_float(w[u] << 16);
      v[2 * u + 1] = __uint_as_float(w[u] & 0xffff0000u);
    }
  } else if constexpr (VEC % 4 == 0 && DT == QW_F32) {
#pragma unroll
    for (int u = 0; u < VEC; u += 4) {
      const float4 q = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i + u);
      v[u] = q.x;
      v[u + 1] = q.y;
      v[u + 2] = q.z;
      v[u + 3] = q.w;
    }
  } else if constexpr (VEC % 4 == 0 && DT == QW_F16) {
#pragma unroll
    for (int u = 0; u < VEC; u += 4) {
      const uint2 q = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p) + i + u);
      v[u] = f16_to_f32(q.x & 0xffffu);
      v[u + 1] = f16_to_f32(q.x >> 16);
      v[u + 2] = f16_to_f32(q.y & 0xffffu);
      v[u + 3] = f16_to_f32(q.y >> 16);
    }
  } else if constexpr (VEC == 4 && DT == QW_BF16) {
    const uint2 q = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p) + i);
    v[0] = __uint_as_float(q.x << 16);
    v[1] = __uint_as_float(q.x & 0xffff0000u);
    v[2] = __uint_as_float(q.y << 16);
    v[3] = __uint_as_float(q.y & 0xffff0000u);
  } else {
#pragma unroll
    for (int u = 0; u < VEC; ++u) v[u] = load_act<DT>(p, i + u);
  }
}

// Stores VEC fp32 values as activations of dtype DT (rounded to nearest even
// for bf16) from element i, in one store where VEC allows.
template <int DT, int VEC>
__device__ __forceinline__ void store_vec(void* p, int64_t i, const float (&v)[VEC]) {
  if constexpr (VEC == 8 && DT == QW_BF16) {
    uint32_t w[4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      w[u] = pack_half2<QW_BF16>(v[2 * u], v[2 * u + 1]);
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(p) + i) = make_uint4(w[0], w[1], w[2], w[3]);
  } else if constexpr (VEC % 4 == 0 && DT == QW_F32) {
#pragma unroll
    for (int u = 0; u < VEC; u += 4)
      *reinterpret_cast<float4*>(static_cast<float*>(p) + i + u) = make_float4(v[u], v[u + 1], v[u + 2], v[u + 3]);
  } else if constexpr (VEC % 4 == 0 && DT == QW_F16) {
#pragma unroll
    for (int u = 0; u < VEC; u += 4) {
      const uint32_t lo = pack_half2<QW_F16>(v[u], v[u + 1]);
      const uint32_t hi = pack_half2<QW_F16>(v[u + 2], v[u + 3]);
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p) + i + u) = make_uint2(lo, hi);
    }
  } else if constexpr (VEC == 4 && DT == QW_BF16) {
    const uint32_t lo = pack_half2<QW_BF16>(v[0], v[1]);
    const uint32_t hi = pack_half2<QW_BF16>(v[2], v[3]);
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p) + i) = make_uint2(lo, hi);
  } else {
#pragma unroll
    for (int u = 0; u < VEC; ++u) store_act<DT>(p, i + u, v[u]);
  }
}

// Tile t of a grid laid over the row blocks of E groups, group e holding rows
// [offsets[e], offsets[e+1]) clamped to [0, rows), in tiles of `gran` rows:
// returns the group (or -1 when t is past the last tile) and sets *local to the
// tile's index within it.  Every lane of the wave computes the same answer
// (wave prefix sums over 64 groups at a time), so a grid of
// ceil(rows / gran) + E tiles covers any distribution of rows.
// With stride > 1 only the groups start, start + stride, ... take part (the
// groups one XCD owns); the returned index is the group's own.
__device__ __forceinline__ int find_tile(const int32_t* __restrict__ offsets, int E, int rows, int gran, int t,
                                         int* local, int start = 0, int stride = 1) {
  const int lane = threadIdx.x % kWave;
  int carry = 0;
  const int groups = start < E ? (E - start + stride - 1) / stride : 0;
  for (int i0 = 0; i0 < groups; i0 += kWave) {
    const int e = start + stride * (i0 + lane);
    int n = 0;
    if (e < E) {
      const int lo = min(max(offsets[e], 0), rows), hi = min(offsets[e + 1], rows);
      n = hi > lo ? (hi - lo + gran - 1) / gran : 0;
    }
    int incl = n;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int v = __shfl_up(incl, o, kWave);
      if (lane >= o) incl += v;
    }
    const unsigned long long hit = __ballot(carry + incl > t);
    if (hit) {
      const int l = __ffsll(static_cast<long long>(hit)) - 1;
      *local = t - carry - __shfl(incl - n, l, kWave);
      return start + stride * (i0 + l);
    }
    carry += __shfl(incl, kWave - 1, kWave);
  }
  return -1;
}

// Value of another lane of the same 16-lane row (DPP; gfx9 controls), or the
// lane's own value where the control writes nothing.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(static_cast<int>(v), static_cast<int>(v), CTRL, 0xf, 0xf, false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i of 8 <- lane 7 - i
constexpr int kDppMirror = 0x140;      // lane i of 16 <- lane 15 - i

// Maximum over the wave, in every lane.  A maximum is exact in any order, so
// the lanes of each 16-lane row are combined with DPP moves (quad xor 1 and 2,
// half-row mirror, row mirror: no LDS round trips) and the four row maxima
// are read from lanes 15, 31, 47 and 63.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, __uint_as_float(dpp_u32<kDppXor1>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp_u32<kDppXor2>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp_u32<kDppHalfMirror>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(dpp_u32<kDppMirror>(__float_as_uint(v))));
  const int b = __float_as_int(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(b, 15));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(b, 31));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(b, 47));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(b, 63));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

template <int CTRL>
__device__ __forceinline__ uint64_t dpp_max_u64(uint64_t v) {
  const uint64_t o = (static_cast<uint64_t>(dpp_u32<CTRL>(static_cast<uint32_t>(v >> 32))) << 32) |
                     dpp_u32<CTRL>(static_cast<uint32_t>(v));
  return o > v ? o : v;
}

// Maximum of a 64-bit key over the wave, in every lane (as wave_max).
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  v = dpp_max_u64<kDppXor1>(v);
  v = dpp_max_u64<kDppXor2>(v);
  v = dpp_max_u64<kDppHalfMirror>(v);
  v = dpp_max_u64<kDppMirror>(v);
  const int hi = static_cast<int>(v >> 32), lo = static_cast<int>(v);
  uint64_t r = 0;
#pragma unroll
  for (int row = 0; row < 4; ++row) {
    const uint64_t x = (static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(hi, 16 * row + 15))) << 32) |
                       static_cast<uint32_t>(__builtin_amdgcn_readlane(lo, 16 * row + 15));
    r = x > r ? x : r;
  }
  return r;
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

// Sums V = 2^L values over the 64 lanes of the wave with 6 - L + (V - 1)
// shuffles instead of 6 V: at each of the first L steps a lane keeps half of
// its values, adds the partner's copies of them and hands over the other half.
// Afterwards every lane holds the full sum of value index lane >> (6 - L).
template <int V>
constexpr int log2i() {
  int l = 0;
  while ((1 << l) < V) ++l;
  return l;
}

// One step of reduce_scatter over the first N of V values (all indices are
// compile-time constants, so the values stay in registers).
template <int V, int N>
__device__ __forceinline__ void rs_step(float (&v)[V], int lane) {
  if constexpr (N > 1) {
    constexpr int half = N / 2;
    constexpr int o = 32 * N / V;  // lane bit that picks the half this lane keeps
    const bool upper = lane & o;
#pragma unroll
    for (int i = 0; i < half; ++i) {
      const float give = upper ? v[i] : v[i + half];
      const float keep = upper ? v[i + half] : v[i];
      v[i] = keep + __shfl_xor(give, o, kWave);
    }
    rs_step<V, half>(v, lane);
  }
}

template <int V>
__device__ __forceinline__ float reduce_scatter(float (&v)[V], int lane) {
  static_assert(V >= 1 && V <= 64 && (V & (V - 1)) == 0, "V must be a power of two <= 64");
  rs_step<V, V>(v, lane);
  float r = v[0];
#pragma unroll
  for (int o = 32 / V; o >= 1; o >>= 1) r += __shfl_xor(r, o, kWave);
  return r;
}

// Block-wide exclusive scan of one integer per thread; *total gets the sum.
template <typename T>
__device__ T block_exclusive_scan(T v, T* warp_tot, T* total) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  T incl = v;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const T n = __shfl_up(incl, o, kWave);
    if (lane >= o) incl += n;
  }
  if (lane == kWave - 1) warp_tot[wave] = incl;
  __syncthreads();
  if (wave == 0) {
    const int nw = blockDim.x / kWave;
    const T w = lane < nw ? warp_tot[lane] : T(0);
    T wi = w;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const T n = __shfl_up(wi, o, kWave);
      if (lane >= o) wi += n;
    }
    if (lane < nw) warp_tot[lane] = wi - w;
    if (lane == nw - 1) *total = wi;
  }
  __syncthreads();
  const T r = warp_tot[wave] + incl - v;
  __syncthreads();
  return r;
}

__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + __expf(-g)); }

// silu(g) = g * sigmoid(g) with the hardware reciprocal (v_rcp_f32, 1 ulp)
// instead of an IEEE division: a few ulp of fp32 in all, below the bf16/fp16
// rounding that follows, and about a third of the instructions (the prefill
// gate/up epilogue forms 80 of these per lane per tile while its compute unit
// streams nothing).  Limits as the quotient: g -> -inf gives -0 (NaN at -inf
// itself), g -> +inf gives g.
__device__ __forceinline__ float silu_fast(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }

// silu(gate) * up with the rounding points of tensors held in activation dtype
// DT: gate and up are rounded (they are stored projections), silu(gate) is
// rounded, and the caller rounds the product when it stores it.
template <int DT>
__device__ __forceinline__ float swiglu_act(float g, float u) {
  const float gr = round_act<DT>(g);
  return round_act<DT>(silu_f32(gr)) * round_act<DT>(u);
}
__device__ __forceinline__ float swiglu_bf16(float g, float u) { return swiglu_act<QW_BF16>(g, u); }

// Two SwiGLU values with the rounding points of swiglu_act (and silu_fast),
// returned as the packed 16-bit pair (element 0 in the low half) the caller
// stores.  bf16: each rounding of a pair is one v_cvt_pk_bf16_f32, and a bf16
// pair widens to fp32 with a shift and a mask.
template <int DT>
__device__ __forceinline__ uint32_t swiglu_pack2(float g0, float g1, float u0, float u1) {
  static_assert(DT == QW_BF16 || DT == QW_F16, "16-bit activations");
  if constexpr (DT == QW_BF16) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    auto round2 = [](float& a, float& b) {
      uint32_t w = pack_half2<QW_BF16>(a, b);
      // opaque to the optimiser: seeing that each half is used alone, it
      // would split the pair conversion into one per value
      asm("" : "+v"(w));
      a = __uint_as_float(w << 16);
      b = __uint_as_float(w & 0xffff0000u);
    };
    round2(g0, g1);
    round2(u0, u1);
    float s0 = silu_fast(g0), s1 = silu_fast(g1);
    round2(s0, s1);
    const bf16x2_t h = {static_cast<__bf16>(s0 * u0), static_cast<__bf16>(s1 * u1)};
    return __builtin_bit_cast(uint32_t, h);
  } else {
    auto one = [](float g, float u) {
      return f32_to_f16(round_to_f16(silu_fast(round_to_f16(g))) * round_to_f16(u));
    };
    return one(g0, u0) | (static_cast<uint32_t>(one(g1, u1)) << 16);
  }
}

// Workgroup barrier that orders LDS only.  __syncthreads() also waits for every
// outstanding global load of the wave (vmcnt(0)); this one lets global loads
// stay in flight across the barrier.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

}  // namespace qw
