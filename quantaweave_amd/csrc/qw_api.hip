// C ABI entry points (include/qwmoe.h): argument checks, workspace carving and
// kernel selection.  No entry point allocates device memory or synchronises.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "qw_ffn.h"

namespace qw {

static thread_local char g_error[512] = "";

int set_error(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return status;
}

void clear_error() { g_error[0] = '\0'; }

// Implemented in the kernel files.
int route(const void* x, int xdt, int64_t x_stride, const void* w, int wdt, int64_t T, int64_t D, int64_t E,
          int64_t K, float temperature, const float* bias, float* logits, float* probs, int32_t* top_idx,
          float* top_w, float* partial, size_t partial_bytes, hipStream_t stream, bool select_logits = false);
size_t route_workspace_bytes(int64_t T, int64_t D, int64_t E);
int route_from_logits(const float* logits, int64_t T, int64_t E, int64_t K, const float* bias, float* probs,
                      int32_t* top_idx, float* top_w, hipStream_t stream);
size_t plan_workspace_bytes(int64_t T, int64_t K, int64_t E);
bool route_plan_small_fits(int64_t T, int64_t E, int64_t K);
int route_plan_small(const void* x, int xdt, int64_t x_stride, const void* w, int wdt, int64_t T, int64_t D,
                     int64_t E, int64_t K, float temperature, const float* bias, bool select_logits, float* logits,
                     float* probs, int32_t* top_idx, float* top_w, int64_t capacity, int32_t* counts,
                     int32_t* kept_counts, int32_t* kept_offsets, int32_t* totals, int32_t* slot_token,
                     float* slot_weight, int32_t* route_slot, int32_t* dropped_token, int32_t* dropped_expert,
                     const float* cast_x, uint16_t* cast_out, int cast_dtype, float* partial,
                     size_t partial_bytes, hipStream_t stream);
int plan(const int32_t* top_idx, const float* top_w, int64_t T, int64_t K, int64_t E, int64_t capacity,
         int32_t* counts, int32_t* kept_counts, int32_t* kept_offsets, int32_t* slot_token, float* slot_weight,
         int32_t* route_slot, int32_t* dropped_token, int32_t* dropped_expert, int32_t* totals, void* ws,
         size_t ws_bytes, hipStream_t stream);
int permute(const void* x, int dtype, int64_t D, const int32_t* slot_token, const int32_t* totals, int64_t max_rows,
            void* out, hipStream_t stream);
int combine(const void* y, int dtype, const int32_t* route_slot, const int32_t* top_idx, int64_t T, int64_t K,
            int64_t D, void* out, hipStream_t stream);
int decode_combine(const void* y, int dtype, const int32_t* route_slot, const float* top_w, const float* residual,
                   int64_t T, int64_t K, int64_t D, float* out, hipStream_t stream);
int cast_half(const float* x, int64_t n, uint16_t* out, int dtype, hipStream_t stream);
int pack_bf16_tiles(const void* w, int64_t E, int64_t rows, int64_t cols, void* out, hipStream_t stream);
size_t balance_workspace_bytes(int64_t T, int64_t E);
int balance_ws(const float* probs, const int32_t* counts, int64_t T, int64_t K, int64_t E, float* importance,
               float* bal, void* ws, size_t ws_bytes, hipStream_t stream);
int balance(const float* probs, const int32_t* counts, int64_t T, int64_t K, int64_t E, float* importance,
            float* bal, hipStream_t stream, float* scratch_importance);
int quantize(const void* w, int wdt, int64_t rows, int64_t cols, int bits, int64_t group, void* qweight, float* scales,
             hipStream_t stream);
int dequantize(const void* qweight, const float* scales, int bits, int64_t rows, int64_t cols, int64_t group,
               float* out, hipStream_t stream);
int grouped_matmul_generic(const void* x, int act, const WView& w, int wfmt, int64_t E, const int32_t* offsets,
                           int64_t rows, void* out, hipStream_t stream);
int combine_weighted(const void* y, int dtype, const int32_t* route_slot, const int32_t* top_idx, const float* top_w,
                     int64_t T, int64_t K, int64_t D, void* out, int out_dtype, hipStream_t stream);
int combine_static(const void* y, int dtype, const int32_t* route_slot, const int32_t* top_idx, const float* top_w,
                   int64_t T, int64_t K, int64_t D, void* out, int out_dtype, hipStream_t stream);
int grouped_matmul_backward(const void* gy, const void* x, const void* w, int dtype, int64_t E, int64_t N, int64_t K,
                            const int32_t* offsets, int64_t rows, int64_t max_rows_per_expert, void* gx, int accumulate,
                            void* gw, int gw_dtype, void* ws, size_t ws_bytes, hipStream_t stream);
size_t grouped_backward_workspace_bytes(int64_t E, int64_t N, int64_t K, int64_t rows, int dtype);
bool gemm_rows_fits(int64_t K, int64_t rows, int64_t E);
int gemm_grouped_forward(const void* x, const void* w, int dtype, int64_t E, int64_t N, int64_t K,
                         const int32_t* offsets, int64_t rows, int64_t rows_per_expert, void* out, hipStream_t stream);
int swiglu(const void* g, const void* u, int dtype, int64_t n, void* h, hipStream_t stream);
int swiglu_backward(const void* dh, const void* g, const void* u, int dtype, int64_t n, void* dg, void* du,
                    hipStream_t stream);
int combine_backward(const void* grad_out, int out_dtype, const void* y, int y_dtype, const int32_t* route_slot,
                     const float* top_w, int64_t T, int64_t K, int64_t D, void* grad_y, float* grad_top_w,
                     hipStream_t stream);
int route_backward(const float* probs, const int32_t* top_idx, const float* top_w, const float* grad_top_w,
                   const float* grad_probs, const float* grad_balance, const int32_t* counts, int64_t T, int64_t E,
                   int64_t K, float temperature, float* out, hipStream_t stream);

static size_t act_size(int dt) { return dt == QW_F32 ? 4 : 2; }

size_t experts_workspace_bytes(int64_t max_rows, int64_t E, int64_t D, int64_t F, int act) {
  (void)E;
  Carver c(nullptr);
  c.take<char>(static_cast<size_t>(max_rows) * F * act_size(act));  // hidden
  c.take<float>(static_cast<size_t>(max_rows) * D);                  // split-K partials (decode)
  return c.used + 256;
}

int experts(const void* x, int act, const int32_t* row_index, const int32_t* offsets, int64_t E, int64_t D, int64_t F,
            int64_t max_rows, int wfmt, int64_t group_in, int64_t group_ff, const void* gate_w, const float* gate_s,
            const void* up_w, const float* up_s, const void* down_w, const float* down_s, const float* row_weight,
            void* y, void* ws, size_t ws_bytes, hipStream_t stream, int64_t avg_rows, int64_t row_cap,
            void* save_gate = nullptr, void* save_up = nullptr, void* save_y = nullptr,
            void* hidden_out = nullptr, int path = QW_PATH_AUTO) {
  QW_REQUIRE(path >= QW_PATH_AUTO && path <= QW_PATH_STREAM, "unknown kernel path %d", path);
  QW_REQUIRE(act == QW_F32 || act == QW_BF16 || act == QW_F16, "activation dtype must be f32, bf16 or f16");
  QW_REQUIRE(wfmt >= QW_F32 && wfmt <= QW_F16T, "unknown weight format %d", wfmt);
  QW_REQUIRE(E >= 1 && E <= 65535, "experts out of range");
  QW_REQUIRE((wfmt != QW_BF16T && wfmt != QW_F16T) || (D % 64 == 0 && F % 64 == 0),
             "tiled weights need d_model and d_ff multiples of 64 (got %lld, %lld)", (long long)D, (long long)F);
  QW_REQUIRE(D >= 1 && D <= INT32_MAX / 2 && F >= 1 && F <= INT32_MAX / 2, "d_model/d_ff out of range");
  QW_REQUIRE(max_rows >= 0 && max_rows <= INT32_MAX, "max_rows out of range");
  if (wfmt == QW_I8 || wfmt == QW_U4) {
    QW_REQUIRE(group_in >= 1 && group_ff >= 1, "quantised weights need positive group sizes");
    QW_REQUIRE(wfmt == QW_I8 || (group_in % 2 == 0 && group_ff % 2 == 0),
               "group_size must be even for 4-bit weights");
    QW_REQUIRE(gate_s && up_s && down_s, "quantised weights need scales");
  }
  if (max_rows == 0) return QW_OK;
  QW_REQUIRE(x && offsets && gate_w && up_w && down_w && y, "experts pointers are required");
  const size_t need = experts_workspace_bytes(max_rows, E, D, F, act);
  if (ws_bytes < need || !ws)
    return set_error(QW_ERR_WORKSPACE, "experts workspace needs %zu bytes, got %zu", need, ws_bytes);
  Carver c(ws);
  FfnArgs a{};
  a.x = x;
  a.row_index = row_index;
  a.offsets = offsets;
  a.experts = E;
  a.d_model = D;
  a.d_ff = F;
  a.max_rows = max_rows;
  a.act = act;
  a.wfmt = wfmt;
  a.gate = make_wview(wfmt, gate_w, gate_s, F, D, group_in);
  a.up = make_wview(wfmt, up_w, up_s, F, D, group_in);
  a.down = make_wview(wfmt, down_w, down_s, D, F, group_ff);
  a.row_weight = row_weight;
  a.hidden = c.take<char>(static_cast<size_t>(max_rows) * F * act_size(act));
  if (hidden_out) a.hidden = hidden_out;
  a.partial = c.take<float>(static_cast<size_t>(max_rows) * D);
  a.save_gate = save_gate;
  a.save_up = save_up;
  a.save_y = save_y;
  a.y = y;
  a.avg_rows = avg_rows;
  a.row_cap = row_cap;
  bool handled = false;
  int st = QW_OK;
  switch (path) {
    case QW_PATH_GENERAL:
      return launch_ffn_generic(a, stream);
    case QW_PATH_STREAM:
      a.avg_rows = 0;  // the family is chosen: no row-count threshold
      st = launch_ffn_gemv(a, stream, &handled);
      if (st || handled) return st;
      return set_error(QW_ERR_UNSUPPORTED, "the weight-streaming kernels do not take this shape or format");
    case QW_PATH_MFMA:
      a.avg_rows = std::max<int64_t>(a.avg_rows, 16);
      st = launch_ffn_mfma(a, stream, &handled);
      if (st || handled) return st;
      st = launch_ffn_f32(a, stream, &handled);
      if (st || handled) return st;
      return set_error(QW_ERR_UNSUPPORTED, "the matrix-core kernels do not take this shape or format");
    default:
      st = launch_ffn_gemv(a, stream, &handled);
      if (st || handled) return st;
      st = launch_ffn_mfma(a, stream, &handled);
      if (st || handled) return st;
      st = launch_ffn_f32(a, stream, &handled);
      if (st || handled) return st;
      return launch_ffn_generic(a, stream);
  }
}

size_t forward_workspace_bytes(int64_t T, int64_t D, int64_t E, int64_t K, int64_t F, int act) {
  const int64_t R = T * K;
  Carver c(nullptr);
  c.take<float>(static_cast<size_t>(T) * E);  // logits
  c.take<int32_t>(R);                           // slot_token
  c.take<float>(R);                             // slot_weight
  c.take<int32_t>(R);                           // route_slot
  c.take<int32_t>(E + 1);                       // kept_offsets
  c.take<char>(static_cast<size_t>(R) * D * act_size(act));  // y
  c.take<char>(plan_workspace_bytes(T, K, E));
  c.take<char>(experts_workspace_bytes(R, E, D, F, act));
  c.take<char>(route_workspace_bytes(T, D, E));
  return c.used + 256;
}

// The decode step keeps its plan in the workspace: one carve serves both the
// size query and the call.
struct DecodeWs {
  float* logits;
  int32_t *counts, *kept_counts, *kept_offsets, *totals;
  int32_t *slot_token, *route_slot, *dropped_token, *dropped_expert;
  float* slot_weight;
  uint16_t* xc;
  char* y;
  char* plan_ws;
  size_t plan_bytes;
  char* exp_ws;
  size_t exp_bytes;
  float* route_ws;
  size_t route_bytes;
  size_t used;
};

static DecodeWs carve_decode(void* base, int64_t T, int64_t D, int64_t E, int64_t K, int64_t F, int act) {
  const int64_t R = T * K;
  Carver c(base);
  DecodeWs w{};
  w.logits = c.take<float>(static_cast<size_t>(T) * E);
  w.counts = c.take<int32_t>(E);
  w.kept_counts = c.take<int32_t>(E);
  w.kept_offsets = c.take<int32_t>(E + 1);
  w.totals = c.take<int32_t>(2);
  w.slot_token = c.take<int32_t>(R);
  w.route_slot = c.take<int32_t>(R);
  w.dropped_token = c.take<int32_t>(R);
  w.dropped_expert = c.take<int32_t>(R);
  w.slot_weight = c.take<float>(R);
  w.xc = is_half(act) ? c.take<uint16_t>(static_cast<size_t>(T) * D) : nullptr;
  w.y = c.take<char>(static_cast<size_t>(R) * D * act_size(act));
  w.plan_bytes = plan_workspace_bytes(T, K, E);
  w.plan_ws = c.take<char>(w.plan_bytes);
  w.exp_bytes = experts_workspace_bytes(R, E, D, F, act);
  w.exp_ws = c.take<char>(w.exp_bytes);
  w.route_bytes = route_workspace_bytes(T, D, E);
  w.route_ws = reinterpret_cast<float*>(c.take<char>(w.route_bytes));
  w.used = c.used + 256;
  return w;
}

// ---------------------------------------------------------------------------
// Library-owned scratch of the allocation-free decode step
// (qw_moe_decode_step_noalloc): one array per device, kept until the process
// ends.  In host code `scratch` names a host-side stand-in, not device
// memory: its device address on each GPU comes from hipGetSymbolAddress,
// made once per device with that device current, and only that address is
// ever handed to kernels.
// ---------------------------------------------------------------------------
constexpr size_t kNoAllocScratchBytes = size_t(32) << 20;  // 32 MiB per device
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

static std::atomic<void*> g_scratch_ptr[kMaxDevices];

// Looks up the device address of `scratch` on the current device (once per
// device; qw_init).  The lookup can load the library's code object on that
// device, which allocates its global memory, so it must not happen inside a
// graph capture: the allocation-free entry point does it only outside one.
static int scratch_lookup(int dev, void** out) {
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    QW_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return set_error(QW_ERR_HIP, "hipGetSymbolAddress returned no address for the scratch array");
    g_scratch_ptr[dev].store(p, std::memory_order_release);  // the same address whoever stores it first
  }
  *out = p;
  return QW_OK;
}

static int current_device(int* dev) {
  QW_HIP_CHECK(hipGetDevice(dev));
  if (*dev < 0 || *dev >= kMaxDevices)
    return set_error(QW_ERR_UNSUPPORTED, "device %d is beyond the library's table", *dev);
  return QW_OK;
}

}  // namespace qw

using namespace qw;

extern "C" {

const char* qw_last_error(void) { return g_error; }

int qw_abi_version(void) { return 1; }

int64_t qw_moe_capacity(int64_t tokens, int64_t top_k, int64_t experts, double capacity_factor,
                        double capacity_scale, int64_t min_capacity, int drop_overflow) {
  if (tokens < 0 || top_k < 1 || experts < 1 || min_capacity < 1 || capacity_factor < 0) {
    set_error(QW_ERR_INVALID, "bad capacity arguments");
    return QW_ERR_INVALID;
  }
  if (capacity_factor > 0 && drop_overflow) {
    // Python: num_tokens * top_k / num_experts * capacity_factor * capacity_scale,
    // int*int is exact, `/` is true division in double, then left to right.
    const double v = static_cast<double>(tokens * top_k) / static_cast<double>(experts) * capacity_factor *
                     capacity_scale;
    const double c = std::ceil(v);
    if (!(c < 9.2e18)) {
      set_error(QW_ERR_INVALID, "capacity overflows int64");
      return QW_ERR_INVALID;
    }
    const int64_t ci = static_cast<int64_t>(c);
    return ci > min_capacity ? ci : min_capacity;
  }
  return tokens * top_k;
}

size_t qw_moe_route_workspace_bytes(int64_t tokens, int64_t d_model, int64_t experts) {
  if (tokens < 0 || d_model < 1 || experts < 1) return 0;
  return route_workspace_bytes(tokens, d_model, experts);
}

int qw_moe_route(const void* x, int x_dtype, int64_t x_row_stride, const void* router_w, int w_dtype, int64_t tokens,
                 int64_t d_model, int64_t experts, int64_t top_k, float temperature, const float* expert_bias,
                 float* logits, float* probs, int32_t* top_idx, float* top_w, void* workspace,
                 size_t workspace_bytes, void* stream) {
  clear_error();
  return route(x, x_dtype, x_row_stride, router_w, w_dtype, tokens, d_model, experts, top_k, temperature, expert_bias,
               logits, probs, top_idx, top_w, static_cast<float*>(workspace), workspace_bytes, as_stream(stream));
}

int qw_moe_route_from_logits(const float* logits, int64_t tokens, int64_t experts, int64_t top_k,
                             const float* expert_bias, float* probs, int32_t* top_idx, float* top_w, void* stream) {
  clear_error();
  return route_from_logits(logits, tokens, experts, top_k, expert_bias, probs, top_idx, top_w, as_stream(stream));
}

size_t qw_moe_plan_workspace_bytes(int64_t tokens, int64_t top_k, int64_t experts) {
  if (tokens < 0 || top_k < 1 || experts < 1) return 0;
  return plan_workspace_bytes(tokens, top_k, experts);
}

int qw_moe_plan(const int32_t* top_idx, const float* top_w, int64_t tokens, int64_t top_k, int64_t experts,
                int64_t capacity, int32_t* counts, int32_t* kept_counts, int32_t* kept_offsets, int32_t* slot_token,
                float* slot_weight, int32_t* route_slot, int32_t* dropped_token, int32_t* dropped_expert,
                int32_t* totals, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  return plan(top_idx, top_w, tokens, top_k, experts, capacity, counts, kept_counts, kept_offsets, slot_token,
              slot_weight, route_slot, dropped_token, dropped_expert, totals, workspace, workspace_bytes,
              as_stream(stream));
}

int qw_moe_permute(const void* x, int dtype, int64_t d_model, const int32_t* slot_token, const int32_t* totals,
                   int64_t max_rows, void* out, void* stream) {
  clear_error();
  return permute(x, dtype, d_model, slot_token, totals, max_rows, out, as_stream(stream));
}

size_t qw_moe_experts_workspace_bytes(int64_t max_rows, int64_t experts, int64_t d_model, int64_t d_ff,
                                      int act_dtype) {
  if (max_rows < 0 || experts < 1 || d_model < 1 || d_ff < 1) return 0;
  return experts_workspace_bytes(max_rows, experts, d_model, d_ff, act_dtype);
}

int qw_moe_experts(const void* x, int act_dtype, const int32_t* row_index, const int32_t* kept_offsets,
                   int64_t experts, int64_t d_model, int64_t d_ff, int64_t max_rows, int64_t max_rows_per_expert,
                   int w_format, int64_t group_in,
                   int64_t group_ff, const void* gate_w, const float* gate_scales, const void* up_w,
                   const float* up_scales, const void* down_w, const float* down_scales, const float* row_weight,
                   void* y, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  QW_REQUIRE(max_rows_per_expert >= 0, "max_rows_per_expert must be >= 0");
  const int64_t cap = (max_rows_per_expert > 0 && max_rows_per_expert < max_rows) ? max_rows_per_expert : max_rows;
  int64_t avg = experts > 0 ? (max_rows + experts - 1) / experts : 0;
  if (avg > cap) avg = cap;
  return qw::experts(x, act_dtype, row_index, kept_offsets, experts, d_model, d_ff, max_rows, w_format, group_in,
                     group_ff, gate_w, gate_scales, up_w, up_scales, down_w, down_scales, row_weight, y, workspace,
                     workspace_bytes, as_stream(stream), avg, cap);
}

int qw_moe_experts_on_path(int path, const void* x, int act_dtype, const int32_t* row_index,
                           const int32_t* kept_offsets, int64_t experts, int64_t d_model, int64_t d_ff,
                           int64_t max_rows, int64_t max_rows_per_expert, int w_format, int64_t group_in,
                           int64_t group_ff, const void* gate_w, const float* gate_scales, const void* up_w,
                           const float* up_scales, const void* down_w, const float* down_scales,
                           const float* row_weight, void* y, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  QW_REQUIRE(max_rows_per_expert >= 0, "max_rows_per_expert must be >= 0");
  const int64_t cap = (max_rows_per_expert > 0 && max_rows_per_expert < max_rows) ? max_rows_per_expert : max_rows;
  int64_t avg = experts > 0 ? (max_rows + experts - 1) / experts : 0;
  if (avg > cap) avg = cap;
  return qw::experts(x, act_dtype, row_index, kept_offsets, experts, d_model, d_ff, max_rows, w_format, group_in,
                     group_ff, gate_w, gate_scales, up_w, up_scales, down_w, down_scales, row_weight, y, workspace,
                     workspace_bytes, as_stream(stream), avg, cap, nullptr, nullptr, nullptr, nullptr, path);
}

int qw_moe_combine(const void* y, int dtype, const int32_t* route_slot, const int32_t* top_idx, int64_t tokens,
                   int64_t top_k, int64_t d_model, void* out, void* stream) {
  clear_error();
  return combine(y, dtype, route_slot, top_idx, tokens, top_k, d_model, out, as_stream(stream));
}

int qw_moe_balance(const float* probs, const int32_t* counts, int64_t tokens, int64_t top_k, int64_t experts,
                   float* importance, float* balance_out, void* stream) {
  clear_error();
  QW_REQUIRE(importance != nullptr, "importance buffer [experts] is required");
  return balance(probs, counts, tokens, top_k, experts, importance, balance_out, as_stream(stream), nullptr);
}

size_t qw_moe_balance_workspace_bytes(int64_t tokens, int64_t experts) {
  if (tokens < 1 || experts < 1) return 0;
  return balance_workspace_bytes(tokens, experts);
}

int qw_moe_balance_ws(const float* probs, const int32_t* counts, int64_t tokens, int64_t top_k, int64_t experts,
                      float* importance, float* balance_out, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  return balance_ws(probs, counts, tokens, top_k, experts, importance, balance_out, workspace, workspace_bytes,
                    as_stream(stream));
}

size_t qw_moe_forward_workspace_bytes(int64_t tokens, int64_t d_model, int64_t experts, int64_t top_k, int64_t d_ff,
                                      int act_dtype) {
  if (tokens < 0 || d_model < 1 || experts < 1 || top_k < 1 || d_ff < 1) return 0;
  return forward_workspace_bytes(tokens, d_model, experts, top_k, d_ff, act_dtype);
}

int qw_moe_forward(const void* x, int act_dtype, int64_t tokens, int64_t d_model, const void* router_w,
                   int router_dtype, float temperature, const float* expert_bias, int64_t experts, int64_t top_k,
                   int64_t capacity, int64_t d_ff, int w_format, int64_t group_in, int64_t group_ff,
                   const void* gate_w, const float* gate_scales, const void* up_w, const float* up_scales,
                   const void* down_w, const float* down_scales, void* out, float* probs, int32_t* top_idx,
                   float* top_w, int32_t* counts, int32_t* kept_counts, int32_t* totals, int32_t* dropped_token,
                   int32_t* dropped_expert, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  QW_REQUIRE(act_dtype == QW_F32 || act_dtype == QW_BF16 || act_dtype == QW_F16,
             "activation dtype must be f32, bf16 or f16");
  QW_REQUIRE(tokens >= 0 && top_k >= 1 && experts >= 1 && d_model >= 1 && d_ff >= 1, "bad forward sizes");
  QW_REQUIRE(capacity >= 0, "capacity must be >= 0");
  QW_REQUIRE(probs && top_idx && top_w && counts && kept_counts && totals, "forward outputs are required");
  if (tokens == 0) return QW_OK;
  QW_REQUIRE(out && dropped_token && dropped_expert, "forward outputs are required");
  const size_t need = forward_workspace_bytes(tokens, d_model, experts, top_k, d_ff, act_dtype);
  if (!workspace || workspace_bytes < need)
    return set_error(QW_ERR_WORKSPACE, "forward workspace needs %zu bytes, got %zu", need, workspace_bytes);
  hipStream_t s = as_stream(stream);
  const int64_t R = tokens * top_k;
  Carver c(workspace);
  float* logits = c.take<float>(static_cast<size_t>(tokens) * experts);
  int32_t* slot_token = c.take<int32_t>(R);
  float* slot_weight = c.take<float>(R);
  int32_t* route_slot = c.take<int32_t>(R);
  int32_t* kept_offsets = c.take<int32_t>(experts + 1);
  char* y = c.take<char>(static_cast<size_t>(R) * d_model * act_size(act_dtype));
  const size_t plan_ws = plan_workspace_bytes(tokens, top_k, experts);
  char* pws = c.take<char>(plan_ws);
  const int64_t max_rows = std::min<int64_t>(R, capacity * experts);
  const size_t exp_ws = experts_workspace_bytes(R, experts, d_model, d_ff, act_dtype);
  char* ews = c.take<char>(exp_ws);
  const size_t route_ws = route_workspace_bytes(tokens, d_model, experts);
  float* rws = reinterpret_cast<float*>(c.take<char>(route_ws));
  int st;
  if (route_plan_small_fits(tokens, experts, top_k)) {
    st = route_plan_small(x, act_dtype, d_model, router_w, router_dtype, tokens, d_model, experts, top_k, temperature,
                          expert_bias, false, logits, probs, top_idx, top_w, capacity, counts, kept_counts,
                          kept_offsets, totals, slot_token, slot_weight, route_slot, dropped_token, dropped_expert,
                          nullptr, nullptr, act_dtype, rws, route_ws, s);
    if (st) return st;
  } else {
    st = route(x, act_dtype, d_model, router_w, router_dtype, tokens, d_model, experts, top_k, temperature,
               expert_bias, logits, probs, top_idx, top_w, rws, route_ws, s);
    if (st) return st;
    st = plan(top_idx, top_w, tokens, top_k, experts, capacity, counts, kept_counts, kept_offsets, slot_token,
              slot_weight, route_slot, dropped_token, dropped_expert, totals, pws, plan_ws, s);
    if (st) return st;
  }
  // The experts store unweighted rows and the combine applies the route
  // weights: it computes the same bf16(bf16(y) * w) per route that the
  // expert kernels would store, and the down projection's epilogue then waits
  // on no weight loads.
  if (max_rows > 0) {
    const int64_t avg = (R + experts - 1) / experts;
    st = qw::experts(x, act_dtype, slot_token, kept_offsets, experts, d_model, d_ff, max_rows, w_format, group_in,
                     group_ff, gate_w, gate_scales, up_w, up_scales, down_w, down_scales, nullptr, y, ews, exp_ws, s,
                     avg < capacity ? avg : capacity, std::min<int64_t>(capacity, R));
    if (st) return st;
  }
  return combine_weighted(y, act_dtype, route_slot, top_idx, top_w, tokens, top_k, d_model, out, act_dtype, s);
}

size_t qw_moe_decode_step_workspace_bytes(int64_t tokens, int64_t d_model, int64_t experts, int64_t top_k,
                                          int64_t d_ff, int compute_dtype) {
  if (tokens < 0 || d_model < 1 || experts < 1 || top_k < 1 || d_ff < 1) return 0;
  if (compute_dtype != QW_F32 && compute_dtype != QW_BF16 && compute_dtype != QW_F16) return 0;
  return carve_decode(nullptr, tokens, d_model, experts, top_k, d_ff, compute_dtype).used;
}

int qw_moe_decode_step(const float* x, const float* residual, int64_t tokens, int64_t d_model,
                       const float* router_w, float temperature, const float* expert_bias, int64_t experts,
                       int64_t top_k, int64_t d_ff, int compute_dtype, int w_format, int64_t group_in,
                       int64_t group_ff, const void* gate_w, const float* gate_scales, const void* up_w,
                       const float* up_scales, const void* down_w, const float* down_scales, float* out,
                       float* probs, int32_t* top_idx, float* top_w, void* workspace, size_t workspace_bytes,
                       void* stream) {
  clear_error();
  QW_REQUIRE(compute_dtype == QW_F32 || compute_dtype == QW_BF16 || compute_dtype == QW_F16,
             "compute dtype must be f32, bf16 or f16");
  QW_REQUIRE(tokens >= 0 && top_k >= 1 && experts >= 1 && d_model >= 1 && d_ff >= 1, "bad decode step sizes");
  QW_REQUIRE(top_k <= experts, "top_k must be between 1 and num_experts (got %lld, %lld)", (long long)top_k,
             (long long)experts);
  if (tokens == 0) return QW_OK;
  QW_REQUIRE(x && router_w && out && top_idx && top_w, "x, router_w, out, top_idx and top_w are required");
  const DecodeWs need = carve_decode(nullptr, tokens, d_model, experts, top_k, d_ff, compute_dtype);
  if (!workspace || workspace_bytes < need.used)
    return set_error(QW_ERR_WORKSPACE, "decode step workspace needs %zu bytes, got %zu", need.used, workspace_bytes);
  hipStream_t s = as_stream(stream);
  const int64_t R = tokens * top_k;
  const DecodeWs w = carve_decode(workspace, tokens, d_model, experts, top_k, d_ff, compute_dtype);
  // capacity R: every route keeps its slot
  const void* xc = is_half(compute_dtype) ? static_cast<const void*>(w.xc) : static_cast<const void*>(x);
  int st;
  if (route_plan_small_fits(tokens, experts, top_k)) {
    st = route_plan_small(x, QW_F32, d_model, router_w, QW_F32, tokens, d_model, experts, top_k, temperature,
                          expert_bias, /*select_logits=*/true, w.logits, probs, top_idx, top_w, R, w.counts,
                          w.kept_counts, w.kept_offsets, w.totals, w.slot_token, w.slot_weight, w.route_slot,
                          w.dropped_token, w.dropped_expert, x, is_half(compute_dtype) ? w.xc : nullptr,
                          compute_dtype, w.route_ws, w.route_bytes, s);
    if (st) return st;
  } else {
    st = route(x, QW_F32, d_model, router_w, QW_F32, tokens, d_model, experts, top_k, temperature, expert_bias,
               w.logits, probs, top_idx, top_w, w.route_ws, w.route_bytes, s, /*select_logits=*/true);
    if (st) return st;
    st = plan(top_idx, top_w, tokens, top_k, experts, R, w.counts, w.kept_counts, w.kept_offsets, w.slot_token,
              w.slot_weight, w.route_slot, w.dropped_token, w.dropped_expert, w.totals, w.plan_ws, w.plan_bytes, s);
    if (st) return st;
    if (is_half(compute_dtype)) {
      st = cast_half(x, tokens * d_model, w.xc, compute_dtype, s);
      if (st) return st;
    }
  }
  const int64_t avg = (R + experts - 1) / experts;
  st = qw::experts(xc, compute_dtype, w.slot_token, w.kept_offsets, experts, d_model, d_ff, R, w_format, group_in,
                   group_ff, gate_w, gate_scales, up_w, up_scales, down_w, down_scales, nullptr, w.y, w.exp_ws,
                   w.exp_bytes, s, avg, std::min<int64_t>(tokens, R));
  if (st) return st;
  return decode_combine(w.y, compute_dtype, w.route_slot, top_w, residual, tokens, top_k, d_model, out, s);
}

int qw_init(void) {
  clear_error();
  int dev = 0;
  if (const int st = current_device(&dev)) return st;
  void* p = nullptr;
  return scratch_lookup(dev, &p);
}

size_t qw_moe_decode_step_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

int qw_moe_decode_step_noalloc(const float* x, const float* residual, int64_t tokens, int64_t d_model,
                               const float* router_w, float temperature, const float* expert_bias, int64_t experts,
                               int64_t top_k, int64_t d_ff, int compute_dtype, int w_format, int64_t group_in,
                               int64_t group_ff, const void* gate_w, const float* gate_scales, const void* up_w,
                               const float* up_scales, const void* down_w, const float* down_scales, float* out,
                               float* probs, int32_t* top_idx, float* top_w, void* stream) {
  clear_error();
  QW_REQUIRE(compute_dtype == QW_F32 || compute_dtype == QW_BF16 || compute_dtype == QW_F16,
             "compute dtype must be f32, bf16 or f16");
  QW_REQUIRE(tokens >= 0 && top_k >= 1 && experts >= 1 && d_model >= 1 && d_ff >= 1, "bad decode step sizes");
  // sizes first: an oversized call is refused before any device work
  const size_t need = carve_decode(nullptr, tokens, d_model, experts, top_k, d_ff, compute_dtype).used;
  QW_REQUIRE(need <= kNoAllocScratchBytes,
             "this decode step needs %zu bytes of scratch; the allocation-free entry point has %zu per device "
             "(use qw_moe_decode_step with a workspace)",
             need, kNoAllocScratchBytes);
  if (tokens == 0) return QW_OK;
  hipStream_t s = as_stream(stream);
  if (s != nullptr) {  // the scratch address is per device: the stream must be on the current device
    int cur = 0, sdev = 0;
    QW_HIP_CHECK(hipGetDevice(&cur));
    QW_HIP_CHECK(hipStreamGetDevice(s, &sdev));
    QW_REQUIRE(sdev == cur, "the stream belongs to device %d but device %d is current", sdev, cur);
  }
  int dev = 0;
  if (const int st = current_device(&dev)) return st;
  void* ws = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!ws) {
    // not set up on this device: look the array up now unless the stream is
    // being captured (the lookup may load the code object and allocate)
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    QW_HIP_CHECK(hipStreamIsCapturing(s, &cap));
    QW_REQUIRE(cap == hipStreamCaptureStatusNone,
               "qw_moe_decode_step_noalloc: call qw_init() on device %d outside graph capture before capturing it",
               dev);
    if (const int st = scratch_lookup(dev, &ws)) return st;
  }
  return qw_moe_decode_step(x, residual, tokens, d_model, router_w, temperature, expert_bias, experts, top_k, d_ff,
                            compute_dtype, w_format, group_in, group_ff, gate_w, gate_scales, up_w, up_scales, down_w,
                            down_scales, out, probs, top_idx, top_w, ws, kNoAllocScratchBytes, stream);
}

int qw_quantize(const void* w, int w_dtype, int64_t out_features, int64_t in_features, int bits, int64_t group_size,
                void* qweight, float* scales, void* stream) {
  clear_error();
  return quantize(w, w_dtype, out_features, in_features, bits, group_size, qweight, scales, as_stream(stream));
}

int qw_dequantize(const void* qweight, const float* scales, int bits, int64_t out_features, int64_t in_features,
                  int64_t group_size, float* out, void* stream) {
  clear_error();
  return dequantize(qweight, scales, bits, out_features, in_features, group_size, out, as_stream(stream));
}

int qw_pack_bf16_tiles(const void* w, int64_t experts, int64_t out_features, int64_t in_features, void* tiled,
                       void* stream) {
  clear_error();
  return pack_bf16_tiles(w, experts, out_features, in_features, tiled, as_stream(stream));
}

int qw_grouped_matmul(const void* x, int act_dtype, const void* w, int w_format, const float* scales, int64_t group,
                      int64_t experts, int64_t out_features, int64_t in_features, const int32_t* offsets,
                      int64_t rows, int64_t max_rows_per_expert, void* out, void* stream) {
  clear_error();
  QW_REQUIRE(act_dtype == QW_F32 || act_dtype == QW_BF16 || act_dtype == QW_F16,
             "grouped_matmul dtype must be f32, bf16 or f16");
  QW_REQUIRE(w_format >= QW_F32 && w_format <= QW_F16T, "unknown weight format %d", w_format);
  QW_REQUIRE((w_format != QW_BF16T && w_format != QW_F16T) || (out_features % 8 == 0 && in_features % 64 == 0),
             "tiled weights need out_features %% 8 == 0 and in_features %% 64 == 0");
  QW_REQUIRE(experts >= 1 && experts <= 65535 && out_features >= 1 && in_features >= 1 && rows >= 0 &&
                 out_features <= INT32_MAX / 2 && in_features <= INT32_MAX / 2 && rows <= INT32_MAX,
             "bad grouped_matmul sizes");
  if (w_format == QW_I8 || w_format == QW_U4) {
    QW_REQUIRE(group >= 1 && (w_format == QW_I8 || group % 2 == 0), "bad group size for quantised weights");
    QW_REQUIRE(scales != nullptr, "quantised weights need scales");
  }
  QW_REQUIRE(max_rows_per_expert >= 0, "max_rows_per_expert must be >= 0");
  if (rows == 0) return QW_OK;
  QW_REQUIRE(x && w && offsets && out, "grouped_matmul pointers are required");
  const int64_t per = max_rows_per_expert > 0 && max_rows_per_expert < rows ? max_rows_per_expert : rows;
  if (is_half(act_dtype) && w_format == act_dtype && gemm_rows_fits(in_features, rows, experts) &&
      ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(out)) & 15) == 0)
    return gemm_grouped_forward(x, w, act_dtype, experts, out_features, in_features, offsets, rows, per, out, as_stream(stream));
  if (act_dtype == QW_F32 && w_format == QW_F32) {
    bool handled = false;
    const int st = grouped_matmul_f32(static_cast<const float*>(x), static_cast<const float*>(w), experts, out_features,
                                      in_features, offsets, rows, static_cast<float*>(out), as_stream(stream), &handled);
    if (st || handled) return st;
  }
  const WView v = make_wview(w_format, w, scales, out_features, in_features, group);
  return grouped_matmul_generic(x, act_dtype, v, w_format, experts, offsets, rows, out, as_stream(stream));
}

int qw_moe_experts_save(const void* x, int act_dtype, const int32_t* row_index, const int32_t* kept_offsets,
                        int64_t experts, int64_t d_model, int64_t d_ff, int64_t max_rows,
                        int64_t max_rows_per_expert, int w_format, int64_t group_in, int64_t group_ff,
                        const void* gate_w, const float* gate_scales, const void* up_w, const float* up_scales,
                        const void* down_w, const float* down_scales, const float* row_weight, void* y,
                        void* gate_out, void* up_out, void* hidden_out, void* y_unweighted, void* workspace,
                        size_t workspace_bytes, void* stream) {
  clear_error();
  QW_REQUIRE(max_rows_per_expert >= 0, "max_rows_per_expert must be >= 0");
  QW_REQUIRE(gate_out && up_out && hidden_out && y_unweighted, "the saved activation buffers are required");
  const int64_t cap = (max_rows_per_expert > 0 && max_rows_per_expert < max_rows) ? max_rows_per_expert : max_rows;
  int64_t avg = experts > 0 ? (max_rows + experts - 1) / experts : 0;
  if (avg > cap) avg = cap;
  return qw::experts(x, act_dtype, row_index, kept_offsets, experts, d_model, d_ff, max_rows, w_format, group_in,
                     group_ff, gate_w, gate_scales, up_w, up_scales, down_w, down_scales, row_weight, y, workspace,
                     workspace_bytes, as_stream(stream), avg, cap, gate_out, up_out, y_unweighted, hidden_out);
}

int qw_moe_combine_weighted(const void* y, int y_dtype, const int32_t* route_slot, const int32_t* top_idx,
                            const float* top_w, int64_t tokens, int64_t top_k, int64_t d_model, void* out,
                            int out_dtype, void* stream) {
  clear_error();
  return combine_weighted(y, y_dtype, route_slot, top_idx, top_w, tokens, top_k, d_model, out, out_dtype,
                          as_stream(stream));
}

int qw_moe_combine_static(const void* y, int y_dtype, const int32_t* route_slot, const int32_t* top_idx,
                          const float* top_w, int64_t tokens, int64_t top_k, int64_t d_model, void* out,
                          int out_dtype, void* stream) {
  clear_error();
  return combine_static(y, y_dtype, route_slot, top_idx, top_w, tokens, top_k, d_model, out, out_dtype,
                        as_stream(stream));
}

size_t qw_grouped_matmul_backward_workspace_bytes(int64_t experts, int64_t out_features, int64_t in_features,
                                                  int64_t rows, int dtype) {
  if (experts < 1 || out_features < 1 || in_features < 1 || rows < 0) return 0;
  return grouped_backward_workspace_bytes(experts, out_features, in_features, rows, dtype);
}

int qw_grouped_matmul_backward(const void* grad_out, const void* x, const void* w, int dtype, int64_t experts,
                               int64_t out_features, int64_t in_features, const int32_t* offsets, int64_t rows,
                               int64_t max_rows_per_expert, void* grad_x, int accumulate_grad_x, void* grad_w,
                               int grad_w_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  return grouped_matmul_backward(grad_out, x, w, dtype, experts, out_features, in_features, offsets, rows,
                                 max_rows_per_expert, grad_x, accumulate_grad_x, grad_w, grad_w_dtype, workspace,
                                 workspace_bytes, as_stream(stream));
}

int qw_swiglu(const void* gate, const void* up, int dtype, int64_t n, void* hidden, void* stream) {
  clear_error();
  return swiglu(gate, up, dtype, n, hidden, as_stream(stream));
}

int qw_swiglu_backward(const void* grad_hidden, const void* gate, const void* up, int dtype, int64_t n,
                       void* grad_gate, void* grad_up, void* stream) {
  clear_error();
  return swiglu_backward(grad_hidden, gate, up, dtype, n, grad_gate, grad_up, as_stream(stream));
}

int qw_moe_combine_backward(const void* grad_out, int out_dtype, const void* y, int y_dtype,
                            const int32_t* route_slot, const float* top_w, int64_t tokens, int64_t top_k,
                            int64_t d_model, void* grad_y, float* grad_top_w, void* stream) {
  clear_error();
  return combine_backward(grad_out, out_dtype, y, y_dtype, route_slot, top_w, tokens, top_k, d_model, grad_y,
                          grad_top_w, as_stream(stream));
}

int qw_moe_route_backward(const float* probs, const int32_t* top_idx, const float* top_w, const float* grad_top_w,
                          const float* grad_probs, const float* grad_balance, const int32_t* counts, int64_t tokens,
                          int64_t experts, int64_t top_k, float temperature, float* grad_scores, void* stream) {
  clear_error();
  return route_backward(probs, top_idx, top_w, grad_top_w, grad_probs, grad_balance, counts, tokens, experts, top_k,
                        temperature, grad_scores, as_stream(stream));
}

}  // extern "C"
