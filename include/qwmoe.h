/*
 * qwmoe.h — C ABI of the MI355X (gfx950) routed-MoE expert-FFN forward path.
 *
 * Drop-in boundary for QuantaWeave's MoE layer.  Every entry point is
 * `extern "C"`, takes plain device pointers, sizes and a HIP stream
 * (`void* stream`, a hipStream_t; NULL is the null stream), is stream-ordered,
 * never synchronises the host, and returns an int status (0 = ok, < 0 = error;
 * the message is in qw_last_error(), which is thread-local).
 *
 * Ownership: every pointer is caller-owned device memory.  The library never
 * allocates device memory; entry points that need scratch take an explicit
 * `workspace` whose size the caller obtains from the matching
 * qw_*_workspace_bytes() function.  Apart from the one allocation-free entry
 * point (qw_moe_decode_step_noalloc, whose scratch is a static per-device
 * array) and two read-only per-device caches filled on first use (that
 * array's address, and the occupancy figure the int4/int8 decode kernels size
 * their grid by), the library keeps no mutable global state, so calls on
 * different streams do not interfere (calls that share a workspace must be
 * ordered on one stream).
 *
 * Reference citations are paths inside the QuantaWeave source tree.
 */
#ifndef QWMOE_H
#define QWMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element formats.  QW_F32/QW_BF16/QW_F16 describe activations and plain
 * weights (QW_F16: IEEE binary16, the reference's fp16 autocast and
 * precision="fp16" decode, src/moe_kernels.py:179-183, src/fast_decode.py:77-80).
 * QW_I8: int8 weights [out, padded] with fp32 scales [out, padded/group].
 * QW_U4: int4 weights packed two per byte [out, padded/2] — even input column
 * in the low nibble, odd column in the high nibble, each stored as q + 8 — with
 * fp32 scales [out, padded/group].  Layouts are exactly those of
 * src/quantization.py:36-40, :53-58.
 * QW_BF16T: bf16 weights [out, in] (out % 8 == 0, in % 64 == 0) rearranged
 * into 1 KiB tiles [out/8][in/64][64][8]: 16-byte piece i of tile (rb, kb)
 * holds W[r][64*kb + 8*p .. 8*p + 7] with r = 8*rb + i/8 and
 * p = (i % 8) ^ ((r / 2) % 8).  One tile is what an 8-row, 64-column operand
 * slice of the MFMA kernels holds in LDS, so it streams as one contiguous KiB.
 * No reference counterpart: it is a cache of QW_BF16 weights made by
 * qw_pack_bf16_tiles.  QW_F16T: QW_F16 weights in the same tiles (the packing
 * moves 16-bit elements, so qw_pack_bf16_tiles makes them too). */
enum qw_dtype { QW_F32 = 0, QW_BF16 = 1, QW_I8 = 2, QW_U4 = 3, QW_BF16T = 4, QW_F16 = 5, QW_F16T = 6 };

/* Status codes.  INVALID maps to ValueError, the others to RuntimeError. */
enum qw_status {
  QW_OK = 0,
  QW_ERR_INVALID = -1,     /* bad argument: size, dtype, null pointer, range */
  QW_ERR_UNSUPPORTED = -2, /* valid but not implemented for this shape/format */
  QW_ERR_HIP = -3,         /* a HIP runtime call or kernel launch failed */
  QW_ERR_WORKSPACE = -4    /* workspace missing or smaller than required */
};

/* Thread-local text of the last error raised on this thread ("" if none). */
const char* qw_last_error(void);

/* ABI revision of this library (bumped on any signature change). */
int qw_abi_version(void);

/* Route slots per expert.  Replaces TopKMoE.capacity,
 * src/quantweave_moe_model.py:100-111: when capacity_factor > 0 and
 * drop_overflow != 0 it is max(min_capacity,
 * ceil(tokens*top_k/experts*capacity_factor*capacity_scale)) evaluated in
 * double, left to right; otherwise tokens*top_k.  Returns < 0 on bad input. */
int64_t qw_moe_capacity(int64_t tokens, int64_t top_k, int64_t experts, double capacity_factor,
                        double capacity_scale, int64_t min_capacity, int drop_overflow);

/* Router, softmax, top-k and renormalisation.  Replaces
 * src/quantweave_moe_model.py:124-137:
 *   logits = (x.float() @ router_w.float().T) / temperature      [T, E] fp32
 *   probs  = softmax(logits)                                     [T, E] fp32
 *   top_idx, w = topk(probs, k)            (expert_bias == NULL)
 *   top_idx = topk(logits + expert_bias, k).indices; w = probs.gather(top_idx)
 *   top_w  = w / w.sum(-1)                                       [T, k] fp32
 * x: [tokens, d_model] (QW_F32, QW_BF16 or QW_F16) with row stride x_row_stride
 * elements; router_w: [experts, d_model] contiguous (QW_F32, QW_BF16 or
 * QW_F16).  Both are widened to fp32 (the reference's `.float()`).
 * Top-k order is descending, ties resolved towards the lower expert index.
 * 1 <= top_k <= experts <= 1024.  The router GEMM is split over d_model; its
 * fp32 partial sums go to `workspace` and are added in a fixed order. */
size_t qw_moe_route_workspace_bytes(int64_t tokens, int64_t d_model, int64_t experts);
int qw_moe_route(const void* x, int x_dtype, int64_t x_row_stride, const void* router_w, int w_dtype,
                 int64_t tokens, int64_t d_model, int64_t experts, int64_t top_k, float temperature,
                 const float* expert_bias, float* logits, float* probs, int32_t* top_idx, float* top_w,
                 void* workspace, size_t workspace_bytes, void* stream);

/* The softmax/top-k/renormalise half of qw_moe_route on caller-supplied fp32
 * logits [tokens, experts] (already divided by the temperature).  With
 * identical logits this is the routing the bit-exact parity contract covers.
 * src/quantweave_moe_model.py:129-137. */
int qw_moe_route_from_logits(const float* logits, int64_t tokens, int64_t experts, int64_t top_k,
                             const float* expert_bias, float* probs, int32_t* top_idx, float* top_w,
                             void* stream);

/* Capacity plan.  Replaces TopKMoE._plan, src/quantweave_moe_model.py:166-188.
 * Routes r = token*top_k + j are ordered by (expert ascending, weight
 * descending, route id ascending); the first `capacity` routes of each expert
 * are kept.  Outputs (R = tokens*top_k):
 *   counts[E]        routes per expert before capacity (bincount)
 *   kept_counts[E]   min(counts, capacity)
 *   kept_offsets[E+1] exclusive scan of kept_counts (kept_offsets[E] = kept)
 *   slot_token[R]    token of each kept route, in plan order   ("tokens")
 *   slot_weight[R]   renormalised weight of each kept route    ("weights")
 *   route_slot[R]    slot of route r, or -1 when it was dropped
 *   dropped_token[R], dropped_expert[R]  dropped routes in plan order
 *   totals[2]        {kept routes, overflow routes}
 * Entries past totals[0] / totals[1] are left unwritten. */
size_t qw_moe_plan_workspace_bytes(int64_t tokens, int64_t top_k, int64_t experts);
int qw_moe_plan(const int32_t* top_idx, const float* top_w, int64_t tokens, int64_t top_k, int64_t experts,
                int64_t capacity, int32_t* counts, int32_t* kept_counts, int32_t* kept_offsets,
                int32_t* slot_token, float* slot_weight, int32_t* route_slot, int32_t* dropped_token,
                int32_t* dropped_expert, int32_t* totals, void* workspace, size_t workspace_bytes, void* stream);

/* Gather kept rows into plan order: out[s] = x[slot_token[s]] for
 * s < totals[0] (src/quantweave_moe_model.py:195, `flat_hidden[tokens]`).
 * x and out are contiguous [*, d_model] of `dtype`. */
int qw_moe_permute(const void* x, int dtype, int64_t d_model, const int32_t* slot_token, const int32_t* totals,
                   int64_t max_rows, void* out, void* stream);

/* Grouped SwiGLU experts over plan-ordered rows.  Replaces
 * moe_kernels.grouped_swiglu (src/moe_kernels.py:186-195), the per-expert loop
 * (src/quantweave_moe_model.py:203-211) and, for quantised experts,
 * QuantizedLinear.forward (src/quantization.py:61-72):
 *   y[s] = down_e( silu(gate_e(x_s)) * up_e(x_s) ) * row_weight[s]
 * for every s in [kept_offsets[e], kept_offsets[e+1]) of expert e, where x_s is
 * x[row_index[s]] (row_index == NULL: x[s]).  row_weight may be NULL (factor 1).
 * Weights per expert, nn.Linear [out, in] layout, stacked over experts:
 *   QW_F32 / QW_BF16 : gate_w, up_w [E, d_ff, d_model]; down_w [E, d_model, d_ff]
 *   QW_F16           : the same layout in fp16
 *   QW_BF16T/QW_F16T : the same matrices in tiles (d_model and d_ff multiples of 64)
 *   QW_I8 / QW_U4    : qweight and fp32 scales stacked the same way, group sizes
 *                      group_in (gate/up, over d_model) and group_ff (down)
 * act_dtype: QW_F32, QW_BF16 or QW_F16 (x and y).  Weights of another float
 * type are rounded to act_dtype (the reference's `.to(dtype)` of the stacked
 * weights); the matrix-core and weight-streaming kernels take 16-bit weights of
 * act_dtype itself or quantised ones.  Quantised weights are dequantised
 * to fp32, rounded to act_dtype, and multiplied with fp32 accumulation.
 * max_rows bounds kept_offsets[E] (rows of y and of the hidden workspace);
 * max_rows_per_expert bounds every expert's row count (the capacity; 0 when
 * unknown, then max_rows) and sizes the launch grids. */
size_t qw_moe_experts_workspace_bytes(int64_t max_rows, int64_t experts, int64_t d_model, int64_t d_ff,
                                      int act_dtype);
int qw_moe_experts(const void* x, int act_dtype, const int32_t* row_index, const int32_t* kept_offsets,
                   int64_t experts, int64_t d_model, int64_t d_ff, int64_t max_rows, int64_t max_rows_per_expert,
                   int w_format,
                   int64_t group_in, int64_t group_ff, const void* gate_w, const float* gate_scales,
                   const void* up_w, const float* up_scales, const void* down_w, const float* down_scales,
                   const float* row_weight, void* y, void* workspace, size_t workspace_bytes, void* stream);

/* Kernel families of the grouped SwiGLU (qw_moe_experts_on_path). */
enum qw_ffn_path {
  QW_PATH_AUTO = 0,    /* what qw_moe_experts picks for the shape */
  QW_PATH_GENERAL = 1, /* the general kernel: every format and shape */
  QW_PATH_MFMA = 2,    /* the matrix-core kernels (bf16/fp16 prefill; fp32) */
  QW_PATH_STREAM = 3   /* the weight-streaming decode kernels */
};

/* qw_moe_experts with the kernel family chosen by the caller instead of by
 * the row count.  A family that does not take the given formats or shape
 * returns QW_ERR_UNSUPPORTED and launches nothing.  Every family computes
 * the same arithmetic (fp32 accumulation, the same rounding points), so
 * results agree within accumulation order.  No reference counterpart: it
 * lets a caller or a test pin one kernel (the reference's grouped executor
 * has a single Triton kernel, src/moe_kernels.py:186-195). */
int qw_moe_experts_on_path(int path, const void* x, int act_dtype, const int32_t* row_index,
                           const int32_t* kept_offsets, int64_t experts, int64_t d_model, int64_t d_ff,
                           int64_t max_rows, int64_t max_rows_per_expert, int w_format, int64_t group_in,
                           int64_t group_ff, const void* gate_w, const float* gate_scales, const void* up_w,
                           const float* up_scales, const void* down_w, const float* down_scales,
                           const float* row_weight, void* y, void* workspace, size_t workspace_bytes, void* stream);

/* Weighted combine.  Replaces `output.index_add_(0, tokens, expert_output)`
 * (src/quantweave_moe_model.py:192, :200-201, :210-211): out[t] starts at zero
 * and adds y[route_slot[t*k+j]] of every kept route of token t in ascending
 * expert order (the plan order of `tokens`) in fp32, rounded to `dtype` once,
 * as torch's index_add_ does for a bf16 output.  out: [tokens, d_model]. */
int qw_moe_combine(const void* y, int dtype, const int32_t* route_slot, const int32_t* top_idx, int64_t tokens,
                   int64_t top_k, int64_t d_model, void* out, void* stream);

/* Load-balance loss (src/quantweave_moe_model.py:152-154):
 * importance[e] = mean_t probs[t, e]; balance = E * sum_e importance[e] *
 * counts[e] / (tokens*top_k).  importance [experts] receives the means
 * (required). */
int qw_moe_balance(const float* probs, const int32_t* counts, int64_t tokens, int64_t top_k, int64_t experts,
                   float* importance, float* balance, void* stream);

/* qw_moe_balance with a caller workspace of qw_moe_balance_workspace_bytes:
 * the same quantities, the importance summed from per-64-token partial sums
 * in a fixed order (deterministic; the probs rows are read coalesced by many
 * workgroups).  No reference counterpart beyond qw_moe_balance (:152-154). */
size_t qw_moe_balance_workspace_bytes(int64_t tokens, int64_t experts);
int qw_moe_balance_ws(const float* probs, const int32_t* counts, int64_t tokens, int64_t top_k, int64_t experts,
                      float* importance, float* balance, void* workspace, size_t workspace_bytes, void* stream);

/* Whole MoE layer forward (TopKMoE.forward, src/quantweave_moe_model.py:113-164,
 * dynamic-dispatch branch): route -> plan -> grouped SwiGLU -> combine, no host
 * synchronisation.  `out` [tokens, d_model] has act_dtype.  Outputs as for the
 * calls above; probs/top_idx/top_w/counts/kept_counts/totals/dropped_* are
 * required.  `capacity` comes from qw_moe_capacity. */
size_t qw_moe_forward_workspace_bytes(int64_t tokens, int64_t d_model, int64_t experts, int64_t top_k,
                                      int64_t d_ff, int act_dtype);
int qw_moe_forward(const void* x, int act_dtype, int64_t tokens, int64_t d_model, const void* router_w,
                   int router_dtype, float temperature, const float* expert_bias, int64_t experts,
                   int64_t top_k, int64_t capacity, int64_t d_ff, int w_format, int64_t group_in,
                   int64_t group_ff, const void* gate_w, const float* gate_scales, const void* up_w,
                   const float* up_scales, const void* down_w, const float* down_scales, void* out,
                   float* probs, int32_t* top_idx, float* top_w, int32_t* counts, int32_t* kept_counts,
                   int32_t* totals, int32_t* dropped_token, int32_t* dropped_expert, void* workspace,
                   size_t workspace_bytes, void* stream);

/* One decode step of a MoE layer, the routed-expert lines of
 * FastDecoder._step (src/fast_decode.py:170-177), with the experts kept in
 * their stored format (the reference stacks dense dequantised copies,
 * src/fast_decode.py:64-73, :121-123):
 *   scores = x @ router_w^T / temperature           (fp32, x and router_w fp32)
 *   probs = softmax(scores)
 *   idx = topk(scores + expert_bias, top_k)          (scores alone with no bias;
 *                                                      equal keys: lower expert)
 *   w = probs[idx] / sum(probs[idx])
 *   y_j = down(silu(gate(x_c)) * up(x_c)) of expert idx_j, x_c = x in
 *         compute_dtype (QW_BF16: round to nearest even; QW_F32: x itself)
 *   out = residual + ((y_0 * w_0 + y_1 * w_1) + ...)  (fp32; no residual when NULL)
 * No capacity: every route is evaluated.  x, residual, out: fp32 [tokens, d_model];
 * out may be residual (in place).  probs [tokens, experts] may be NULL; top_idx
 * and top_w [tokens, top_k] are required.  Nothing is allocated, copied to the
 * host or cleared with a memset, so the call can be captured in a HIP graph. */
size_t qw_moe_decode_step_workspace_bytes(int64_t tokens, int64_t d_model, int64_t experts, int64_t top_k,
                                          int64_t d_ff, int compute_dtype);
int qw_moe_decode_step(const float* x, const float* residual, int64_t tokens, int64_t d_model,
                       const float* router_w, float temperature, const float* expert_bias, int64_t experts,
                       int64_t top_k, int64_t d_ff, int compute_dtype, int w_format, int64_t group_in,
                       int64_t group_ff, const void* gate_w, const float* gate_scales, const void* up_w,
                       const float* up_scales, const void* down_w, const float* down_scales, float* out,
                       float* probs, int32_t* top_idx, float* top_w, void* workspace, size_t workspace_bytes,
                       void* stream);

/* Library set-up for the current device: looks up the device address of the
 * allocation-free entry point's static scratch array (which may load the
 * library's code object on that device and so allocate its global memory).
 * Call it once per device, outside graph capture, before a graph captures
 * qw_moe_decode_step_noalloc; calling it again is cheap.  No counterpart in
 * the reference (no other entry point needs it). */
int qw_init(void);

/* qw_moe_decode_step without a workspace argument: its scratch is a
 * library-owned array of qw_moe_decode_step_noalloc_scratch_bytes() (32 MiB)
 * on each device, so the call performs no allocation of any kind (it calls no
 * hipMalloc, and torch allocates nothing for it).  No counterpart in the
 * reference: it is for callers that cannot allocate — code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation.  The caller
 * still passes inputs and outputs, exactly as for qw_moe_decode_step, whose
 * results it reproduces bit for bit.  A step whose workspace would exceed the
 * array (qw_moe_decode_step_workspace_bytes) is refused with QW_ERR_INVALID
 * before any device work.  The stream must belong to the current device.
 * Every call on one device shares that device's array and leaves its last
 * contents there (every value a step reads it first writes, so nothing needs
 * clearing); calls that overlap on one device — on different streams or
 * threads without ordering — race.  The array's address is looked up by
 * qw_init(); a call on a device where that has not happened does it first,
 * unless the stream is being captured, in which case the call is refused
 * (QW_ERR_INVALID) so that nothing is loaded or allocated under capture. */
size_t qw_moe_decode_step_noalloc_scratch_bytes(void);
int qw_moe_decode_step_noalloc(const float* x, const float* residual, int64_t tokens, int64_t d_model,
                               const float* router_w, float temperature, const float* expert_bias, int64_t experts,
                               int64_t top_k, int64_t d_ff, int compute_dtype, int w_format, int64_t group_in,
                               int64_t group_ff, const void* gate_w, const float* gate_scales, const void* up_w,
                               const float* up_scales, const void* down_w, const float* down_scales, float* out,
                               float* probs, int32_t* top_idx, float* top_w, void* stream);

/* Weight-only quantisation, QuantizedLinear.from_linear
 * (src/quantization.py:43-59): w [out, in] fp32 or bf16 is zero-padded to
 * padded = ceil(in/group)*group columns; per group scale =
 * max(amax/limit, 1e-8) (limit 127 for bits 8, 7 for bits 4);
 * q = clamp(round_half_even(w/scale), -limit-(bits==4), limit).
 * bits 8: qweight int8 [out, padded]; bits 4: uint8 [out, padded/2] with
 * (q+8) of even columns in the low nibble.  scales fp32 [out, padded/group]. */
int qw_quantize(const void* w, int w_dtype, int64_t out_features, int64_t in_features, int bits,
                int64_t group_size, void* qweight, float* scales, void* stream);

/* QuantizedLinear.dequantize (src/quantization.py:61-69): out fp32
 * [out, in] = q * scale per group, padding columns dropped. */
int qw_dequantize(const void* qweight, const float* scales, int bits, int64_t out_features, int64_t in_features,
                  int64_t group_size, float* out, void* stream);

/* Rearranges bf16 (or fp16) weights w [experts, out_features, in_features]
 * (nn.Linear layout, stacked) into the QW_BF16T (QW_F16T) tiles of the same
 * size; the packing moves 16-bit elements and ignores their type.  No reference
 * counterpart (the reference's Triton kernels read nn.Linear weights as
 * stored); callers pack once per weight update and pass QW_BF16T. */
int qw_pack_bf16_tiles(const void* w, int64_t experts, int64_t out_features, int64_t in_features, void* tiled,
                       void* stream);

/* Grouped matmul forward, moe_kernels.grouped_matmul (src/moe_kernels.py:118-135,
 * :167-171): out[rows of e] = x[rows of e] @ w[e]^T with rows of e =
 * [offsets[e], offsets[e+1]); w [E, out_features, in_features] in w_format
 * (QW_I8 / QW_U4 with fp32 scales and group size `group`, as
 * QuantizedLinear.forward, src/quantization.py:71-72); x and out have
 * act_dtype (QW_F32, QW_BF16 or QW_F16); fp32 accumulation, quantised weights rounded
 * to act_dtype before the multiply.  max_rows_per_expert bounds every
 * expert's row count (0: rows); bf16 (fp16) with plain bf16 (fp16) weights and
 * in_features % 64 == 0 runs on the matrix cores. */
int qw_grouped_matmul(const void* x, int act_dtype, const void* w, int w_format, const float* scales, int64_t group,
                      int64_t experts, int64_t out_features, int64_t in_features, const int32_t* offsets,
                      int64_t rows, int64_t max_rows_per_expert, void* out, void* stream);

/* The accumulation of the capacity-free static dispatch, replacing the loop
 * of TopKMoE._static_output (src/quantweave_moe_model.py:235-245):
 * out[t] = sum over the routes of t in ascending expert order of
 * y[slot] * top_w.to(out_dtype), each product and each add rounded to
 * out_dtype (`output = output + expert(x) * dense_weights[:, e].to(dtype)`;
 * the experts a token does not use add exact zeros).  y holds the unweighted
 * expert rows of a capacity-free plan. */
int qw_moe_combine_static(const void* y, int y_dtype, const int32_t* route_slot, const int32_t* top_idx,
                          const float* top_w, int64_t tokens, int64_t top_k, int64_t d_model, void* out,
                          int out_dtype, void* stream);

/* ------------------------------------------------------------------------
 * Training: the backward pass of the grouped expert matmuls and of the MoE
 * layer's routing and combine.  All gradients are fp32-accumulated; bf16
 * and fp16 tensors are rounded where torch's ops round them.
 * ------------------------------------------------------------------------ */

/* Backward of qw_grouped_matmul with plain weights, _GroupedMatmul.backward
 * (src/moe_kernels.py:146-164) and _grouped_dw_kernel (:66-89):
 *   grad_x[r]   = grad_out[r] @ w[e]            (r in [offsets[e], offsets[e+1]))
 *   grad_w[e]   = grad_out[rows of e]^T @ x[rows of e]   (exactly 0 without rows)
 * grad_out [rows, out_features], x [rows, in_features], w [E, out, in], all of
 * `dtype` (QW_F32, QW_BF16 or QW_F16).  grad_x or grad_w may be NULL (not computed).
 * grad_w has grad_w_dtype: `dtype`, or QW_F32 for fp32 parameters multiplied
 * in bf16 (the gradient is then not rounded to bf16).
 * accumulate_grad_x != 0 adds to grad_x instead of overwriting it.
 * max_rows_per_expert bounds every expert's row count (0: `rows`).
 * bf16 or fp16 with a workspace of qw_grouped_matmul_backward_workspace_bytes runs on
 * the matrix cores (grad_x when out_features % 64 == 0; grad_w always): the
 * weights and the row blocks are transposed into the workspace first.  fp32,
 * or no workspace, runs the vector-ALU kernels. */
size_t qw_grouped_matmul_backward_workspace_bytes(int64_t experts, int64_t out_features, int64_t in_features,
                                                  int64_t rows, int dtype);
int qw_grouped_matmul_backward(const void* grad_out, const void* x, const void* w, int dtype, int64_t experts,
                               int64_t out_features, int64_t in_features, const int32_t* offsets, int64_t rows,
                               int64_t max_rows_per_expert, void* grad_x, int accumulate_grad_x, void* grad_w,
                               int grad_w_dtype, void* workspace, size_t workspace_bytes, void* stream);

/* qw_moe_experts that also keeps what its backward needs, for training
 * (the activations autograd saves for SparseSwiGLU.forward,
 * src/quantweave_moe_model.py:59-60): gate_out / up_out [max_rows, d_ff] the
 * gate and up projections before the SiLU, hidden_out [max_rows, d_ff] the
 * SiLU product, y_unweighted [max_rows, d_model] the expert rows before
 * row_weight; all act_dtype, plan-ordered.  y and the other arguments as for
 * qw_moe_experts, with identical results. */
int qw_moe_experts_save(const void* x, int act_dtype, const int32_t* row_index, const int32_t* kept_offsets,
                        int64_t experts, int64_t d_model, int64_t d_ff, int64_t max_rows,
                        int64_t max_rows_per_expert, int w_format, int64_t group_in, int64_t group_ff,
                        const void* gate_w, const float* gate_scales, const void* up_w, const float* up_scales,
                        const void* down_w, const float* down_scales, const float* row_weight, void* y,
                        void* gate_out, void* up_out, void* hidden_out, void* y_unweighted, void* workspace,
                        size_t workspace_bytes, void* stream);

/* hidden = silu(gate) * up over n elements, `F.silu(gate) * up` of
 * grouped_swiglu (src/moe_kernels.py:194); bf16 rounds silu and the product. */
int qw_swiglu(const void* gate, const void* up, int dtype, int64_t n, void* hidden, void* stream);

/* Its derivative: grad_up = grad_hidden * silu(gate); grad_gate =
 * (grad_hidden * up) * silu'(gate). */
int qw_swiglu_backward(const void* grad_hidden, const void* gate, const void* up, int dtype, int64_t n,
                       void* grad_gate, void* grad_up, void* stream);

/* Combine with router weights and a separate output dtype,
 * `output.index_add_(0, tokens, (expert_output * weights[:, None]).to(out))`
 * (src/quantweave_moe_model.py:201-202): out[t] = sum over the kept routes of
 * t in ascending expert order of (y[slot] * top_w).to(out_dtype), added in
 * fp32 and rounded to out_dtype once.  top_w == NULL: weight 1 (then this is also the
 * backward of the row gather flat[tokens], :192, with out_dtype fp32). */
int qw_moe_combine_weighted(const void* y, int y_dtype, const int32_t* route_slot, const int32_t* top_idx,
                            const float* top_w, int64_t tokens, int64_t top_k, int64_t d_model, void* out,
                            int out_dtype, void* stream);

/* Backward of qw_moe_combine_weighted: for every kept route (t, j) with slot s,
 * grad_y[s] = grad_out[t] * top_w[t, j] (y_dtype) and grad_top_w[t, j] =
 * sum_c grad_out[t, c] * y[s, c]; dropped routes get grad_top_w = 0.
 * top_k <= 64. */
int qw_moe_combine_backward(const void* grad_out, int out_dtype, const void* y, int y_dtype,
                            const int32_t* route_slot, const float* top_w, int64_t tokens, int64_t top_k,
                            int64_t d_model, void* grad_y, float* grad_top_w, void* stream);

/* Backward of the routing (src/quantweave_moe_model.py:126-135, :152-154):
 * from the gradients of the renormalised top-k weights (grad_top_w), of the
 * router probabilities (grad_probs, NULL = 0) and of the balance loss
 * (grad_balance, a device scalar, NULL = 0; needs `counts`, the per-expert
 * route counts of the plan), computes grad_scores [tokens, experts] = the
 * gradient with respect to x @ router_w^T (before the temperature).  The
 * expert bias only steers selection and gets no gradient.  top_k <= 64. */
int qw_moe_route_backward(const float* probs, const int32_t* top_idx, const float* top_w, const float* grad_top_w,
                          const float* grad_probs, const float* grad_balance, const int32_t* counts, int64_t tokens,
                          int64_t experts, int64_t top_k, float temperature, float* grad_scores, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QWMOE_H */
