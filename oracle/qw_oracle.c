/*
 * CPU oracle for the routed MoE expert-FFN forward path — TEST INFRASTRUCTURE.
 *
 * A plain-C restatement of the reference algorithm, used only by tests/,
 * __graft_entry__.smoke() and bench.py's CPU-baseline leg, as the reference
 * the GPU results are compared with.  It
 * is never linked into or called by the product library.
 *
 * Built with -ffp-contract=off and no fast-math: every float operation below
 * is one IEEE-754 single-precision operation in the written order.
 *
 * Functions and the reference lines they restate:
 *   orc_expf, orc_softmax_row  softmax of src/quantweave_moe_model.py:129 with
 *                              an exactly specified exp and summation order
 *   orc_route_from_logits      :129-137 (softmax, topk / biased topk, renorm;
 *                              topk's tie order and the renormalising sum
 *                              are torch-ROCm's, which the reference runs)
 *   orc_route_select_probs     the same selection from given probabilities
 *   orc_route_select           the same with the decode step's selection,
 *                              src/fast_decode.py:170-174 (topk of the
 *                              scores, biased or not)
 *   orc_router_logits          :128 (fp32 logits, double accumulation)
 *   orc_capacity               :100-111
 *   orc_plan                   :166-188 (two stable argsorts == one stable
 *                              sort by (expert, -weight, route))
 *   orc_quantize               src/quantization.py:43-59
 *   orc_dequantize             src/quantization.py:61-69
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---- exp and softmax --------------------------------------------------- */

static float as_float(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint32_t as_uint(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* e^x for x <= 0: n = rint(x*log2(e)); r = x - n*ln2 (two-part ln2, fma);
 * e^r by the degree-7 Taylor polynomial 1/i! in Horner form (fma);
 * times 2^n via the exponent field, in two steps below 2^-126. */
float orc_expf(float x) {
  if (!(x >= -104.0f)) return (x != x) ? x : 0.0f;
  const float n = rintf(x * 1.4426950216293335f);
  float r = fmaf(-n, 0.693145751953125f, x);
  r = fmaf(-n, 1.428606765330187e-06f, r);
  float p = 0.00019841270113829523f;
  p = fmaf(p, r, 0.0013888889225199819f);
  p = fmaf(p, r, 0.008333333767950535f);
  p = fmaf(p, r, 0.0416666679084301f);
  p = fmaf(p, r, 0.1666666716337204f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const int ni = (int)n;
  if (ni >= -126) return p * as_float((uint32_t)(ni + 127) << 23);
  return (p * as_float((uint32_t)(ni + 127 + 64) << 23)) * 5.421010862427522e-20f;
}

/* softmax of one row of E logits.  Summation order: the row is dealt to 64
 * lanes (expert e to lane e % 64); each lane sums its experts in index order;
 * then 6 butterfly rounds: v[l] = v[l] + v[l ^ o] for o = 32, 16, 8, 4, 2, 1;
 * the sum is lane 0's value.  p_e = q_e / sum (IEEE division). */
void orc_softmax_row(const float* logits, int E, float* probs) {
  float m = -INFINITY;
  int has_nan = 0;
  for (int e = 0; e < E; ++e) {
    if (logits[e] != logits[e]) has_nan = 1;
    else if (logits[e] > m) m = logits[e];
  }
  if (has_nan) m = NAN;
  float lane[64];
  for (int l = 0; l < 64; ++l) lane[l] = 0.0f;
  for (int e = 0; e < E; ++e) {
    probs[e] = orc_expf(logits[e] - m);
  }
  for (int l = 0; l < 64; ++l) {
    float s = 0.0f;
    for (int e = l; e < E; e += 64) s = s + probs[e];
    lane[l] = s;
  }
  for (int o = 32; o >= 1; o >>= 1) {
    float nxt[64];
    for (int l = 0; l < 64; ++l) nxt[l] = lane[l] + lane[l ^ o];
    memcpy(lane, nxt, sizeof(lane));
  }
  const float s = lane[0];
  for (int e = 0; e < E; ++e) probs[e] = probs[e] / s;
}

/* Total order key: -inf < ... < -0 < +0 < ... < +inf < NaN. */
static uint32_t sort_key(float f) {
  uint32_t u = as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

/* torch.topk's comparison (GTOp with NaN handling): NaN above numbers. */
static int topk_greater(float a, float b) { return (a != a && b == b) || a > b; }

/* torch.topk's order (torch-ROCm, measured on the device and pinned by
 * tests/golden/torch_rocm_routing.npz): the chosen values above the k-th
 * value in index order, then the k-th value's ties in index order, sorted for
 * k <= 32 by the 32-wide bitonic network of
 * aten/src/ATen/native/cuda/SortUtils.cuh (bitonicSort / bitonicSwap, GTOp,
 * invalid entries last), for larger k stably.  kv, idx, pv hold the k choices
 * (any order) and are rewritten in torch's order. */
static void topk_torch_order(int k, float* kv, int32_t* idx, float* pv) {
  float K[1024], P[1024];
  int32_t V[1024];
  int valid[1024];
  /* the split compares radix-select keys (sort_key: -0 below +0); the
   * network compares floats (-0 equal to +0) */
  uint32_t kth = sort_key(kv[0]);
  for (int j = 0; j < k; ++j)
    if (sort_key(kv[j]) < kth) kth = sort_key(kv[j]); /* the smallest chosen value */
  int n = 0;
  for (int pass = 0; pass < 2; ++pass) {
    for (int e = -1;;) { /* next chosen expert above e in index order */
      int best = -1;
      for (int j = 0; j < k; ++j) {
        const int grp = sort_key(kv[j]) > kth ? 0 : 1;
        if (grp != pass || idx[j] <= e) continue;
        if (best < 0 || idx[j] < idx[best]) best = j;
      }
      if (best < 0) break;
      K[n] = kv[best];
      V[n] = idx[best];
      P[n] = pv[best];
      valid[n] = 1;
      ++n;
      e = idx[best];
    }
  }
  if (k > 32) { /* torch sorts longer selections stably */
    for (int i = 1; i < n; ++i)
      for (int j = i; j > 0 && topk_greater(K[j], K[j - 1]); --j) {
        float tk = K[j]; K[j] = K[j - 1]; K[j - 1] = tk;
        int32_t tv = V[j]; V[j] = V[j - 1]; V[j - 1] = tv;
        float tp = P[j]; P[j] = P[j - 1]; P[j - 1] = tp;
      }
    for (int j = 0; j < k; ++j) {
      kv[j] = K[j];
      idx[j] = V[j];
      pv[j] = P[j];
    }
    return;
  }
  for (int i = n; i < 32; ++i) {
    K[i] = 0.0f;
    V[i] = 0;
    P[i] = 0.0f;
    valid[i] = 0;
  }
  for (unsigned size = 2; size <= 32; size *= 2) {
    for (unsigned stride = size / 2; stride > 0; stride /= 2) {
      for (unsigned t = 0; t < 16; ++t) {
        const unsigned a = 2 * t - (t & (stride - 1)), b = a + stride;
        const int dir = size < 32 && (t & (size / 2)) != 0;
        const int swap = (topk_greater(K[a], K[b]) && valid[a]) || !valid[b];
        if (swap == dir) {
          float tk = K[a]; K[a] = K[b]; K[b] = tk;
          int32_t tv = V[a]; V[a] = V[b]; V[b] = tv;
          float tp = P[a]; P[a] = P[b]; P[b] = tp;
          int tvl = valid[a]; valid[a] = valid[b]; valid[b] = tvl;
        }
      }
    }
  }
  for (int j = 0; j < k; ++j) {
    kv[j] = K[j];
    idx[j] = V[j];
    pv[j] = P[j];
  }
}

/* w.sum(-1) of k < 128 values as torch-ROCm reduces a contiguous last
 * dimension (aten/src/ATen/native/cuda/Reduce.cuh): B = 2^floor(log2 k)
 * threads (at most 64), thread i holding w_i + w_{i+B} (w_i alone when
 * i + B >= k), then adjacent pairs in a tree. */
float orc_topk_weight_sum(const float* w, int k) {
  int B = 1;
  while (B * 2 <= k && B < 64) B *= 2;
  float v[64];
  for (int i = 0; i < B; ++i) v[i] = (i + B < k) ? w[i] + w[i + B] : w[i];
  for (int n = B; n > 1; n /= 2)
    for (int i = 0; i < n / 2; ++i) v[i] = v[2 * i] + v[2 * i + 1];
  return v[0];
}

/* One token's selection from its probabilities p (and logits l): indices =
 * topk(key, k) with key = l + bias when a bias is given, else l when
 * select_logits, else p; chosen by (key descending, index ascending), which
 * is the set torch.topk chooses, then put in torch.topk's order; w = p[idx] /
 * torch's sum of the chosen p (orc_topk_weight_sum; the plain sum in choice
 * order beyond 128 choices). */
static void select_row(const float* l, const float* p, int E, int K, const float* bias, int select_logits,
                       uint32_t* key, char* taken, float* kv, int32_t* top_idx, float* top_w) {
  for (int e = 0; e < E; ++e) {
    key[e] = sort_key(bias ? l[e] + bias[e] : (select_logits ? l[e] : p[e]));
    taken[e] = 0;
  }
  for (int j = 0; j < K; ++j) {
    int best = -1;
    for (int e = 0; e < E; ++e) {
      if (taken[e]) continue;
      if (best < 0 || key[e] > key[best]) best = e;
    }
    taken[best] = 1;
    top_idx[j] = best;
    top_w[j] = p[best];
    kv[j] = bias ? l[best] + bias[best] : (select_logits ? l[best] : p[best]);
  }
  if (K >= 2 && K <= 1024) topk_torch_order(K, kv, top_idx, top_w);
  float sum;
  if (K < 128) {
    sum = orc_topk_weight_sum(top_w, K);
  } else {
    sum = top_w[0];
    for (int j = 1; j < K; ++j) sum = sum + top_w[j];
  }
  for (int j = 0; j < K; ++j) top_w[j] = top_w[j] / sum;
}

/* probs = softmax(logits), then select_row per token. */
void orc_route_select(const float* logits, int T, int E, int K, const float* bias, int select_logits,
                      float* probs, int32_t* top_idx, float* top_w) {
  uint32_t* key = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)E);
  char* taken = (char*)malloc((size_t)E);
  float* kv = (float*)malloc(sizeof(float) * (size_t)K);
  for (int t = 0; t < T; ++t) {
    orc_softmax_row(logits + (size_t)t * E, E, probs + (size_t)t * E);
    select_row(logits + (size_t)t * E, probs + (size_t)t * E, E, K, bias, select_logits, key, taken, kv,
               top_idx + (size_t)t * K, top_w + (size_t)t * K);
  }
  free(key);
  free(taken);
  free(kv);
}

/* The same selection from given probabilities (softmax computed elsewhere,
 * e.g. by torch on the device). */
void orc_route_select_probs(const float* logits, const float* probs, int T, int E, int K, const float* bias,
                            int select_logits, int32_t* top_idx, float* top_w) {
  uint32_t* key = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)E);
  char* taken = (char*)malloc((size_t)E);
  float* kv = (float*)malloc(sizeof(float) * (size_t)K);
  for (int t = 0; t < T; ++t)
    select_row(logits + (size_t)t * E, probs + (size_t)t * E, E, K, bias, select_logits, key, taken, kv,
               top_idx + (size_t)t * K, top_w + (size_t)t * K);
  free(key);
  free(taken);
  free(kv);
}

void orc_route_from_logits(const float* logits, int T, int E, int K, const float* bias, float* probs,
                           int32_t* top_idx, float* top_w) {
  orc_route_select(logits, T, E, K, bias, 0, probs, top_idx, top_w);
}

/* logits[t, e] = (sum_k x[t,k] * w[e,k], in double, rounded to float) / temperature */
void orc_router_logits(const float* x, const float* w, int T, int D, int E, float temperature, float* logits) {
  for (int t = 0; t < T; ++t)
    for (int e = 0; e < E; ++e) {
      double acc = 0.0;
      for (int k = 0; k < D; ++k) acc += (double)x[(size_t)t * D + k] * (double)w[(size_t)e * D + k];
      logits[(size_t)t * E + e] = (float)acc / temperature;
    }
}

/* ---- capacity and plan ------------------------------------------------- */

int64_t orc_capacity(int64_t tokens, int64_t top_k, int64_t experts, double capacity_factor, double capacity_scale,
                     int64_t min_capacity, int drop_overflow) {
  if (capacity_factor > 0 && drop_overflow) {
    double v = (double)(tokens * top_k) / (double)experts * capacity_factor * capacity_scale;
    int64_t c = (int64_t)ceil(v);
    return c > min_capacity ? c : min_capacity;
  }
  return tokens * top_k;
}

typedef struct {
  int32_t expert;
  uint32_t wkey; /* sort_key(weight): larger weight -> larger key */
  int32_t route;
} plan_item;

static int plan_cmp(const void* a, const void* b) {
  const plan_item* x = (const plan_item*)a;
  const plan_item* y = (const plan_item*)b;
  if (x->expert != y->expert) return x->expert < y->expert ? -1 : 1;
  if (x->wkey != y->wkey) return x->wkey > y->wkey ? -1 : 1; /* weight descending */
  return x->route < y->route ? -1 : (x->route > y->route); /* stability: route ascending */
}

/* Outputs as qw_moe_plan.  Returns the number of kept routes. */
int orc_plan(const int32_t* top_idx, const float* top_w, int T, int K, int E, int64_t capacity, int32_t* counts,
             int32_t* kept_counts, int32_t* kept_offsets, int32_t* slot_token, float* slot_weight,
             int32_t* route_slot, int32_t* dropped_token, int32_t* dropped_expert, int32_t* totals) {
  const int R = T * K;
  plan_item* items = (plan_item*)malloc(sizeof(plan_item) * (size_t)(R > 0 ? R : 1));
  for (int e = 0; e < E; ++e) counts[e] = 0;
  for (int r = 0; r < R; ++r) {
    items[r].expert = top_idx[r];
    items[r].wkey = sort_key(top_w[r]);
    items[r].route = r;
    counts[top_idx[r]] += 1;
  }
  qsort(items, (size_t)R, sizeof(plan_item), plan_cmp);
  int off = 0;
  for (int e = 0; e < E; ++e) {
    kept_counts[e] = counts[e] < capacity ? counts[e] : (int32_t)capacity;
    kept_offsets[e] = off;
    off += kept_counts[e];
  }
  kept_offsets[E] = off;
  /* position of the i-th sorted route inside its expert = i - first index of its expert */
  int kept = 0, dropped = 0, start = 0;
  for (int i = 0; i < R; ++i) {
    if (i > 0 && items[i].expert != items[i - 1].expert) start = i;
    const int position = i - start;
    const int r = items[i].route;
    if (position < capacity) {
      slot_token[kept] = r / K;
      slot_weight[kept] = top_w[r];
      route_slot[r] = kept;
      ++kept;
    } else {
      dropped_token[dropped] = r / K;
      dropped_expert[dropped] = items[i].expert;
      route_slot[r] = -1;
      ++dropped;
    }
  }
  totals[0] = kept;
  totals[1] = dropped;
  free(items);
  return kept;
}

/* ---- weight-only quantisation ------------------------------------------ */

/* w fp32 [rows, cols] -> qweight (int8 [rows, padded] or uint8 [rows, padded/2])
 * and scales fp32 [rows, padded/group]. */
void orc_quantize(const float* w, int64_t rows, int64_t cols, int bits, int64_t group, void* qweight, float* scales) {
  const int64_t groups = (cols + group - 1) / group;
  const int64_t padded = groups * group;
  const float limit = bits == 8 ? 127.0f : 7.0f;
  const float lo = bits == 8 ? -127.0f : -8.0f;
  for (int64_t row = 0; row < rows; ++row) {
    for (int64_t g = 0; g < groups; ++g) {
      float amax = 0.0f;
      for (int64_t c = g * group; c < (g + 1) * group; ++c) {
        const float v = c < cols ? fabsf(w[row * cols + c]) : 0.0f;
        if (v > amax) amax = v;
      }
      float s = amax / limit;
      if (s < 1e-8f) s = 1e-8f;
      scales[row * groups + g] = s;
      for (int64_t c = g * group; c < (g + 1) * group; ++c) {
        const float v = c < cols ? w[row * cols + c] : 0.0f;
        float q = rintf(v / s);
        if (q < lo) q = lo;
        if (q > limit) q = limit;
        if (bits == 8) {
          ((int8_t*)qweight)[row * padded + c] = (int8_t)q;
        } else {
          uint8_t* b = (uint8_t*)qweight + row * (padded / 2) + c / 2;
          const uint8_t u = (uint8_t)((int)q + 8);
          if (c % 2 == 0) *b = (uint8_t)((*b & 0xF0) | u);
          else *b = (uint8_t)((*b & 0x0F) | (u << 4));
        }
      }
    }
  }
}

void orc_dequantize(const void* qweight, const float* scales, int bits, int64_t rows, int64_t cols, int64_t group,
                    float* out) {
  const int64_t groups = (cols + group - 1) / group;
  const int64_t padded = groups * group;
  for (int64_t row = 0; row < rows; ++row)
    for (int64_t c = 0; c < cols; ++c) {
      float q;
      if (bits == 8) {
        q = (float)((const int8_t*)qweight)[row * padded + c];
      } else {
        const uint8_t b = ((const uint8_t*)qweight)[row * (padded / 2) + c / 2];
        q = (float)((c % 2 == 0) ? (b & 0xF) : (b >> 4)) - 8.0f;
      }
      out[row * cols + c] = q * scales[row * groups + c / group];
    }
}
