/*
 * CPU oracle for the routing and token-permute stages of the FP8 block-scale MoE.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker that the HIP kernels are compared
 * against; it is never linked into the product library, and the product never calls it.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 *
 * It restates, in plain scalar C, the semantics that every reference solution implements
 * (the flashinfer-bench definition itself is not vendored in the reference):
 *
 *   DeepSeek-V3 no-aux routing (routing_method 0):
 *     R1  s = sigmoid(logit) in fp32
 *           goal_full_shape/fable-5.1/moe_fp8_fwd/MOEDIR/moe_common.cuh:282
 *           kda05_reproduction_single_shape/fable-5.1/moe_fp8_fwd/t14107/moe_kernel.cu:526
 *     R2  v = s + float(bias_bf16)                                   moe_common.cuh:283
 *     R3  group score = sum of the two largest v of the group,
 *         a duplicated maximum counts twice                          moe_common.cuh:288-305
 *     R4  keep topk_group groups, ties -> lower group index          moe_common.cuh:306-313
 *     R5  top_k experts by v among kept groups, ties -> lower index  moe_common.cuh:320-337
 *     R6  w = s / (sum of selected s + 1e-20) * routed_scaling_factor
 *           (unbiased s)                                             moe_common.cuh:339-363
 *           goal_full_shape/opus-4.8/moe_fp8_fwd/MOEDIR/main.py:65-66 (the s / wsum * rsf order)
 *     L1  local expert le = ge - local_expert_offset, valid iff 0 <= le < E_local
 *           goal_full_shape/opus-4.8/moe_fp8_fwd/MOEDIR/main.py:59-62
 *     P1  per local expert: ascending token list (torch.nonzero order) with the pair weights.
 *
 *   Softmax top-k renormalised routing (routing_method 1, the Qwen3-style geometry; the
 *   reference has no code for it): experts are ranked by logit (softmax is monotone, so the
 *   ranking equals the softmax ranking), ties -> lower index, and w_k = e_k / sum(e_sel) with
 *   e_k = exp(x_k - x_max); the softmax denominator cancels in the renormalisation.
 *
 * Precision conventions this oracle fixes (the kernels follow them exactly, so indices and
 * weights are bit-identical):
 *   - R1 is an fp32 sigmoid built from the steps of sigmoid_f32 below (Cody-Waite range
 *     reduction and a Taylor polynomial for exp, carried as a two-float value, then a
 *     Newton-corrected reciprocal of 1 + e^-x). Every step is an IEEE fp32 operation (fmaf
 *     where a product feeds an add, correctly rounded division, ldexpf), so the GPU gives the
 *     same bits. It is within 1 ulp of the correctly rounded sigmoid and within 2 ulp of
 *     torch.sigmoid (tests/test_oracle.py); the reference's 1/(1+expf(-x)) is an fp32 sigmoid
 *     of the same kind.
 *   - softmax weights use exp_f32 (the high part of the same exp) of x_k - x_max.
 *   - the selected-s sum is accumulated in selection order (descending v, ties lower index),
 *     in fp32, starting from 0.0f; then 1e-20f is added; w = (s / sum) * rsf in fp32.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float bf16_to_float(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/*
 * exp(y) = 2^n (ph + pl), |pl| <= ulp(ph): n = rint(y log2 e), r = y - n ln2 in two steps
 * (Cody-Waite: LN2_HI has 16 significant bits, LN2_LO = ln2 - LN2_HI), e^r = 1 + r q(r) with q
 * the Taylor series of (e^r - 1) / r to degree 6 (truncation < 2^-27 for |r| <= ln2 / 2), and
 * the rounding error of the final 1 + r q recovered exactly by a second fma. y is clamped to
 * [-104, 88], where e^y stays finite.
 */
static const float kL2E = 1.44269504088896341f;
static const float kLn2Hi = 0.693145751953125f;
static const float kLn2Lo = 1.428606765330187045e-06f;

static void exp_parts(float y, float* ph, float* pl, int* n_out) {
  y = fminf(fmaxf(y, -104.0f), 88.0f);
  const float n = rintf(y * kL2E);
  float r = fmaf(-n, kLn2Hi, y);
  r = fmaf(-n, kLn2Lo, r);
  float q = 1.0f / 5040.0f;
  q = fmaf(q, r, 1.0f / 720.0f);
  q = fmaf(q, r, 1.0f / 120.0f);
  q = fmaf(q, r, 1.0f / 24.0f);
  q = fmaf(q, r, 1.0f / 6.0f);
  q = fmaf(q, r, 0.5f);
  q = fmaf(q, r, 1.0f);
  const float h = fmaf(r, q, 1.0f);
  *ph = h;
  *pl = fmaf(r, q, 1.0f - h); /* 1 - h is exact (h in [0.70, 1.42]) */
  *n_out = (int)n;
}

float oracle_exp_f32(float y) {
  float ph, pl;
  int n;
  exp_parts(y, &ph, &pl, &n);
  return ldexpf(ph, n);
}

/*
 * sigmoid(x) = 1 / d with d = 1 + e^-x held as dh + dl (Fast2Sum of 1 and the high part, plus
 * the low part), s0 = RN(1 / dh), then one Newton step s0 + s0 (1 - s0 dh - s0 dl). Below
 * x = -87, 1 + e^-x equals e^-x to far below an ulp and the result is e^x.
 */
float oracle_sigmoid_f32(float x) {
  float ph, pl;
  int n;
  exp_parts(x < -87.0f ? x : -x, &ph, &pl, &n);
  if (x < -87.0f) return ldexpf(ph, n);
  const float eh = ldexpf(ph, n), el = ldexpf(pl, n);
  const float dh = 1.0f + eh;
  const float dl = (eh >= 1.0f ? (eh - dh) + 1.0f : (1.0f - dh) + eh) + el;
  const float s0 = 1.0f / dh;
  const float res = fmaf(-s0, dl, fmaf(-s0, dh, 1.0f));
  return fmaf(s0, res, s0);
}

/* Batch forms for the pinning tests. */
void oracle_sigmoid_batch(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = oracle_sigmoid_f32(x[i]);
}
void oracle_exp_batch(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = oracle_exp_f32(x[i]);
}

/* Returns 1 if (va, ia) ranks before (vb, ib): larger value first, ties -> lower index. */
static int better(float va, int ia, float vb, int ib) { return va > vb || (va == vb && ia < ib); }

/*
 * DeepSeek no-aux routing for one batch.
 * logits fp32 [T, E], bias bf16 bits [E] (may be NULL -> zeros).
 * Outputs: topk_idx int32 [T, top_k] global expert ids in selection order,
 *          topk_w fp32 [T, top_k].
 * Returns 0, or -1 on unsupported geometry.
 */
int oracle_route_ds(const float* logits, const uint16_t* bias, int T, int E, int n_group,
                    int topk_group, int top_k, float rsf, int32_t* topk_idx, float* topk_w) {
  if (E <= 0 || E > 1024 || n_group <= 0 || E % n_group || topk_group > n_group || top_k > 64) return -1;
  const int gs = E / n_group;
  float s[1024], v[1024], gscore[1024];
  int kept[1024], taken[1024];
  for (int t = 0; t < T; ++t) {
    const float* x = logits + (size_t)t * E;
    for (int e = 0; e < E; ++e) {
      s[e] = oracle_sigmoid_f32(x[e]);
      v[e] = s[e] + (bias ? bf16_to_float(bias[e]) : 0.0f);
    }
    for (int g = 0; g < n_group; ++g) {
      /* top-2 of the group as a multiset: the first maximum (lowest index) is removed */
      int i1 = g * gs;
      for (int e = g * gs + 1; e < (g + 1) * gs; ++e)
        if (v[e] > v[i1]) i1 = e;
      float m2 = -INFINITY;
      for (int e = g * gs; e < (g + 1) * gs; ++e)
        if (e != i1 && v[e] > m2) m2 = v[e];
      gscore[g] = gs > 1 ? v[i1] + m2 : v[i1];
    }
    for (int g = 0; g < n_group; ++g) {
      int rank = 0;
      for (int h = 0; h < n_group; ++h) rank += better(gscore[h], h, gscore[g], g);
      kept[g] = rank < topk_group;
    }
    for (int e = 0; e < E; ++e) taken[e] = 0;
    float sum = 0.0f;
    float sel_s[64];
    for (int k = 0; k < top_k; ++k) {
      int best = -1;
      for (int e = 0; e < E; ++e) {
        if (!kept[e / gs] || taken[e]) continue;
        if (best < 0 || better(v[e], e, v[best], best)) best = e;
      }
      if (best < 0) return -1;
      taken[best] = 1;
      topk_idx[(size_t)t * top_k + k] = best;
      sel_s[k] = s[best];
      sum += s[best];
    }
    sum += 1e-20f;
    for (int k = 0; k < top_k; ++k) topk_w[(size_t)t * top_k + k] = sel_s[k] / sum * rsf;
  }
  return 0;
}

/* Softmax top-k, renormalised over the selected experts (no groups, bias or scaling). */
int oracle_route_softmax(const float* logits, int T, int E, int top_k, int32_t* topk_idx,
                         float* topk_w) {
  if (E <= 0 || E > 1024 || top_k > 64 || top_k > E) return -1;
  int taken[1024];
  for (int t = 0; t < T; ++t) {
    const float* x = logits + (size_t)t * E;
    for (int e = 0; e < E; ++e) taken[e] = 0;
    float xs[64];
    for (int k = 0; k < top_k; ++k) {
      int best = -1;
      for (int e = 0; e < E; ++e) {
        if (taken[e]) continue;
        if (best < 0 || better(x[e], e, x[best], best)) best = e;
      }
      taken[best] = 1;
      topk_idx[(size_t)t * top_k + k] = best;
      xs[k] = x[best];
    }
    float ex[64], sum = 0.0f;
    for (int k = 0; k < top_k; ++k) {
      ex[k] = oracle_exp_f32(xs[k] - xs[0]);
      sum += ex[k];
    }
    for (int k = 0; k < top_k; ++k) topk_w[(size_t)t * top_k + k] = ex[k] / sum;
  }
  return 0;
}

/*
 * Stable counting sort of the local (token, expert) pairs by local expert (P1).
 * counts [E_local], offsets [E_local + 1], sorted_tok / sorted_w [>= offsets[E_local]],
 * pair_of [T, top_k]: the pair row of slot (t, k), or -1 when the expert is not local.
 * Returns the number of local pairs.
 */
int oracle_permute(const int32_t* topk_idx, const float* topk_w, int T, int top_k,
                   int local_offset, int E_local, int32_t* counts, int32_t* offsets,
                   int32_t* sorted_tok, float* sorted_w, int32_t* pair_of) {
  for (int e = 0; e < E_local; ++e) counts[e] = 0;
  for (size_t i = 0; i < (size_t)T * top_k; ++i) {
    int le = topk_idx[i] - local_offset;
    if (le >= 0 && le < E_local) counts[le]++;
  }
  offsets[0] = 0;
  for (int e = 0; e < E_local; ++e) offsets[e + 1] = offsets[e] + counts[e];
  /* fill cursor per expert; walking tokens in ascending order makes each segment ascending */
  int32_t cursor[1024];
  if (E_local > 1024) return -1;
  for (int e = 0; e < E_local; ++e) cursor[e] = offsets[e];
  for (int t = 0; t < T; ++t) {
    for (int k = 0; k < top_k; ++k) {
      size_t i = (size_t)t * top_k + k;
      int le = topk_idx[i] - local_offset;
      if (le >= 0 && le < E_local) {
        int p = cursor[le]++;
        sorted_tok[p] = t;
        sorted_w[p] = topk_w[i];
        pair_of[i] = p;
      } else {
        pair_of[i] = -1;
      }
    }
  }
  return offsets[E_local];
}
