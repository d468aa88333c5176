/*
 * sa_oracle.c — CPU oracle for the KV-cache decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker).  Loaded by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg; never by the
 * product library.  Build: oracle/Makefile (gcc -O2 -ffp-contract=off).
 *
 * Reference paths below are relative to the reference checkout.
 */
#include "sa_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* FP16 codec                                                                */
/* ------------------------------------------------------------------------ */

static uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, sizeof u);
  return u;
}

static float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, sizeof f);
  return f;
}

/* cpp/src/attention_reference.cpp:11-28.  The rounding adds half an FP16 ulp
 * (0x1000 in fp32 mantissa units) and truncates; a carry out of the 10-bit
 * field lands on the exponent's lowest bit through a bitwise OR, which is
 * why e.g. 1.99999f encodes as 1.0.  Overflow saturates to infinity and NaN
 * encodes as infinity; values below the subnormal range flush to zero. */
uint16_t sao_float_to_half(float value) {
  const uint32_t in = f32_bits(value);
  const uint32_t sign = (in >> 16) & 0x8000u;
  const int biased = (int)((in >> 23) & 0xffu) - 112; /* 127 - 15 */
  uint32_t frac = in & 0x7fffffu;
  if (biased <= 0) {
    if (biased < -10) return (uint16_t)sign;
    frac = (frac | 0x800000u) >> (1 - biased);
    return (uint16_t)(sign | ((frac + 0x1000u) >> 13));
  }
  if (biased >= 31) return (uint16_t)(sign | 0x7c00u);
  const uint32_t rounded = (frac + 0x1000u) >> 13; /* may be 0x400 */
  return (uint16_t)(sign | ((uint32_t)biased << 10) | rounded);
}

/* cpp/src/attention_reference.cpp:30-53: exact decode.  Subnormal halves are
 * renormalised; infinities and NaNs keep their payload bits. */
float sao_half_to_float(uint16_t h) {
  const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  const uint32_t exp5 = ((uint32_t)h >> 10) & 0x1fu;
  uint32_t frac = (uint32_t)h & 0x3ffu;
  if (exp5 == 31) return bits_f32(sign | 0x7f800000u | (frac << 13));
  if (exp5 != 0) return bits_f32(sign | ((exp5 + 112u) << 23) | (frac << 13));
  if (frac == 0) return bits_f32(sign);
  uint32_t e = 113; /* exponent of 2^-14 */
  while (!(frac & 0x400u)) {
    frac <<= 1;
    --e;
  }
  return bits_f32(sign | (e << 23) | ((frac & 0x3ffu) << 13));
}

/* IEEE-754 binary32 -> binary16, round to nearest, ties to even; NaN stays
 * a quiet NaN.  Written from the format definition. */
uint16_t sao_float_to_half_rne(float value) {
  const uint32_t in = f32_bits(value);
  const uint32_t sign = (in >> 16) & 0x8000u;
  const uint32_t mag = in & 0x7fffffffu;
  if (mag >= 0x7f800000u) { /* inf or NaN */
    if (mag == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | 0x7e00u | ((mag >> 13) & 0x3ffu));
  }
  if (mag >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 */
  const int e = (int)(mag >> 23) - 127;
  uint32_t mant = (mag & 0x7fffffu) | 0x800000u;
  int shift; /* bits to drop from the 24-bit significand */
  uint32_t base;
  if (e >= -14) {
    shift = 13;
    base = (uint32_t)(e + 15) << 10;
    mant &= 0x7fffffu; /* implicit bit carried by the exponent field */
  } else {
    if (e < -25) return (uint16_t)sign; /* below half of the least subnormal */
    shift = -e - 1;                      /* 14 .. 24 */
    base = 0;
  }
  const uint32_t kept = mant >> shift;
  const uint32_t rest = mant & ((1u << shift) - 1u);
  const uint32_t half = 1u << (shift - 1);
  uint32_t out = base + kept; /* a mantissa carry rolls into the exponent */
  if (rest > half || (rest == half && (kept & 1u))) out += 1u;
  return (uint16_t)(sign | out);
}

/* ------------------------------------------------------------------------ */
/* Stable index sort, descending by key ("left > right" comparator)          */
/* ------------------------------------------------------------------------ */

typedef int (*greater_fn)(const void* keys, size_t a, size_t b);

static int greater_f32(const void* keys, size_t a, size_t b) {
  const float* k = (const float*)keys;
  return k[a] > k[b];
}

/* The builder's received-mass order: the reference's a > b for numbers; NaN,
 * which a > b leaves unordered (std::stable_sort then has no defined
 * result), after every number.  The GPU builders rank the same way. */
static int greater_mass(const void* keys, size_t a, size_t b) {
  const float* k = (const float*)keys;
  return k[a] > k[b] || (k[a] == k[a] && k[b] != k[b]);
}

static int greater_f64(const void* keys, size_t a, size_t b) {
  const double* k = (const double*)keys;
  return k[a] > k[b];
}

/* Bottom-up merge sort: an element of the right run is taken only when it
 * is strictly greater than the head of the left run, so equal keys keep
 * their input order (the std::stable_sort contract the reference uses). */
static void stable_sort_desc(size_t* idx, size_t n, const void* keys,
                             greater_fn greater) {
  if (n < 2) return;
  size_t* tmp = (size_t*)malloc(n * sizeof(size_t));
  if (!tmp) abort();
  size_t* src = idx;
  size_t* dst = tmp;
  for (size_t width = 1; width < n; width *= 2) {
    for (size_t lo = 0; lo < n; lo += 2 * width) {
      size_t mid = lo + width < n ? lo + width : n;
      size_t hi = lo + 2 * width < n ? lo + 2 * width : n;
      size_t i = lo, j = mid, o = lo;
      while (i < mid && j < hi) {
        if (greater(keys, src[j], src[i])) dst[o++] = src[j++];
        else dst[o++] = src[i++];
      }
      while (i < mid) dst[o++] = src[i++];
      while (j < hi) dst[o++] = src[j++];
    }
    size_t* t = src;
    src = dst;
    dst = t;
  }
  if (src != idx) memcpy(idx, src, n * sizeof(size_t));
  free(tmp);
}

/* ------------------------------------------------------------------------ */
/* C1 attention                                                              */
/* ------------------------------------------------------------------------ */

/* cpp/src/attention_reference.cpp:55-96.  Per query head: sequential fp32
 * dot over head_dim, logit = dot * scale, running max; exp(logit - max)
 * summed in token order; out += (p / denominator) * v in token order. */
int sao_attention_reference(const uint16_t* kv, const float* query,
                            size_t tokens, size_t query_heads, size_t kv_heads,
                            size_t head_dim, float scale, float* out) {
  if (!kv || !query || !out || kv_heads == 0 || tokens == 0 ||
      query_heads % kv_heads != 0)
    return SAO_EINVAL;
  const size_t group = query_heads / kv_heads;
  const size_t token_stride = 2 * kv_heads * head_dim;
  float* logits = (float*)malloc(tokens * sizeof(float));
  if (!logits) return SAO_EINVAL;
  memset(out, 0, query_heads * head_dim * sizeof(float));
  for (size_t h = 0; h < query_heads; ++h) {
    const size_t g = h / group;
    const float* q = query + h * head_dim;
    float maximum = -INFINITY;
    for (size_t t = 0; t < tokens; ++t) {
      const uint16_t* k = kv + t * token_stride + g * head_dim;
      float dot = 0.0f;
      for (size_t d = 0; d < head_dim; ++d) dot += q[d] * sao_half_to_float(k[d]);
      logits[t] = dot * scale;
      if (logits[t] > maximum) maximum = logits[t];
    }
    float denominator = 0.0f;
    for (size_t t = 0; t < tokens; ++t) {
      logits[t] = expf(logits[t] - maximum);
      denominator += logits[t];
    }
    float* o = out + h * head_dim;
    for (size_t t = 0; t < tokens; ++t) {
      const uint16_t* v = kv + t * token_stride + kv_heads * head_dim + g * head_dim;
      const float w = logits[t] / denominator;
      for (size_t d = 0; d < head_dim; ++d) o[d] += w * sao_half_to_float(v[d]);
    }
  }
  free(logits);
  return SAO_OK;
}

/* ------------------------------------------------------------------------ */
/* C2 representatives and selection                                          */
/* ------------------------------------------------------------------------ */

/* cpp/src/selection.cpp:12-94. */
/* The reference's std::exp(float) (selection.cpp:53) is glibc's expf.  This
 * restates the method of glibc 2.35 (sysdeps/ieee754/flt-32/e_expf.c with the
 * data of e_exp2f_data.c, the ARM optimized-routines expf): in double,
 * z = x * 32/ln2, k = z rounded to the nearest integer (by adding and
 * subtracting 1.5 * 2^52), r = z - k, 2^(k/32) = 2^((k mod 32)/32) * 2^(k div 32)
 * from a 32-entry table (gen_expf_table.py), and 2^(r/32) by a degree-3
 * polynomial; the double result is rounded to float.  x86-64 glibc runs the
 * variant built for FMA: r and the polynomial steps below are fused
 * multiply-adds.  With exactly these fusions the result equals this
 * container's libm expf on every float in [-110, 90] (all 2,240,806,914 of
 * them; without the fusion in r, 2 differ).  Test infrastructure, restated
 * so that the GPU builder can run the same operations. */
static const uint64_t kExpfTab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

void sao_expf_glibc_table(uint64_t* out) { memcpy(out, kExpfTab, sizeof kExpfTab); }

float sao_expf_glibc(float x) {
  static const double kInvLn2N = 0x1.71547652b82fep+0 * 32;
  static const double kShift = 0x1.8p+52;
  static const double kC0 = 0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0);
  static const double kC1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32.0);
  static const double kC2 = 0x1.62e42ff0c52d6p-1 / 32.0;
  if (x != x) return x + x;
  if (x > 0x1.62e42ep6f) return INFINITY;  /* above log(2^128) */
  if (x < -0x1.9fe368p6f) return 0.0f;     /* below log(2^-150) */
  const double xd = (double)x;
  const double z = kInvLn2N * xd;
  const double kd_shifted = z + kShift;
  uint64_t ki;
  memcpy(&ki, &kd_shifted, sizeof ki);
  const double kd = kd_shifted - kShift;
  const double r = fma(kInvLn2N, xd, -kd);
  uint64_t t = kExpfTab[ki % 32] + (ki << 47);
  double s;
  memcpy(&s, &t, sizeof s);
  const double p = fma(kC0, r, kC1);
  const double r2 = r * r;
  double y = fma(kC2, r, 1.0);
  y = fma(p, r2, y);
  y = y * s;
  return (float)y;
}

long long sao_expf_glibc_mismatches(uint32_t first_bits, uint32_t last_bits, uint32_t stride) {
  long long bad = 0;
  if (stride == 0) stride = 1;
  for (uint64_t u = first_bits; u <= last_bits; u += stride) {
    const uint32_t bits = (uint32_t)u;
    float x, a, b;
    memcpy(&x, &bits, sizeof x);
    a = sao_expf_glibc(x);
    b = expf(x);
    if (memcmp(&a, &b, sizeof a) != 0) ++bad;
  }
  return bad;
}

/* The reference's builder (selection.cpp:12-94) with the exponential as a
 * parameter; received (optional) gets the [Hq][tokens] attention mass. */
static int build_lcr(const float* prompt_queries, const uint16_t* kv, size_t tokens,
                     size_t query_heads, size_t kv_heads, size_t head_dim,
                     size_t block_tokens, size_t local_window, size_t topk,
                     float* values, size_t* offsets, float (*expfn)(float),
                     float* received_out) {
  if (!prompt_queries || !kv || !values || tokens == 0 || kv_heads == 0 ||
      block_tokens == 0 || query_heads % kv_heads != 0 ||
      tokens % block_tokens != 0 || local_window == 0 || topk == 0 ||
      topk > block_tokens)
    return SAO_EINVAL;
  const size_t group = query_heads / kv_heads;
  const size_t blocks = tokens / block_tokens;
  const size_t token_stride = 2 * kv_heads * head_dim;
  const float scale = 1.0f / sqrtf((float)head_dim);
  float* received = (float*)calloc(query_heads * tokens, sizeof(float));
  float* logits = (float*)malloc(local_window * sizeof(float));
  size_t* order = (size_t*)malloc(block_tokens * sizeof(size_t));
  if (!received || !logits || !order) abort();
  for (size_t h = 0; h < query_heads; ++h) {
    const size_t g = h / group;
    for (size_t qp = 0; qp < tokens; ++qp) {
      const size_t start = qp + 1 > local_window ? qp + 1 - local_window : 0;
      const size_t count = qp - start + 1;
      const float* q = prompt_queries + (h * tokens + qp) * head_dim;
      float maximum = -INFINITY;
      for (size_t w = 0; w < count; ++w) {
        const uint16_t* k = kv + (start + w) * token_stride + g * head_dim;
        float dot = 0.0f;
        for (size_t d = 0; d < head_dim; ++d) dot += q[d] * sao_half_to_float(k[d]);
        logits[w] = dot * scale;
        if (logits[w] > maximum) maximum = logits[w];
      }
      float denominator = 0.0f;
      for (size_t w = 0; w < count; ++w) {
        logits[w] = expfn(logits[w] - maximum);
        denominator += logits[w];
      }
      for (size_t w = 0; w < count; ++w)
        received[h * tokens + start + w] += logits[w] / denominator;
    }
  }
  for (size_t h = 0; h < query_heads; ++h) {
    const size_t g = h / group;
    for (size_t b = 0; b < blocks; ++b) {
      for (size_t i = 0; i < block_tokens; ++i) order[i] = i;
      stable_sort_desc(order, block_tokens, received + h * tokens + b * block_tokens,
                       greater_mass);
      if (offsets)
        for (size_t r = 0; r < topk; ++r) offsets[(h * blocks + b) * topk + r] = order[r];
      for (size_t d = 0; d < head_dim; ++d) {
        float sum = 0.0f;
        for (size_t r = 0; r < topk; ++r) {
          const size_t t = b * block_tokens + order[r];
          sum += sao_half_to_float(kv[t * token_stride + g * head_dim + d]);
        }
        values[(h * blocks + b) * head_dim + d] = sum / (float)topk;
      }
    }
  }
  if (received_out) memcpy(received_out, received, query_heads * tokens * sizeof(float));
  free(order);
  free(logits);
  free(received);
  return SAO_OK;
}

static float expf_libm(float x) { return expf(x); }

int sao_build_local_causal_representatives(
    const float* prompt_queries, const uint16_t* kv, size_t tokens,
    size_t query_heads, size_t kv_heads, size_t head_dim, size_t block_tokens,
    size_t local_window, size_t topk, float* values, size_t* offsets) {
  return build_lcr(prompt_queries, kv, tokens, query_heads, kv_heads, head_dim, block_tokens,
                   local_window, topk, values, offsets, expf_libm, NULL);
}

int sao_build_local_causal_representatives_restated(
    const float* prompt_queries, const uint16_t* kv, size_t tokens,
    size_t query_heads, size_t kv_heads, size_t head_dim, size_t block_tokens,
    size_t local_window, size_t topk, float* values, size_t* offsets,
    float* received) {
  return build_lcr(prompt_queries, kv, tokens, query_heads, kv_heads, head_dim, block_tokens,
                   local_window, topk, values, offsets, sao_expf_glibc, received);
}

int sao_mean_key_representatives(const uint16_t* kv, size_t tokens,
                                 size_t kv_heads, size_t head_dim,
                                 size_t block_tokens, float* values) {
  if (!kv || !values || block_tokens == 0 || tokens % block_tokens != 0)
    return SAO_EINVAL;
  const size_t blocks = tokens / block_tokens;
  const size_t token_stride = 2 * kv_heads * head_dim;
  for (size_t g = 0; g < kv_heads; ++g)
    for (size_t b = 0; b < blocks; ++b)
      for (size_t d = 0; d < head_dim; ++d) {
        float sum = 0.0f;
        for (size_t t = 0; t < block_tokens; ++t)
          sum += sao_half_to_float(kv[(b * block_tokens + t) * token_stride + g * head_dim + d]);
        values[(g * blocks + b) * head_dim + d] = sum / (float)block_tokens;
      }
  return SAO_OK;
}

/* Budgeted selection over precomputed mean head scores: init blocks
 * [0, init), local blocks [n - local, n), then the best remaining blocks by
 * stable descending score until the budget is met; ids ascending.
 * cpp/src/selection.cpp:118-145. */
static size_t budget_select(const float* scores, size_t n, size_t budget,
                            size_t init_blocks, size_t local_blocks, size_t* ids) {
  unsigned char* chosen = (unsigned char*)calloc(n, 1);
  size_t* ranked = (size_t*)malloc(n * sizeof(size_t));
  if (!chosen || !ranked) abort();
  const size_t init_n = init_blocks < n ? init_blocks : n;
  const size_t local_n = local_blocks < n ? local_blocks : n;
  for (size_t b = 0; b < init_n; ++b) chosen[b] = 1;
  for (size_t b = n - local_n; b < n; ++b) chosen[b] = 1;
  for (size_t b = 0; b < n; ++b) ranked[b] = b;
  stable_sort_desc(ranked, n, scores, greater_f32);
  size_t count = 0;
  for (size_t b = 0; b < n; ++b) count += chosen[b];
  for (size_t r = 0; r < n && count != budget; ++r) {
    if (!chosen[ranked[r]]) {
      chosen[ranked[r]] = 1;
      ++count;
    }
  }
  size_t out = 0;
  for (size_t b = 0; b < n; ++b)
    if (chosen[b]) ids[out++] = b;
  free(ranked);
  free(chosen);
  return out;
}

/* cpp/src/selection.cpp:96-147. */
int sao_select_shared_blocks(const float* query, const float* representatives,
                             size_t query_heads, size_t blocks,
                             size_t head_dim, size_t budget_blocks,
                             size_t init_blocks, size_t local_blocks,
                             size_t* ids, size_t* count, float* scores) {
  if (!query || !representatives || !ids || !count || query_heads == 0 ||
      blocks == 0 || head_dim == 0 || budget_blocks == 0 ||
      budget_blocks > blocks || init_blocks + local_blocks > budget_blocks)
    return SAO_EINVAL;
  float* mean = (float*)calloc(blocks, sizeof(float));
  if (!mean) abort();
  for (size_t h = 0; h < query_heads; ++h) {
    for (size_t b = 0; b < blocks; ++b) {
      const float* r = representatives + (h * blocks + b) * head_dim;
      const float* q = query + h * head_dim;
      float dot = 0.0f;
      for (size_t d = 0; d < head_dim; ++d) dot += q[d] * r[d];
      mean[b] += dot / (float)query_heads;
    }
  }
  *count = budget_select(mean, blocks, budget_blocks, init_blocks, local_blocks, ids);
  if (scores) memcpy(scores, mean, blocks * sizeof(float));
  free(mean);
  return SAO_OK;
}

/* ------------------------------------------------------------------------ */
/* Batched paged path                                                        */
/* ------------------------------------------------------------------------ */

int sao_paged_score_select(const float* query, const float* reps,
                           const int32_t* sealed, size_t batch,
                           size_t query_heads, size_t kv_heads,
                           size_t head_dim, size_t rep_heads,
                           size_t rep_stride, size_t select_groups,
                           size_t budget, size_t init_blocks,
                           size_t local_blocks, int32_t* selected,
                           int32_t* counts, size_t sel_stride, float* scores) {
  if (!query || !reps || !sealed || !selected || !counts || kv_heads == 0 ||
      query_heads % kv_heads != 0 || select_groups == 0 ||
      kv_heads % select_groups != 0 ||
      (rep_heads != kv_heads && rep_heads != query_heads) || budget == 0 ||
      init_blocks + local_blocks > budget || sel_stride < budget)
    return SAO_EINVAL;
  const size_t group = query_heads / kv_heads;
  const size_t heads_per_sel = query_heads / select_groups;
  float* mean = (float*)malloc((rep_stride ? rep_stride : 1) * sizeof(float));
  size_t* ids = (size_t*)malloc((rep_stride ? rep_stride : 1) * sizeof(size_t));
  if (!mean || !ids) abort();
  int status = SAO_OK;
  for (size_t s = 0; s < batch && status == SAO_OK; ++s) {
    if (sealed[s] < 0 || (size_t)sealed[s] > rep_stride) {
      status = SAO_EINVAL;
      break;
    }
    const size_t n = (size_t)sealed[s];
    for (size_t sg = 0; sg < select_groups; ++sg) {
      for (size_t b = 0; b < n; ++b) mean[b] = 0.0f;
      for (size_t hi = 0; hi < heads_per_sel; ++hi) {
        const size_t h = sg * heads_per_sel + hi;
        const size_t rh = rep_heads == query_heads ? h : h / group;
        const float* q = query + (s * query_heads + h) * head_dim;
        const float* r = reps + (s * rep_heads + rh) * head_dim * rep_stride;
        for (size_t b = 0; b < n; ++b) {
          float dot = 0.0f;
          for (size_t d = 0; d < head_dim; ++d) dot += q[d] * r[d * rep_stride + b];
          mean[b] += dot / (float)heads_per_sel;
        }
      }
      size_t c = 0;
      if (n > 0) {
        if (budget >= n) {
          for (size_t b = 0; b < n; ++b) ids[b] = b;
          c = n;
        } else {
          c = budget_select(mean, n, budget, init_blocks, local_blocks, ids);
        }
      }
      int32_t* out = selected + (s * select_groups + sg) * sel_stride;
      for (size_t i = 0; i < c; ++i) out[i] = (int32_t)ids[i];
      counts[s * select_groups + sg] = (int32_t)c;
      if (scores) {
        float* so = scores + (s * select_groups + sg) * rep_stride;
        for (size_t b = 0; b < n; ++b) so[b] = mean[b];
      }
    }
  }
  free(ids);
  free(mean);
  return status;
}

int sao_paged_sparse_attention(const uint16_t* pool, size_t page_tokens,
                               const int32_t* block_table,
                               size_t table_stride, const int32_t* seq_len,
                               const int32_t* sealed, const int32_t* selected,
                               const int32_t* counts, size_t sel_stride,
                               size_t select_groups, const float* query,
                               size_t batch, size_t query_heads,
                               size_t kv_heads, size_t head_dim, float scale,
                               float* out) {
  if (!pool || !block_table || !seq_len || !sealed || !selected || !counts ||
      !query || !out || kv_heads == 0 || page_tokens == 0 ||
      query_heads % kv_heads != 0 || select_groups == 0 ||
      kv_heads % select_groups != 0)
    return SAO_EINVAL;
  const size_t group = query_heads / kv_heads;
  const size_t token_elems = 2 * kv_heads * head_dim;
  const size_t page_elems = page_tokens * token_elems;
  const size_t kv_per_sel = kv_heads / select_groups;
  size_t max_tokens = 0;
  for (size_t s = 0; s < batch; ++s) {
    const size_t tail = (size_t)seq_len[s] - (size_t)sealed[s] * page_tokens;
    size_t m = 0;
    for (size_t sg = 0; sg < select_groups; ++sg) {
      const size_t c = (size_t)counts[s * select_groups + sg];
      if (c > m) m = c;
    }
    if (m * page_tokens + tail > max_tokens) max_tokens = m * page_tokens + tail;
  }
  /* One KV head's gathered tokens as a 1-KV-head problem [t][K: D][V: D]. */
  uint16_t* gathered = (uint16_t*)malloc((max_tokens ? max_tokens : 1) * 2 * head_dim * sizeof(uint16_t));
  if (!gathered) abort();
  for (size_t s = 0; s < batch; ++s) {
    if (seq_len[s] < 0 || sealed[s] < 0 ||
        (size_t)sealed[s] * page_tokens > (size_t)seq_len[s]) {
      free(gathered);
      return SAO_EINVAL;
    }
    const int32_t* table = block_table + s * table_stride;
    for (size_t g = 0; g < kv_heads; ++g) {
      const size_t sg = g / kv_per_sel;
      const int32_t* ids = selected + (s * select_groups + sg) * sel_stride;
      const size_t c = (size_t)counts[s * select_groups + sg];
      size_t n = 0;
      for (size_t i = 0; i < c; ++i) {
        const uint16_t* page = pool + (size_t)table[ids[i]] * page_elems;
        for (size_t t = 0; t < page_tokens; ++t, ++n) {
          memcpy(gathered + n * 2 * head_dim, page + t * token_elems + g * head_dim,
                 head_dim * sizeof(uint16_t));
          memcpy(gathered + n * 2 * head_dim + head_dim,
                 page + t * token_elems + kv_heads * head_dim + g * head_dim,
                 head_dim * sizeof(uint16_t));
        }
      }
      for (size_t t = (size_t)sealed[s] * page_tokens; t < (size_t)seq_len[s]; ++t, ++n) {
        const uint16_t* tok = pool + (size_t)table[t / page_tokens] * page_elems +
                              (t % page_tokens) * token_elems;
        memcpy(gathered + n * 2 * head_dim, tok + g * head_dim, head_dim * sizeof(uint16_t));
        memcpy(gathered + n * 2 * head_dim + head_dim, tok + kv_heads * head_dim + g * head_dim,
               head_dim * sizeof(uint16_t));
      }
      float* o = out + (s * query_heads + g * group) * head_dim;
      if (n == 0) {
        memset(o, 0, group * head_dim * sizeof(float));
        continue;
      }
      sao_attention_reference(gathered, query + (s * query_heads + g * group) * head_dim, n,
                              group, 1, head_dim, scale, o);
    }
  }
  free(gathered);
  return SAO_OK;
}

int sao_paged_append(uint16_t* pool, size_t page_tokens,
                     const int32_t* block_table, size_t table_stride,
                     int32_t* seq_len, const float* k, const float* v,
                     const uint16_t* k16, const uint16_t* v16, size_t batch,
                     size_t kv_heads, size_t head_dim) {
  if (!pool || !block_table || !seq_len || page_tokens == 0 ||
      !((k && v) || (k16 && v16)))
    return SAO_EINVAL;
  const size_t token_elems = 2 * kv_heads * head_dim;
  const size_t width = kv_heads * head_dim;
  for (size_t s = 0; s < batch; ++s) {
    const size_t t = (size_t)seq_len[s];
    if (t / page_tokens >= table_stride) return SAO_EINVAL;
    uint16_t* dst = pool + (size_t)block_table[s * table_stride + t / page_tokens] *
                               page_tokens * token_elems +
                    (t % page_tokens) * token_elems;
    for (size_t i = 0; i < width; ++i) {
      dst[i] = k16 ? k16[s * width + i] : sao_float_to_half_rne(k[s * width + i]);
      dst[width + i] = v16 ? v16[s * width + i] : sao_float_to_half_rne(v[s * width + i]);
    }
    seq_len[s] += 1;
  }
  return SAO_OK;
}

int sao_paged_seal(const uint16_t* pool, size_t page_tokens,
                   const int32_t* block_table, size_t table_stride,
                   const int32_t* seq_len, int32_t* sealed,
                   int32_t* generation, float* reps, size_t rep_heads,
                   size_t rep_stride, size_t batch, size_t query_heads,
                   size_t kv_heads, size_t head_dim, size_t local_tokens) {
  if (!pool || !block_table || !seq_len || !sealed || !reps || kv_heads == 0 ||
      page_tokens == 0 || query_heads % kv_heads != 0 ||
      (rep_heads != kv_heads && rep_heads != query_heads))
    return SAO_EINVAL;
  const size_t group = query_heads / kv_heads;
  const size_t token_elems = 2 * kv_heads * head_dim;
  for (size_t s = 0; s < batch; ++s) {
    while ((size_t)seq_len[s] >= (size_t)sealed[s] * page_tokens + local_tokens + page_tokens) {
      const size_t b = (size_t)sealed[s];
      if (b >= rep_stride || b >= table_stride) return SAO_EINVAL;
      const uint16_t* page = pool + (size_t)block_table[s * table_stride + b] * page_tokens * token_elems;
      for (size_t g = 0; g < kv_heads; ++g)
        for (size_t d = 0; d < head_dim; ++d) {
          float sum = 0.0f;
          for (size_t t = 0; t < page_tokens; ++t)
            sum += sao_half_to_float(page[t * token_elems + g * head_dim + d]);
          const float rep = sum / (float)page_tokens;
          if (rep_heads == kv_heads) {
            reps[((s * rep_heads + g) * head_dim + d) * rep_stride + b] = rep;
          } else {
            for (size_t j = 0; j < group; ++j)
              reps[((s * rep_heads + g * group + j) * head_dim + d) * rep_stride + b] = rep;
          }
        }
      sealed[s] += 1;
      if (generation) generation[s] += 1;
    }
  }
  return SAO_OK;
}

void sao_pack_blocks(const uint16_t* pool, size_t page_elems,
                     const int32_t* pages, size_t count, uint16_t* out) {
  for (size_t i = 0; i < count; ++i)
    memcpy(out + i * page_elems, pool + (size_t)pages[i] * page_elems,
           page_elems * sizeof(uint16_t));
}

/* ------------------------------------------------------------------------ */
/* Decode-tail lifecycle                                                     */
/* ------------------------------------------------------------------------ */

/* cpp/src/kv_lifecycle_main.cpp:93-102: for each rank the first strict
 * maximum among tokens not picked yet. */
void sao_topk_argmax(const float* scores, size_t n, size_t k, size_t* top) {
  for (size_t r = 0; r < k; ++r) {
    size_t best = n;
    for (size_t t = 0; t < n; ++t) {
      int taken = 0;
      for (size_t j = 0; j < r; ++j) taken |= top[j] == t;
      if (taken) continue;
      if (best == n || scores[t] > scores[best]) best = t;
    }
    top[r] = best;
  }
}

static uint16_t lifecycle_value(size_t layer, size_t token, size_t value) {
  return (uint16_t)((layer * 1009 + token * 37 + value * 13) & 0xffffu);
}

/* cpp/src/kv_lifecycle_main.cpp:20-45, 61-62, 83-141 with the NVMe store
 * replaced by an in-memory byte check of every sealed block. */
int sao_run_synthetic_lifecycle(size_t layers, size_t decode_tokens,
                                sao_lifecycle_result* result) {
  enum { Q_HEADS = 16, KV_HEADS = 8, HEAD_DIM = 128, BLOCK = 32, LOCAL = 32 };
  const size_t token_values = 2 * KV_HEADS * HEAD_DIM;
  const size_t block_bytes = BLOCK * token_values * sizeof(uint16_t);
  const size_t cap = LOCAL + BLOCK; /* the tail never holds more */
  const size_t initial_blocks = 16;
  const size_t capacity_blocks = initial_blocks + (decode_tokens + 31) / 32 + 1;
  uint16_t* kv = (uint16_t*)malloc(cap * token_values * sizeof(uint16_t));
  float* score = (float*)malloc(Q_HEADS * cap * sizeof(float));
  if (!kv || !score || !result) abort();
  memset(result, 0, sizeof *result);
  uint64_t fnv = 1469598103934665603ull;
  int mismatch = 0;
  for (size_t layer = 0; layer < layers; ++layer) {
    size_t tokens = 0, sealed = 0, generation = 0;
    for (size_t step = 0; step < LOCAL + decode_tokens; ++step) {
      const size_t token = step; /* absolute token position */
      for (size_t v = 0; v < token_values; ++v)
        kv[tokens * token_values + v] = lifecycle_value(layer, token, v);
      ++tokens;
      for (size_t h = 0; h < Q_HEADS; ++h) {
        score[h * cap + tokens - 1] = 0.0f;
        for (size_t old = 0; old < tokens; ++old)
          score[h * cap + old] += (float)(((h + 3) * (old + 5) + token) % 97) / 97.0f;
      }
      if (step < LOCAL) continue; /* initial fill has no seal check */
      while (tokens >= LOCAL + BLOCK) {
        for (size_t h = 0; h < Q_HEADS; ++h) {
          size_t top[4];
          sao_topk_argmax(score + h * cap, BLOCK, 4, top);
          result->representative_head_audits += top[0] < BLOCK;
        }
        /* the sealed block must equal the closed form of the readback check */
        const size_t first = sealed * BLOCK;
        for (size_t t = 0; t < BLOCK; ++t)
          for (size_t v = 0; v < token_values; ++v) {
            const uint16_t x = kv[t * token_values + v];
            mismatch |= x != lifecycle_value(layer, first + t, v);
            fnv = (fnv ^ (x & 0xffu)) * 1099511628211ull;
            fnv = (fnv ^ (x >> 8)) * 1099511628211ull;
          }
        memmove(kv, kv + BLOCK * token_values, (tokens - BLOCK) * token_values * sizeof(uint16_t));
        for (size_t h = 0; h < Q_HEADS; ++h)
          memmove(score + h * cap, score + h * cap + BLOCK, (tokens - BLOCK) * sizeof(float));
        tokens -= BLOCK;
        ++sealed;
        ++generation;
        ++result->sealed_blocks;
      }
    }
    if (tokens < LOCAL || tokens >= LOCAL + BLOCK) mismatch = 1; /* unbounded tail */
    if (layer == 0) {
      result->resident_tail_tokens = tokens;
      result->generation = generation;
    }
  }
  result->store_bytes = layers * capacity_blocks * block_bytes;
  result->sealed_bytes_fnv = fnv;
  free(score);
  free(kv);
  return mismatch ? 1 : SAO_OK;
}

/* ------------------------------------------------------------------------ */
/* History prediction and miss correction                                    */
/* ------------------------------------------------------------------------ */

static int contains(const size_t* set, size_t n, size_t value) {
  for (size_t i = 0; i < n; ++i)
    if (set[i] == value) return 1;
  return 0;
}

static int cmp_size(const void* a, const void* b) {
  const size_t x = *(const size_t*)a, y = *(const size_t*)b;
  return x < y ? -1 : x > y;
}

/* cpp/src/pipeline_main.cpp:686-717. */
int sao_compare_prediction(const size_t* predicted, const size_t* oracle,
                           size_t n, size_t* hits, size_t* misses,
                           size_t* replacement_slots, size_t* miss_count) {
  size_t evicted = 0, missing = 0;
  *hits = 0;
  for (size_t slot = 0; slot < n; ++slot) {
    if (contains(oracle, n, predicted[slot])) ++*hits;
    else replacement_slots[evicted++] = slot;
  }
  for (size_t i = 0; i < n; ++i)
    if (!contains(predicted, n, oracle[i])) misses[missing++] = oracle[i];
  *miss_count = missing;
  if (missing != evicted) return SAO_EINVAL;
  size_t* corrected = (size_t*)malloc((n ? n : 1) * sizeof(size_t));
  if (!corrected) abort();
  memcpy(corrected, predicted, n * sizeof(size_t));
  for (size_t m = 0; m < missing; ++m) corrected[replacement_slots[m]] = misses[m];
  qsort(corrected, n, sizeof(size_t), cmp_size);
  /* the sorted corrected set is compared with the oracle as given (the
   * reference's oracle sets are produced in ascending order) */
  const int differ = memcmp(corrected, oracle, n * sizeof(size_t)) != 0;
  free(corrected);
  return differ ? 2 : SAO_OK;
}

/* cpp/src/pipeline_main.cpp:439-447. */
void sao_oracle_blocks(size_t step, size_t layer, size_t out[4]) {
  const size_t phase = step / 2;
  size_t first = 1 + (layer * 3 + phase) % 13;
  size_t second = 1 + (layer * 7 + phase * 2 + 5) % 13;
  if (second == first) second = 1 + second % 13;
  out[0] = 0;
  out[1] = first;
  out[2] = second;
  out[3] = 15;
  qsort(out, 4, sizeof(size_t), cmp_size);
}

/* cpp/src/pipeline_main.cpp:432-437. */
int sao_valid_ticket(size_t ticket_token, size_t ticket_layer,
                     size_t ticket_generation, const size_t ticket_blocks[4],
                     size_t token, size_t layer, size_t generation,
                     const size_t blocks[4]) {
  return ticket_token == token && ticket_layer == layer &&
         ticket_generation == generation &&
         memcmp(ticket_blocks, blocks, 4 * sizeof(size_t)) == 0;
}

/* ------------------------------------------------------------------------ */
/* Reference fixtures                                                        */
/* ------------------------------------------------------------------------ */

/* cpp/src/attention_main.cpp:131-156. */
void sao_fixture_c1(size_t tokens, size_t query_heads, size_t kv_heads,
                    size_t head_dim, uint16_t* kv, float* query) {
  for (size_t t = 0; t < tokens; ++t)
    for (size_t half = 0; half < 2; ++half)
      for (size_t g = 0; g < kv_heads; ++g)
        for (size_t d = 0; d < head_dim; ++d) {
          const float x = (float)(t * 17 + g * 13 + d * 3 + half * 19) * 0.013f;
          kv[t * 2 * kv_heads * head_dim + half * kv_heads * head_dim + g * head_dim + d] =
              sao_float_to_half(sinf(x) * 0.25f);
        }
  for (size_t i = 0; i < query_heads * head_dim; ++i)
    query[i] = cosf((float)(i * 7) * 0.009f) * 0.2f;
}

/* cpp/src/selection_main.cpp:113-147 (== cpp/src/pipeline_main.cpp:588-623). */
void sao_fixture_c2(size_t tokens, size_t query_heads, size_t kv_heads,
                    size_t head_dim, uint16_t* kv, float* prompt_queries) {
  const size_t group = query_heads / kv_heads;
  for (size_t t = 0; t < tokens; ++t)
    for (size_t half = 0; half < 2; ++half)
      for (size_t g = 0; g < kv_heads; ++g)
        for (size_t d = 0; d < head_dim; ++d) {
          const float x = (float)(t * 11 + g * 17 + d * 5 + half * 23) * 0.007f;
          kv[t * 2 * kv_heads * head_dim + half * kv_heads * head_dim + g * head_dim + d] =
              sao_float_to_half(sinf(x) * 0.2f);
        }
  for (size_t h = 0; h < query_heads; ++h) {
    const size_t g = h / group;
    for (size_t t = 0; t < tokens; ++t)
      for (size_t d = 0; d < head_dim; ++d) {
        const float key = sao_half_to_float(kv[t * 2 * kv_heads * head_dim + g * head_dim + d]);
        const float wiggle = cosf((float)(h * 19 + t * 7 + d * 3) * 0.011f);
        prompt_queries[(h * tokens + t) * head_dim + d] = key * 0.85f + wiggle * 0.03f;
      }
  }
}

size_t sao_p1_query_position(size_t tokens, size_t step, size_t layer) {
  return tokens - 1 - ((step * 17 + layer * 11) % 256);
}

/* cpp/src/pipeline_main.cpp:502-574 with the selection of :480-499
 * (select_shared_blocks(query, reps, 16, 16, 128, 4, 1, 1)). */
int sao_p1_dense_audit(const uint16_t* kv, const float* prompt_queries,
                       const float* representatives, size_t steps,
                       size_t layers, double* mass, double* recall) {
  enum { TOKENS = 512, BLOCKS = 16, BLOCK = 32, QH = 16, KVH = 8, D = 128 };
  const size_t group = QH / KVH;
  const float scale = 1.0f / sqrtf((float)D);
  float logits[TOKENS];
  float query[QH * D];
  double total_mass = 0.0, total_recall = 0.0;
  size_t audits = 0;
  for (size_t step = 0; step < steps; ++step) {
    for (size_t layer = 0; layer < layers; ++layer) {
      const size_t pos = sao_p1_query_position(TOKENS, step, layer);
      for (size_t h = 0; h < QH; ++h)
        memcpy(query + h * D, prompt_queries + (h * TOKENS + pos) * D, D * sizeof(float));
      size_t selected[BLOCKS], count = 0;
      if (sao_select_shared_blocks(query, representatives, QH, BLOCKS, D, 4, 1, 1,
                                   selected, &count, NULL) != SAO_OK || count != 4)
        return SAO_EINVAL;
      double block_mass[BLOCKS] = {0};
      for (size_t h = 0; h < QH; ++h) {
        const size_t g = h / group;
        float maximum = -INFINITY;
        for (size_t t = 0; t < TOKENS; ++t) {
          const uint16_t* k = kv + t * 2 * KVH * D + g * D;
          float dot = 0.0f;
          for (size_t d = 0; d < D; ++d) dot += query[h * D + d] * sao_half_to_float(k[d]);
          logits[t] = dot * scale;
          if (logits[t] > maximum) maximum = logits[t];
        }
        double denominator = 0.0;
        for (size_t t = 0; t < TOKENS; ++t) {
          logits[t] = expf(logits[t] - maximum);
          denominator += logits[t];
        }
        for (size_t t = 0; t < TOKENS; ++t)
          block_mass[t / BLOCK] += logits[t] / denominator / (double)QH;
      }
      double selected_mass = 0.0;
      for (size_t i = 0; i < 4; ++i) selected_mass += block_mass[selected[i]];
      unsigned char oracle_chosen[BLOCKS] = {0};
      oracle_chosen[0] = 1;
      oracle_chosen[BLOCKS - 1] = 1;
      size_t ranked[BLOCKS];
      for (size_t b = 0; b < BLOCKS; ++b) ranked[b] = b;
      stable_sort_desc(ranked, BLOCKS, block_mass, greater_f64);
      size_t chosen = 2;
      for (size_t r = 0; r < BLOCKS && chosen != 4; ++r)
        if (!oracle_chosen[ranked[r]]) {
          oracle_chosen[ranked[r]] = 1;
          ++chosen;
        }
      size_t hits = 0;
      for (size_t i = 0; i < 4; ++i) hits += oracle_chosen[selected[i]];
      total_mass += selected_mass;
      total_recall += (double)hits / 4.0;
      ++audits;
    }
  }
  *mass = total_mass / (double)audits;
  *recall = total_recall / (double)audits;
  return SAO_OK;
}

/* ------------------------------------------------------------------------ */
/* Synthetic data                                                            */
/* ------------------------------------------------------------------------ */

/* splitmix64 output function (Steele, Lea, Flood 2014). */
uint64_t sao_mix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

/* Sum of four 16-bit uniforms, centred (exact integer), times 1/sigma with
 * sigma = sqrt(4 * (65536^2 - 1) / 12). */
float sao_synth_normal(uint64_t seed, uint64_t index) {
  const uint64_t h = sao_mix64(sao_mix64(seed) ^ index);
  const int32_t sum = (int32_t)(h & 0xffffu) + (int32_t)((h >> 16) & 0xffffu) +
                      (int32_t)((h >> 32) & 0xffffu) + (int32_t)(h >> 48) - 131070;
  return (float)sum * 2.6428937e-05f;
}

void sao_synth_fill_half(uint64_t seed, uint64_t first_index, size_t count,
                         uint16_t* out) {
  for (size_t i = 0; i < count; ++i)
    out[i] = sao_float_to_half_rne(sao_synth_normal(seed, first_index + i));
}

void sao_synth_fill_float(uint64_t seed, uint64_t first_index, size_t count,
                          float* out) {
  for (size_t i = 0; i < count; ++i) out[i] = sao_synth_normal(seed, first_index + i);
}

/* ------------------------------------------------------------------------ */
/* Query producer / output consumer around attention                        */
/* (cpp/src/qwen_layer_main.cpp:125-183 kernels, :600-645 host order;       */
/*  cpp/src/qwen_chain_main.cpp:365-399)                                    */
/* ------------------------------------------------------------------------ */

/* rms_norm (qwen_layer_main.cpp:125-143): out = x * (1/sqrt(mean(x^2) + eps))
 * * w, sums in double here (the reference's order is a 256-thread tree). */
int sao_rms_norm(const float* x, const float* w, float* out, size_t rows, size_t width, float eps) {
  if (!x || !w || !out || width == 0) return -1;
  for (size_t r = 0; r < rows; ++r) {
    const float* xr = x + r * width;
    double ss = 0.0;
    for (size_t i = 0; i < width; ++i) ss += (double)xr[i] * (double)xr[i];
    const double inv = 1.0 / sqrt(ss / (double)width + (double)eps);
    for (size_t i = 0; i < width; ++i) out[r * width + i] = (float)((double)xr[i] * inv * (double)w[i]);
  }
  return 0;
}

/* The projections (cublasSgemm with CUBLAS_OP_T on the row-major [out][in]
 * weight, qwen_layer_main.cpp:578-584): y[r][o] = sum_i x[r][i] w[o][i]
 * (+ residual[r][o], the residual add of :644-645), sums in double. */
int sao_linear(const float* x, const float* w, const float* residual, float* y, size_t rows, size_t in,
               size_t out) {
  if (!x || !w || !y || in == 0) return -1;
  for (size_t r = 0; r < rows; ++r)
    for (size_t o = 0; o < out; ++o) {
      double acc = 0.0;
      for (size_t i = 0; i < in; ++i) acc += (double)x[r * in + i] * (double)w[o * in + i];
      if (residual) acc += (double)residual[r * out + o];
      y[r * out + o] = (float)acc;
    }
  return 0;
}

/* RoPE frequencies: theta^(-2i/d) for i < d/2, correctly rounded to fp32
 * (the reference evaluates powf(theta, -2.0f * i / width) on the GPU,
 * qwen_layer_main.cpp:162-164, within its 2-ulp bound of this). */
void sao_rope_inv_freq(float theta, size_t head_dim, float* inv_freq) {
  for (size_t i = 0; i < head_dim / 2; ++i)
    inv_freq[i] = (float)pow((double)theta, -2.0 * (double)i / (double)head_dim);
}

/* head_rms then rope, in place, on x [rows][heads][head_dim]
 * (qwen_layer_main.cpp:145-172): every head row is normalised with w, then
 * dims d and d + head_dim/2 are rotated by angle = position[r] * inv_freq[i]
 * (fp32 product, as the reference forms it); cos and sin of that fp32 angle
 * in double.  positions NULL: no rotation (the value projection). */
int sao_qk_norm_rope(float* x, const float* w, const int32_t* positions, size_t rows, size_t heads,
                     size_t head_dim, float theta, float eps) {
  if (!x || head_dim == 0 || head_dim % 2 || head_dim > 512) return -1;
  float inv_freq[256];
  sao_rope_inv_freq(theta, head_dim, inv_freq);
  const size_t half = head_dim / 2;
  float row[512];
  for (size_t r = 0; r < rows; ++r)
    for (size_t h = 0; h < heads; ++h) {
      float* v = x + (r * heads + h) * head_dim;
      if (w) {
        double ss = 0.0;
        for (size_t d = 0; d < head_dim; ++d) ss += (double)v[d] * (double)v[d];
        const double inv = 1.0 / sqrt(ss / (double)head_dim + (double)eps);
        for (size_t d = 0; d < head_dim; ++d) v[d] = (float)((double)v[d] * inv * (double)w[d]);
      }
      if (!positions) continue;
      memcpy(row, v, head_dim * sizeof(float));
      for (size_t d = 0; d < head_dim; ++d) {
        const size_t i = d < half ? d : d - half;
        const float angle = (float)positions[r] * inv_freq[i];
        const double c = cos((double)angle), sn = sin((double)angle);
        const double rotated = d < half ? -(double)row[d + half] : (double)row[d - half];
        v[d] = (float)((double)row[d] * c + rotated * sn);
      }
    }
  return 0;
}
