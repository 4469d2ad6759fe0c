/*
 * CPU oracle, C part.  TEST INFRASTRUCTURE ONLY: the product path never links,
 * loads or calls this file.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, as the checker.
 *
 * These functions pin the parts of the reference path whose results depend on
 * the floating-point evaluation order (block-mask selection near the top-p
 * threshold, exact-FP32 role clustering).  Each fixes one canonical order that
 * the HIP kernels follow as well, so GPU and oracle agree bit for bit:
 *
 *   - dot products: sequential fmaf over d = 0..D-1 starting from +0.0f;
 *   - sums over clusters: sequential in index order;
 *   - exp: spr_oracle_expf below (Cody-Waite range reduction + degree-7
 *     Taylor polynomial, written from the textbook method; pinned against
 *     numpy's float64 exp in tests/test_oracle.py);
 *   - sort: descending value, ties broken by ascending index.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no -ffast-math).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <float.h>

/* e^x in fp32.  x < -87 returns 0 (keeps every nonzero result normal, so
 * the final scaling by 2^n is exact); x > 89 returns +inf.  The scaling is
 * applied as 2^(n - n/2) * 2^(n/2) so that n = 128 (x up to ln(FLT_MAX))
 * stays finite. */
float spr_oracle_expf(float x) {
  if (x != x) return x;
  if (x < -87.0f) return 0.0f;
  if (x > 89.0f) return INFINITY;
  const float log2e = 1.44269504088896341f;
  const float ln2_hi = 0.693145751953125f;        /* 12 significant bits: n*ln2_hi exact */
  const float ln2_lo = 1.428606765330187045e-06f; /* ln2 - ln2_hi */
  float n = rintf(x * log2e);
  float r = fmaf(-n, ln2_hi, x);
  r = fmaf(-n, ln2_lo, r);
  /* Taylor coefficients 1/k!, k = 7..0, Horner with fmaf. */
  float p = 1.98412698412698413e-04f;
  p = fmaf(p, r, 1.38888888888888889e-03f);
  p = fmaf(p, r, 8.33333333333333333e-03f);
  p = fmaf(p, r, 4.16666666666666667e-02f);
  p = fmaf(p, r, 1.66666666666666667e-01f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  int ni = (int)n;
  int nb = ni >> 1, na = ni - nb;
  uint32_t bits_a = (uint32_t)(na + 127) << 23, bits_b = (uint32_t)(nb + 127) << 23;
  float sa, sb;
  memcpy(&sa, &bits_a, sizeof(sa));
  memcpy(&sb, &bits_b, sizeof(sb));
  return (p * sa) * sb;
}

void spr_oracle_expf_array(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = spr_oracle_expf(x[i]);
}

/* Round fp32 to bfloat16 (nearest even), returned as fp32. */
static float bf16r(float f) {
  uint32_t u;
  memcpy(&u, &f, sizeof(u));
  if ((u & 0x7fffffffu) > 0x7f800000u) return f;
  u += 0x7fffu + ((u >> 16) & 1u);
  u &= 0xffff0000u;
  memcpy(&f, &u, sizeof(f));
  return f;
}

typedef struct {
  float value;
  int32_t index;
} keyed_t;

static int cmp_desc_then_index(const void* a, const void* b) {
  const keyed_t* x = (const keyed_t*)a;
  const keyed_t* y = (const keyed_t*)b;
  if (x->value > y->value) return -1;
  if (x->value < y->value) return 1;
  return (x->index > y->index) - (x->index < y->index);
}

/*
 * Top-p cluster-pair map (reference: kmeans_utils.py:1710-1742 identify_dynamic_map
 * with weighted_softmax :1698-1707), canonical fp32 order.
 *   qc [bh, qn, d], kc [bh, kn, d] fp32; k_sizes [bh, kn] int32
 *   map [bh, qn, kn] uint8 (0/1)
 *   cum_out/order_out (optional, [bh, qn, kn]) expose the running sum and the
 *   sorted order for near-threshold analysis.
 *   bf16 != 0 reproduces torch's bfloat16 dtype flow for bf16 centroids: the
 *   matmul output and the scaled scores are bf16, weighted_softmax returns
 *   bf16 probabilities (.to(input_dtype)), cumsum writes bf16 partial sums of
 *   an fp32 accumulator, and `cumsum > p` compares in bf16 (p rounded to bf16).
 */
void oracle_topp_map(const float* qc, const float* kc, const int32_t* k_sizes,
                     int64_t bh, int32_t qn, int32_t kn, int32_t d,
                     float sqrt_d, float p, int32_t preserve_len, int32_t bf16,
                     uint8_t* map, float* cum_out, int32_t* order_out) {
  const float thr = bf16 ? bf16r(p) : p;
  float* s = (float*)malloc(sizeof(float) * kn);
  float* we = (float*)malloc(sizeof(float) * kn);
  keyed_t* keyed = (keyed_t*)malloc(sizeof(keyed_t) * kn);
  for (int64_t h = 0; h < bh; ++h) {
    for (int32_t i = 0; i < qn; ++i) {
      const float* q = qc + (h * qn + i) * (int64_t)d;
      float m = -INFINITY;
      for (int32_t j = 0; j < kn; ++j) {
        const float* k = kc + (h * kn + j) * (int64_t)d;
        float acc = 0.0f;
        for (int32_t t = 0; t < d; ++t) acc = fmaf(q[t], k[t], acc);
        s[j] = bf16 ? bf16r(bf16r(acc) / sqrt_d) : acc / sqrt_d;
        if (s[j] > m) m = s[j];
      }
      float sum = 0.0f;
      for (int32_t j = 0; j < kn; ++j) {
        float w = (float)k_sizes[h * kn + j];
        we[j] = w * spr_oracle_expf(s[j] - m);
        sum = sum + we[j];
      }
      float denom = sum > 1e-12f ? sum : 1e-12f;
      for (int32_t j = 0; j < kn; ++j) {
        float prob = we[j] / denom;
        keyed[j].value = bf16 ? bf16r(prob) : prob;
        keyed[j].index = j;
      }
      qsort(keyed, kn, sizeof(keyed_t), cmp_desc_then_index);
      uint8_t* row = map + (h * qn + i) * (int64_t)kn;
      memset(row, 0, kn);
      float cum = 0.0f;
      float prev = 0.0f;
      for (int32_t r = 0; r < kn; ++r) {
        cum = cum + keyed[r].value;
        float shown = bf16 ? bf16r(cum) : cum;
        int remove = (r > 0) && (prev > thr);
        if (r < preserve_len) remove = 0;
        row[keyed[r].index] = remove ? 0 : 1;
        if (cum_out) cum_out[(h * qn + i) * (int64_t)kn + r] = shown;
        if (order_out) order_out[(h * qn + i) * (int64_t)kn + r] = keyed[r].index;
        prev = shown;
      }
    }
  }
  free(s);
  free(we);
  free(keyed);
}

/*
 * Budget selector (reference: n8_ops.cu:271-322 selector_budget_kernel for
 * mode 0; selector_budget.py:10-54 and n8_v6.py:1088-1111 for mode 1).
 * Scores sorted descending, ties by ascending index.
 *   mode 0: walk positive-cost clusters; keep while the running cost fits; the
 *           first positive-cost cluster that does not fit is added afterwards
 *           if the budget is positive and not yet reached.
 *   mode 1: keep = positive & prefix-cost <= budget; then the cluster at sorted
 *           position `count` (number kept) is added if the kept cost is below
 *           the budget and some positive cluster is left unkept.
 * out [bh, qn+1, kn+1]: header row/column set as the reference does.
 */
void oracle_select_budget(const float* scores, const int32_t* sizes,
                          const int32_t* budgets, int64_t bh, int32_t qn,
                          int32_t kn, int32_t mode, uint8_t* out) {
  keyed_t* keyed = (keyed_t*)malloc(sizeof(keyed_t) * kn);
  const int64_t stride = (int64_t)kn + 1;
  memset(out, 0, (size_t)(bh * (qn + 1) * stride));
  for (int64_t h = 0; h < bh; ++h) {
    uint8_t* head = out + h * (qn + 1) * stride;
    head[0] = 1;
    for (int32_t i = 0; i < qn; ++i) {
      const float* srow = scores + (h * qn + i) * (int64_t)kn;
      for (int32_t j = 0; j < kn; ++j) {
        keyed[j].value = srow[j];
        keyed[j].index = j;
      }
      qsort(keyed, kn, sizeof(keyed_t), cmp_desc_then_index);
      uint8_t* row = head + (int64_t)(i + 1) * stride;
      row[0] = 1;
      const int32_t budget = budgets[h * qn + i];
      if (mode == 0) {
        int32_t selected = 0;
        int32_t crossing = -1;
        for (int32_t r = 0; r < kn; ++r) {
          int32_t c = keyed[r].index;
          int32_t cost = sizes[h * kn + c];
          if (cost <= 0) continue;
          if (crossing < 0 && selected + cost <= budget) {
            row[c + 1] = 1;
            selected += cost;
          } else if (crossing < 0) {
            crossing = c;
          }
        }
        if (budget > 0 && selected < budget && crossing >= 0) row[crossing + 1] = 1;
      } else {
        int64_t cum = 0;
        int64_t selected = 0;
        int32_t count = 0;
        int32_t valid = 0;
        for (int32_t r = 0; r < kn; ++r) {
          int32_t c = keyed[r].index;
          int32_t cost = sizes[h * kn + c];
          if (cost > 0) {
            valid += 1;
            cum += cost;
            if (cum <= budget) {
              row[c + 1] = 1;
              selected += cost;
              count += 1;
            }
          }
        }
        if (budget > 0 && selected < budget && count < valid && count < kn) {
          row[keyed[count].index + 1] = 1;
        }
      }
    }
  }
  free(keyed);
}

/*
 * One exact-FP32 Lloyd step at D=64 (reference: n8_ops.cu:198-269).
 * Distance: sequential fmaf over r of (p[r]-c[r])^2; ties to the lower index.
 * Sums are accumulated in double (exact for these inputs), then
 * mean = (float)(sum / count); empty clusters keep the previous centroid.
 */
void oracle_role_step64(const float* features, const float* centroids,
                        int64_t bh, int64_t n, int32_t c, int32_t* labels,
                        float* out_centroids, int32_t* sizes, float* best_dist) {
  const int D = 64;
  double* sums = (double*)calloc((size_t)(c * D), sizeof(double));
  for (int64_t h = 0; h < bh; ++h) {
    memset(sums, 0, sizeof(double) * (size_t)(c * D));
    int32_t* sz = sizes + h * c;
    memset(sz, 0, sizeof(int32_t) * (size_t)c);
    for (int64_t t = 0; t < n; ++t) {
      const float* p = features + (h * n + t) * D;
      float bestd = FLT_MAX;
      int32_t besti = 0x7fffffff;
      for (int32_t k = 0; k < c; ++k) {
        const float* q = centroids + (h * c + k) * D;
        float dist = 0.0f;
        for (int r = 0; r < D; ++r) {
          float delta = p[r] - q[r];
          dist = fmaf(delta, delta, dist);
        }
        if (dist < bestd || (dist == bestd && k < besti)) {
          bestd = dist;
          besti = k;
        }
      }
      labels[h * n + t] = besti;
      if (best_dist) best_dist[h * n + t] = bestd;
      sz[besti] += 1;
      for (int r = 0; r < D; ++r) sums[besti * D + r] += (double)p[r];
    }
    for (int32_t k = 0; k < c; ++k) {
      for (int r = 0; r < D; ++r) {
        int64_t o = (h * c + k) * D + r;
        out_centroids[o] = sz[k] > 0 ? (float)(sums[k * D + r] / (double)sz[k])
                                     : centroids[o];
      }
    }
  }
  free(sums);
}
