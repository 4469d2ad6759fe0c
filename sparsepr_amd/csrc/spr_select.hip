// Block selection: top-p cluster-pair map, exact budget selector, mask
// compaction into a kept-cluster schedule, kept-pair density.
//
// Replaces:
//   identify_dynamic_map + weighted_softmax   (src/sparsepr/kmeans_utils.py:1710-1742, :1698-1707)
//   svg_ear_select_budget(_schedule)          (kernels/n8_ext/csrc/n8_ops.cu:271-322, :541-638)
//   exact_budget_dynamic_map_triton           (kernels/triton/selector_budget.py:10-54, :131-171)
//   compact_selected_clusters                 (n8_ops.cu:324-355, :617-638)
//   density_calculation                       (kmeans_utils.py:285-303)
//
// The top-p map must be reproducible bit for bit on the CPU (the decision
// `cumsum > p` flips with the last ulp near the threshold), so every step has a
// fixed fp32 evaluation order, with contraction disabled:
//   score = (sequential fmaf over d of qc*kc) / sqrt(D)
//   w_j e_j = size_j * canonical_expf(score_j - max)      (spr_common.h)
//   denom  = max(sum_j in index order, 1e-12)
//   prob_j = w_j e_j / denom
//   order  = descending prob, ties by ascending index
//   keep rank r iff r == 0 or cumsum(prob[order[0..r-1]]) <= p (r < preserve kept too).
// With bf16 centroids (score_bf16 = 1) the reference's tensors are bf16 along the
// way and the kernel rounds at the same points: matmul output and scaled score,
// the softmax output (weighted_softmax returns input_dtype), each cumsum output,
// and the threshold (a python float compared against a bf16 tensor is cast to bf16).
#pragma clang fp contract(off)

#include <type_traits>

#include "spr_common.h"

namespace {

constexpr int SEL_THREADS = 256;
constexpr int MAX_KC = 4096;

__device__ __forceinline__ float bf16r(float f) { return spr::bf16_to_f32(spr::f32_to_bf16(f)); }

__device__ __forceinline__ bool ranks_before(float pa, int ia, float pb, int ib) {
  return pa > pb || (pa == pb && ia < ib);
}

__device__ float block_max(float v, float* scratch) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) scratch[wave] = v;
  __syncthreads();
  float m = scratch[0];
  for (int w = 1; w < static_cast<int>(blockDim.x >> 6); ++w) m = fmaxf(m, scratch[w]);
  __syncthreads();
  return m;
}

// score(q, k) = sum_t q[t] k[t], sequential fused multiply-adds in t.  The key
// centroid's row is read with 16-byte loads, 32 floats issued ahead of their
// multiply-adds (16-byte aligned rows), so the chain does not wait on one load
// per step.
__device__ __forceinline__ float row_dot(const float* q_row, const float* kr, int d) {
  float acc = 0.0f;
  if ((d & 3) == 0 && (reinterpret_cast<uintptr_t>(kr) & 15) == 0) {
    const spr::f32x4* k4 = reinterpret_cast<const spr::f32x4*>(kr);
    const spr::f32x4* q4 = reinterpret_cast<const spr::f32x4*>(q_row);
    const int n4 = d >> 2;
    for (int t = 0; t < n4; t += 8) {
      spr::f32x4 kv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) kv[u] = t + u < n4 ? k4[t + u] : spr::f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (t + u < n4) {
          const spr::f32x4 qv = q4[t + u];
#pragma unroll
          for (int e = 0; e < 4; ++e) acc = __builtin_fmaf(qv[e], kv[u][e], acc);
        }
      }
    }
  } else {
    for (int t = 0; t < d; ++t) acc = __builtin_fmaf(q_row[t], kr[t], acc);
  }
  return acc;
}

// Sort key of (value, index) under ranks_before: ascending keys are descending values,
// ties by ascending index.  The high word is the value's order-preserving unsigned image
// (-0 taken as +0, so that equal values tie as under ==), complemented; the low word is
// the index.  (NaN values, which ranks_before leaves unordered, get a fixed place.)
__device__ __forceinline__ uint64_t rank_key(float v, int32_t i) {
  uint32_t b = __float_as_uint(v);
  if ((b << 1) == 0u) b = 0u;
  const uint32_t up = (b & 0x80000000u) ? ~b : (b | 0x80000000u);  // ascending in v
  return (static_cast<uint64_t>(~up) << 32) | static_cast<uint32_t>(i);
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int mask) {
  const int lo = __shfl_xor(static_cast<int>(static_cast<uint32_t>(v)), mask, 64);
  const int hi = __shfl_xor(static_cast<int>(static_cast<uint32_t>(v >> 32)), mask, 64);
  return (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo);
}

// One exchange stage (run length SIZE, partner distance STRIDE) of a bitonic network over
// 64 E keys, lane l holding positions l E .. l E + E - 1; keys end up ascending.  Strides
// below E exchange inside the lane, the others with lane ^ (STRIDE / E) by shuffles (then
// SIZE > STRIDE >= E, so a run's direction, position & SIZE, comes from the lane bits).
template <int E, int SIZE, int STRIDE>
__device__ __forceinline__ void bitonic_stage(uint64_t (&k)[E], int lane) {
  if constexpr (STRIDE >= E) {
    constexpr int LX = STRIDE / E;
    const bool take_min = ((lane & LX) == 0) == (((lane * E) & SIZE) == 0);
#pragma unroll
    for (int r = 0; r < E; ++r) {
      const uint64_t o = shfl_xor_u64(k[r], LX);
      k[r] = (take_min ? o < k[r] : o > k[r]) ? o : k[r];
    }
  } else {
#pragma unroll
    for (int r = 0; r < E; ++r) {
      if ((r & STRIDE) == 0) {
        constexpr bool IN_LANE = SIZE < E;
        const bool ascending = IN_LANE ? (r & SIZE) == 0 : ((lane * E) & SIZE) == 0;
        const uint64_t a = k[r], b = k[r | STRIDE];
        const bool sw = ascending ? b < a : a < b;
        k[r] = sw ? b : a;
        k[r | STRIDE] = sw ? a : b;
      }
    }
  }
}

// The whole network from stage (SIZE, STRIDE) on, every index a compile-time constant.
template <int E, int SIZE, int STRIDE>
__device__ __forceinline__ void bitonic_from(uint64_t (&k)[E], int lane) {
  bitonic_stage<E, SIZE, STRIDE>(k, lane);
  if constexpr (STRIDE > 1) {
    bitonic_from<E, SIZE, STRIDE / 2>(k, lane);
  } else if constexpr (SIZE < 64 * E) {
    bitonic_from<E, 2 * SIZE, SIZE>(k, lane);
  }
}

// Sorts 64 E keys held E per lane (lane l: positions l E .. l E + E - 1), ascending.
template <int E>
__device__ __forceinline__ void wave_sort_keys(uint64_t (&k)[E], int lane) {
  bitonic_from<E, 2, 1>(k, lane);
}

// Sorts the n2 (a power of two, n2 <= 64 E) (value, index) pairs in LDS so that
// ranks_before holds along the array.  One wave, in registers (wave_sort_keys; positions
// past n2 hold the largest key); then the values (bit for bit, read back through the
// sorted indices) and indices are stored in rank order.  The order is total, so the
// result equals a rank sort's.  Only the calling wave touches the arrays.
template <int E>
__device__ void wave_rank_sort(float* v, int32_t* idx, int n2) {
  const int lane = threadIdx.x & 63;
  uint64_t k[E];
#pragma unroll
  for (int r = 0; r < E; ++r) {
    const int pos = lane * E + r;
    k[r] = pos < n2 ? rank_key(v[pos], idx[pos]) : ~0ull;
  }
  wave_sort_keys<E>(k, lane);
  float val[E];
#pragma unroll
  for (int r = 0; r < E; ++r) {
    const int pos = lane * E + r;
    val[r] = pos < n2 ? v[static_cast<uint32_t>(k[r])] : 0.0f;
  }
#pragma unroll
  for (int r = 0; r < E; ++r) {
    const int pos = lane * E + r;
    if (pos < n2) {
      v[pos] = val[r];
      idx[pos] = static_cast<int32_t>(static_cast<uint32_t>(k[r]));
    }
  }
}

// Calls f(std::integral_constant<int, E>) with E = n2 / 64 (at least 1), the register
// count per lane of wave_rank_sort, for n2 a power of two up to 4096.
template <typename F>
void by_sort_width(int n2, F&& f) {
  if (n2 <= 64) f(std::integral_constant<int, 1>{});
  else if (n2 <= 128) f(std::integral_constant<int, 2>{});
  else if (n2 <= 256) f(std::integral_constant<int, 4>{});
  else if (n2 <= 512) f(std::integral_constant<int, 8>{});
  else if (n2 <= 1024) f(std::integral_constant<int, 16>{});
  else if (n2 <= 2048) f(std::integral_constant<int, 32>{});
  else f(std::integral_constant<int, 64>{});
}

__device__ __forceinline__ int pow2_at_least(int n) {
  int n2 = 1;
  while (n2 < n) n2 <<= 1;
  return n2;
}

// One workgroup per (bh, q-cluster) row.
//   scores, max, weighted exp, sum (index order, one wave reading 64 values per step
//   into registers), probabilities;
//   sort by (probability desc, index asc): one wave's bitonic network in registers
//   (the order is total, so the result equals a rank sort's);
//   the shown cumsum of the sorted probabilities never decreases (terms >= 0,
//   bf16 rounding monotone), so "remove rank r when r > 0 and the cumsum through
//   r - 1 exceeds p" keeps exactly the ranks below cut = max(first such r,
//   preserve): one wave walks the chain up to the crossing only, 64 values at a time.
// Dynamic LDS: 2 x n2 floats/ints (n2 = kn rounded up to a power of two).
template <int E>  // n2 <= 64 E
__global__ __launch_bounds__(SEL_THREADS) void topp_map_kernel(const float* __restrict__ qc,
                                                               const float* __restrict__ kc,
                                                               const int32_t* __restrict__ k_sizes,
                                                               int32_t qn, int32_t kn, int32_t d, float sqrt_d,
                                                               float p, int32_t preserve, int32_t score_bf16,
                                                               uint8_t* __restrict__ map,
                                                               int32_t* __restrict__ budgets) {
  __shared__ __attribute__((aligned(16))) float q_row[512];
  extern __shared__ __attribute__((aligned(16))) uint8_t sel_dyn[];
  __shared__ float scratch[SEL_THREADS / 64];
  __shared__ float denom_s;
  __shared__ int32_t cut_s;
  __shared__ unsigned long long budget_s;

  const int n2 = pow2_at_least(kn);
  float* sorted_val = reinterpret_cast<float*>(sel_dyn);         // [n2]: weighted exps, then probabilities
  int32_t* sorted_idx = reinterpret_cast<int32_t*>(sorted_val + n2);  // [n2]
  const int lane = threadIdx.x & 63;
  const bool wave0 = threadIdx.x < 64;
  const int64_t row = blockIdx.x;  // bh * qn + q
  const int64_t bh = row / qn;
  const float* qrow = qc + row * d;
  const float* kb = kc + bh * kn * static_cast<int64_t>(d);
  const int32_t* sz = k_sizes + bh * kn;
  for (int t = threadIdx.x; t < d; t += blockDim.x) q_row[t] = qrow[t];
  __syncthreads();

  float local_max = -__builtin_huge_valf();
  for (int j = threadIdx.x; j < kn; j += blockDim.x) {
    const float acc = row_dot(q_row, kb + static_cast<int64_t>(j) * d, d);
    const float sc = score_bf16 ? bf16r(bf16r(acc) / sqrt_d) : acc / sqrt_d;
    sorted_val[j] = sc;
    local_max = fmaxf(local_max, sc);
  }
  const float m = block_max(local_max, scratch);

  for (int j = threadIdx.x; j < kn; j += blockDim.x) {
    const float w = static_cast<float>(sz[j]);
    sorted_val[j] = w * spr::canonical_expf(sorted_val[j] - m);
  }
  __syncthreads();
  if (wave0) {  // sum in index order
    float sum = 0.0f;
    for (int base = 0; base < kn; base += 64) {
      const float x = base + lane < kn ? sorted_val[base + lane] : 0.0f;
      const int n = min(64, kn - base);
      for (int u = 0; u < n; ++u) sum = sum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), u));
    }
    if (lane == 0) denom_s = sum > 1e-12f ? sum : 1e-12f;
  }
  __syncthreads();
  const float denom = denom_s;
  for (int j = threadIdx.x; j < n2; j += blockDim.x) {
    if (j < kn) {
      const float prob = sorted_val[j] / denom;
      sorted_val[j] = score_bf16 ? bf16r(prob) : prob;
    } else {
      sorted_val[j] = -__builtin_huge_valf();  // padding sorts last
    }
    sorted_idx[j] = j;
  }
  __syncthreads();
  if (wave0) wave_rank_sort<E>(sorted_val, sorted_idx, n2);
  __syncthreads();

  if (wave0) {
    const float thr = score_bf16 ? bf16r(p) : p;
    float cum = 0.0f;
    float prev = 0.0f;  // shown cumsum through rank r - 1
    int cut = kn;
    bool done = false;
    for (int base = 0; base < kn && !done; base += 64) {
      const float x = base + lane < kn ? sorted_val[base + lane] : 0.0f;
      const int n = min(64, kn - base);
      for (int u = 0; u < n; ++u) {
        const int r = base + u;
        if (r > 0 && prev > thr) {
          cut = r > preserve ? r : preserve;
          done = true;
          break;
        }
        cum = cum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), u));
        prev = score_bf16 ? bf16r(cum) : cum;
      }
    }
    if (lane == 0) {
      cut_s = cut < kn ? cut : kn;
      budget_s = 0;
    }
  }
  __syncthreads();
  const int cut = cut_s;
  if (map != nullptr) {
    uint8_t* out = map + row * kn;
    for (int r = threadIdx.x; r < kn; r += blockDim.x) out[sorted_idx[r]] = r < cut ? 1 : 0;
  }
  if (budgets != nullptr) {
    // key-token budget of the kept clusters (n8_v6.py:226-230): sum of their sizes;
    // integers, so the summation order does not matter
    unsigned long long part = 0;
    for (int r = threadIdx.x; r < cut; r += blockDim.x) part += static_cast<unsigned long long>(max(sz[sorted_idx[r]], 0));
    if (part != 0) atomicAdd(&budget_s, part);
    __syncthreads();
    if (threadIdx.x == 0) budgets[row] = static_cast<int32_t>(min(budget_s, 0x7FFFFFFFull));
  }
}

// One wave per (bh, q) row of scores [bh, qn, kn].
// mode 0: n8_ops.cu semantics, mode 1: selector_budget.py / CPU-fallback semantics.
// Both walk the clusters in (score desc, index asc) order, skip empty ones, and keep a
// cluster while the running cost of the non-empty clusters so far stays within the
// budget; the running cost only grows, so that is the set {non-empty r : cum_r <= budget}
// with cum the inclusive prefix sum of the non-empty costs in sorted order.  They differ
// in the one extra cluster taken when the budget is not met: mode 0 the first non-empty
// cluster past it (the crossing), mode 1 the cluster at sorted position `count`.
// The row's keys are sorted in registers (wave_sort_keys: lane l holds ranks
// l E .. l E + E - 1), the prefix sum runs over those ranks where they lie (lane totals
// scanned across the wave), and the kept flags go through an LDS byte row to the map row
// and the ascending schedule.
// Dynamic LDS: kn bytes rounded up to 16.
template <int E>  // kn <= 64 E
__global__ __launch_bounds__(64) void select_budget_kernel(
    const float* __restrict__ scores, const int32_t* __restrict__ sizes, const int32_t* __restrict__ budgets,
    int32_t qn, int32_t kn, int32_t mode, uint8_t* __restrict__ out, int32_t* __restrict__ ids,
    int32_t* __restrict__ counts) {
  extern __shared__ __attribute__((aligned(16))) uint8_t keep[];
  const int64_t row = blockIdx.x;
  const int64_t bh = row / qn;
  const int32_t q = static_cast<int32_t>(row - bh * qn);
  const float* srow = scores + row * kn;
  const int32_t* sz = sizes + bh * kn;
  const int lane = threadIdx.x;
  const int32_t budget = budgets[row];
  for (int j = 4 * lane; j < kn; j += 256) *reinterpret_cast<uint32_t*>(keep + j) = 0u;
  uint64_t k[E];
#pragma unroll
  for (int r = 0; r < E; ++r) {
    const int pos = lane * E + r;
    k[r] = pos < kn ? rank_key(srow[pos], pos) : ~0ull;  // padding sorts last
  }
  wave_sort_keys<E>(k, lane);
  // costs in rank order; the exclusive prefix of the non-empty costs before this lane's ranks
  int32_t cost[E];
  long long tot = 0;
#pragma unroll
  for (int r = 0; r < E; ++r) {
    cost[r] = lane * E + r < kn ? sz[static_cast<uint32_t>(k[r])] : 0;
    tot += max(cost[r], 0);
  }
  long long incl = tot;
  for (int o = 1; o < 64; o <<= 1) {
    const long long up = __shfl_up(incl, o, 64);
    if (lane >= o) incl += up;
  }
  long long cum = incl - tot;
  long long sel = 0;
  int32_t cnt = 0, valid = 0, cross = 0x7FFFFFFF;
  __syncthreads();  // the cleared flags are stored before any is set
#pragma unroll
  for (int r = 0; r < E; ++r) {
    const int rank = lane * E + r;
    if (rank < kn && cost[r] > 0) {
      cum += cost[r];
      ++valid;
      if (cum <= budget) {
        keep[static_cast<uint32_t>(k[r])] = 1;
        sel += cost[r];
        ++cnt;
      } else {
        cross = min(cross, rank);
      }
    }
  }
  for (int o = 32; o > 0; o >>= 1) {
    sel += __shfl_xor(sel, o, 64);
    cnt += __shfl_xor(cnt, o, 64);
    valid += __shfl_xor(valid, o, 64);
    cross = min(cross, __shfl_xor(cross, o, 64));
  }
  // the one extra cluster, at rank `crossing` (mode 0) or `count` (mode 1), set by its lane
  int32_t extra = -1;
  if (mode == 0) {
    if (budget > 0 && sel < budget && cross != 0x7FFFFFFF) extra = cross;
  } else {
    if (budget > 0 && sel < budget && cnt < valid && cnt < kn) extra = cnt;
  }
  if (extra >= 0 && extra / E == lane) {
#pragma unroll
    for (int r = 0; r < E; ++r) {
      if (r == extra % E) keep[static_cast<uint32_t>(k[r])] = 1;
    }
  }
  __syncthreads();
  const int64_t stride = static_cast<int64_t>(kn) + 1;
  uint8_t* orow = out + (bh * (qn + 1) + q + 1) * stride;
  for (int j = lane; j <= kn; j += 64) orow[j] = (j == 0) ? 1 : keep[j - 1];
  if (q == 0) {
    uint8_t* head = out + bh * (qn + 1) * stride;
    for (int j = lane; j <= kn; j += 64) head[j] = (j == 0) ? 1 : 0;
  }
  if (ids != nullptr && counts != nullptr) {
    // ascending compaction of the kept flags
    int32_t* irow = ids + row * kn;
    int32_t base = 0;
    for (int c0 = 0; c0 < kn; c0 += 64) {
      const int c = c0 + lane;
      const bool kc = c < kn && keep[c];
      const uint64_t bits = __ballot(kc);
      const int pos = __popcll(bits & ((1ull << lane) - 1ull));
      if (kc) irow[base + pos] = c;
      base += __popcll(bits);
    }
    if (lane == 0) counts[row] = base;
  }
}

// One wave per row of a bool mask [rows, kn]: ascending kept ids + count.
__global__ __launch_bounds__(64) void compact_kernel(const uint8_t* __restrict__ mask, int64_t rows, int32_t kn,
                                                     int32_t* __restrict__ ids, int32_t* __restrict__ counts) {
  const int64_t row = blockIdx.x;
  if (row >= rows) return;
  const int lane = threadIdx.x;
  const uint8_t* m = mask + row * kn;
  int32_t* irow = ids + row * kn;
  int32_t base = 0;
  for (int c0 = 0; c0 < kn; c0 += 64) {
    const int c = c0 + lane;
    const bool k = c < kn && m[c] != 0;
    const uint64_t bits = __ballot(k);
    const int pos = __popcll(bits & ((1ull << lane) - 1ull));
    if (k) irow[base + pos] = c;
    base += __popcll(bits);
  }
  if (lane == 0) counts[row] = base;
}

// One workgroup per (cfg, head): kept pairs / all pairs, exact int64 sums.
__global__ __launch_bounds__(256) void density_kernel(const uint8_t* __restrict__ map,
                                                      const int32_t* __restrict__ q_sizes,
                                                      const int32_t* __restrict__ k_sizes, int32_t qn,
                                                      int32_t kn, float* __restrict__ out) {
  __shared__ long long red[3][4];
  extern __shared__ int32_t qk_sizes[];  // [qn] then [kn]
  const int64_t h = blockIdx.x;
  const int tid = threadIdx.x;
  const uint8_t* m = map + h * qn * static_cast<int64_t>(kn);
  const int32_t* qs = q_sizes + h * qn;
  const int32_t* ks = k_sizes + h * kn;
  int32_t* sq = qk_sizes;
  int32_t* sk = qk_sizes + qn;
  long long kept = 0, qsum = 0, ksum = 0;
  for (int i = tid; i < qn; i += blockDim.x) {
    sq[i] = qs[i];
    qsum += qs[i];
  }
  for (int j = tid; j < kn; j += blockDim.x) {
    sk[j] = ks[j];
    ksum += ks[j];
  }
  __syncthreads();
  // sum over (i, j) of map[i][j] ? qs[i] * ks[j] : 0, walked as 16-byte vectors of the
  // map when rows are whole vectors (every load independent), else byte by byte
  if ((kn & 15) == 0 && (reinterpret_cast<uintptr_t>(m) & 15) == 0) {
    const int vpr = kn >> 4;
    const int total = qn * vpr;
    const uint4* mv = reinterpret_cast<const uint4*>(m);
    for (int v = tid; v < total; v += blockDim.x) {
      const int i = v / vpr;
      const int j0 = (v - i * vpr) << 4;
      const uint4 w = mv[v];
      const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
      long long rs = 0;
#pragma unroll
      for (int b = 0; b < 16; ++b) rs += ((ws[b >> 2] >> (8 * (b & 3))) & 0xFFu) ? sk[j0 + b] : 0;
      kept += rs * sq[i];
    }
  } else {
    for (int e = tid; e < qn * kn; e += blockDim.x) {
      const int i = e / kn;
      const int j = e - i * kn;
      kept += m[e] ? static_cast<long long>(sk[j]) * sq[i] : 0;
    }
  }
  for (int o = 32; o > 0; o >>= 1) {
    kept += __shfl_xor(kept, o, 64);
    qsum += __shfl_xor(qsum, o, 64);
    ksum += __shfl_xor(ksum, o, 64);
  }
  if ((tid & 63) == 0) {
    red[0][tid >> 6] = kept;
    red[1][tid >> 6] = qsum;
    red[2][tid >> 6] = ksum;
  }
  __syncthreads();
  if (tid == 0) {
    long long a = 0, b = 0, c = 0;
    for (int w = 0; w < static_cast<int>(blockDim.x) / 64; ++w) {
      a += red[0][w];
      b += red[1][w];
      c += red[2][w];
    }
    const double all = static_cast<double>(b) * static_cast<double>(c);
    out[h] = all > 0.0 ? static_cast<float>(static_cast<double>(a) / all) : 0.0f;
  }
}

}  // namespace

// map uint8 [bh, qn, kn] from centroids qc [bh, qn, d], kc [bh, kn, d] (fp32
// values; bf16 centroids are passed widened to fp32 with score_bf16 = 1) and
// int32 key-cluster sizes [bh, kn].  sqrt_d is the divisor (float(sqrt(d))).
extern "C" int spr_topp_map(const float* qc, const float* kc, const int32_t* k_sizes, int64_t bh, int32_t qn,
                            int32_t kn, int32_t d, float sqrt_d, float p, int32_t preserve, int32_t score_bf16,
                            uint8_t* map, int32_t* budgets, hipStream_t stream) {
  SPR_REQUIRE(bh >= 0 && qn >= 0 && kn >= 1, "spr_topp_map: bad size");
  SPR_REQUIRE(kn <= MAX_KC, "spr_topp_map: %d key clusters exceed %d", kn, MAX_KC);
  SPR_REQUIRE(d >= 1 && d <= 512, "spr_topp_map: head dim %d outside [1, 512]", d);
  if (bh == 0 || qn == 0) return SPR_OK;
  SPR_REQUIRE(qc && kc && k_sizes && (map || budgets), "spr_topp_map: null pointer");
  int n2 = 1;
  while (n2 < kn) n2 <<= 1;
  const size_t lds = static_cast<size_t>(n2) * 8;  // at most 32 KB (kn <= 4096)
  by_sort_width(n2, [&](auto e) {
    topp_map_kernel<decltype(e)::value><<<dim3(static_cast<uint32_t>(bh * qn)), SEL_THREADS, lds, stream>>>(
        qc, kc, k_sizes, qn, kn, d, sqrt_d, p, preserve, score_bf16, map, budgets);
  });
  SPR_LAUNCHED("topp_map_kernel");
  return SPR_OK;
}

// out uint8 [bh, qn + 1, kn + 1] (header row/column as the reference);
// ids int32 [bh, qn, kn] and counts int32 [bh, qn] optional (both or neither).
extern "C" int spr_select_budget(const float* scores, const int32_t* sizes, const int32_t* budgets, int64_t bh,
                                 int32_t qn, int32_t kn, int32_t mode, uint8_t* out, int32_t* ids,
                                 int32_t* counts, hipStream_t stream) {
  SPR_REQUIRE(bh >= 0 && qn >= 0 && kn >= 1, "spr_select_budget: bad size");
  SPR_REQUIRE(kn <= MAX_KC, "spr_select_budget: %d key clusters exceed %d", kn, MAX_KC);
  SPR_REQUIRE(mode == 0 || mode == 1, "spr_select_budget: mode must be 0 or 1");
  SPR_REQUIRE((ids == nullptr) == (counts == nullptr), "spr_select_budget: ids and counts go together");
  if (bh == 0) return SPR_OK;
  SPR_REQUIRE(scores && sizes && budgets && out, "spr_select_budget: null pointer");
  if (qn == 0) return SPR_OK;
  int n2 = 1;
  while (n2 < kn) n2 <<= 1;
  const size_t lds = (static_cast<size_t>(kn) + 15) & ~size_t(15);  // the kept flags
  by_sort_width(n2, [&](auto e) {
    select_budget_kernel<decltype(e)::value><<<dim3(static_cast<uint32_t>(bh * qn)), 64, lds, stream>>>(
        scores, sizes, budgets, qn, kn, mode, out, ids, counts);
  });
  SPR_LAUNCHED("select_budget_kernel");
  return SPR_OK;
}

extern "C" int spr_compact_selected(const uint8_t* mask, int64_t rows, int32_t kn, int32_t* ids, int32_t* counts,
                                    hipStream_t stream) {
  SPR_REQUIRE(rows >= 0 && kn >= 1, "spr_compact_selected: bad size");
  if (rows == 0) return SPR_OK;
  SPR_REQUIRE(mask && ids && counts, "spr_compact_selected: null pointer");
  SPR_REQUIRE(rows < (int64_t(1) << 31), "spr_compact_selected: too many rows");
  compact_kernel<<<dim3(static_cast<uint32_t>(rows)), 64, 0, stream>>>(mask, rows, kn, ids, counts);
  SPR_LAUNCHED("compact_kernel");
  return SPR_OK;
}

// density[h] = sum_ij map[h,i,j] qs[h,i] ks[h,j] / (sum qs[h] * sum ks[h]) for h < heads.
extern "C" int spr_density(const uint8_t* map, const int32_t* q_sizes, const int32_t* k_sizes, int64_t heads,
                           int32_t qn, int32_t kn, float* out, hipStream_t stream) {
  SPR_REQUIRE(heads >= 0 && qn >= 1 && kn >= 1, "spr_density: bad size");
  if (heads == 0) return SPR_OK;
  SPR_REQUIRE(map && q_sizes && k_sizes && out, "spr_density: null pointer");
  SPR_REQUIRE(static_cast<int64_t>(qn) * kn < (int64_t(1) << 31) && qn + kn <= 16384, "spr_density: map too large");
  density_kernel<<<dim3(static_cast<uint32_t>(heads)), 256, (qn + kn) * sizeof(int32_t), stream>>>(map, q_sizes, k_sizes,
                                                                                                   qn, kn, out);
  SPR_LAUNCHED("density_kernel");
  return SPR_OK;
}
