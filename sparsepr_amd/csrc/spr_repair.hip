// Probe-fitted reduced-rank residual repair: probe selection, fit preparation,
// low-rank apply, exact-probe scatter.
//
// Replaces:
//   select_role_equal_probes(_vectorized), select_first_token_largest_groups
//       (src/sparsepr/models/cosmos3/residual_repair.py:36-260)
//   n8_prepare_output_repair_fit_triton    (kernels/triton/residual_repair.py:798-857, kernel :330-363)
//   n8_prepare_repair_fit_triton           (kernels/triton/residual_repair.py:737-797, kernel :285-327)
//   n8_repair_apply_output_triton          (kernels/triton/residual_repair.py:478-562, kernel :95-155)
//   n8_repair_apply_triton                 (kernels/triton/residual_repair.py:388-475, kernel :10-92)
//   n8_exact_probe_scatter_triton          (kernels/triton/residual_repair.py:656-700, kernel :257-282)
//
// Probe selection runs in two launches.  (1) distance: each token's squared
// distance to its cluster center in fp32 with separate multiply and add, summed
// sequentially within each group of 8 consecutive dims and then by a balanced
// pairwise tree over the groups (a fixed order, so exact ties are reproducible).
// (2) select, one workgroup per head: groups ordered by size (descending,
// stable); in round r every group offers its r-th nearest token (ties by lower
// token id) via an LDS atomicMin over 64-bit (distance bits, token) keys.
#pragma clang fp contract(off)

#include <algorithm>

#include "spr_common.h"
#include <type_traits>

namespace {

using spr::u32x4;

// x[l] + x[l ^ 32] (v_permlane32_swap returns both halves; + is symmetric in them).
__device__ __forceinline__ float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

constexpr int MAX_GROUPS = 2048;

template <typename T>
__device__ __forceinline__ float load_elem(const T* p, int64_t i) {
  if constexpr (sizeof(T) == 2) {
    return spr::bf16_to_f32(p[i]);
  } else {
    return p[i];
  }
}

// Eight consecutive feature values as fp32 (bf16: one 16-byte load; fp32: two).
template <typename T>
struct Feat8 {
  u32x4 w[sizeof(T) == 2 ? 1 : 2];
};

template <typename T>
__device__ __forceinline__ Feat8<T> load_feat8(const T* __restrict__ p) {
  Feat8<T> r;
  const u32x4* q = reinterpret_cast<const u32x4*>(p);
  r.w[0] = q[0];
  if constexpr (sizeof(T) == 4) r.w[1] = q[1];
  return r;
}

// The sequential fp32 sum over the eight dims of (f - c)^2, each term rounded (sub,
// mul, add; no contraction).
template <typename T>
__device__ __forceinline__ float part8(const Feat8<T>& x, spr::f32x4 c0, spr::f32x4 c1) {
  const float cv[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
  float fv[8];
  if constexpr (sizeof(T) == 2) {
    const uint32_t ws[4] = {x.w[0].x, x.w[0].y, x.w[0].z, x.w[0].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      fv[2 * e] = spr::bf16_lo(ws[e]);
      fv[2 * e + 1] = spr::bf16_hi(ws[e]);
    }
  } else {
    const uint32_t ws[8] = {x.w[0].x, x.w[0].y, x.w[0].z, x.w[0].w, x.w[1].x, x.w[1].y, x.w[1].z, x.w[1].w};
#pragma unroll
    for (int e = 0; e < 8; ++e) fv[e] = __uint_as_float(ws[e]);
  }
  float acc = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    // plain operators: the file-level contract(off) keeps mul and add apart
    const float diff = fv[e] - cv[e];
    const float sq = diff * diff;
    acc = acc + sq;
  }
  return acc;
}

// dist[bh, t] = sum_d (f[t, d] - center[label[t], d])^2 in fp32, each term rounded
// (sub, mul, add; no contraction): sequential within each group of 8 consecutive
// dims, then a balanced pairwise tree over the groups in index order (the
// reference's torch .sum() fixes no order; this is the canonical one).
template <typename T, int R>
__global__ __launch_bounds__(256) void probe_distance_kernel(const T* __restrict__ f,
                                                             const int32_t* __restrict__ labels,
                                                             const float* __restrict__ centers, int64_t n,
                                                             int32_t groups, float* __restrict__ dist) {
  // R / 8 lanes share a row (coalesced 16- or 32-byte loads); lane k sums dims
  // 8k .. 8k + 7 sequentially, then a butterfly over the row's lanes adds the
  // partials as a balanced pairwise tree in index order (x + y == y + x, so both
  // lanes of every pair hold the same sum).  A wave covers 64 rows in steps of
  // 64 / L rows; it loads its 64 labels once (one per lane) and issues the feature
  // and center loads of U steps before using any of them.  Rows past n load row
  // n - 1 and store nothing; an out-of-range label loads center 0 and uses zeros.
  constexpr int L = R / 8;
  constexpr int RPS = 64 / L;   // rows per wave step
  constexpr int STEPS = 64 / RPS;
  constexpr int U = STEPS < 8 ? STEPS : 8;
  const int64_t bh = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int k = lane % L;
  const int64_t base = static_cast<int64_t>(blockIdx.x) * 256 + (threadIdx.x >> 6) * 64;
  if (base >= n) return;
  const int32_t my_lab = labels[bh * n + std::min<int64_t>(base + lane, n - 1)];
  const spr::f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s0 = 0; s0 < STEPS; s0 += U) {
    Feat8<T> fx[U];
    spr::f32x4 c0[U], c1[U];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t t = std::min<int64_t>(base + (s0 + u) * RPS + lane / L, n - 1);
      fx[u] = load_feat8(f + (bh * n + t) * R + 8 * k);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the feature loads ahead of the label wait
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int32_t lab = __shfl(my_lab, (s0 + u) * RPS + lane / L, 64);
      ok[u] = lab >= 0 && lab < groups;
      const spr::f32x4* crow =
          reinterpret_cast<const spr::f32x4*>(centers + (bh * groups + (ok[u] ? lab : 0)) * R + 8 * k);
      c0[u] = crow[0];
      c1[u] = crow[1];
    }
    float acc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) acc[u] = part8(fx[u], ok[u] ? c0[u] : zero, ok[u] ? c1[u] : zero);
#pragma unroll
    for (int o = 1; o < L; o <<= 1) {
#pragma unroll
      for (int u = 0; u < U; ++u) acc[u] = acc[u] + __shfl_xor(acc[u], o, 64);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t t = base + (s0 + u) * RPS + lane / L;
      if (t < n && k == 0) dist[bh * n + t] = acc[u];
    }
  }
}

// The same distances with the head's centers staged in LDS (groups * R * 4 bytes, at
// most PD_LDS_BYTES).  Read from memory, the centers cost the vector-memory path twice
// the feature bytes; from LDS they cost nothing there.  A 512-thread workgroup stages
// one head's centers once and then walks a slice of that head's rows in 64-row tiles,
// one tile per wave at a time, with the next tile's labels loaded during the current
// one.  Within a center row the 16-byte pieces are stored as [half][lane] (piece 2k + h
// at h * L + k), so the R / 8 lanes of a row read consecutive pieces (no bank
// conflicts).  Results are identical to probe_distance_kernel's (same arithmetic).
constexpr int PD_LDS_BYTES = 65536;
constexpr int PD_LDS_THREADS = 512;

template <typename T, int R>
// four waves per SIMD: two workgroups per CU (at most 128 VGPRs)
__global__ __launch_bounds__(PD_LDS_THREADS) __attribute__((amdgpu_waves_per_eu(4))) void probe_distance_lds_kernel(
    const T* __restrict__ f, const int32_t* __restrict__ labels, const float* __restrict__ centers, int64_t n,
    int32_t groups, int64_t rows_per_block, float* __restrict__ dist) {
  extern __shared__ __align__(16) spr::f32x4 pd_cs[];
  constexpr int L = R / 8;
  constexpr int RPS = 64 / L;
  constexpr int STEPS = 64 / RPS;
  constexpr int U = STEPS < 4 ? STEPS : 4;  // more would spill at 128 VGPRs
  constexpr int WAVES = PD_LDS_THREADS / 64;
  const int64_t bh = blockIdx.y;
  {
    const spr::f32x4* src = reinterpret_cast<const spr::f32x4*>(centers + bh * groups * R);
    for (int i = threadIdx.x; i < groups * (R / 4); i += PD_LDS_THREADS) {
      const int g = i / (R / 4), j = i % (R / 4);  // piece j = 2k + h of center g
      pd_cs[g * (R / 4) + (j & 1) * L + (j >> 1)] = src[i];
    }
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int k = lane % L;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * rows_per_block;
  const int64_t r1 = std::min<int64_t>(n, r0 + rows_per_block);
  const int32_t* lab_h = labels + bh * n;
  const spr::f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  int64_t base = r0 + (threadIdx.x >> 6) * 64;
  int32_t my_lab = base < r1 ? lab_h[std::min<int64_t>(base + lane, r1 - 1)] : 0;
  for (; base < r1; base += WAVES * 64) {
    const int64_t next = base + WAVES * 64;
#pragma unroll
    for (int s0 = 0; s0 < STEPS; s0 += U) {
      Feat8<T> fx[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t t = std::min<int64_t>(base + (s0 + u) * RPS + lane / L, r1 - 1);
        fx[u] = load_feat8(f + (bh * n + t) * R + 8 * k);
      }
      int32_t next_lab = 0;
      if (s0 + U >= STEPS && next < r1) next_lab = lab_h[std::min<int64_t>(next + lane, r1 - 1)];
      __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of the first use
      float acc[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int32_t lab = __shfl(my_lab, (s0 + u) * RPS + lane / L, 64);
        const bool ok = lab >= 0 && lab < groups;
        const spr::f32x4* crow = pd_cs + (ok ? lab : 0) * (R / 4) + k;
        acc[u] = part8(fx[u], ok ? crow[0] : zero, ok ? crow[L] : zero);
      }
#pragma unroll
      for (int o = 1; o < L; o <<= 1) {
#pragma unroll
        for (int u = 0; u < U; ++u) acc[u] = acc[u] + __shfl_xor(acc[u], o, 64);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t t = base + (s0 + u) * RPS + lane / L;
        if (t < r1 && k == 0) dist[bh * n + t] = acc[u];
      }
      if (s0 + U >= STEPS) my_lab = next_lab;
    }
  }
}

// First pass of probe selection for modes 0 and 2, split over many workgroups per head:
// each workgroup reduces its slice of tokens to the smallest (distance bits, token) key
// per group in LDS, then merges those keys into the head's keys in `best` with 64-bit
// global atomicMin.  The minimum over all tokens does not depend on the order.
constexpr int PROBE_SLICE = 2048;  // tokens per workgroup

__global__ void probe_best_init_kernel(unsigned long long* __restrict__ best, int64_t total) {
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x)
    best[e] = ~0ull;
}

__global__ __launch_bounds__(256) void probe_best_kernel(const float* __restrict__ dist,
                                                         const int32_t* __restrict__ labels, int64_t n,
                                                         int32_t groups, int32_t mode,
                                                         unsigned long long* __restrict__ best) {
  __shared__ unsigned long long lb[MAX_GROUPS];
  const int64_t bh = blockIdx.y;
  for (int c = threadIdx.x; c < groups; c += blockDim.x) lb[c] = ~0ull;
  __syncthreads();
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * PROBE_SLICE;
  const int64_t t1 = min(n, t0 + PROBE_SLICE);
  const int32_t* lab = labels + bh * n;
  const float* dd = dist + bh * n;
  for (int64_t t = t0 + threadIdx.x; t < t1; t += blockDim.x) {
    const int32_t c = lab[t];
    if (c < 0 || c >= groups) continue;
    const float dv = (mode == 2) ? 0.0f : dd[t];
    atomicMin(&lb[c], (static_cast<unsigned long long>(__float_as_uint(dv)) << 32) | static_cast<uint32_t>(t));
  }
  __syncthreads();
  for (int c = threadIdx.x; c < groups; c += blockDim.x) {
    if (lb[c] != ~0ull) atomicMin(&best[bh * groups + c], lb[c]);
  }
}

// mode 0: vectorized role-equal (one representative per group, first `count`
//         groups in size order; empty-group slots fall back to token j);
// mode 1: representative rounds until `count` probes (an exhausted group offers
//         its lowest token again, as the reference does);
// mode 2: first token of each of the largest groups, weight = group size.
__global__ __launch_bounds__(256) void probe_select_kernel(const float* __restrict__ dist,
                                                           const int32_t* __restrict__ labels,
                                                           const int32_t* __restrict__ sizes, int64_t n,
                                                           int32_t groups, int32_t count, int32_t mode,
                                                           int32_t* __restrict__ rows, float* __restrict__ weights,
                                                           int32_t* __restrict__ status,
                                                           const unsigned long long* __restrict__ gbest) {
  __shared__ int32_t sz[MAX_GROUPS];
  __shared__ int32_t order[MAX_GROUPS];
  __shared__ unsigned long long best[MAX_GROUPS];
  __shared__ unsigned long long prev[MAX_GROUPS];
  __shared__ int32_t sampled[MAX_GROUPS];
  __shared__ int32_t first_tok[MAX_GROUPS];
  __shared__ int32_t chosen_count;
  __shared__ double wsum;
  const int64_t bh = blockIdx.x;
  const int32_t* lab = labels + bh * n;
  const float* dd = dist + bh * n;
  int32_t* out_rows = rows + bh * count;
  float* out_w = weights + bh * count;

  for (int c = threadIdx.x; c < groups; c += blockDim.x) {
    sz[c] = sizes[bh * groups + c];
    prev[c] = 0ull;
    sampled[c] = 0;
  }
  if (threadIdx.x == 0) chosen_count = 0;
  __syncthreads();
  // stable descending order of group sizes
  for (int c = threadIdx.x; c < groups; c += blockDim.x) {
    const int32_t s = sz[c];
    int rank = 0;
    for (int o = 0; o < groups; ++o) {
      const int32_t so = sz[o];
      rank += (so > s || (so == s && o < c)) ? 1 : 0;
    }
    order[rank] = c;
  }
  __syncthreads();

  // Round r: every non-empty group offers its r-th smallest (distance, token)
  // key.  A group whose members are all taken offers its lowest token id again,
  // as the reference's all-infinite remaining distances do (residual_repair.py:70-98).
  const unsigned long long none = ~0ull;
  for (int c = threadIdx.x; c < groups; c += blockDim.x) first_tok[c] = 0x7fffffff;
  for (int round = 0; round <= count; ++round) {
    if (gbest != nullptr) {  // modes 0 and 2: the keys of the split first pass
      for (int c = threadIdx.x; c < groups; c += blockDim.x) best[c] = gbest[bh * groups + c];
    } else {
      for (int c = threadIdx.x; c < groups; c += blockDim.x) best[c] = none;
      __syncthreads();
      for (int64_t t = threadIdx.x; t < n; t += blockDim.x) {
        const int32_t c = lab[t];
        if (c < 0 || c >= groups) continue;
        const float dv = (mode == 2) ? 0.0f : dd[t];
        const unsigned long long key =
            (static_cast<unsigned long long>(__float_as_uint(dv)) << 32) | static_cast<uint32_t>(t);
        if (round == 0) {
          atomicMin(&best[c], key);
          atomicMin(&first_tok[c], static_cast<int32_t>(t));
        } else if (key > prev[c]) {
          atomicMin(&best[c], key);
        }
      }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      int32_t have = chosen_count;
      for (int j = 0; j < groups && have < count; ++j) {
        const int32_t c = order[j];
        const unsigned long long key = best[c];
        if (sz[c] <= 0) {
          if (mode != 1) {
            out_rows[have] = have;  // empty group: fallback token id = slot
            ++have;
          }
        } else if (key != none) {
          out_rows[have++] = static_cast<int32_t>(key & 0xffffffffull);
        } else {
          out_rows[have++] = first_tok[c];  // exhausted group
        }
      }
      chosen_count = have;
    }
    for (int c = threadIdx.x; c < groups; c += blockDim.x) {
      if (best[c] != none) prev[c] = best[c];
    }
    __syncthreads();
    if (mode != 1 || chosen_count >= count || chosen_count == 0) break;
  }
  if (threadIdx.x == 0 && status != nullptr) status[bh] = chosen_count;
  __syncthreads();

  // weights: group size / probes sampled from the group, normalised to mean 1
  const int32_t have = chosen_count;
  for (int j = threadIdx.x; j < have; j += blockDim.x) {
    const int32_t t = out_rows[j];
    const int32_t c = (t >= 0 && t < n) ? lab[t] : -1;
    if (c >= 0 && c < groups) atomicAdd(&sampled[c], 1);
  }
  __syncthreads();
  for (int j = threadIdx.x; j < have; j += blockDim.x) {
    const int32_t t = out_rows[j];
    const int32_t c = (t >= 0 && t < n) ? lab[t] : -1;
    float w = 0.0f;
    if (c >= 0 && c < groups) {
      const float size = static_cast<float>(sz[c]);
      w = (mode == 2) ? size : __fdiv_rn(size, static_cast<float>(max(sampled[c], 1)));
    }
    out_w[j] = w;
  }
  __syncthreads();
  if (threadIdx.x == 0) {  // the mean in a fixed (sequential) order
    double s = 0.0;
    for (int j = 0; j < have; ++j) s += static_cast<double>(out_w[j]);
    wsum = have > 0 ? s / static_cast<double>(have) : 0.0;
  }
  __syncthreads();
  const float mean = fmaxf(static_cast<float>(wsum), 1e-20f);
  for (int j = threadIdx.x; j < have; j += blockDim.x) out_w[j] = __fdiv_rn(out_w[j], mean);
}

// x_fit = float(base[rows]) (then, with role, float(role[rows]) in columns d .. d + rr of
// rows of d + rr), dense_f = float(dense), y_fit = dense_f - float(base[rows]).
template <typename TB, typename TD>
__global__ void fit_prep_kernel(const TB* __restrict__ base, const TD* __restrict__ dense,
                                const float* __restrict__ role, int32_t rr, const int32_t* __restrict__ rows,
                                int64_t n, int32_t m, int32_t d, float* __restrict__ x_fit,
                                float* __restrict__ dense_f, float* __restrict__ y_fit) {
  const int64_t bh = blockIdx.y;
  const int64_t xp = d + rr;  // x_fit row length
  for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < m * (d + rr); e += gridDim.x * blockDim.x) {
    const int j = e / (d + rr);
    const int c = e - j * (d + rr);
    const int32_t r = rows[bh * m + j];
    const bool ok = r >= 0 && r < n;
    if (c >= d) {
      x_fit[(bh * m + j) * xp + c] = ok ? role[(bh * n + r) * rr + (c - d)] : 0.0f;
      continue;
    }
    const float b = ok ? load_elem(base, (bh * n + r) * d + c) : 0.0f;
    const float y = load_elem(dense, (bh * m + j) * static_cast<int64_t>(d) + c);
    const int64_t o = (bh * m + j) * static_cast<int64_t>(d) + c;
    x_fit[(bh * m + j) * xp + c] = b;
    dense_f[o] = y;
    y_fit[o] = __fsub_rn(y, b);
  }
}

// out = base + alpha * (((base - mu) / sigma) L B^T + mu_y), optional norm cap; with RR
// role features the standardised role row joins the features (L has D + RR rows) and the
// cap stays on the base norm.  One lane per token row (64 rows per wave); L and B are read
// from LDS as wave-uniform broadcasts.  Loops over the head dim are fully unrolled so the
// row stays in registers.
template <int D, int RK, int RR>
__global__ __launch_bounds__(256) void repair_apply_kernel(const uint16_t* __restrict__ base,
                                                           const float* __restrict__ role,
                                                           const float* __restrict__ x_mean,
                                                           const float* __restrict__ x_scale,
                                                           const float* __restrict__ y_mean,
                                                           const float* __restrict__ left,
                                                           const float* __restrict__ basis, int64_t n, float alpha,
                                                           float norm_cap, uint16_t* __restrict__ out) {
  constexpr int P = D + RR;
  __shared__ __attribute__((aligned(16))) float Ls[P][RK];
  __shared__ __attribute__((aligned(16))) float Bs[D][RK];
  __shared__ float mu[P], inv_sd[P], my[D];
  const int64_t bh = blockIdx.y;
  for (int e = threadIdx.x; e < P * RK; e += blockDim.x) Ls[e / RK][e % RK] = left[bh * P * RK + e];
  for (int e = threadIdx.x; e < D * RK; e += blockDim.x) Bs[e / RK][e % RK] = basis[bh * D * RK + e];
  for (int e = threadIdx.x; e < P; e += blockDim.x) {
    mu[e] = x_mean[bh * P + e];
    inv_sd[e] = 1.0f / x_scale[bh * P + e];
  }
  for (int e = threadIdx.x; e < D; e += blockDim.x) my[e] = y_mean[bh * D + e];
  __syncthreads();
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= n) return;
  const u32x4* brow = reinterpret_cast<const u32x4*>(base + (bh * n + t) * D);
  // Up to rank 32 the row stays in registers; at rank 64 the coordinates take them, and each
  // pass over the row reads it again (from the cache)
  constexpr bool HOLD = RK <= 32;
  uint32_t packed[HOLD ? D / 2 : 1];
  if constexpr (HOLD) {
#pragma unroll
    for (int i = 0; i < D / 8; ++i) {
      const u32x4 w = brow[i];
      packed[4 * i] = w.x;
      packed[4 * i + 1] = w.y;
      packed[4 * i + 2] = w.z;
      packed[4 * i + 3] = w.w;
    }
  }
  auto piece = [&](int i) -> u32x4 {  // dims 8 i .. 8 i + 7 as bf16 pairs
    if constexpr (HOLD) {
      return u32x4{packed[4 * i], packed[4 * i + 1], packed[4 * i + 2], packed[4 * i + 3]};
    } else {
      return brow[i];
    }
  };
  float coords[RK];
#pragma unroll
  for (int r = 0; r < RK; ++r) coords[r] = 0.0f;
  float bn = 0.0f;
#pragma unroll
  for (int i = 0; i < D / 8; ++i) {
    const u32x4 w = piece(i);
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int h = 0; h < 4; ++h) {
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int dd = 8 * i + 2 * h + e;
        const float b = e ? spr::bf16_hi(ws[h]) : spr::bf16_lo(ws[h]);
        bn = __builtin_fmaf(b, b, bn);
        const float z = (b - mu[dd]) * inv_sd[dd];
#pragma unroll
        for (int r = 0; r < RK; ++r) coords[r] = __builtin_fmaf(z, Ls[dd][r], coords[r]);
      }
    }
  }
  if constexpr (RR > 0) {
    const float* rrow = role + (bh * n + t) * RR;
#pragma unroll
    for (int c = 0; c < RR; ++c) {
      const float z = (rrow[c] - mu[D + c]) * inv_sd[D + c];
#pragma unroll
      for (int r = 0; r < RK; ++r) coords[r] = __builtin_fmaf(z, Ls[D + c][r], coords[r]);
    }
  }
  float scale = alpha;
  if (norm_cap > 0.0f) {
    float cn = 0.0f;
#pragma unroll
    for (int dd = 0; dd < D; ++dd) {
      float corr = my[dd];
#pragma unroll
      for (int r = 0; r < RK; ++r) corr = __builtin_fmaf(coords[r], Bs[dd][r], corr);
      cn = __builtin_fmaf(corr, corr, cn);
    }
    scale = alpha * fminf(1.0f, norm_cap * sqrtf(bn) / fmaxf(sqrtf(cn), 1e-20f));
  }
  u32x4* orow = reinterpret_cast<u32x4*>(out + (bh * n + t) * D);
#pragma unroll
  for (int i = 0; i < D / 8; ++i) {
    const u32x4 w = piece(i);
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    uint32_t o[4];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      float res[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int dd = 8 * i + 2 * h + e;
        const float b = e ? spr::bf16_hi(ws[h]) : spr::bf16_lo(ws[h]);
        float corr = my[dd];
#pragma unroll
        for (int r = 0; r < RK; ++r) corr = __builtin_fmaf(coords[r], Bs[dd][r], corr);
        res[e] = __builtin_fmaf(scale, corr, b);
      }
      o[h] = spr::pack_bf16x2(res[0], res[1]);
    }
    orow[i] = u32x4{o[0], o[1], o[2], o[3]};
  }
}

// out[bh, rows[j]] = dense[bh, j] cast to the output dtype (bf16 out, fp32 or bf16 in).
// x = hi + lo with hi = bf16(x), lo = bf16(x - hi): eight fp32 values as two
// packed bf16 fragments (about 16 mantissa bits between them).
__device__ __forceinline__ void split_bf16x8(const float (&v)[8], u32x4& hi, u32x4& lo) {
  uint32_t h[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    h[i] = spr::pack_bf16x2_rne(v[2 * i], v[2 * i + 1]);
    l[i] = spr::pack_bf16x2_rne(v[2 * i] - spr::bf16_lo(h[i]), v[2 * i + 1] - spr::bf16_hi(h[i]));
  }
  hi = u32x4{h[0], h[1], h[2], h[3]};
  lo = u32x4{l[0], l[1], l[2], l[3]};
}

// Rank-16 correction on v_mfma_f32_32x32x16_bf16, D = 128: one wave per 32 rows.
// fp32 operands enter as bf16 hi + lo pairs and each product is
// hi*hi + lo*hi + hi*lo (about 16 mantissa bits; the reference's tl.dot runs in
// TF32 by default).
//   coords^T[rank, row] = L^T z^T: A = L^T (32 ranks, 16..31 zero) x 16 dims; B =
//     z^T, where lane (row l % 32, k-half h) holds dims 16s + 8h .. + 7 of its
//     row.  The accumulator gives that lane ranks 8i + 4h + j (i = 0, 1;
//     registers 0..7).
//   corr^T[dim, row] = B coords^T with the rank (k) index of this product in the
//     order rho(h, m) = 8(m / 4) + 4h + m % 4, so registers 0..7 of the coords
//     accumulator are the B operand as they stand; A = basis in the same rank
//     order.  Row a of N-tile nt is dim 32 nt + pi(a), pi swapping bits 2 and 3
//     of a, so lane (row, h) receives exactly the 64 dims it read: register
//     8q + e of tile nt is dim 16(2 nt + q) + 8h + e, and out = b + scale corr
//     needs no exchange.
// Rows stream through LDS: every wave DMAs its own 32-row batches (1 KB, four
// rows, per instruction; buffer range checks return zeros past the end) into a
// private double buffer one batch ahead, so only vmcnt waits order them.  The
// 16-byte pieces of row r sit at slot j ^ (r & 15): the fragment reads of 16
// consecutive rows hit all 64 banks.  Each workgroup (8 waves, one per CU)
// stages the head's factors once and walks 256-row batches.
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, uint8_t* lds, int32_t voff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, 0);
#endif
}

// The A fragment of rank row col of a stored [16][2] block: zeros for col >= 16 (read
// from row col % 16, then selected away, so the load is not divergent).
__device__ __forceinline__ u32x4 lfrag_at(const u32x4 (&blk)[16][2], int col, int part) {
  const u32x4 v = blk[col & 15][part];
  const bool live = col < 16;
  return u32x4{live ? v.x : 0u, live ? v.y : 0u, live ? v.z : 0u, live ? v.w : 0u};
}

// s_waitcnt vmcnt(N) for a compile-time N
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// With RR role features (fp32 [n][RR] per head), each row's standardised role values join
// the coordinates as RR / 16 more k-steps: lane (row, h) loads dims 16s + 8h .. + 7 of its
// role row with two 16-byte loads per step at the top of the batch, before the next batch's
// DMA, so they land while the batch waits and runs its base steps; the explicit waits count
// those loads.  L then has D + RR rows, the statistics D + RR entries.
template <bool CAP, int RR>
__global__ __launch_bounds__(512) void repair_apply_mfma_kernel(const uint16_t* __restrict__ base,
                                                                const float* __restrict__ role,
                                                                const float* __restrict__ x_mean,
                                                                const float* __restrict__ x_scale,
                                                                const float* __restrict__ y_mean,
                                                                const float* __restrict__ left,
                                                                const float* __restrict__ basis, int64_t n,
                                                                float alpha, float norm_cap,
                                                                uint16_t* __restrict__ out) {
  constexpr int D = 128;
  constexpr int RK = 16;
  constexpr int P = D + RR;          // features
  constexpr int RS = RR / 16;        // role k-steps
  constexpr int NR = 2 * RS;         // role loads per lane and batch
  constexpr int ROWB = D * 2;        // bytes per row
  constexpr int TILE = 32 * ROWB;    // one wave's batch
  // [k-step s][k-half h][rank] (hi, lo): L[16s + 8h + e][rank]; the A operand's ranks 16 .. 31
  // are zero and are not stored (lanes with col >= 16 select zeros)
  __shared__ u32x4 lfrag[8 + RS][2][RK][2];
  __shared__ u32x4 bfrag[4][32][2][2];   // [N-tile][row a][k-half h] (hi, lo): basis[32 nt + pi(a)][rho(h, m)]
  __shared__ __attribute__((aligned(16))) float mu[P], inv_sd[P], my[D];
  __shared__ __attribute__((aligned(1024))) uint8_t rows_lds[8][2][TILE];  // [wave][buffer]
  auto lds8 = [](const float* p, float (&x)[8]) {  // 8 consecutive floats, 32-byte aligned
    const spr::f32x4 a = reinterpret_cast<const spr::f32x4*>(p)[0];
    const spr::f32x4 b = reinterpret_cast<const spr::f32x4*>(p)[1];
    x[0] = a[0]; x[1] = a[1]; x[2] = a[2]; x[3] = a[3];
    x[4] = b[0]; x[5] = b[1]; x[6] = b[2]; x[7] = b[3];
  };
  const int64_t bh = blockIdx.y;
  const float* lm = left + bh * P * RK;
  const float* bm = basis + bh * D * RK;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int col = lane & 31;
  const int h = lane >> 5;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  const __amdgpu_buffer_rsrc_t rsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base + bh * n * D), 0, static_cast<int32_t>(n * ROWB),
                                        0x00020000);
  // batch starting at wave row w0 into buffer tile: instruction i moves rows 4i .. 4i + 3
  auto dma = [&](int64_t w0, uint8_t* tile) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = 4 * i + (lane >> 4);
      const int64_t row = w0 + r;
      const int32_t off = row < n ? static_cast<int32_t>(row * ROWB) + (((lane & 15) ^ (r & 15)) << 4)
                                  : static_cast<int32_t>(n * ROWB);  // past the range: reads zeros
      lds_dma16(rsrc, tile + i * 1024, off);
    }
  };
  int64_t w0 = static_cast<int64_t>(blockIdx.x) * 256 + wave * 32;
  if (w0 < n) dma(w0, rows_lds[wave][0]);

  for (int f = tid; f < (8 + RS) * 2 * RK; f += blockDim.x) {
    const int st = f / (2 * RK), hh = (f / RK) % 2, rk = f % RK;
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = rk < RK ? lm[(16 * st + 8 * hh + e) * RK + rk] : 0.0f;
    split_bf16x8(v, lfrag[st][hh][rk][0], lfrag[st][hh][rk][1]);
  }
  for (int f = tid; f < 4 * 32 * 2; f += blockDim.x) {
    const int nt = f / 64, a = (f / 2) % 32, hh = f % 2;
    const int dim = 32 * nt + ((a & ~12) | ((a & 4) << 1) | ((a & 8) >> 1));
    float v[8];
#pragma unroll
    for (int m = 0; m < 8; ++m) v[m] = bm[dim * RK + 8 * (m / 4) + 4 * hh + m % 4];
    split_bf16x8(v, bfrag[nt][a][hh][0], bfrag[nt][a][hh][1]);
  }
  for (int e = tid; e < P; e += blockDim.x) {
    mu[e] = x_mean[bh * P + e];
    inv_sd[e] = 1.0f / x_scale[bh * P + e];
  }
  for (int e = tid; e < D; e += blockDim.x) my[e] = y_mean[bh * D + e];
  __syncthreads();

  // Batch it is DMA'd into buffer it % 2 one batch ahead.  Once its rows are in
  // registers the buffer stages the batch's output: written in the input's swizzled
  // layout, read back in row order, so each store instruction writes 1 KB of
  // consecutive bytes (a store of 16-byte pieces from 32 rows at once runs about 20 %
  // slower).  Vector-memory operations complete in issue order and every batch but a
  // wave's last issues 8 DMAs and 8 stores, so batch it has landed once no more than
  // [stores of it - 1] + [DMA of it + 1] are outstanding.
  for (int it = 0; w0 < n; w0 += stride, ++it) {
    const int buf = it & 1;
    const bool more = w0 + stride < n;
    spr::f32x4 rv[RS > 0 ? RS : 1][2];  // this lane's role values, dims 16 s + 8 h + 4 u ..
    if constexpr (RS > 0) {
      const int64_t row = w0 + col;
      const float* rp = role + (bh * n + (row < n ? row : 0)) * RR + 8 * h;
#pragma unroll
      for (int st = 0; st < RS; ++st) {
#pragma unroll
        for (int u = 0; u < 2; ++u) rv[st][u] = *reinterpret_cast<const spr::f32x4*>(rp + 16 * st + 4 * u);
      }
    }
    if (more) dma(w0 + stride, rows_lds[wave][buf ^ 1]);
    if (it >= 1 && more) {
      wait_vmcnt<16 + NR>();
    } else if (it >= 1 || more) {
      wait_vmcnt<8 + NR>();
    } else {
      wait_vmcnt<NR>();
    }
    uint8_t* tile = rows_lds[wave][buf];
    u32x4 bv[8];  // dims 16s + 8h .. + 7 of row col
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      bv[st] = *reinterpret_cast<const u32x4*>(tile + col * ROWB + (((2 * st + h) ^ (col & 15)) << 4));
    }
    spr::f32x16 cacc = spr::f32x16{};
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      const uint32_t w[4] = {bv[st].x, bv[st].y, bv[st].z, bv[st].w};
      float z[8], m8[8], s8[8];
      lds8(mu + 16 * st + 8 * h, m8);
      lds8(inv_sd + 16 * st + 8 * h, s8);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float b = (e & 1) ? spr::bf16_hi(w[e / 2]) : spr::bf16_lo(w[e / 2]);
        z[e] = (b - m8[e]) * s8[e];
      }
      u32x4 zh, zl;
      split_bf16x8(z, zh, zl);
      const u32x4 ah = lfrag_at(lfrag[st][h], col, 0);
      const u32x4 al = lfrag_at(lfrag[st][h], col, 1);
      cacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(spr::as_bf16x8(ah), spr::as_bf16x8(zh), cacc, 0, 0, 0);
      cacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(spr::as_bf16x8(al), spr::as_bf16x8(zh), cacc, 0, 0, 0);
      cacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(spr::as_bf16x8(ah), spr::as_bf16x8(zl), cacc, 0, 0, 0);
    }
#pragma unroll
    for (int st = 0; st < RS; ++st) {  // role k-steps (rows past n: their values are never stored)
      float z[8], m8[8], s8[8];
      lds8(mu + D + 16 * st + 8 * h, m8);
      lds8(inv_sd + D + 16 * st + 8 * h, s8);
#pragma unroll
      for (int e = 0; e < 8; ++e) z[e] = (rv[st][e / 4][e % 4] - m8[e]) * s8[e];
      u32x4 zh, zl;
      split_bf16x8(z, zh, zl);
      const u32x4 ah = lfrag_at(lfrag[8 + st][h], col, 0);
      const u32x4 al = lfrag_at(lfrag[8 + st][h], col, 1);
      cacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(spr::as_bf16x8(ah), spr::as_bf16x8(zh), cacc, 0, 0, 0);
      cacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(spr::as_bf16x8(al), spr::as_bf16x8(zh), cacc, 0, 0, 0);
      cacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(spr::as_bf16x8(ah), spr::as_bf16x8(zl), cacc, 0, 0, 0);
    }
    u32x4 ch, cl;
    {
      float c[8];
#pragma unroll
      for (int m = 0; m < 8; ++m) c[m] = cacc[m];
      split_bf16x8(c, ch, cl);
    }
    spr::f32x16 acc[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const u32x4 ah = bfrag[nt][col][h][0];
      const u32x4 al = bfrag[nt][col][h][1];
      acc[nt] = spr::f32x16{};
      acc[nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(spr::as_bf16x8(ah), spr::as_bf16x8(ch), acc[nt], 0, 0, 0);
      acc[nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(spr::as_bf16x8(al), spr::as_bf16x8(ch), acc[nt], 0, 0, 0);
      acc[nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(spr::as_bf16x8(ah), spr::as_bf16x8(cl), acc[nt], 0, 0, 0);
    }
    // corr = acc + y_mean; with CAP, norms over the row's 128 dims (this lane's 64 and lane l ^ 32's)
    float bn = 0.0f, cn = 0.0f;
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      float y8[2][8];
      lds8(my + 32 * nt + 8 * h, y8[0]);
      lds8(my + 32 * nt + 16 + 8 * h, y8[1]);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int st = 2 * nt + r / 8, e = r % 8;
        acc[nt][r] += y8[r / 8][e];
        if constexpr (CAP) {
          const uint32_t w = (e / 2 == 0) ? bv[st].x : (e / 2 == 1) ? bv[st].y : (e / 2 == 2) ? bv[st].z : bv[st].w;
          const float b = (e & 1) ? spr::bf16_hi(w) : spr::bf16_lo(w);
          bn = __builtin_fmaf(b, b, bn);
          cn = __builtin_fmaf(acc[nt][r], acc[nt][r], cn);
        }
      }
    }
    float scale = alpha;
    if constexpr (CAP) {
      bn = sum_xor32(bn);
      cn = sum_xor32(cn);
      scale = alpha * fminf(1.0f, norm_cap * sqrtf(bn) / fmaxf(sqrtf(cn), 1e-20f));
    }
    // output rows into the batch's buffer (its input is in registers), then out in row order
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      const uint32_t w[4] = {bv[st].x, bv[st].y, bv[st].z, bv[st].w};
      uint32_t o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o[i] = spr::pack_bf16x2(__builtin_fmaf(scale, acc[st / 2][8 * (st % 2) + 2 * i], spr::bf16_lo(w[i])),
                                __builtin_fmaf(scale, acc[st / 2][8 * (st % 2) + 2 * i + 1], spr::bf16_hi(w[i])));
      }
      *reinterpret_cast<u32x4*>(tile + col * ROWB + (((2 * st + h) ^ (col & 15)) << 4)) = u32x4{o[0], o[1], o[2], o[3]};
    }
    uint16_t* obase = out + (bh * n + w0) * D;
#pragma unroll
    for (int i = 0; i < 8; ++i) {  // instruction i: rows 4i .. 4i + 3, piece lane % 16 of each
      const int r = 4 * i + (lane >> 4), j = lane & 15;
      const u32x4 o = *reinterpret_cast<const u32x4*>(tile + r * ROWB + ((j ^ (r & 15)) << 4));
      if (w0 + r < n) *reinterpret_cast<u32x4*>(obase + r * D + 8 * j) = o;
    }
  }
}

template <typename TD>
__global__ void probe_scatter_kernel(const TD* __restrict__ dense, const int32_t* __restrict__ rows, int64_t n,
                                     int32_t m, int32_t d, uint16_t* __restrict__ out) {
  const int64_t bh = blockIdx.y;
  for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < m * d; e += gridDim.x * blockDim.x) {
    const int j = e / d;
    const int c = e - j * d;
    const int32_t r = rows[bh * m + j];
    if (r < 0 || r >= n) continue;
    // A row listed more than once takes its last entry, as a sequential assignment would;
    // the other entries' threads write nothing, so the result does not depend on timing.
    bool later = false;
    for (int jj = j + 1; jj < m && !later; ++jj) later = rows[bh * m + jj] == r;
    if (later) continue;
    const float v = load_elem(dense, (bh * m + j) * static_cast<int64_t>(d) + c);
    out[(bh * n + r) * d + c] = spr::f32_to_bf16(v);
  }
}

}  // namespace

// ------------------------------------------------------------------------------ C ABI

// dist fp32 [bh, n] for features [bh, n, r] (dtype 0 bf16 / 2 fp32), labels int32
// [bh, n], centers fp32 [bh, groups, r].  r in {64, 128}.
extern "C" int spr_probe_distances(const void* features, int32_t dtype, const int32_t* labels, const float* centers,
                                   int64_t bh, int64_t n, int32_t groups, int32_t r, float* dist, hipStream_t stream) {
  SPR_REQUIRE(bh >= 0 && n >= 0 && groups >= 1, "spr_probe_distances: bad size");
  SPR_REQUIRE(bh <= 65535, "spr_probe_distances: bh exceeds 65535");
  if (bh == 0 || n == 0) return SPR_OK;
  SPR_REQUIRE(features && labels && centers && dist, "spr_probe_distances: null pointer");
  const size_t lds = static_cast<size_t>(groups) * r * sizeof(float);
  const bool staged = lds <= PD_LDS_BYTES;
  // staged: one round of two workgroups per CU over the chip's 256 CUs, slices whole tiles
  const int64_t slices = std::max<int64_t>(1, std::min<int64_t>(spr::ceil_div(n, 64 * 8), 512 / bh));
  const int64_t per_slice = spr::ceil_div(spr::ceil_div(n, slices), 64) * 64;
  const dim3 sgrid(static_cast<uint32_t>(spr::ceil_div(n, per_slice)), static_cast<uint32_t>(bh));
  const dim3 grid(static_cast<uint32_t>(spr::ceil_div(n, 256)), static_cast<uint32_t>(bh));
#define SPR_PD(T, RR)                                                                                               \
  do {                                                                                                               \
    if (staged)                                                                                                      \
      probe_distance_lds_kernel<T, RR><<<sgrid, PD_LDS_THREADS, lds, stream>>>(                                      \
          static_cast<const T*>(features), labels, centers, n, groups, per_slice, dist);                             \
    else                                                                                                             \
      probe_distance_kernel<T, RR><<<grid, 256, 0, stream>>>(static_cast<const T*>(features), labels, centers, n,   \
                                                              groups, dist);                                         \
  } while (0)
  if (dtype == 0 && r == 128) SPR_PD(uint16_t, 128);
  else if (dtype == 0 && r == 64) SPR_PD(uint16_t, 64);
  else if (dtype == 2 && r == 128) SPR_PD(float, 128);
  else if (dtype == 2 && r == 64) SPR_PD(float, 64);
  else SPR_REQUIRE(false, "spr_probe_distances: dtype %d / dim %d not supported", dtype, r);
#undef SPR_PD
  SPR_LAUNCHED("probe_distance_kernel");
  return SPR_OK;
}

extern "C" size_t spr_probe_select_workspace(int64_t bh, int32_t groups) {
  return (bh <= 0 || groups <= 0) ? 0 : static_cast<size_t>(bh) * groups * sizeof(unsigned long long);
}

// rows int32 [bh, count], weights fp32 [bh, count]; filled int32 [bh] (nullable)
// receives the number of rows found (count unless mode 1 ran out of tokens).
// dist may be null for mode 2.  workspace (spr_probe_select_workspace bytes, nullable)
// lets modes 0 and 2 split the pass over the tokens across many workgroups per head.
extern "C" int spr_probe_select(const float* dist, const int32_t* labels, const int32_t* sizes, int64_t bh, int64_t n,
                                int32_t groups, int32_t count, int32_t mode, int32_t* rows, float* weights,
                                int32_t* filled, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  SPR_REQUIRE(bh >= 0 && n >= 0 && groups >= 1 && count >= 0, "spr_probe_select: bad size");
  SPR_REQUIRE(groups <= MAX_GROUPS, "spr_probe_select: %d groups exceed %d", groups, MAX_GROUPS);
  SPR_REQUIRE(mode >= 0 && mode <= 2, "spr_probe_select: mode must be 0, 1 or 2");
  SPR_REQUIRE(mode == 1 || count <= groups, "spr_probe_select: rows=%d > groups=%d needs mode 1", count, groups);
  SPR_REQUIRE(n < (int64_t(1) << 31), "spr_probe_select: n too large");
  SPR_REQUIRE(count <= n, "spr_probe_select: more probes than tokens");
  if (bh == 0 || count == 0) return SPR_OK;
  SPR_REQUIRE(labels && sizes && rows && weights && (dist || mode == 2), "spr_probe_select: null pointer");
  SPR_REQUIRE(bh <= 65535, "spr_probe_select: too many heads");
  unsigned long long* gbest = nullptr;
  if (workspace != nullptr && mode != 1) {
    if (workspace_bytes < spr_probe_select_workspace(bh, groups)) {
      spr_set_error("spr_probe_select: workspace too small (%zu < %zu)", workspace_bytes,
                    spr_probe_select_workspace(bh, groups));
      return SPR_EWORKSPACE;
    }
    gbest = static_cast<unsigned long long*>(workspace);
    const int64_t total = bh * groups;
    probe_best_init_kernel<<<dim3(static_cast<uint32_t>(spr::ceil_div(total, 256))), 256, 0, stream>>>(gbest, total);
    SPR_LAUNCHED("probe_best_init_kernel");
    if (n > 0) {
      const dim3 grid(static_cast<uint32_t>(spr::ceil_div(n, PROBE_SLICE)), static_cast<uint32_t>(bh));
      probe_best_kernel<<<grid, 256, 0, stream>>>(dist, labels, n, groups, mode, gbest);
      SPR_LAUNCHED("probe_best_kernel");
    }
  }
  probe_select_kernel<<<dim3(static_cast<uint32_t>(bh)), 256, 0, stream>>>(dist, labels, sizes, n, groups, count,
                                                                           mode, rows, weights, filled, gbest);
  SPR_LAUNCHED("probe_select_kernel");
  return SPR_OK;
}

// base [bh, n, d] (dtype 0 bf16 / 2 fp32), dense [bh, m, d] (dense_dtype 0/2), rows int32
// [bh, m], role fp32 [bh, n, role_dim] (nullable when role_dim is 0) -> x_fit fp32
// [bh, m, d + role_dim] = [base[rows], role[rows]], dense_f, y_fit fp32 [bh, m, d]
// (n8_prepare_repair_fit_triton; role_dim 0 is the output-only preparation).
extern "C" int spr_repair_fit_prep_role(const void* base, int32_t base_dtype, const float* role, int32_t role_dim,
                                        const void* dense, int32_t dense_dtype, const int32_t* rows, int64_t bh,
                                        int64_t n, int32_t m, int32_t d, float* x_fit, float* dense_f, float* y_fit,
                                        hipStream_t stream) {
  SPR_REQUIRE(bh >= 0 && n >= 0 && m >= 0 && d >= 1 && role_dim >= 0, "spr_repair_fit_prep: bad size");
  SPR_REQUIRE(bh <= 65535, "spr_repair_fit_prep: bh exceeds 65535");
  if (bh == 0 || m == 0) return SPR_OK;
  SPR_REQUIRE(base && dense && rows && x_fit && dense_f && y_fit && (role || role_dim == 0),
              "spr_repair_fit_prep: null pointer");
  dim3 grid(static_cast<uint32_t>(spr::ceil_div(static_cast<int64_t>(m) * (d + role_dim), 256)),
            static_cast<uint32_t>(bh));
#define SPR_FP(TB, TD)                                                                                          \
  fit_prep_kernel<TB, TD><<<grid, 256, 0, stream>>>(static_cast<const TB*>(base), static_cast<const TD*>(dense), \
                                                    role, role_dim, rows, n, m, d, x_fit, dense_f, y_fit)
  if (base_dtype == 0 && dense_dtype == 0) SPR_FP(uint16_t, uint16_t);
  else if (base_dtype == 0 && dense_dtype == 2) SPR_FP(uint16_t, float);
  else if (base_dtype == 2 && dense_dtype == 0) SPR_FP(float, uint16_t);
  else if (base_dtype == 2 && dense_dtype == 2) SPR_FP(float, float);
  else SPR_REQUIRE(false, "spr_repair_fit_prep: unsupported dtypes");
#undef SPR_FP
  SPR_LAUNCHED("fit_prep_kernel");
  return SPR_OK;
}

// base [bh, n, d] (dtype 0 bf16 / 2 fp32), dense [bh, m, d] (dense_dtype 0/2), rows
// int32 [bh, m] -> x_fit, dense_f, y_fit fp32 [bh, m, d].
extern "C" int spr_repair_fit_prep(const void* base, int32_t base_dtype, const void* dense, int32_t dense_dtype,
                                   const int32_t* rows, int64_t bh, int64_t n, int32_t m, int32_t d, float* x_fit,
                                   float* dense_f, float* y_fit, hipStream_t stream) {
  return spr_repair_fit_prep_role(base, base_dtype, nullptr, 0, dense, dense_dtype, rows, bh, n, m, d, x_fit, dense_f,
                                  y_fit, stream);
}

// bf16 base/out [bh, n, d]; role fp32 [bh, n, role_dim] (nullable when role_dim is 0);
// x_mean, x_scale fp32 [bh, d + role_dim]; y_mean fp32 [bh, d]; left fp32
// [bh, d + role_dim, rank]; basis fp32 [bh, d, rank]; d in {64, 128}, rank in {16, 32, 64}
// (rank 16 at d = 128 on the MFMA kernel, the others one lane per row), role_dim in
// {0, 16, 32, 48, 64}.
extern "C" int spr_repair_apply_role(const void* base, const float* role, int32_t role_dim, const float* x_mean,
                                     const float* x_scale, const float* y_mean, const float* left, const float* basis,
                                     int64_t bh, int64_t n, int32_t d, int32_t rank, float alpha, float norm_cap,
                                     void* out, hipStream_t stream) {
  SPR_REQUIRE(bh >= 0 && n >= 0, "spr_repair_apply: bad size");
  SPR_REQUIRE((d == 128 || d == 64) && (rank == 16 || rank == 32 || rank == 64),
              "spr_repair_apply: requires D in {64, 128}, rank in {16, 32, 64} (got %d, %d)", d, rank);
  SPR_REQUIRE(role_dim >= 0 && role_dim <= 64 && role_dim % 16 == 0,
              "spr_repair_apply: role_dim must be 0, 16, 32, 48 or 64 (got %d)", role_dim);
  SPR_REQUIRE(bh <= 65535, "spr_repair_apply: bh exceeds 65535");
  if (bh == 0 || n == 0) return SPR_OK;
  SPR_REQUIRE(base && x_mean && x_scale && y_mean && left && basis && out && (role || role_dim == 0),
              "spr_repair_apply: null pointer");
  SPR_REQUIRE(reinterpret_cast<uintptr_t>(base) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(role) % 16 == 0,
              "spr_repair_apply: base/out/role must be 16-byte aligned");
  const uint16_t* b16 = static_cast<const uint16_t*>(base);
  uint16_t* o16 = static_cast<uint16_t*>(out);
  if (rank != 16) {
    dim3 grid(static_cast<uint32_t>(spr::ceil_div(n, 256)), static_cast<uint32_t>(bh));
    auto lane_rows = [&](auto dd, auto rk) {
      constexpr int DD = decltype(dd)::value, RKK = decltype(rk)::value;
      switch (role_dim) {
        case 0: repair_apply_kernel<DD, RKK, 0><<<grid, 256, 0, stream>>>(b16, role, x_mean, x_scale, y_mean, left,
                                                                            basis, n, alpha, norm_cap, o16); break;
        case 16: repair_apply_kernel<DD, RKK, 16><<<grid, 256, 0, stream>>>(b16, role, x_mean, x_scale, y_mean, left,
                                                                              basis, n, alpha, norm_cap, o16); break;
        case 32: repair_apply_kernel<DD, RKK, 32><<<grid, 256, 0, stream>>>(b16, role, x_mean, x_scale, y_mean, left,
                                                                              basis, n, alpha, norm_cap, o16); break;
        case 48: repair_apply_kernel<DD, RKK, 48><<<grid, 256, 0, stream>>>(b16, role, x_mean, x_scale, y_mean, left,
                                                                              basis, n, alpha, norm_cap, o16); break;
        default: repair_apply_kernel<DD, RKK, 64><<<grid, 256, 0, stream>>>(b16, role, x_mean, x_scale, y_mean, left,
                                                                              basis, n, alpha, norm_cap, o16); break;
      }
    };
    using R32 = std::integral_constant<int, 32>;
    using R64 = std::integral_constant<int, 64>;
    if (d == 128) {
      if (rank == 32) lane_rows(std::integral_constant<int, 128>{}, R32{}); else lane_rows(std::integral_constant<int, 128>{}, R64{});
    } else {
      if (rank == 32) lane_rows(std::integral_constant<int, 64>{}, R32{}); else lane_rows(std::integral_constant<int, 64>{}, R64{});
    }
  } else if (d == 128) {
    SPR_REQUIRE(n * 256 < (int64_t(1) << 31), "spr_repair_apply: a head's rows exceed 2 GiB");
    // one resident workgroup per CU (256 CUs), each walking 256-row batches of one head
    const int64_t per_head = std::max<int64_t>(1, std::min<int64_t>(spr::ceil_div(n, 256), 256 / bh));
    dim3 grid(static_cast<uint32_t>(per_head), static_cast<uint32_t>(bh));
#define SPR_RA(CAP, RR)                                                                                           \
  repair_apply_mfma_kernel<CAP, RR><<<grid, 512, 0, stream>>>(b16, role, x_mean, x_scale, y_mean, left, basis, n, \
                                                              alpha, norm_cap, o16)
#define SPR_RA_CAP(RR)          \
  do {                          \
    if (norm_cap > 0.0f)        \
      SPR_RA(true, RR);         \
    else                        \
      SPR_RA(false, RR);        \
  } while (0)
    switch (role_dim) {
      case 0: SPR_RA_CAP(0); break;
      case 16: SPR_RA_CAP(16); break;
      case 32: SPR_RA_CAP(32); break;
      case 48: SPR_RA_CAP(48); break;
      default: SPR_RA_CAP(64); break;
    }
#undef SPR_RA_CAP
#undef SPR_RA
  } else {
    dim3 grid(static_cast<uint32_t>(spr::ceil_div(n, 256)), static_cast<uint32_t>(bh));
#define SPR_RA64(RR)                                                                                                \
  repair_apply_kernel<64, 16, RR><<<grid, 256, 0, stream>>>(b16, role, x_mean, x_scale, y_mean, left, basis, n, alpha, \
                                                            norm_cap, o16)
    switch (role_dim) {
      case 0: SPR_RA64(0); break;
      case 16: SPR_RA64(16); break;
      case 32: SPR_RA64(32); break;
      case 48: SPR_RA64(48); break;
      default: SPR_RA64(64); break;
    }
#undef SPR_RA64
  }
  SPR_LAUNCHED("repair_apply_kernel");
  return SPR_OK;
}

// bf16 base/out [bh, n, d]; x_mean, x_scale, y_mean fp32 [bh, d]; left, basis fp32
// [bh, d, rank]; d in {64, 128}, rank 16 (the output-only form of spr_repair_apply_role).
extern "C" int spr_repair_apply(const void* base, const float* x_mean, const float* x_scale, const float* y_mean,
                                const float* left, const float* basis, int64_t bh, int64_t n, int32_t d, int32_t rank,
                                float alpha, float norm_cap, void* out, hipStream_t stream) {
  return spr_repair_apply_role(base, nullptr, 0, x_mean, x_scale, y_mean, left, basis, bh, n, d, rank, alpha,
                               norm_cap, out, stream);
}

// out bf16 [bh, n, d]; out[b, rows[b, j]] = dense[b, j] (dense_dtype 0 bf16 / 2 fp32).
extern "C" int spr_probe_scatter(const void* dense, int32_t dense_dtype, const int32_t* rows, int64_t bh, int64_t n,
                                 int32_t m, int32_t d, void* out, hipStream_t stream) {
  SPR_REQUIRE(bh >= 0 && n >= 0 && m >= 0 && d >= 1, "spr_probe_scatter: bad size");
  SPR_REQUIRE(bh <= 65535, "spr_probe_scatter: bh exceeds 65535");
  if (bh == 0 || m == 0) return SPR_OK;
  SPR_REQUIRE(dense && rows && out, "spr_probe_scatter: null pointer");
  dim3 grid(static_cast<uint32_t>(spr::ceil_div(static_cast<int64_t>(m) * d, 256)), static_cast<uint32_t>(bh));
  if (dense_dtype == 0) {
    probe_scatter_kernel<uint16_t><<<grid, 256, 0, stream>>>(static_cast<const uint16_t*>(dense), rows, n, m, d,
                                                             static_cast<uint16_t*>(out));
  } else if (dense_dtype == 2) {
    probe_scatter_kernel<float><<<grid, 256, 0, stream>>>(static_cast<const float*>(dense), rows, n, m, d,
                                                          static_cast<uint16_t*>(out));
  } else {
    SPR_REQUIRE(false, "spr_probe_scatter: unsupported dense dtype %d", dense_dtype);
  }
  SPR_LAUNCHED("probe_scatter_kernel");
  return SPR_OK;
}
