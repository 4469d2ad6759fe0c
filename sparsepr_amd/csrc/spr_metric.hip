// Role metrics and their factors for the N8 router (N8V6Core.route).
//
// Replaces (src/sparsepr/models/cosmos3/operator_kmeans.py):
//   covariance / key_metric_from_queries / value_metric_from_values (:62-92, :491-498)
//   query_metric_from_key_centroids (:517-531)
//   metric_factor (:95-151)
//   warm_subspace_metric_factor with every orthogonalisation (each_qr, final_qr,
//     each_cholesky_qr(2), cholesky_qr) and every finish (full, rayleigh_cholesky, diagonal,
//     previous_scale) (:219-477), cholesky_with_device_fallback (:154-216)
//   project_tokens / normalize_rows_rms and the compiled K-centroid projection
//     (:534-555; src/sparsepr/models/common/n8_v6.py:141-178)
// and the per-head recovery of N8V6Core._updated_factor (n8_v6.py:478-519).
//
// role_metric_kernel   out = post_scale / count * sum over the used rows of (x - mean)(x - mean)^T,
//                      one 32 x 32 output tile per workgroup, rows staged in LDS, fp32.
// warm_factor_kernel   one 1024-thread workgroup per head with the metric (128 x 128), the basis
//                      and its image in LDS: metric . basis products, column normalisation,
//                      Gram, Cholesky (one wave), triangular solves, Householder QR (columns
//                      register resident, one barrier per reflector), Rayleigh matrix,
//                      fallback Cholesky, all fp32.  The full finish hands the Rayleigh
//                      matrix to spr_sym_top_eig and warm_full_finish_kernel.
// factor_scale_kernel  eigenvectors x sqrt(max(lambda, 0) / max(mean lambda, 1e-12)).
// project_rows_kernel  one wave per row: p = x . F (fp32, or both operands rounded to TF32 as
//                      a "high"-precision fp32 matmul does, or to bf16 as a "medium" one
//                      does), / a per-head divisor, optional row-RMS normalisation, times a
//                      weight, into columns of a wider row.
#include "spr_common.h"

extern "C" int spr_sym_top_eig(const float* mats, int64_t bh, int32_t n, int32_t rank, int32_t symmetrize,
                               float* vecs, float* vals, hipStream_t stream);

namespace {

constexpr int MET_MAX_D = 128;
constexpr int MET_MAX_R = 64;

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_read(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
// Sum over the wave, uniform result.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_mov<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_mov<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp_mov<0x124>(v);  // row_ror 4
  v += dpp_mov<0x128>(v);  // row_ror 8
  return (lane_read(v, 0) + lane_read(v, 16)) + (lane_read(v, 32) + lane_read(v, 48));
}
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
__device__ __forceinline__ float tf32_rna(float v) {
  return __uint_as_float((__float_as_uint(v) + 0x1000u) & 0xFFFFE000u);
}

template <typename T>
__device__ __forceinline__ float load_f32(const T* p);
template <>
__device__ __forceinline__ float load_f32<uint16_t>(const uint16_t* p) {
  return __uint_as_float(static_cast<uint32_t>(*p) << 16);
}
template <>
__device__ __forceinline__ float load_f32<float>(const float* p) {
  return *p;
}

// ---------------------------------------------------------------- covariance
// grid (bh, tiles^2): tile (ti, tj) of the d x d output; rows used: rows[0 .. count) when
// rows is given (the same positions for every head), else all n rows, each only when
// sizes[h, r] > 0 (sizes nullable).  Rows go in stages of RB: the stage's row indices and
// validity are loaded once into LDS, then every thread loads its 2 x RB / 8 elements of
// the two column blocks (independent loads), the next stage's while the current one is
// summed.  The column means (center) take one such pass first: thread t sums column t % 32
// over the stage rows r = t / 32 (mod 8), and the eight partial sums are added in order.
template <typename T>
__global__ __launch_bounds__(256) void role_metric_kernel(const T* __restrict__ x, int64_t n, int32_t d,
                                                          const int32_t* __restrict__ rows, int32_t count,
                                                          const int32_t* __restrict__ sizes, int32_t center,
                                                          float post_scale, float* __restrict__ out) {
  // rows per stage: each stage waits on a row-index load and then a value load, so larger
  // stages mean fewer waits; the sums run over the rows in the same order for any RB
  constexpr int RB = 192;
  constexpr int PER = RB * 32 / 256;  // elements per thread and column block per stage (24)
  __shared__ float ta[RB][33];
  __shared__ float tb[RB][33];
  __shared__ int64_t ridx[2][RB];  // row of each stage row (-1: not used)
  __shared__ float part[8][64];
  __shared__ float mean_a[32], mean_b[32];
  __shared__ int32_t used_s;
  const int t = threadIdx.x;
  const int64_t h = blockIdx.x;
  const int tiles = (d + 31) / 32;
  const int ti = blockIdx.y / tiles, tj = blockIdx.y % tiles;
  const T* xh = x + h * n * d;
  const int32_t* sz = sizes != nullptr ? sizes + h * n : nullptr;
  const int64_t total = rows != nullptr ? count : n;
  const int64_t nstage = (total + RB - 1) / RB;
  const int cc = t & 31, rg = t >> 5;  // column in the block, row group (rows rg + 8 i)
  const int ca = 32 * ti + cc, cb = 32 * tj + cc;
  // the row indices of stage s into ridx[s & 1] (threads 0 .. RB - 1)
  auto stage_rows = [&](int64_t st) {
    if (t < RB) {
      const int64_t r = st * RB + t;
      int64_t row = -1;
      if (r < total) {
        row = rows != nullptr ? rows[r] : r;
        if (sz != nullptr && !(sz[row] > 0)) row = -1;
      }
      ridx[st & 1][t] = row;
    }
  };
  auto load_vals = [&](int64_t st, float (&va)[PER], float (&vb)[PER]) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int64_t row = ridx[st & 1][rg + 8 * i];
      va[i] = (row >= 0 && ca < d) ? load_f32(xh + row * d + ca) : 0.0f;
      vb[i] = (row >= 0 && cb < d) ? load_f32(xh + row * d + cb) : 0.0f;
    }
  };
  // ---- column means and the used-row count
  if (t == 0) used_s = 0;
  float sa = 0.0f, sb = 0.0f;
  int32_t used = 0;
  const bool need_means = center || sz != nullptr;
  if (need_means) {
    for (int64_t st = 0; st < nstage; ++st) {
      stage_rows(st);
      __syncthreads();
      float va[PER], vb[PER];
      load_vals(st, va, vb);
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        sa += va[i];
        sb += vb[i];
      }
      if (t < RB) used += ridx[st & 1][t] >= 0 ? 1 : 0;
      __syncthreads();  // ridx[st & 1] is rewritten two stages on
    }
    part[rg][cc] = sa;
    part[rg][32 + cc] = sb;
    if (t < RB) atomicAdd(&used_s, used);  // integer: order-independent
    __syncthreads();
    if (t < 64) {
      float m = 0.0f;
      for (int g = 0; g < 8; ++g) m += part[g][t];
      const float cnt = static_cast<float>(used_s > 0 ? used_s : 1);
      m = center ? m / cnt : 0.0f;
      if (t < 32) mean_a[t] = m; else mean_b[t - 32] = m;
    }
  } else {
    if (t < 32) {
      mean_a[t] = 0.0f;
      mean_b[t] = 0.0f;
    }
    if (t == 0) used_s = static_cast<int32_t>(total);
  }
  __syncthreads();
  // ---- (x - mean_a)^T (x - mean_b) over the used rows
  const int a = t >> 4, b = t & 15;  // outputs (2a, 2a + 1) x (2b, 2b + 1) of the tile
  float s00 = 0.0f, s01 = 0.0f, s10 = 0.0f, s11 = 0.0f;
  float va[PER], vb[PER];
  if (nstage > 0) {
    stage_rows(0);
    __syncthreads();
    load_vals(0, va, vb);
  }
  for (int64_t st = 0; st < nstage; ++st) {
    // stage st's values (in registers) into the tiles; stage st + 1's rows into the other
    // ridx slot, then its values into registers while the tiles are summed
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int64_t row = ridx[st & 1][rg + 8 * i];
      ta[rg + 8 * i][cc] = row >= 0 ? va[i] - mean_a[cc] : 0.0f;
      tb[rg + 8 * i][cc] = row >= 0 ? vb[i] - mean_b[cc] : 0.0f;
    }
    if (st + 1 < nstage) stage_rows(st + 1);
    __syncthreads();
    if (st + 1 < nstage) load_vals(st + 1, va, vb);
    const int rows_here = static_cast<int>(total - st * RB < RB ? total - st * RB : RB);
    for (int rr = 0; rr < rows_here; ++rr) {
      const float u0 = ta[rr][2 * a], u1 = ta[rr][2 * a + 1];
      const float v0 = tb[rr][2 * b], v1 = tb[rr][2 * b + 1];
      s00 = __builtin_fmaf(u0, v0, s00);
      s01 = __builtin_fmaf(u0, v1, s01);
      s10 = __builtin_fmaf(u1, v0, s10);
      s11 = __builtin_fmaf(u1, v1, s11);
    }
    __syncthreads();
  }
  const float cnt = static_cast<float>(used_s > 0 ? used_s : 1);
  const float acc[2][2] = {{s00, s01}, {s10, s11}};
#pragma unroll
  for (int u = 0; u < 2; ++u) {
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      const int gi = 32 * ti + 2 * a + u, gj = 32 * tj + 2 * b + v;
      if (gi < d && gj < d) out[(h * d + gi) * d + gj] = acc[u][v] / cnt * post_scale;
    }
  }
}

// ---------------------------------------------------------------- cold factor scaling
// factor [n][r] holds the eigenvectors (ascending); vals [r] the eigenvalues (ascending):
// factor *= sqrt(max(lambda, 0) / max(mean_r max(lambda, 0), 1e-12)).
__global__ __launch_bounds__(256) void factor_scale_kernel(float* __restrict__ factor, const float* __restrict__ vals,
                                                           int32_t n, int32_t r) {
  __shared__ float scale_s[MET_MAX_R];
  const int64_t h = blockIdx.x;
  const float* lv = vals + h * r;
  if (threadIdx.x == 0) {
    float s = 0.0f;
    for (int c = 0; c < r; ++c) s += fmaxf(lv[c], 0.0f);
    const float norm = fmaxf(s / static_cast<float>(r), 1e-12f);
    for (int c = 0; c < r; ++c) scale_s[c] = sqrtf(fmaxf(lv[c], 0.0f) / norm);
  }
  __syncthreads();
  float* f = factor + h * n * r;
  for (int e = threadIdx.x; e < n * r; e += blockDim.x) f[e] *= scale_s[e % r];
}

// ---------------------------------------------------------------- warm subspace update
constexpr int WF_THREADS = 1024;
// Rows are 16-byte aligned for vector reads and 4 banks apart, so the eight rows one wave
// reads at a time fall in distinct banks.
constexpr int LDM = MET_MAX_D + 4;  // metric row
constexpr int LDB = MET_MAX_R + 4;  // basis row

enum WarmOrtho { ORTHO_EACH_CQR = 0, ORTHO_EACH_CQR2 = 1, ORTHO_FINAL_CQR = 2, ORTHO_EACH_QR = 3, ORTHO_FINAL_QR = 4 };
enum WarmRitz { RITZ_RAYLEIGH_CHOLESKY = 0, RITZ_DIAGONAL = 1, RITZ_PREVIOUS_SCALE = 2, RITZ_FULL = 3 };

struct WarmSmem {
  __attribute__((aligned(16))) float m[MET_MAX_D * LDM];  // metric
  __attribute__((aligned(16))) float b[MET_MAX_D * LDB];  // basis
  __attribute__((aligned(16))) float w[MET_MAX_D * LDB];  // metric . basis, scratch
  __attribute__((aligned(16))) float g[MET_MAX_R * LDB];  // Gram / Rayleigh matrix, its Cholesky factor (lower)
  __attribute__((aligned(16))) float lcol[MET_MAX_R];     // the Cholesky column in flight
  float colv[MET_MAX_R];      // per-column values (norms, diagonal Ritz values, scales)
  float tau[MET_MAX_R];       // Householder scalars
  float scal[4];
  int32_t fail;
};

// Sum over the 8 lanes 8g .. 8g + 7 (every lane of the group gets the same value).
__device__ __forceinline__ float sum8(float v) {
  v += dpp_mov<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_mov<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp_mov<0x141>(v);  // row_half_mirror
  return v;
}

// w = m . b (n x n times n x r); thread t: row t / 8, columns 8 (t % 8) .. + 7, the sum over
// j in index order; m read four entries at a time, b eight columns at a time
__device__ __forceinline__ void wf_apply(WarmSmem& s, int n, int r) {
  const int t = threadIdx.x, i = t >> 3, c0 = 8 * (t & 7);
  if (i < n && c0 < r) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    auto step = [&](float mij, int j) {
      const spr::f32x4 b0 = *reinterpret_cast<const spr::f32x4*>(&s.b[j * LDB + c0]);
      const spr::f32x4 b1 = *reinterpret_cast<const spr::f32x4*>(&s.b[j * LDB + c0 + 4]);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        acc[u] = __builtin_fmaf(mij, b0[u], acc[u]);
        acc[4 + u] = __builtin_fmaf(mij, b1[u], acc[4 + u]);
      }
    };
    int j = 0;
    for (; j + 4 <= n; j += 4) {
      const spr::f32x4 mv = *reinterpret_cast<const spr::f32x4*>(&s.m[i * LDM + j]);
#pragma unroll
      for (int u = 0; u < 4; ++u) step(mv[u], j + u);
    }
    for (; j < n; ++j) step(s.m[i * LDM + j], j);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (c0 + u < r) s.w[i * LDB + c0 + u] = acc[u];
    }
  }
  __syncthreads();
}

// column norms of src (n x r) into colv, clamped at 1e-12
__device__ __forceinline__ void wf_colnorms(WarmSmem& s, const float* src, int n, int r) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  for (int col = wv; col < r; col += WF_THREADS / 64) {
    const float v0 = lane < n ? src[lane * LDB + col] : 0.0f;
    const float v1 = lane + 64 < n ? src[(lane + 64) * LDB + col] : 0.0f;
    const float ss = wave_sum(v0 * v0 + v1 * v1);
    if (lane == 0) s.colv[col] = fmaxf(sqrtf(ss), 1e-12f);
  }
  __syncthreads();
}

// g = a^T c (r x r), or 0.5 (a^T c + c^T a) when symmetrize; thread t owns the 2 x 2 tile
// at (2 (t / 32), 2 (t % 32)), sums over the rows in index order; tiles on or above the
// diagonal are computed and mirrored, so g is exactly symmetric
__device__ __forceinline__ void wf_gram(WarmSmem& s, const float* a, const float* c, int n, int r, bool symmetrize) {
  const int t = threadIdx.x, p0 = 2 * (t >> 5), q0 = 2 * (t & 31);
  if (p0 < r && q0 < r && p0 <= q0) {
    float acc[2][2] = {{0, 0}, {0, 0}}, acc2[2][2] = {{0, 0}, {0, 0}};
    for (int i = 0; i < n; ++i) {
      const float2 ap = *reinterpret_cast<const float2*>(&a[i * LDB + p0]);
      const float2 cq = *reinterpret_cast<const float2*>(&c[i * LDB + q0]);
      acc[0][0] = __builtin_fmaf(ap.x, cq.x, acc[0][0]);
      acc[0][1] = __builtin_fmaf(ap.x, cq.y, acc[0][1]);
      acc[1][0] = __builtin_fmaf(ap.y, cq.x, acc[1][0]);
      acc[1][1] = __builtin_fmaf(ap.y, cq.y, acc[1][1]);
      if (symmetrize) {
        const float2 aq = *reinterpret_cast<const float2*>(&a[i * LDB + q0]);
        const float2 cp = *reinterpret_cast<const float2*>(&c[i * LDB + p0]);
        acc2[0][0] = __builtin_fmaf(aq.x, cp.x, acc2[0][0]);
        acc2[0][1] = __builtin_fmaf(aq.y, cp.x, acc2[0][1]);
        acc2[1][0] = __builtin_fmaf(aq.x, cp.y, acc2[1][0]);
        acc2[1][1] = __builtin_fmaf(aq.y, cp.y, acc2[1][1]);
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int v = 0; v < 2; ++v) {
        const int p = p0 + u, q = q0 + v;
        if (p < r && q < r && p <= q) {
          const float val = symmetrize ? 0.5f * (acc[u][v] + acc2[u][v]) : acc[u][v];
          s.g[p * LDB + q] = val;
          s.g[q * LDB + p] = val;
        }
      }
    }
  }
  __syncthreads();
}

// In-place lower Cholesky of src[0..r) + shift I into g, by wave 0: lane = row, the row in
// registers; each column of L goes through LDS once and comes back as broadcast reads
// (a readlane per entry instead measured twice as slow).  Sets *fail (0 = every pivot
// finite and positive).  Only the lower triangle of g is written; on failure the factor is
// undefined.  Kept out of line (it is called from several places and is fully unrolled);
// its LDS pointers carry their address space, so the accesses stay LDS instructions.
typedef __attribute__((address_space(3))) float lds_f32;
typedef __attribute__((address_space(3))) int32_t lds_i32;
template <int RMAX>
__device__ __noinline__ void wf_cholesky_wave(const lds_f32* src, lds_f32* g, lds_f32* lcol, lds_i32* fail, int r,
                                              float shift) {
  const int lane = threadIdx.x & 63;
  float row[RMAX];
#pragma unroll
  for (int j = 0; j < RMAX; ++j) {
    row[j] = (lane < r && j <= lane && j < r) ? src[lane * LDB + j] + (j == lane ? shift : 0.0f) : 0.0f;
  }
  bool ok = true;
#pragma unroll
  for (int k = 0; k < RMAX; ++k) {
    if (k < r) {
      const float piv = lane_read(row[k], k);
      ok = ok && (piv > 0.0f) && (piv < __builtin_huge_valf());
      const float lkk = sqrtf(fmaxf(piv, 1e-30f));
      const float lik = lane > k ? row[k] / lkk : 0.0f;
      row[k] = lane == k ? lkk : (lane > k ? lik : row[k]);
      lcol[lane] = lik;
      wave_sync();
#pragma unroll
      for (int j = k + 1; j < RMAX; ++j) row[j] -= lik * lcol[j];  // entries past the lane are unused
      wave_sync();
    }
  }
#pragma unroll
  for (int j = 0; j < RMAX; ++j) {
    if (lane < r && j <= lane) g[lane * LDB + j] = row[j];
  }
  if (lane == 0) *fail = ok ? 0 : 1;
}
__device__ __forceinline__ bool wf_cholesky(WarmSmem& s, const float* src, int r, float shift) {
  if (threadIdx.x < 64) {
    // generic to LDS address space (the pointers point into the workgroup's LDS); the
    // unrolled loops stop at r rounded up to 16
    const lds_f32* a = (const lds_f32*)src;
    lds_f32* g = (lds_f32*)s.g;
    lds_f32* lc = (lds_f32*)s.lcol;
    lds_i32* f = (lds_i32*)&s.fail;
    if (r <= 16) {
      wf_cholesky_wave<16>(a, g, lc, f, r, shift);
    } else if (r <= 32) {
      wf_cholesky_wave<32>(a, g, lc, f, r, shift);
    } else if (r <= 48) {
      wf_cholesky_wave<48>(a, g, lc, f, r, shift);
    } else {
      wf_cholesky_wave<MET_MAX_R>(a, g, lc, f, r, shift);
    }
  }
  __syncthreads();
  return s.fail == 0;
}

// b = w L^-T: row i solves L y = w_i by forward substitution (identity L when ok is false).
// Threads 8 i .. 8 i + 7 share the row; thread 8 i + u keeps y[c] for c = u mod 8 in
// registers, and each step sums the eight partial dot products (DPP) before the division.
// Out of line for the same reason as the Cholesky.
template <int RMAX>
__device__ __noinline__ void wf_solve_rows(const lds_f32* g, const lds_f32* w, lds_f32* b, int n, int r, bool ok) {
  const int t = threadIdx.x, i = t >> 3, u = t & 7;
  float y[RMAX / 8];
#pragma unroll
  for (int q = 0; q < RMAX / 8; ++q) y[q] = 0.0f;
#pragma unroll
  for (int c = 0; c < RMAX; ++c) {
    if (c < r) {
      float part = 0.0f;
#pragma unroll
      for (int q = 0; q < RMAX / 8; ++q) {
        if (8 * q < c) {
          const int k = 8 * q + u;
          part = k < c ? __builtin_fmaf(g[c * LDB + k], y[q], part) : part;
        }
      }
      const float tot = sum8(part);
      const float wic = i < n ? w[i * LDB + c] : 0.0f;
      const float yc = ok ? (wic - tot) / g[c * LDB + c] : wic;
      if (u == (c & 7)) y[c >> 3] = yc;
    }
  }
  if (i < n) {
#pragma unroll
    for (int q = 0; q < RMAX / 8; ++q) {
      if (8 * q + u < r) b[i * LDB + 8 * q + u] = y[q];
    }
  }
}

// Cholesky-QR of src (n x r) into s.b (operator_kmeans.py:326-358): columns normalised
// (norm clamped at 1e-12), Gram, jitter = max(mean diag, 1e-12) * ridge on the diagonal,
// Cholesky (identity on failure), b = normalised . L^-T.  Returns whether it failed.
__device__ __forceinline__ bool wf_cholesky_qr(WarmSmem& s, const float* src, int n, int r, float ridge) {
  wf_colnorms(s, src, n, r);
  // normalised columns into w (src may be w itself: each element read then written by one thread)
  for (int e = threadIdx.x; e < n * r; e += WF_THREADS) {
    const int i = e / r, c = e - i * r;
    s.w[i * LDB + c] = src[i * LDB + c] / s.colv[c];
  }
  __syncthreads();
  // w^T w is symmetric as computed (each tile pair sums the same products in the same
  // order), so symmetrising would return it unchanged
  wf_gram(s, s.w, s.w, n, r, false);
  if (threadIdx.x == 0) {
    float tr = 0.0f;
    for (int c = 0; c < r; ++c) tr += s.g[c * LDB + c];
    s.scal[0] = fmaxf(tr / static_cast<float>(r), 1e-12f) * ridge;
  }
  __syncthreads();
  const bool ok = wf_cholesky(s, s.g, r, s.scal[0]);  // in place
  const lds_f32* gl = (const lds_f32*)s.g;
  const lds_f32* wl = (const lds_f32*)s.w;
  lds_f32* bl = (lds_f32*)s.b;
  if (r <= 16) {
    wf_solve_rows<16>(gl, wl, bl, n, r, ok);
  } else if (r <= 32) {
    wf_solve_rows<32>(gl, wl, bl, n, r, ok);
  } else if (r <= 48) {
    wf_solve_rows<48>(gl, wl, bl, n, r, ok);
  } else {
    wf_solve_rows<MET_MAX_R>(gl, wl, bl, n, r, ok);
  }
  __syncthreads();
  return !ok;
}

// Householder QR of a (n x r, rows of LDB floats) into q (n x r), as LAPACK geqrf + orgqr
// (torch.linalg.qr, mode "reduced"): reflector k is H_k = I - tau_k v v^T with v[k] = 1,
// v[i > k] = x[i] / (alpha - beta), beta = -sign(alpha) sqrt(alpha^2 + |x below|^2)
// (alpha = x[k]; sign(+-0) = +), tau_k = (beta - alpha) / beta, and tau_k = 0 when x is zero
// below the pivot; Q = H_0 ... H_{r-1} [I; 0].  Column j belongs to wave j % 16 and stays in
// its registers (lane l: rows l and l + 64); the owner of column k + 1 forms reflector k + 1
// as soon as H_k has been applied to it, so each reflector costs one barrier.  The
// reflectors overwrite a (column k below the diagonal), tau goes to tau; Q is formed
// backwards from them without barriers, each wave on its own columns.
constexpr int QR_WAVES = WF_THREADS / 64;
constexpr int QR_COLS = MET_MAX_R / QR_WAVES;
__device__ __forceinline__ void qr_reflector(float x0, float x1, int k, int n, lds_f32* a, lds_f32* tau) {
  const int lane = threadIdx.x & 63, i0 = lane, i1 = lane + 64;
  const float below = (i0 > k && i0 < n ? x0 * x0 : 0.0f) + (i1 > k && i1 < n ? x1 * x1 : 0.0f);
  const float sigma = wave_sum(below);
  const float alpha = lane_read(k < 64 ? x0 : x1, k & 63);
  float tk = 0.0f, sk = 0.0f;
  if (sigma != 0.0f) {
    const float nrm = sqrtf(alpha * alpha + sigma);
    const float beta = alpha >= 0.0f ? -nrm : nrm;
    tk = (beta - alpha) / beta;
    sk = 1.0f / (alpha - beta);
  }
  if (i0 > k && i0 < n) a[i0 * LDB + k] = x0 * sk;
  if (i1 > k && i1 < n) a[i1 * LDB + k] = x1 * sk;
  if (lane == 0) tau[k] = tk;
}
__device__ __noinline__ void wf_householder_qr(lds_f32* a, lds_f32* q, lds_f32* tau, int n, int r) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, i0 = lane, i1 = lane + 64;
  float col[QR_COLS][2];
#pragma unroll
  for (int c = 0; c < QR_COLS; ++c) {
    const int j = wv + QR_WAVES * c;
    col[c][0] = j < r && i0 < n ? a[i0 * LDB + j] : 0.0f;
    col[c][1] = j < r && i1 < n ? a[i1 * LDB + j] : 0.0f;
  }
  if (wv == 0) qr_reflector(col[0][0], col[0][1], 0, n, a, tau);
  __syncthreads();
  for (int k = 0; k < r; ++k) {
    const float v0 = i0 == k ? 1.0f : (i0 > k && i0 < n ? a[i0 * LDB + k] : 0.0f);
    const float v1 = i1 == k ? 1.0f : (i1 > k && i1 < n ? a[i1 * LDB + k] : 0.0f);
    const float tk = tau[k];
#pragma unroll
    for (int c = 0; c < QR_COLS; ++c) {
      const int j = wv + QR_WAVES * c;
      if (j > k && j < r) {
        const float dot = wave_sum(v0 * col[c][0] + v1 * col[c][1]);
        col[c][0] = __builtin_fmaf(-tk * dot, v0, col[c][0]);
        col[c][1] = __builtin_fmaf(-tk * dot, v1, col[c][1]);
        if (j == k + 1) qr_reflector(col[c][0], col[c][1], k + 1, n, a, tau);
      }
    }
    __syncthreads();
  }
  float qc[QR_COLS][2];
#pragma unroll
  for (int c = 0; c < QR_COLS; ++c) qc[c][0] = qc[c][1] = 0.0f;
  for (int k = r - 1; k >= 0; --k) {
    const float v0 = i0 == k ? 1.0f : (i0 > k && i0 < n ? a[i0 * LDB + k] : 0.0f);
    const float v1 = i1 == k ? 1.0f : (i1 > k && i1 < n ? a[i1 * LDB + k] : 0.0f);
    const float tk = tau[k];
#pragma unroll
    for (int c = 0; c < QR_COLS; ++c) {
      const int j = wv + QR_WAVES * c;
      if (j > k && j < r) {
        const float dot = wave_sum(v0 * qc[c][0] + v1 * qc[c][1]);
        qc[c][0] = __builtin_fmaf(-tk * dot, v0, qc[c][0]);
        qc[c][1] = __builtin_fmaf(-tk * dot, v1, qc[c][1]);
      } else if (j == k) {
        qc[c][0] = (i0 == k ? 1.0f : 0.0f) - tk * v0;
        qc[c][1] = (i1 == k ? 1.0f : 0.0f) - tk * v1;
      }
    }
  }
#pragma unroll
  for (int c = 0; c < QR_COLS; ++c) {
    const int j = wv + QR_WAVES * c;
    if (j < r) {
      if (i0 < n) q[i0 * LDB + j] = qc[c][0];
      if (i1 < n) q[i1 * LDB + j] = qc[c][1];
    }
  }
  __syncthreads();
}
__device__ __forceinline__ void wf_qr(WarmSmem& s, int n, int r) {  // s.w -> s.b
  wf_householder_qr((lds_f32*)s.w, (lds_f32*)s.b, (lds_f32*)s.tau, n, r);
}

// One head per workgroup.  metric [n][n]; prev_state [n][r] (the previous basis, or the cold
// factor); prev_factor [n][r] (nullable: the previous factor); outputs factor, state [n][r]
// and recovered[h] (1 = a Cholesky failed or a result is not finite; then, when prev_factor
// is given, factor and state are the previous ones).  The full finish instead writes the
// basis [n][r], the Rayleigh matrix [r][r] (diag(1 .. r) when it is not finite, so the
// eigensolver only sees finite input) and the Cholesky failure flag into the workspace
// arrays full_basis / full_ray / full_flag, for warm_full_finish_kernel.
__global__ __launch_bounds__(WF_THREADS, 1) void warm_factor_kernel(
    const float* __restrict__ metric, const float* __restrict__ prev_state, const float* __restrict__ prev_factor,
    int32_t n, int32_t r, int32_t power_iters, int32_t ortho, int32_t ritz, float rayleigh_ridge, float cqr_ridge,
    float* __restrict__ factor, float* __restrict__ state, uint8_t* __restrict__ recovered,
    float* __restrict__ full_basis, float* __restrict__ full_ray, int32_t* __restrict__ full_flag) {
  __shared__ WarmSmem s;
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int64_t h = blockIdx.x;
  const float* mh = metric + h * n * n;
  const float* ps = prev_state + h * n * r;
  const float* pf = prev_factor != nullptr ? prev_factor + h * n * r : nullptr;
  for (int e = t; e < n * n; e += WF_THREADS) s.m[(e / n) * LDM + (e % n)] = mh[e];
  for (int e = t; e < n * r; e += WF_THREADS) s.b[(e / r) * LDB + (e % r)] = ps[e];
  __syncthreads();
  bool failed = false;
  // previous column scales (only the previous_scale finish uses them), then the
  // column-normalised previous basis, or (each_qr) the Householder QR of the previous one
  wf_colnorms(s, s.b, n, r);
  __shared__ float prev_scale[MET_MAX_R];
  if (t < r) prev_scale[t] = s.colv[t];
  for (int e = t; e < n * r; e += WF_THREADS) {
    const int i = e / r, c = e - i * r;
    if (ortho == ORTHO_EACH_QR) {
      s.w[i * LDB + c] = s.b[i * LDB + c];
    } else {
      s.b[i * LDB + c] /= s.colv[c];
    }
  }
  __syncthreads();
  if (ortho == ORTHO_EACH_QR) wf_qr(s, n, r);
  __shared__ float diag_vals[MET_MAX_R];
  for (int it = 0; it < power_iters; ++it) {
    wf_apply(s, n, r);  // w = m b
    if (ritz == RITZ_DIAGONAL && it == power_iters - 1) {
      for (int col = wv; col < r; col += WF_THREADS / 64) {
        float acc = 0.0f;
        if (lane < n) acc += s.b[lane * LDB + col] * s.w[lane * LDB + col];
        if (lane + 64 < n) acc += s.b[(lane + 64) * LDB + col] * s.w[(lane + 64) * LDB + col];
        const float dsum = wave_sum(acc);
        if (lane == 0) diag_vals[col] = dsum;
      }
      __syncthreads();
    }
    if (ortho == ORTHO_EACH_QR) {
      wf_qr(s, n, r);
    } else if (ortho == ORTHO_FINAL_CQR || ortho == ORTHO_FINAL_QR) {
      // unorthogonalised power step: columns rescaled to unit norm
      wf_colnorms(s, s.w, n, r);
      for (int e = t; e < n * r; e += WF_THREADS) {
        const int i = e / r, c = e - i * r;
        s.b[i * LDB + c] = s.w[i * LDB + c] / s.colv[c];
      }
      __syncthreads();
    } else {
      failed |= wf_cholesky_qr(s, s.w, n, r, cqr_ridge);
      if (ortho == ORTHO_EACH_CQR2 && it == power_iters - 1) {
        // the corrective pass: same calibrated ridge floor (operator_kmeans.py:380-392)
        for (int e = t; e < n * r; e += WF_THREADS) {
          const int i = e / r, c = e - i * r;
          s.w[i * LDB + c] = s.b[i * LDB + c];
        }
        __syncthreads();
        failed |= wf_cholesky_qr(s, s.w, n, r, fmaxf(cqr_ridge, 1e-5f));
      }
    }
  }
  if (ortho == ORTHO_FINAL_CQR || ortho == ORTHO_FINAL_QR) {
    for (int e = t; e < n * r; e += WF_THREADS) {
      const int i = e / r, c = e - i * r;
      s.w[i * LDB + c] = s.b[i * LDB + c];
    }
    __syncthreads();
    if (ortho == ORTHO_FINAL_QR) {
      wf_qr(s, n, r);
    } else {
      failed |= wf_cholesky_qr(s, s.w, n, r, 1e-6f);
    }
  }
  if (ritz == RITZ_FULL) {
    // Rayleigh matrix R = b^T (m b), symmetrised, the basis and the failure flag to the
    // workspace; the reduced eigh and the factor follow in their own launches
    wf_apply(s, n, r);
    wf_gram(s, s.b, s.w, n, r, true);
    __shared__ int32_t ray_bad;
    if (t == 0) ray_bad = 0;
    __syncthreads();
    for (int e = t; e < r * r; e += WF_THREADS) {
      if (!(fabsf(s.g[(e / r) * LDB + (e % r)]) < __builtin_huge_valf())) ray_bad = 1;
    }
    __syncthreads();
    float* bo = full_basis + h * n * r;
    float* ro = full_ray + h * r * r;
    for (int e = t; e < n * r; e += WF_THREADS) bo[e] = s.b[(e / r) * LDB + (e % r)];
    for (int e = t; e < r * r; e += WF_THREADS) {
      const int p = e / r, q = e - p * r;
      ro[e] = ray_bad ? (p == q ? static_cast<float>(p + 1) : 0.0f) : s.g[p * LDB + q];
    }
    if (t == 0) full_flag[h] = failed ? 1 : 0;
    return;
  }
  // finish: the factor goes to w, the basis stays in b
  if (ritz == RITZ_PREVIOUS_SCALE || ritz == RITZ_DIAGONAL) {
    if (t == 0) {
      if (ritz == RITZ_DIAGONAL) {
        float sum = 0.0f;
        for (int c = 0; c < r; ++c) sum += fmaxf(diag_vals[c], 0.0f);
        const float norm = fmaxf(sum / static_cast<float>(r), 1e-12f);
        for (int c = 0; c < r; ++c) s.colv[c] = sqrtf(fmaxf(diag_vals[c], 0.0f) / norm);
      } else {
        for (int c = 0; c < r; ++c) s.colv[c] = prev_scale[c];
      }
    }
    __syncthreads();
    for (int e = t; e < n * r; e += WF_THREADS) {
      const int i = e / r, c = e - i * r;
      s.w[i * LDB + c] = s.b[i * LDB + c] * s.colv[c];
    }
    __syncthreads();
  } else {
    // Rayleigh matrix R = b^T (m b), symmetrised; normalizer = max(mean diag R, 1e-12);
    // L = chol(R + normalizer ridge I), else chol(R + normalizer max(1e-2, ridge) I), else I
    // with the head marked failed (operator_kmeans.py:154-216, :442-458)
    wf_apply(s, n, r);
    wf_gram(s, s.b, s.w, n, r, true);
    if (t == 0) {
      float tr = 0.0f;
      for (int c = 0; c < r; ++c) tr += s.g[c * LDB + c];
      s.scal[1] = fmaxf(tr / static_cast<float>(r), 1e-12f);
    }
    __syncthreads();
    // R is kept in w (m b is dead) for the fallback factorisation; the chosen factor goes
    // to the metric region, which is no longer needed
    for (int e = t; e < r * r; e += WF_THREADS) {
      const int p = e / r, q = e - p * r;
      s.w[p * LDB + q] = s.g[p * LDB + q];
    }
    __syncthreads();
    const float normalizer = s.scal[1];
    bool ok = true;
    float* l_primary = s.m;  // [r][r]
    {
      ok = wf_cholesky(s, s.w, r, normalizer * rayleigh_ridge);
      for (int e = t; e < r * r; e += WF_THREADS) l_primary[e] = s.g[(e / r) * LDB + (e % r)];
      __syncthreads();
    }
    if (!ok) {
      ok = wf_cholesky(s, s.w, r, normalizer * fmaxf(1e-2f, rayleigh_ridge));
      if (ok) {
        for (int e = t; e < r * r; e += WF_THREADS) l_primary[e] = s.g[(e / r) * LDB + (e % r)];
      } else {
        for (int e = t; e < r * r; e += WF_THREADS) l_primary[e] = (e / r == e % r) ? 1.0f : 0.0f;
        failed = true;
      }
      __syncthreads();
    }
    // factor = b L / sqrt(normalizer), L lower (entries above the diagonal are zero)
    const float inv = 1.0f / sqrtf(normalizer);
    for (int e = t; e < n * r; e += WF_THREADS) {
      const int i = e / r, c = e - i * r;
      float acc = 0.0f;
      for (int k = c; k < r; ++k) acc = __builtin_fmaf(s.b[i * LDB + k], l_primary[k * r + c], acc);
      s.w[i * LDB + c] = acc * inv;
    }
    __syncthreads();
  }
  // recovery: a failed factorisation or a non-finite factor or basis keeps the previous ones
  __shared__ int32_t nonfinite;
  if (t == 0) nonfinite = 0;
  __syncthreads();
  for (int e = t; e < n * r; e += WF_THREADS) {
    const int i = e / r, c = e - i * r;
    const float fv = s.w[i * LDB + c], bv = s.b[i * LDB + c];
    if (!(fabsf(fv) < __builtin_huge_valf()) || !(fabsf(bv) < __builtin_huge_valf())) nonfinite = 1;
  }
  __syncthreads();
  const bool rec = failed || nonfinite != 0;
  const bool keep_prev = rec && pf != nullptr;
  float* fo = factor + h * n * r;
  float* so = state + h * n * r;
  for (int e = t; e < n * r; e += WF_THREADS) {
    const int i = e / r, c = e - i * r;
    fo[e] = keep_prev ? pf[e] : s.w[i * LDB + c];
    so[e] = keep_prev ? ps[e] : s.b[i * LDB + c];
  }
  if (t == 0 && recovered != nullptr) recovered[h] = rec ? 1 : 0;
}

// The full Rayleigh-Ritz finish (operator_kmeans.py:460-466) for one head per workgroup:
// factor = basis . U . diag(sqrt(max(lambda, 0) / max(mean max(lambda, 0), 1e-12))) with U,
// lambda the eigenpairs of the Rayleigh matrix in ascending order; then the recovery of
// warm_factor_kernel (a failed Cholesky-QR, or a factor or basis that is not finite).
__global__ __launch_bounds__(256) void warm_full_finish_kernel(
    const float* __restrict__ basis, const float* __restrict__ vecs, const float* __restrict__ vals,
    const int32_t* __restrict__ flag, const float* __restrict__ prev_state, const float* __restrict__ prev_factor,
    int32_t n, int32_t r, float* __restrict__ factor, float* __restrict__ state, uint8_t* __restrict__ recovered) {
  __shared__ float u[MET_MAX_R * (MET_MAX_R + 1)];
  __shared__ float f[MET_MAX_D * MET_MAX_R];
  __shared__ float scale[MET_MAX_R];
  __shared__ int32_t nonfinite;
  const int t = threadIdx.x;
  const int64_t h = blockIdx.x;
  const float* bh_ = basis + h * n * r;
  const float* uh = vecs + h * r * r;
  if (t == 0) {
    const float* lh = vals + h * r;
    float sum = 0.0f;
    for (int c = 0; c < r; ++c) sum += fmaxf(lh[c], 0.0f);
    const float norm = fmaxf(sum / static_cast<float>(r), 1e-12f);
    for (int c = 0; c < r; ++c) scale[c] = sqrtf(fmaxf(lh[c], 0.0f) / norm);
    nonfinite = 0;
  }
  for (int e = t; e < r * r; e += 256) u[(e / r) * (MET_MAX_R + 1) + (e % r)] = uh[e];
  __syncthreads();
  for (int e = t; e < n * r; e += 256) {
    const int i = e / r, c = e - i * r;
    float acc = 0.0f;
    for (int k = 0; k < r; ++k) acc = __builtin_fmaf(bh_[i * r + k], u[k * (MET_MAX_R + 1) + c], acc);
    const float fv = acc * scale[c];
    f[e] = fv;
    if (!(fabsf(fv) < __builtin_huge_valf()) || !(fabsf(bh_[e]) < __builtin_huge_valf())) nonfinite = 1;
  }
  __syncthreads();
  const bool rec = flag[h] != 0 || nonfinite != 0;
  const bool keep_prev = rec && prev_factor != nullptr;
  for (int e = t; e < n * r; e += 256) {
    factor[h * n * r + e] = keep_prev ? prev_factor[h * n * r + e] : f[e];
    state[h * n * r + e] = keep_prev ? prev_state[h * n * r + e] : bh_[e];
  }
  if (t == 0 && recovered != nullptr) recovered[h] = rec ? 1 : 0;
}

// ---------------------------------------------------------------- row projections
// one wave per (head, row): lane c < r computes sum_j x[row][j] F[j][c] in index order
// (fmaf), then divides by div[h] (nullable) and, with row_rms, by
// max(sqrt(mean_c p_c^2), eps).
// precision 0: fp32 operands; 1: both rounded to TF32; 2: both rounded to bf16 (nearest even).
// out[row][out_col + c] (rows of out_ld floats) = weight * (p_c / div[h]).
__global__ __launch_bounds__(256) void project_rows_kernel(const float* __restrict__ x, const float* __restrict__ f,
                                                           const float* __restrict__ div, int64_t m, int32_t d,
                                                           int32_t r, int32_t precision, int32_t row_rms, float eps,
                                                           int32_t out_ld, int32_t out_col, float weight,
                                                           float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t h = blockIdx.y;
  if (row >= m) return;
  const float* xr = x + (h * m + row) * d;
  const float* fh = f + h * d * r;
  float acc = 0.0f;
  if (lane < r) {
    // the loads of 16 steps are issued before their multiply-adds, so the chain waits on
    // one memory latency per 16 steps instead of one per step
    constexpr int JB = 16;
    for (int j0 = 0; j0 < d; j0 += JB) {
      float xv[JB], fv[JB];
#pragma unroll
      for (int u = 0; u < JB; ++u) {
        const int j = min(j0 + u, d - 1);
        xv[u] = xr[j];
        fv[u] = fh[j * r + lane];
      }
#pragma unroll
      for (int u = 0; u < JB; ++u) {
        if (j0 + u < d) {
          float a = xv[u], b = fv[u];
          if (precision == 1) {
            a = tf32_rna(a);
            b = tf32_rna(b);
          } else if (precision == 2) {
            a = spr::bf16_to_f32(spr::f32_to_bf16(a));
            b = spr::bf16_to_f32(spr::f32_to_bf16(b));
          }
          acc = __builtin_fmaf(a, b, acc);
        }
      }
    }
    if (div != nullptr) acc = acc / div[h];
  }
  if (row_rms) {
    const float ms = wave_sum(lane < r ? acc * acc : 0.0f) / static_cast<float>(r);
    acc = acc / fmaxf(sqrtf(ms), eps);
  }
  if (lane < r) out[(h * m + row) * out_ld + out_col + lane] = weight == 1.0f ? acc : weight * acc;
}

}  // namespace

// x (dtype 0 bf16 / 2 fp32) [bh, n, d], d <= 128; rows int32 [count] (nullable: all n rows);
// sizes int32 [bh, n] (nullable; only with rows == NULL: rows with size <= 0 are skipped and
// not counted); center: subtract the used rows' mean; out fp32 [bh, d, d] =
// post_scale / max(used, 1) * sum (x - mean)(x - mean)^T.
extern "C" int spr_role_metric(const void* x, int32_t dtype, int64_t bh, int64_t n, int32_t d, const int32_t* rows,
                               int32_t count, const int32_t* sizes, int32_t center, float post_scale, float* out,
                               hipStream_t stream) {
  SPR_REQUIRE(bh >= 0 && n >= 0 && d >= 1 && d <= MET_MAX_D, "spr_role_metric: bad size (d=%d)", d);
  SPR_REQUIRE(dtype == 0 || dtype == 2, "spr_role_metric: dtype must be 0 (bf16) or 2 (fp32)");
  SPR_REQUIRE(rows == nullptr || sizes == nullptr, "spr_role_metric: rows and sizes are exclusive");
  SPR_REQUIRE(rows == nullptr || count >= 0, "spr_role_metric: negative count");
  SPR_REQUIRE(bh <= 65535, "spr_role_metric: too many heads");
  if (bh == 0) return SPR_OK;
  SPR_REQUIRE(x && out, "spr_role_metric: null pointer");
  const int tiles = (d + 31) / 32;
  dim3 grid(static_cast<uint32_t>(bh), static_cast<uint32_t>(tiles * tiles));
  if (dtype == 0) {
    role_metric_kernel<uint16_t><<<grid, 256, 0, stream>>>(static_cast<const uint16_t*>(x), n, d, rows, count, sizes,
                                                            center, post_scale, out);
  } else {
    role_metric_kernel<float><<<grid, 256, 0, stream>>>(static_cast<const float*>(x), n, d, rows, count, sizes, center,
                                                         post_scale, out);
  }
  SPR_LAUNCHED("role_metric_kernel");
  return SPR_OK;
}

extern "C" size_t spr_metric_factor_workspace(int64_t bh, int32_t rank) {
  return static_cast<size_t>(bh > 0 ? bh : 0) * static_cast<size_t>(rank > 0 ? rank : 0) * sizeof(float);
}

// metric fp32 [bh, n, n] -> factor fp32 [bh, n, rank]: the top-rank eigenvectors of
// 0.5 (M + M^T) (ascending eigenvalue order), column c scaled by
// sqrt(max(lambda_c, 0) / max(mean max(lambda, 0), 1e-12)); workspace: the eigenvalues.
extern "C" int spr_metric_factor(const float* metric, int64_t bh, int32_t n, int32_t rank, float* factor,
                                 void* workspace, size_t workspace_bytes, hipStream_t stream) {
  SPR_REQUIRE(rank >= 1 && rank <= MET_MAX_R && rank <= n, "spr_metric_factor: rank %d outside [1, min(64, n)]",
              rank);
  if (bh <= 0) return SPR_OK;
  if (workspace_bytes < spr_metric_factor_workspace(bh, rank)) {
    spr_set_error("spr_metric_factor: workspace %zu < %zu bytes", workspace_bytes,
                  spr_metric_factor_workspace(bh, rank));
    return SPR_EWORKSPACE;
  }
  float* vals = static_cast<float*>(workspace);
  const int st = spr_sym_top_eig(metric, bh, n, rank, 1, factor, vals, stream);
  if (st != SPR_OK) return st;
  factor_scale_kernel<<<dim3(static_cast<uint32_t>(bh)), 256, 0, stream>>>(factor, vals, n, rank);
  SPR_LAUNCHED("factor_scale_kernel");
  return SPR_OK;
}

// Workspace of spr_warm_metric_factor_ex: the full finish (ritz 3) keeps, per head, the
// basis [n][rank], the Rayleigh matrix and its eigenvectors [rank][rank], the eigenvalues
// [rank] and a flag; the other finishes need none.
extern "C" size_t spr_warm_metric_factor_workspace(int64_t bh, int32_t n, int32_t rank, int32_t ritz) {
  if (ritz != RITZ_FULL || bh <= 0 || n <= 0 || rank <= 0) return 0;
  const size_t per = static_cast<size_t>(n) * rank + 2 * static_cast<size_t>(rank) * rank + rank + 1;
  return static_cast<size_t>(bh) * per * sizeof(float);
}

// warm_subspace_metric_factor + the per-head recovery of N8V6Core._updated_factor.
// ortho: 0 each_cholesky_qr, 1 each_cholesky_qr2, 2 cholesky_qr (once, after the
// normalised power steps), 3 each_qr, 4 final_qr (Householder QR); ritz: 0 rayleigh_cholesky,
// 1 diagonal, 2 previous_scale, 3 full (three launches: the subspace kernel, spr_sym_top_eig
// on the Rayleigh matrices, the finish).
extern "C" int spr_warm_metric_factor_ex(const float* metric, const float* prev_state, const float* prev_factor,
                                         int64_t bh, int32_t n, int32_t rank, int32_t power_iters, int32_t ortho,
                                         int32_t ritz, float rayleigh_ridge, float cqr_ridge, float* factor,
                                         float* state, uint8_t* recovered, void* workspace, size_t workspace_bytes,
                                         hipStream_t stream) {
  SPR_REQUIRE(bh >= 0 && n >= 1 && n <= MET_MAX_D, "spr_warm_metric_factor: n=%d outside [1, %d]", n, MET_MAX_D);
  SPR_REQUIRE(rank >= 1 && rank <= MET_MAX_R && rank <= n, "spr_warm_metric_factor: rank %d outside [1, 64]", rank);
  SPR_REQUIRE(power_iters >= 1, "spr_warm_metric_factor: power_iters must be positive");
  SPR_REQUIRE(ortho >= 0 && ortho <= 4 && ritz >= 0 && ritz <= 3, "spr_warm_metric_factor: bad mode");
  SPR_REQUIRE(rayleigh_ridge > 0.0f && cqr_ridge > 0.0f, "spr_warm_metric_factor: ridges must be positive");
  SPR_REQUIRE(bh <= 65535, "spr_warm_metric_factor: too many heads");
  if (bh == 0) return SPR_OK;
  SPR_REQUIRE(metric && prev_state && factor && state, "spr_warm_metric_factor: null pointer");
  const size_t need = spr_warm_metric_factor_workspace(bh, n, rank, ritz);
  if (workspace_bytes < need || (need > 0 && workspace == nullptr)) {
    spr_set_error("spr_warm_metric_factor: the full finish needs a workspace of %zu bytes (got %zu)", need,
                  workspace_bytes);
    return SPR_EWORKSPACE;
  }
  float* fb = nullptr;
  float* fr = nullptr;
  float* fv = nullptr;
  float* fl = nullptr;
  int32_t* ff = nullptr;
  if (ritz == RITZ_FULL) {
    fb = static_cast<float*>(workspace);
    fr = fb + bh * n * rank;
    fv = fr + bh * rank * rank;
    fl = fv + bh * rank * rank;
    ff = reinterpret_cast<int32_t*>(fl + bh * rank);
  }
  warm_factor_kernel<<<dim3(static_cast<uint32_t>(bh)), WF_THREADS, 0, stream>>>(
      metric, prev_state, prev_factor, n, rank, power_iters, ortho, ritz, rayleigh_ridge, cqr_ridge, factor, state,
      recovered, fb, fr, ff);
  SPR_LAUNCHED("warm_factor_kernel");
  if (ritz == RITZ_FULL) {
    const int st = spr_sym_top_eig(fr, bh, rank, rank, 1, fv, fl, stream);
    if (st != SPR_OK) return st;
    warm_full_finish_kernel<<<dim3(static_cast<uint32_t>(bh)), 256, 0, stream>>>(
        fb, fv, fl, ff, prev_state, prev_factor, n, rank, factor, state, recovered);
    SPR_LAUNCHED("warm_full_finish_kernel");
  }
  return SPR_OK;
}

extern "C" int spr_warm_metric_factor(const float* metric, const float* prev_state, const float* prev_factor,
                                      int64_t bh, int32_t n, int32_t rank, int32_t power_iters, int32_t ortho,
                                      int32_t ritz, float rayleigh_ridge, float cqr_ridge, float* factor, float* state,
                                      uint8_t* recovered, hipStream_t stream) {
  return spr_warm_metric_factor_ex(metric, prev_state, prev_factor, bh, n, rank, power_iters, ortho, ritz,
                                   rayleigh_ridge, cqr_ridge, factor, state, recovered, nullptr, 0, stream);
}

// out fp32 [bh, m, r] = (x [bh, m, d] . factor [bh, d, r]) / div[h] (div nullable), with
// tf32 = 1 both operands rounded to TF32 first; row_rms = 1 divides each row by
// max(sqrt(mean p^2), eps).  d <= 128, r <= 64.
extern "C" int spr_project_rows_ex(const float* x, const float* factor, const float* div, int64_t bh, int64_t m,
                                   int32_t d, int32_t r, int32_t precision, int32_t row_rms, float eps, float weight,
                                   float* out, int32_t out_ld, int32_t out_col, hipStream_t stream) {
  SPR_REQUIRE(bh >= 0 && m >= 0 && d >= 1 && d <= MET_MAX_D && r >= 1 && r <= 64, "spr_project_rows: bad size");
  SPR_REQUIRE(bh <= 65535, "spr_project_rows: too many heads");
  SPR_REQUIRE(precision >= 0 && precision <= 2, "spr_project_rows: precision must be 0, 1 or 2 (got %d)", precision);
  SPR_REQUIRE(out_col >= 0 && out_ld >= out_col + r, "spr_project_rows: columns %d + %d exceed rows of %d", out_col,
              r, out_ld);
  if (bh == 0 || m == 0) return SPR_OK;
  SPR_REQUIRE(x && factor && out, "spr_project_rows: null pointer");
  dim3 grid(static_cast<uint32_t>(spr::ceil_div(m, 4)), static_cast<uint32_t>(bh));
  project_rows_kernel<<<grid, 256, 0, stream>>>(x, factor, div, m, d, r, precision, row_rms, eps, out_ld, out_col,
                                                weight, out);
  SPR_LAUNCHED("project_rows_kernel");
  return SPR_OK;
}

extern "C" int spr_project_rows(const float* x, const float* factor, const float* div, int64_t bh, int64_t m,
                                int32_t d, int32_t r, int32_t tf32, int32_t row_rms, float eps, float* out,
                                hipStream_t stream) {
  return spr_project_rows_ex(x, factor, div, bh, m, d, r, tf32 ? 1 : 0, row_rms, eps, 1.0f, out, r, 0, stream);
}
