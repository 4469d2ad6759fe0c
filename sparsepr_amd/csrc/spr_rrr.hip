// Weighted ridge reduced-rank residual fit.
//
// Replaces _fit_reduced_rank_residual_fp32 (src/sparsepr/models/cosmos3/residual_repair.py:317-465)
// for every configuration it accepts with M, D <= 128, P <= 128 (or, in the dual form M < P,
// up to 256 while 64 ceil(P / 64) (M | 1) <= 16512) and rank <= 64:
//   weighted (or, without weights, plain mean and unbiased std) standardisation (:364-384);
//   the ridge solve in primal form for M >= P (:424-434) and in dual form for M < P (:386-423);
//   the output basis of the raw residual or of the fitted values (:435-462): the
//   top-r eigenvectors of the weighted output gram, which span the same subspace as the
//   "skinny" row-gram / SVD routes (:468-506);
//   left = weight basis (primal) or x_w^T dual basis (dual) (:463-464).
// recover_nonfinite_rrr_state (:509-587) is rrr_recover_kernel: a per-head finite test of the
// five state tensors and a select against the previous state (or a zero correction).
//
// Per head, in fp32:
//   w_sum = max(sum w, 1e-20); x_mean = sum w x / w_sum; x_scale = max(sqrt(sum w
//   (x - x_mean)^2 / w_sum), 1e-5) (no weights: w = 1, variance over m - 1);
//   y_mean = sum w y / w_sum; x_w = (x - x_mean) / x_scale * sqrt(w); y_w = (y - y_mean) * sqrt(w);
//   primal: G = x_w^T x_w + ridge I (p x p); dual: G = x_w x_w^T + ridge I (m x m);
//   raw basis: top-`rank` eigenvectors of B = y_w^T y_w (ascending eigenvalue order, as eigh);
//   fitted basis: of B = F^T F with F = x_w G^-1 x_w^T y_w (primal) or y_w - ridge G^-1 y_w (dual);
//   Z = y_w basis; left = G^-1 x_w^T Z (primal) or x_w^T G^-1 Z (dual).
//
// Launches, stream ordered (raw basis: four; fitted basis: seven):
//   rrr_stats_kernel   one workgroup per head: the weighted statistics.
//   rrr_gram_kernel    10 workgroups per matrix per head: one 32 x 32 lower tile of G or B
//                      each, mirrored, into the workspace.
//   rrr_factor_kernel  one or two workgroups per head:
//     eigen:   B is held in registers (thread t owns row t / 8, columns t % 8 + 8 q) and
//              reduced to tridiagonal form by Householder reflections (two barriers per
//              column); the top eigenvalues come from 64-way multisection on Sturm counts
//              (one wave per eigenvalue), their vectors from inverse iteration on the
//              tridiagonal matrix (pivoted LU, three steps, members of a cluster
//              orthogonalised against each other as they are computed), the reflections are
//              applied back, and a Cholesky-QR pass makes the basis orthonormal to rounding.
//     Cholesky: factor of G, register resident, one barrier per column, written over G.
//   rrr_fitted_kernel  (fitted basis) F into the workspace, then rrr_gram_kernel for B and
//                      the eigen part of rrr_factor_kernel.
//   rrr_solve_kernel   one workgroup per head: Z = y_w basis, then the substitutions
//                      (one wave per basis column, refined once against an fp64 residual)
//                      and the x_w products of the form in use.
#include "spr_common.h"

namespace {

constexpr int RRR_MAX = 128;  // M, P, D at most
constexpr int RRR_MAX_RANK = 16;   // basis columns per solve block (and the top-16 route's rank)
constexpr int RRR_MAX_FIT_RANK = 64;  // largest fitted rank
constexpr int RRR_THREADS = 1024;
constexpr int RRR_MAT = RRR_MAX * RRR_MAX;  // one workspace matrix (floats)
constexpr int RRR_LS = RRR_MAX + 1;         // padded LDS row: rows i and i + 1 start one bank apart

// ---- lane reductions (DPP within rows of 16 lanes, readlane across rows)
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_read(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
// Sum over the 8 lanes 8g .. 8g + 7 (every lane of the group gets the same value).
__device__ __forceinline__ float sum8(float v) {
  v += dpp_mov<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_mov<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp_mov<0x141>(v);  // row_half_mirror
  return v;
}
// Sum over the wave, uniform result.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_mov<0xB1>(v);
  v += dpp_mov<0x4E>(v);
  v += dpp_mov<0x124>(v);  // row_ror 4
  v += dpp_mov<0x128>(v);  // row_ror 8
  return (lane_read(v, 0) + lane_read(v, 16)) + (lane_read(v, 32) + lane_read(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_mov<0xB1>(v));
  v = fmaxf(v, dpp_mov<0x4E>(v));
  v = fmaxf(v, dpp_mov<0x124>(v));
  v = fmaxf(v, dpp_mov<0x128>(v));
  return fmaxf(fmaxf(lane_read(v, 0), lane_read(v, 16)), fmaxf(lane_read(v, 32), lane_read(v, 48)));
}
// LDS written by some lanes of a wave, then read by others of the same wave.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
// a[q] for a runtime q as an OR of masked bit patterns: a select chain over the
// array gets folded into one load from a selected address, which keeps the array
// on the stack.
__device__ __forceinline__ float pick16(const float (&a)[16], int q) {
  int v = 0;
#pragma unroll
  for (int u = 0; u < 16; ++u) v |= __float_as_int(a[u]) & -static_cast<int>(q == u);
  return __int_as_float(v);
}

// ---- statistics: one workgroup of 256 threads per head.  w == nullptr: unit weights,
// the variance over m - 1 (torch.std), NaN at m = 1 as there.
__device__ __forceinline__ float clamp_min_nan(float v, float lo) { return v != v ? v : fmaxf(v, lo); }

__global__ __launch_bounds__(256) void rrr_stats_kernel(const float* __restrict__ x, const float* __restrict__ y,
                                                        const float* __restrict__ w, int32_t m, int32_t p, int32_t d,
                                                        float* __restrict__ x_mean, float* __restrict__ x_scale,
                                                        float* __restrict__ y_mean) {
  const int t = threadIdx.x;
  const int64_t h = blockIdx.x;
  const float* xh = x + h * m * p;
  const float* yh = y + h * m * d;
  const float* wh = w != nullptr ? w + h * m : nullptr;
  float ws = static_cast<float>(m), var_div = static_cast<float>(m - 1);
  if (wh != nullptr) {
    ws = 0.0f;
    for (int r = 0; r < m; ++r) ws += wh[r];
    ws = fmaxf(ws, 1e-20f);
    var_div = ws;
  }
  for (int col = t; col < p + d; col += 256) {  // features, then outputs
    if (col < p) {
      float s = 0.0f;
#pragma unroll 8
      for (int r = 0; r < m; ++r) s += (wh != nullptr ? wh[r] : 1.0f) * xh[r * p + col];
      const float mean = s / ws;
      float v = 0.0f;
#pragma unroll 8
      for (int r = 0; r < m; ++r) {
        const float dv = xh[r * p + col] - mean;
        v += (wh != nullptr ? wh[r] : 1.0f) * (dv * dv);
      }
      x_mean[h * p + col] = mean;
      x_scale[h * p + col] = clamp_min_nan(sqrtf(v / var_div), 1e-5f);
    } else {
      const int c = col - p;
      float s = 0.0f;
#pragma unroll 8
      for (int r = 0; r < m; ++r) s += (wh != nullptr ? wh[r] : 1.0f) * yh[r * d + c];
      y_mean[h * d + c] = s / ws;
    }
  }
}

// Workspace per head: three 128 x 128 fp32 matrices.  Slot 0: G, then its Cholesky
// factor; slot 1: B; slot 2: F (fitted basis only).
constexpr int RRR_SLOTS = 3;
__device__ __forceinline__ float* ws_slot(float* ws, int64_t h, int slot) {
  return ws + (h * RRR_SLOTS + slot) * RRR_MAT;
}

// ---- Gram matrices, 32 x 32 lower tiles (10 per 128 x 128 matrix), mirrored; zero outside
// the matrix.  The element (r, c) of the matrix whose Gram is summed over r:
//   GRAM_PRIMAL   x_w[r][c]   (r < m, c < p)  -> G = x_w^T x_w + ridge I, slot 0
//   GRAM_DUAL     x_w[c][r]   (r < p, c < m)  -> G = x_w x_w^T + ridge I, slot 0
//   GRAM_RESIDUAL y_w[r][c]   (r < m, c < d)  -> B = y_w^T y_w, slot 1
//   GRAM_PLAIN    a[r][c]     (r < m, c < d)  -> B = a^T a, slot 1 (row stride a_ld, head stride a_hs)
// blockIdx.y / 10 picks kind0 or kind1, blockIdx.y % 10 the tile.
enum GramKind : int32_t { GRAM_PRIMAL = 0, GRAM_DUAL = 1, GRAM_RESIDUAL = 2, GRAM_PLAIN = 3 };

__global__ __launch_bounds__(256) void rrr_gram_kernel(const float* __restrict__ x, const float* __restrict__ y,
                                                       const float* __restrict__ w, int32_t m, int32_t p, int32_t d,
                                                       float ridge, const float* __restrict__ x_mean,
                                                       const float* __restrict__ x_scale,
                                                       const float* __restrict__ y_mean, const float* __restrict__ a,
                                                       int64_t a_hs, int32_t a_ld, int32_t kind0, int32_t kind1,
                                                       float* __restrict__ ws) {
  __shared__ float pa[RRR_MAX][33];
  __shared__ float pb[RRR_MAX][33];
  const int t = threadIdx.x;
  const int64_t h = blockIdx.x;
  const int kind = blockIdx.y < 10 ? kind0 : kind1;
  const int lt = blockIdx.y % 10;
  const int ti = lt >= 6 ? 3 : (lt >= 3 ? 2 : (lt >= 1 ? 1 : 0));
  const int tj = lt - ti * (ti + 1) / 2;
  const int rows = kind == GRAM_DUAL ? p : m;
  const int cols = kind == GRAM_PRIMAL ? p : (kind == GRAM_DUAL ? m : d);
  const float* xh = x + h * m * p;
  const float* yh = y + h * m * d;
  const float* wh = w != nullptr ? w + h * m : nullptr;
  const float* xm = x_mean + h * p;
  const float* xs = x_scale + h * p;
  const float* ym = y_mean + h * d;
  const float* ah = a != nullptr ? a + h * a_hs : nullptr;
  auto elem = [&](int r, int cc) -> float {
    switch (kind) {
      case GRAM_PRIMAL:
        return (xh[r * p + cc] - xm[cc]) / xs[cc] * (wh != nullptr ? sqrtf(wh[r]) : 1.0f);
      case GRAM_DUAL:
        return (xh[cc * p + r] - xm[r]) / xs[r] * (wh != nullptr ? sqrtf(wh[cc]) : 1.0f);
      case GRAM_RESIDUAL:
        return (yh[r * d + cc] - ym[cc]) * (wh != nullptr ? sqrtf(wh[r]) : 1.0f);
      default:
        return ah[static_cast<int64_t>(r) * a_ld + cc];
    }
  };
  const int ta = t >> 4, tb = t & 15;
  float s00 = 0.0f, s01 = 0.0f, s10 = 0.0f, s11 = 0.0f;
  for (int r0 = 0; r0 < rows; r0 += RRR_MAX) {  // the summed rows, 128 at a time (dual: p <= 256)
    if (r0 > 0) __syncthreads();
    for (int e = t; e < RRR_MAX * 32; e += 256) {
      const int r = e >> 5, cc = e & 31;
      const int ci = 32 * ti + cc, cj = 32 * tj + cc;
      pa[r][cc] = (r0 + r < rows && ci < cols) ? elem(r0 + r, ci) : 0.0f;
      pb[r][cc] = (r0 + r < rows && cj < cols) ? elem(r0 + r, cj) : 0.0f;
    }
    __syncthreads();
    const int nr = min(rows - r0, RRR_MAX);
    for (int r = 0; r < nr; ++r) {
      const float u0 = pa[r][2 * ta], u1 = pa[r][2 * ta + 1];
      const float v0 = pb[r][2 * tb], v1 = pb[r][2 * tb + 1];
      s00 += u0 * v0;
      s01 += u0 * v1;
      s10 += u1 * v0;
      s11 += u1 * v1;
    }
  }
  const bool is_g = kind == GRAM_PRIMAL || kind == GRAM_DUAL;
  float* out = ws_slot(ws, h, is_g ? 0 : 1);
  const float acc[2][2] = {{s00, s01}, {s10, s11}};
#pragma unroll
  for (int u = 0; u < 2; ++u) {
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      const int gi = 32 * ti + 2 * ta + u, gj = 32 * tj + 2 * tb + v;
      const float val = acc[u][v] + ((is_g && gi == gj && gi < cols) ? ridge : 0.0f);
      out[gi * RRR_MAX + gj] = val;
      if (ti != tj) out[gj * RRR_MAX + gi] = val;
    }
  }
}

// ---- eigen path LDS layout (floats).  Householder columns and the p vectors are
// stored permuted, j -> (j % 8) * 17 + j / 8, so that lane c's sixteen values
// (j = c + 8 q) are consecutive and the eight lane groups start in distinct banks.
constexpr int HV_STRIDE = 136;
__device__ __forceinline__ int hv_perm(int j) { return (j & 7) * 17 + (j >> 3); }
// LDS layout (floats) of the eigen solver for at most MAXR vectors.  Regions that are
// dead after a phase are reused by a later one: the LU factors hold the back-transformed
// vectors, the tridiagonal eigenvectors the Gram matrix and its factor, the Householder
// columns the final basis.
template <int MAXR>
struct EigLayout {
  static_assert(MAXR >= 16 && MAXR <= 64 && MAXR % 16 == 0, "MAXR in {16, 32, 48, 64}");
  static constexpr int HV = 0;                        // [128][136] Householder columns (raw, permuted)
  static constexpr int DD = HV + RRR_MAX * HV_STRIDE;  // tridiagonal diagonal
  static constexpr int EE = DD + RRR_MAX;             // off-diagonal
  static constexpr int TAU = EE + RRR_MAX;            // reflector tau
  static constexpr int SCL = TAU + RRR_MAX;           // reflector scale: v_j = raw_j * scl (j > k + 1)
  static constexpr int PB = SCL + RRR_MAX;            // [2][136] p = tau A v (permuted)
  static constexpr int PART = PB + 2 * HV_STRIDE;     // [2][16] per-wave p . v
  static constexpr int LAM = PART + 32;               // [MAXR] eigenvalues, descending
  static constexpr int LU = LAM + MAXR;               // [5][128][16] LU of T - lambda_s I, 16 vectors at a time
  static constexpr int X = LU + 5 * RRR_MAX * 16;     // [128][XS] eigenvectors of T
  static constexpr int XS = MAXR + 1;                 // X row stride: column reads hit distinct banks
  static constexpr int FLOATS = X + RRR_MAX * XS;
  static constexpr int VB = LU;                       // [MAXR][128] eigenvectors of B (after inverse iteration)
  static constexpr int S = X;                         // [MAXR][MAXR] Gram, then R (after back-transformation)
  static constexpr int Q = HV;                        // [128][MAXR] orthonormal basis
  static_assert(MAXR * RRR_MAX <= 5 * RRR_MAX * 16, "VB must fit in the LU region");
};

// Top-`rank` eigenpairs of the symmetric n x n matrix bmat (row stride ld; entries
// outside n x n are treated as zero).  symmetrize: use 0.5 (A + A^T).  basis [n][rank]
// gets the eigenvectors in ascending eigenvalue order (as torch.linalg.eigh's last
// `rank` columns); vals [rank] (nullable) their Rayleigh quotients, ascending.
template <int MAXR>
__device__ __forceinline__ void rrr_eigen(float* sm, const float* __restrict__ bmat, int ld, int n, int rank, bool symmetrize,
                          float* __restrict__ basis, float* __restrict__ vals) {
  using L = EigLayout<MAXR>;
  const int t = threadIdx.x, i = t >> 3, c = t & 7, lane = t & 63, wv = t >> 6;
  float* hv = sm + L::HV;
  float* dd = sm + L::DD;
  float* ee = sm + L::EE;
  float* tau = sm + L::TAU;
  float* scl = sm + L::SCL;

  float a[16];
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int j = c + 8 * q;
    float v = 0.0f;
    if (i < n && j < n) {
      v = bmat[i * ld + j];
      if (symmetrize) v = 0.5f * (v + bmat[j * ld + i]);
    }
    a[q] = v;
  }
  for (int e = t; e < L::PART + 32; e += RRR_THREADS) sm[e] = 0.0f;  // columns, p buffers, partials
  __syncthreads();
  // ---- Householder tridiagonalisation (lower), A <- H A H column by column.
  // Columns go in blocks of eight: during block kb, a[q] holds column c + 8 (q + kb),
  // so the column being reduced is a[0] of the lanes with c = k % 8 (the array shifts
  // down one register per block).  Columns <= k read zeros from the column and p
  // buffers, so their updates are no-ops without masks; groups of four registers that
  // are past the end are skipped, and so are waves whose rows are all <= k.
  int kb = 0;
  for (; 8 * kb + 2 < n; ++kb) {
    if (kb > 0) {
#pragma unroll
      for (int q = 0; q < 15; ++q) a[q] = a[q + 1];
      a[15] = 0.0f;
    }
    const int nq = 16 - kb;  // registers still in the matrix
    for (int kc = 0; kc < 8; ++kc) {
      const int k = 8 * kb + kc;
      if (k + 2 >= n) break;
      if (c == kc) {
        hv[k * HV_STRIDE + hv_perm(i)] = i > k ? a[0] : 0.0f;  // zero on and above the diagonal
        if (i == k) dd[k] = a[0];
      }
      __syncthreads();
      const float* col = hv + k * HV_STRIDE;
      const float c0 = col[hv_perm(lane)], c1 = col[hv_perm(lane + 64)];
      const float x0 = lane > k + 1 ? c0 : 0.0f;
      const float x1 = lane + 64 > k + 1 ? c1 : 0.0f;
      const float sigma = wave_sum(x0 * x0 + x1 * x1);
      const float alpha = col[hv_perm(k + 1)];
      float tk = 0.0f, sk = 0.0f, beta = alpha;
      if (sigma != 0.0f) {
        const float nrm = __builtin_amdgcn_sqrtf(alpha * alpha + sigma);
        beta = alpha >= 0.0f ? -nrm : nrm;
        tk = (beta - alpha) * __builtin_amdgcn_rcpf(beta);
        sk = __builtin_amdgcn_rcpf(alpha - beta);
      }
      if (t == 0) {
        ee[k] = beta;
        tau[k] = tk;
        scl[k] = sk;
      }
      const bool live = 8 * wv + 7 > k;  // this wave holds rows below k
      float* pb = sm + L::PB + (k & 1) * HV_STRIDE;
      float* pt = sm + L::PART + (k & 1) * 16;
      float v[16];
      float pr = 0.0f, vi = 0.0f;
      if (live) {
        const float* cq = col + c * 17 + kb;
        float cv[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) cv[q] = cq[q];
        // v_{k+1} = 1 sits in register 0 of lane kc + 1, or register 1 of lane 0 (kc = 7)
        const bool one0 = c == kc + 1, one1 = kc == 7 && c == 0;
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          if (4 * g4 < nq) {
            asm volatile("" ::: "memory");
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const int q = 4 * g4 + u;
              const float vq = cv[q] * sk;
              v[q] = q == 0 ? (one0 ? 1.0f : vq) : (q == 1 ? (one1 ? 1.0f : vq) : vq);
              pr = fmaf(a[q], v[q], pr);
            }
          }
        }
        pr = sum8(pr) * tk;
        vi = i == k + 1 ? 1.0f : col[hv_perm(i)] * sk;
        const float kp = wave_sum((c == 0 && i > k) ? pr * vi : 0.0f);
        if (c == 0) pb[hv_perm(i)] = i > k ? pr : 0.0f;
        if (lane == 0) pt[wv] = kp;
      } else {
        if (c == 0) pb[hv_perm(i)] = 0.0f;
        if (lane == 0) pt[wv] = 0.0f;
      }
      __syncthreads();
      if (live) {
        const float4* p4 = reinterpret_cast<const float4*>(pt);
        const float4 s0 = p4[0], s1 = p4[1], s2 = p4[2], s3 = p4[3];
        const float ks = ((s0.x + s0.y) + (s0.z + s0.w)) + ((s1.x + s1.y) + (s1.z + s1.w)) +
                         (((s2.x + s2.y) + (s2.z + s2.w)) + ((s3.x + s3.y) + (s3.z + s3.w)));
        const float kk = 0.5f * tk * ks;
        const float wi = i > k ? pr - kk * vi : 0.0f;
        const float* pq = pb + c * 17 + kb;
        float pv[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) pv[q] = pq[q];
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          if (4 * g4 < nq) {
            asm volatile("" ::: "memory");
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const int q = 4 * g4 + u;
              const float wj = fmaf(-kk, v[q], pv[q]);
              a[q] = fmaf(-vi, wj, fmaf(-wi, v[q], a[q]));
            }
          }
        }
      }
    }
  }
  // trailing 2 x 2 (or 1 x 1) block: column j sits in register j / 8 - (kb - 1)
  {
    const int sh = kb > 0 ? kb - 1 : 0;
    if (n >= 2) {
      if (i == n - 2 && c == ((n - 2) & 7)) dd[n - 2] = pick16(a, ((n - 2) >> 3) - sh);
      if (i == n - 1 && c == ((n - 1) & 7)) dd[n - 1] = pick16(a, ((n - 1) >> 3) - sh);
      if (i == n - 1 && c == ((n - 2) & 7)) ee[n - 2] = pick16(a, ((n - 2) >> 3) - sh);
    } else if (t == 0) {
      dd[0] = a[0];
    }
  }
  __syncthreads();

  // ---- bounds of the spectrum (every wave, lanes over the rows, same values everywhere)
  float lo, hi, tnorm, e2max;
  {
    float lo_l = 3.4e38f, hi_l = -3.4e38f, tn_l = 0.0f, e2_l = 0.0f;
    for (int j = lane; j < n; j += 64) {
      const float el = j > 0 ? fabsf(ee[j - 1]) : 0.0f;
      const float er = j + 1 < n ? fabsf(ee[j]) : 0.0f;
      lo_l = fminf(lo_l, dd[j] - (el + er));
      hi_l = fmaxf(hi_l, dd[j] + (el + er));
      tn_l = fmaxf(tn_l, fabsf(dd[j]) + el + er);
      e2_l = fmaxf(e2_l, er * er);
    }
    lo = -wave_max(-lo_l);
    hi = wave_max(hi_l);
    tnorm = wave_max(tn_l);
    e2max = wave_max(e2_l);
  }
  const float pivmin = 1.17549435e-38f * fmaxf(1.0f, e2max);
  const float slack = 2.0f * 1.1920929e-7f * tnorm + pivmin;
  lo -= slack;
  hi += slack;

  // ---- top eigenvalues by multisection on Sturm counts: the 16 lanes of group g of
  // wave w evaluate 16 points inside the bracket of the (4 w + g + 1)-th largest
  // eigenvalue, which shrinks 17-fold per round; five rounds leave it about
  // 1.4e-6 (hi - lo) wide, which inverse iteration does not need to be narrower.
  float* lam = sm + L::LAM;
  if (4 * wv < rank) {
    const int grp = lane >> 4, gl = lane & 15;
    const int sv = 4 * wv + grp;
    const int idx = n - 1 - min(sv, rank - 1);  // ascending index
    float l = lo, u = hi;
    for (int round = 0; round < 5; ++round) {
      const float step = (u - l) * (1.0f / 17.0f);
      const float xq = l + step * static_cast<float>(gl + 1);
      // Sturm count: eigenvalues below xq
      float q = dd[0] - xq;
      if (fabsf(q) < pivmin) q = -pivmin;
      int cnt = q < 0.0f;
#pragma unroll 4
      for (int j = 1; j < n; ++j) {
        const float e = ee[j - 1];
        q = (dd[j] - xq) - (e * e) * __builtin_amdgcn_rcpf(q);
        if (fabsf(q) < pivmin) q = -pivmin;
        cnt += q < 0.0f;
      }
      const uint64_t mask = __ballot(cnt <= idx);
      const int below = __popcll((mask >> (16 * grp)) & 0xFFFFull);  // points at or below the eigenvalue
      const float nl = below > 0 ? l + step * static_cast<float>(below) : l;
      const float nu = below < 16 ? l + step * static_cast<float>(below + 1) : u;
      l = nl;
      u = nu;
    }
    if (gl == 0 && sv < rank) lam[sv] = 0.5f * (l + u);
  }
  __syncthreads();

  // ---- eigenvectors of T by inverse iteration, 16 at a time: lane s of wave 0 computes
  // vector 16 bt + s (column of X), with the pivoted LU of T - lambda I in its own
  // columns of the U / L arrays.  Members of a cluster (eigenvalue gaps below
  // 1e-3 ||T||) are solved together, each with its own shift, and after every solve
  // they are normalised and orthogonalised in order against the members before them
  // (earlier batches are complete): block inverse iteration, which converges to the
  // cluster's invariant subspace.
  float* X = sm + L::X;  // [128][XS]
  constexpr int XS = L::XS;
  if (wv == 0) {
    const float ortol = 1e-3f * tnorm;
    const float ptol = fmaxf(1.1920929e-7f * tnorm, 1e-30f);  // smallest pivot magnitude
    float* RU0 = sm + L::LU;  // [128][16] 1 / pivot
    float* U1 = RU0 + RRR_MAX * 16;
    float* U2 = U1 + RRR_MAX * 16;
    float* LM = U2 + RRR_MAX * 16;
    float* PV = LM + RRR_MAX * 16;
    // the tridiagonal in registers (lane l holds entries l and l + 64), read by readlane
    const float d0 = dd[lane], d1 = dd[lane + 64], e0 = ee[lane], e1 = ee[lane + 64];
    auto dget = [&](int j) {
      const float r0 = lane_read(d0, j & 63), r1 = lane_read(d1, j & 63);
      return j < 64 ? r0 : r1;
    };
    auto eget = [&](int j) {
      const float r0 = lane_read(e0, j & 63), r1 = lane_read(e1, j & 63);
      return j < 64 ? r0 : r1;
    };
    for (int bt = 0; 16 * bt < rank; ++bt) {
      const int sl = lane;  // column of the LU arrays
      const int s = 16 * bt + lane;
      const bool act = lane < 16 && s < rank;
      int mypos = 0;  // members of this vector's cluster before it
      {
        int pos = 0;
        for (int u = 1; u < min(rank, 16 * bt + 16); ++u) {
          pos = (lam[u - 1] - lam[u] < ortol) ? pos + 1 : 0;
          if (u == s) mypos = pos;
        }
      }
      const float lm = act ? lam[s] : 0.0f;
      // a member of a cluster with followers or predecessors
      const bool clustered = act && (mypos > 0 || (s + 1 < rank && lam[s] - lam[s + 1] < ortol));
      {
        const bool mine = act;
        float sc = 1.0f;
        if (mine) {
          float cd = dget(0) - lm;
          float cs = n > 1 ? eget(0) : 0.0f;
          for (int j = 0; j + 1 < n; ++j) {
            const float sub = eget(j);
            const float nd = dget(j + 1) - lm;
            const float ns = j + 2 < n ? eget(j + 1) : 0.0f;
            const bool sw = fabsf(cd) < fabsf(sub);
            const float piv = sw ? sub : cd;
            const float oth = sw ? cd : sub;
            const float l = oth == 0.0f ? 0.0f : oth * __builtin_amdgcn_rcpf(piv);
            const float pv = fabsf(piv) < ptol ? copysignf(ptol, piv) : piv;
            RU0[j * 16 + sl] = __builtin_amdgcn_rcpf(pv);
            U1[j * 16 + sl] = sw ? nd : cs;
            U2[j * 16 + sl] = sw ? ns : 0.0f;
            LM[j * 16 + sl] = l;
            PV[j * 16 + sl] = sw ? 1.0f : 0.0f;
            const float ncd = sw ? cs - l * nd : nd - l * cs;
            cs = sw ? -l * ns : ns;
            cd = ncd;
          }
          const float pv = fabsf(cd) < ptol ? copysignf(ptol, cd) : cd;
          RU0[(n - 1) * 16 + sl] = __builtin_amdgcn_rcpf(pv);
          // start vector: deterministic, distinct per eigenvalue
          for (int j = 0; j < n; ++j) {
            const uint32_t hsh =
                (static_cast<uint32_t>(j) * 2654435761u) ^ (static_cast<uint32_t>(s + 1) * 0x9E3779B9u);
            const uint32_t mix = (hsh ^ (hsh >> 15)) * 0x2C1B3C6Du;
            X[j * XS + s] = static_cast<float>((mix >> 8) & 0xFFFF) * (2.0f / 65535.0f) - 1.0f;
          }
        }
        // Three solves.  Between solves X is only rescaled (by 1 / max |x|, applied as the
        // next forward pass loads it); cluster members are also normalised and
        // orthogonalised against the members before them, by the whole wave, one member
        // at a time.  The norm is taken once, at the end.
        for (int it = 0; it < 3; ++it) {
          if (mine) {
            // P, L: forward elimination of the right-hand side, 8 rows per batch of loads
            float cur = X[s] * sc;
            for (int j0 = 0; j0 + 1 < n; j0 += 8) {
              float nx[8], lv[8], pv[8];
#pragma unroll
              for (int u = 0; u < 8; ++u) {
                const int j = min(j0 + u, RRR_MAX - 2);
                nx[u] = X[(j + 1) * XS + s];
                lv[u] = LM[j * 16 + sl];
                pv[u] = PV[j * 16 + sl];
              }
#pragma unroll
              for (int u = 0; u < 8; ++u) {
                const int j = j0 + u;
                if (j + 1 < n) {
                  const bool sw = pv[u] != 0.0f;
                  const float xn = nx[u] * sc;
                  X[j * XS + s] = sw ? xn : cur;
                  cur = sw ? cur - lv[u] * xn : xn - lv[u] * cur;
                }
              }
            }
            // U: back substitution, tracking the largest magnitude
            float x1 = cur * RU0[(n - 1) * 16 + sl], x2 = 0.0f;
            X[(n - 1) * XS + s] = x1;
            float mx = fabsf(x1);
            for (int j0 = n - 2; j0 >= 0; j0 -= 8) {
              float xi[8], u1[8], u2[8], ru[8];
#pragma unroll
              for (int u = 0; u < 8; ++u) {
                const int j = max(j0 - u, 0);
                xi[u] = X[j * XS + s];
                u1[u] = U1[j * 16 + sl];
                u2[u] = U2[j * 16 + sl];
                ru[u] = RU0[j * 16 + sl];
              }
#pragma unroll
              for (int u = 0; u < 8; ++u) {
                const int j = j0 - u;
                if (j >= 0) {
                  const float xv = (xi[u] - u1[u] * x1 - u2[u] * x2) * ru[u];
                  X[j * XS + s] = xv;
                  mx = fmaxf(mx, fabsf(xv));
                  x2 = x1;
                  x1 = xv;
                }
              }
            }
            sc = mx > 0.0f ? 1.0f / mx : 1.0f;
          }
          wave_sync();
          // cluster members in ascending order: normalised, and orthogonalised against the
          // members before them (which this pass has already normalised)
          uint64_t todo = __ballot(clustered);
          while (todo != 0ull) {
            const int ls = __builtin_ctzll(todo);
            todo &= todo - 1ull;
            const int sv = 16 * bt + ls;
            const int mp = __builtin_amdgcn_readlane(mypos, ls);
            const float scv = lane_read(sc, ls);
            float x0 = lane < n ? X[lane * XS + sv] * scv : 0.0f;
            float x1 = lane + 64 < n ? X[(lane + 64) * XS + sv] * scv : 0.0f;
            for (int o = sv - mp; o < sv; ++o) {
              const float p0 = lane < n ? X[lane * XS + o] : 0.0f;
              const float p1 = lane + 64 < n ? X[(lane + 64) * XS + o] : 0.0f;
              const float dt = wave_sum(x0 * p0 + x1 * p1);
              x0 -= dt * p0;
              x1 -= dt * p1;
            }
            const float nr = sqrtf(wave_sum(x0 * x0 + x1 * x1));
            const float f = nr > 0.0f ? 1.0f / nr : 0.0f;
            if (lane < n) X[lane * XS + sv] = x0 * f;
            if (lane + 64 < n) X[(lane + 64) * XS + sv] = x1 * f;
            if (lane == ls) sc = 1.0f;
            wave_sync();
          }
        }
        if (mine) {
          float ss = 0.0f;
#pragma unroll 8
          for (int j = 0; j < n; ++j) {
            const float xv = X[j * XS + s] * sc;
            ss += xv * xv;
          }
          const float nr = sqrtf(ss);
          const float f = nr > 0.0f ? sc / nr : 0.0f;
#pragma unroll 8
          for (int j = 0; j < n; ++j) X[j * XS + s] *= f;
        }
        wave_sync();
      }
    }
  }
  __syncthreads();

  // ---- back to B's coordinates: y <- H_0 H_1 ... H_{n-3} y, four vectors per wave per pass
  float* vb = sm + L::VB;  // (the LU arrays are dead)
  for (int base = 0; base < rank; base += 64) {
    if (base + 4 * wv < rank) {
      float y0[4], y1[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int sv = base + 4 * wv + u;
        y0[u] = (sv < rank && lane < n) ? X[lane * XS + sv] : 0.0f;
        y1[u] = (sv < rank && lane + 64 < n) ? X[(lane + 64) * XS + sv] : 0.0f;
      }
      const int pl0 = hv_perm(lane), pl1 = hv_perm(lane + 64);
      int k = n - 3;
      float tk = 0.0f, sk = 0.0f, r0 = 0.0f, r1 = 0.0f;
      if (k >= 0) {
        tk = tau[k];
        sk = scl[k];
        r0 = hv[k * HV_STRIDE + pl0];
        r1 = hv[k * HV_STRIDE + pl1];
      }
      for (; k >= 0; --k) {
        // next reflector's data, loaded while this one is applied
        const int kn = max(k - 1, 0);
        const float tn = tau[kn], sn = scl[kn];
        const float n0 = hv[kn * HV_STRIDE + pl0], n1 = hv[kn * HV_STRIDE + pl1];
        if (tk != 0.0f) {
          const float v0 = lane == k + 1 ? 1.0f : r0 * sk;
          const float v1 = lane + 64 == k + 1 ? 1.0f : r1 * sk;
          float dt[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) dt[u] = tk * wave_sum(v0 * y0[u] + v1 * y1[u]);
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            y0[u] -= dt[u] * v0;
            y1[u] -= dt[u] * v1;
          }
        }
        tk = tn;
        sk = sn;
        r0 = n0;
        r1 = n1;
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int sv = base + 4 * wv + u;
        if (sv < rank) {
          vb[sv * RRR_MAX + lane] = y0[u];
          vb[sv * RRR_MAX + lane + 64] = y1[u];
        }
      }
    }
  }
  __syncthreads();

  // ---- Cholesky-QR: S = V^T V = R^T R (R upper, in place), then Q R = V by forward
  // substitution over the columns; Q is orthonormal to rounding.
  float* S = sm + L::S;  // (the tridiagonal eigenvectors are dead)
  for (int col = wv; col < rank; col += RRR_THREADS / 64) {
    const float y0 = vb[col * RRR_MAX + lane], y1 = vb[col * RRR_MAX + lane + 64];
    for (int s2 = 0; s2 <= col; ++s2) {
      const float dt = wave_sum(y0 * vb[s2 * RRR_MAX + lane] + y1 * vb[s2 * RRR_MAX + lane + 64]);
      if (lane == 0) {
        S[s2 * MAXR + col] = dt;
        S[col * MAXR + s2] = dt;
      }
    }
  }
  __syncthreads();
  for (int k = 0; k < rank; ++k) {
    const float rkk = sqrtf(S[k * MAXR + k]);
    __syncthreads();
    if (t >= k && t < rank) S[k * MAXR + t] = t == k ? rkk : S[k * MAXR + t] / rkk;
    __syncthreads();
    for (int e = t; e < rank * rank; e += RRR_THREADS) {
      const int r = e / rank, q = e - r * rank;
      if (r > k && q >= r) S[r * MAXR + q] -= S[k * MAXR + r] * S[k * MAXR + q];
    }
    __syncthreads();
  }
  float* Qm = sm + L::Q;  // [128][MAXR] (the Householder columns are dead)
  if (t < n) {
    for (int col = 0; col < rank; ++col) {
      float acc = vb[col * RRR_MAX + t];
      for (int s2 = 0; s2 < col; ++s2) acc -= Qm[t * MAXR + s2] * S[s2 * MAXR + col];
      Qm[t * MAXR + col] = acc / S[col * MAXR + col];
    }
  }
  __syncthreads();
  // eigenvalue rank col (0 = largest) goes to column rank - 1 - col: ascending order
  for (int e = t; e < n * rank; e += RRR_THREADS) {
    const int r = e / rank, col = e - r * rank;
    basis[r * rank + (rank - 1 - col)] = Qm[r * MAXR + col];
  }
  if (vals != nullptr) {
    // Rayleigh quotients q^T A q (the symmetric part of A gives the same value)
    for (int col = wv; col < rank; col += RRR_THREADS / 64) {
      const float q0 = lane < n ? Qm[lane * MAXR + col] : 0.0f;
      const float q1 = lane + 64 < n ? Qm[(lane + 64) * MAXR + col] : 0.0f;
      float a0 = 0.0f, a1 = 0.0f;
      for (int j = 0; j < n; ++j) {
        const float qj = Qm[j * MAXR + col];
        if (lane < n) a0 += bmat[j * ld + lane] * qj;
        if (lane + 64 < n) a1 += bmat[j * ld + lane + 64] * qj;
      }
      const float lam_c = wave_sum(q0 * a0 + q1 * a1);
      if (lane == 0) vals[rank - 1 - col] = lam_c;
    }
  }
}

// Cholesky of G (p x p, register resident), L written over G (lower triangle).  The
// whole trailing block is updated (it stays symmetric), so a lane needs no per-column
// test.  Columns go in blocks of eight as in the tridiagonalisation (g[0] of lanes
// c = k % 8 is the pivot column, the array shifts down one register per block);
// groups of four registers past the end are skipped, and so are waves whose rows
// are all finished.
__device__ __forceinline__ void rrr_cholesky(float* sm, float* __restrict__ gmat, int p) {
  const int t = threadIdx.x, i = t >> 3, c = t & 7, wv = t >> 6;
  float g[16];
#pragma unroll
  for (int q = 0; q < 16; ++q) g[q] = gmat[i * RRR_MAX + c + 8 * q];
  if (t < 2 * HV_STRIDE) sm[t] = 0.0f;
  __syncthreads();  // G read before L is written over it; column buffers cleared
  for (int kb = 0; 8 * kb < p; ++kb) {
    if (kb > 0) {
#pragma unroll
      for (int q = 0; q < 15; ++q) g[q] = g[q + 1];
      g[15] = 0.0f;
    }
    const int nq = 16 - kb;
    for (int kc = 0; kc < 8; ++kc) {
      const int k = 8 * kb + kc;
      if (k >= p) break;
      float* buf = sm + (k & 1) * HV_STRIDE;
      if (c == kc) buf[hv_perm(i)] = i >= k ? g[0] : 0.0f;
      __syncthreads();
      const float dk = buf[hv_perm(k)];
      if (c == kc && i >= k && i < p) gmat[i * RRR_MAX + k] = g[0] / sqrtf(dk);
      if (8 * wv + 7 > k) {
        const float f = i > k ? buf[hv_perm(i)] * __builtin_amdgcn_rcpf(dk) : 0.0f;
        const float* bq = buf + c * 17 + kb;
        float bv[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) bv[q] = bq[q];
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          if (4 * g4 < nq) {
            asm volatile("" ::: "memory");
#pragma unroll
            for (int u = 0; u < 4; ++u) g[4 * g4 + u] = fmaf(-f, bv[4 * g4 + u], g[4 * g4 + u]);
          }
        }
      }
    }
  }
}

// role = blockIdx.y + role0: 0 the eigenvectors of B (slot 1), 1 the Cholesky factor of the
// ng x ng matrix G (slot 0).  MAXR: the eigen solver's largest rank (16 or 64).
template <int MAXR>
__global__ __launch_bounds__(RRR_THREADS, 1) void rrr_factor_kernel(float* __restrict__ ws, int32_t ng, int32_t d,
                                                                    int32_t rank, int32_t role0,
                                                                    float* __restrict__ basis) {
  __shared__ float sm[EigLayout<MAXR>::FLOATS];
  const int64_t h = blockIdx.x;
  if (blockIdx.y + role0 == 1) {
    rrr_cholesky(sm, ws_slot(ws, h, 0), ng);
  } else {
    rrr_eigen<MAXR>(sm, ws_slot(ws, h, 1), RRR_MAX, d, rank, false, basis + h * d * rank, nullptr);
  }
}
// the factor kernel for a rank (one template per eigen-solver size)
inline void launch_rrr_factor(dim3 grid, hipStream_t stream, float* ws, int32_t ng, int32_t d, int32_t rank,
                              int32_t role0, float* basis) {
  if (rank <= RRR_MAX_RANK) {
    rrr_factor_kernel<RRR_MAX_RANK><<<grid, RRR_THREADS, 0, stream>>>(ws, ng, d, rank, role0, basis);
  } else {
    rrr_factor_kernel<RRR_MAX_FIT_RANK><<<grid, RRR_THREADS, 0, stream>>>(ws, ng, d, rank, role0, basis);
  }
}

// Top-rank eigenpairs of a batch of symmetric matrices, one workgroup per matrix.
template <int MAXR>
__global__ __launch_bounds__(RRR_THREADS, 1) void sym_top_eig_kernel(const float* __restrict__ mats, int32_t n,
                                                                     int32_t rank, int32_t symmetrize,
                                                                     float* __restrict__ vecs,
                                                                     float* __restrict__ vals) {
  __shared__ float sm[EigLayout<MAXR>::FLOATS];
  const int64_t h = blockIdx.x;
  rrr_eigen<MAXR>(sm, mats + h * n * n, n, n, rank, symmetrize != 0, vecs + h * n * rank,
                  vals != nullptr ? vals + h * rank : nullptr);
}

// x_w^T in LDS, [xt_rows(p)][xt_stride(m, p)] in an array of RRR_MAX * RRR_LS floats: feature
// a is row a (rows from p on are zero), token r column r (columns from m on are zero).  Up
// to 128 features: 128 rows of 129.  More features (the dual form, m < p <= 256): 64 ceil(p /
// 64) rows of m | 1 (odd, so that the rows lane + 64 q of one column fall in distinct banks),
// which fits when that product is at most RRR_MAX * RRR_LS.
__host__ __device__ inline int xt_stride(int m, int p) { return p <= RRR_MAX ? RRR_LS : (m | 1); }
__host__ __device__ inline int xt_rows(int p) { return p <= RRR_MAX ? RRR_MAX : 64 * ((p + 63) / 64); }

// L (ng x ng lower, slot 0) into LDS and x_w^T into LDS (the layout above).
__device__ __forceinline__ void load_factor_and_xt(const float* __restrict__ lg, int ng, const float* __restrict__ xh,
                                                   const float* __restrict__ wh, const float* __restrict__ xm,
                                                   const float* __restrict__ xs, int m, int p, float* ls,
                                                   float* xt) {
  const int t = threadIdx.x;
  for (int e = t; e < RRR_MAT; e += RRR_THREADS) {
    const int r = e >> 7, cc = e & 127;
    ls[r * RRR_LS + cc] = (r < ng && cc <= r) ? lg[e] : 0.0f;
  }
  const int xst = xt_stride(m, p), xr = xt_rows(p);
  for (int e = t; e < m * p; e += RRR_THREADS) {  // x in its own order (coalesced reads)
    const int i = e / p, j = e - i * p;
    const float sw = wh != nullptr ? sqrtf(wh[i]) : 1.0f;
    xt[j * xst + i] = (xh[e] - xm[j]) / xs[j] * sw;
  }
  for (int e = t; e < xr * xst; e += RRR_THREADS) {  // the zero padding (disjoint from the above)
    const int j = e / xst, i = e - j * xst;
    if (i >= m || j >= p) xt[e] = 0.0f;
  }
}

// L L^T u = b for one right-hand side held by a wave: entry k in lane k % 64 of b0 (k < 64)
// or b1 (k >= 64).  Entries at or beyond n stay as they are.  Each substitution step is a
// short dependent chain (scale by the reciprocal pivot, broadcast, one FMA per lane); the
// factor entries it needs are read from LDS eight steps at a time ahead of the chain.
__device__ __forceinline__ void chol_solve_wave(const float* ls, int n, int lane, float& b0, float& b1) {
  const float rd0 = lane < n ? 1.0f / ls[lane * RRR_LS + lane] : 0.0f;
  const float rd1 = lane + 64 < n ? 1.0f / ls[(lane + 64) * RRR_LS + lane + 64] : 0.0f;
  for (int k0 = 0; k0 < n; k0 += 8) {  // L y = b: column k of L, rows lane and lane + 64
    float c0[8], c1[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = min(k0 + u, RRR_MAX - 1);
      c0[u] = lane > k ? ls[lane * RRR_LS + k] : 0.0f;
      c1[u] = lane + 64 > k ? ls[(lane + 64) * RRR_LS + k] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = k0 + u;
      if (k < n) {
        const float yk = lane_read(k < 64 ? b0 * rd0 : b1 * rd1, k & 63);
        if (lane == (k & 63)) {
          if (k < 64) b0 = yk;
          else b1 = yk;
        }
        b0 = fmaf(-c0[u], yk, b0);
        b1 = fmaf(-c1[u], yk, b1);
      }
    }
  }
  for (int k0 = n - 1; k0 >= 0; k0 -= 8) {  // L^T u = y: row k of L, columns lane and lane + 64
    float c0[8], c1[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = max(k0 - u, 0);
      c0[u] = lane < k ? ls[k * RRR_LS + lane] : 0.0f;
      c1[u] = lane + 64 < k ? ls[k * RRR_LS + lane + 64] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = k0 - u;
      if (k >= 0) {
        const float xk = lane_read(k < 64 ? b0 * rd0 : b1 * rd1, k & 63);
        if (lane == (k & 63)) {
          if (k < 64) b0 = xk;
          else b1 = xk;
        }
        b0 = fmaf(-c0[u], xk, b0);
        b1 = fmaf(-c1[u], xk, b1);
      }
    }
  }
}

// o = x_w^T u for u over the m rows (held as in chol_solve_wave): feature a (< p) in lane
// a % 64 of o[a / 64].
__device__ __forceinline__ void xt_times(const float* xt, int m, int p, int lane, float b0, float b1,
                                         float (&o)[4]) {
  const int xst = xt_stride(m, p), nfq = xt_rows(p) / 64;
  float l[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int r0 = 0; r0 < m; r0 += 8) {
    float e[4][8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int r = min(r0 + u, xst - 1);
#pragma unroll
      for (int q = 0; q < 4; ++q) e[q][u] = q < nfq ? xt[(lane + 64 * q) * xst + r] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int r = r0 + u;
      if (r < m) {
        const float uu = lane_read(r < 64 ? b0 : b1, r & 63);
#pragma unroll
        for (int q = 0; q < 4; ++q) l[q] += e[q][u] * uu;
      }
    }
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) o[q] = l[q];
}

__device__ __forceinline__ double lane_read_d(double v, int lane) {
  const long long b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_readlane(static_cast<int>(b), lane);
  const int hi = __builtin_amdgcn_readlane(static_cast<int>(b >> 32), lane);
  return __longlong_as_double((static_cast<long long>(hi) << 32) | static_cast<unsigned int>(lo));
}

// G u for the ridge system, in fp64 from x_w (exact fp32 values in xt) rather than from the
// rounded G: dual (u over the m rows): x_w x_w^T u + ridge u; primal (u over the p
// features): x_w^T x_w u + ridge u.  u and the result are held as in chol_solve_wave; the
// middle vector x_w^T u of the dual form (p <= 256 entries) as the output of xt_times.
__device__ __forceinline__ void ridge_apply_f64(const float* xt, bool dual, int m, int p, float ridge, int lane,
                                                float u0, float u1, double& g0, double& g1) {
  const int xst = xt_stride(m, p), nfq = xt_rows(p) / 64;
  double w0 = 0.0, w1 = 0.0;
  if (dual) {
    double v[4] = {0.0, 0.0, 0.0, 0.0};  // v[a] = sum_r x_w[r][a] u[r] = sum_r xt[a][r] u[r]
    for (int k0 = 0; k0 < m; k0 += 8) {
      float e[4][8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int k = min(k0 + u, xst - 1);
#pragma unroll
        for (int q = 0; q < 4; ++q) e[q][u] = q < nfq ? xt[(lane + 64 * q) * xst + k] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int k = k0 + u;
        if (k < m) {
          const double uk = static_cast<double>(lane_read(k < 64 ? u0 : u1, k & 63));
#pragma unroll
          for (int q = 0; q < 4; ++q) v[q] = fma(static_cast<double>(e[q][u]), uk, v[q]);
        }
      }
    }
    for (int k0 = 0; k0 < p; k0 += 8) {  // w[r] = sum_a xt[a][r] v[a], r = lane, lane + 64
      float e0[8], e1[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int k = min(k0 + u, 64 * nfq - 1);
        e0[u] = lane < xst ? xt[k * xst + lane] : 0.0f;
        e1[u] = lane + 64 < xst ? xt[k * xst + lane + 64] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int k = k0 + u;
        if (k < p) {
          const double vq = k < 64 ? v[0] : (k < 128 ? v[1] : (k < 192 ? v[2] : v[3]));
          const double vk = lane_read_d(vq, k & 63);
          w0 = fma(static_cast<double>(e0[u]), vk, w0);
          w1 = fma(static_cast<double>(e1[u]), vk, w1);
        }
      }
    }
  } else {  // p <= 128 < 129 = xst
    double v0 = 0.0, v1 = 0.0;  // v[r] = sum_a x_w[r][a] u[a] = sum_a xt[a][r] u[a]
    for (int k0 = 0; k0 < p; k0 += 8) {
      float e0[8], e1[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int k = min(k0 + u, RRR_MAX - 1);
        e0[u] = xt[k * xst + lane];
        e1[u] = xt[k * xst + lane + 64];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int k = k0 + u;
        if (k < p) {
          const double uk = static_cast<double>(lane_read(k < 64 ? u0 : u1, k & 63));
          v0 = fma(static_cast<double>(e0[u]), uk, v0);
          v1 = fma(static_cast<double>(e1[u]), uk, v1);
        }
      }
    }
    for (int k0 = 0; k0 < m; k0 += 8) {  // w[a] = sum_r xt[a][r] v[r]
      float e0[8], e1[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int k = min(k0 + u, RRR_MAX - 1);
        e0[u] = xt[lane * xst + k];
        e1[u] = xt[(lane + 64) * xst + k];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int k = k0 + u;
        if (k < m) {
          const double vk = lane_read_d(k < 64 ? v0 : v1, k & 63);
          w0 = fma(static_cast<double>(e0[u]), vk, w0);
          w1 = fma(static_cast<double>(e1[u]), vk, w1);
        }
      }
    }
  }
  g0 = w0 + static_cast<double>(ridge) * u0;
  g1 = w1 + static_cast<double>(ridge) * u1;
}

// Solve G u = b (b held as in chol_solve_wave, entries at or beyond ng zero) with the fp32
// Cholesky factor and one step of iterative refinement whose residual b - G u is
// accumulated in fp64 from x_w.  The condition number of G is about the largest eigenvalue
// of the weighted gram over the ridge (1e5 and more for token-count weights), so the plain
// fp32 solve keeps only a few digits; the refinement step multiplies its error by about
// cond * 2^-24.
__device__ __forceinline__ void ridge_solve_refined(const float* ls, const float* xt, bool dual, int m, int p,
                                                    float ridge, int lane, float& b0, float& b1) {
  const int ng = dual ? m : p;
  const float r0 = b0, r1 = b1;
  chol_solve_wave(ls, ng, lane, b0, b1);
  {
    double g0, g1;
    ridge_apply_f64(xt, dual, m, p, ridge, lane, b0, b1, g0, g1);
    float d0 = lane < ng ? static_cast<float>(static_cast<double>(r0) - g0) : 0.0f;
    float d1 = lane + 64 < ng ? static_cast<float>(static_cast<double>(r1) - g1) : 0.0f;
    chol_solve_wave(ls, ng, lane, d0, d1);
    b0 += d0;
    b1 += d1;
  }
}

// The weighted fitted values F [m][d] into slot 2 (row stride 128): one wave per column.
//   dual:   F = y_w - ridge G^-1 y_w;  primal: F = x_w G^-1 x_w^T y_w.
__global__ __launch_bounds__(RRR_THREADS, 1) void rrr_fitted_kernel(const float* __restrict__ x,
                                                                    const float* __restrict__ y,
                                                                    const float* __restrict__ w, int32_t m, int32_t p,
                                                                    int32_t d, float ridge,
                                                                    const float* __restrict__ x_mean,
                                                                    const float* __restrict__ x_scale,
                                                                    const float* __restrict__ y_mean,
                                                                    float* __restrict__ ws) {
  __shared__ float ls[RRR_MAX * RRR_LS];
  __shared__ float xt[RRR_MAX * RRR_LS];
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int64_t h = blockIdx.x;
  const bool dual = m < p;
  const int ng = dual ? m : p;
  const float* wh = w != nullptr ? w + h * m : nullptr;
  const float* yh = y + h * m * d;
  const float* ym = y_mean + h * d;
  load_factor_and_xt(ws_slot(ws, h, 0), ng, x + h * m * p, wh, x_mean + h * p, x_scale + h * p, m, p, ls, xt);
  __syncthreads();
  float* f = ws_slot(ws, h, 2);
  const float sw0 = lane < m ? (wh != nullptr ? sqrtf(wh[lane]) : 1.0f) : 0.0f;
  const float sw1 = lane + 64 < m ? (wh != nullptr ? sqrtf(wh[lane + 64]) : 1.0f) : 0.0f;
  for (int col = wv; col < d; col += RRR_THREADS / 64) {
    const float y0 = lane < m ? (yh[lane * d + col] - ym[col]) * sw0 : 0.0f;
    const float y1 = lane + 64 < m ? (yh[(lane + 64) * d + col] - ym[col]) * sw1 : 0.0f;
    float b0, b1;
    if (dual) {
      b0 = y0;
      b1 = y1;
      ridge_solve_refined(ls, xt, true, m, p, ridge, lane, b0, b1);
      b0 = y0 - ridge * b0;
      b1 = y1 - ridge * b1;
    } else {
      float o[4];
      xt_times(xt, m, p, lane, y0, y1, o);  // x_w^T y_w[:, col] (primal: p <= 128)
      b0 = o[0];
      b1 = o[1];
      ridge_solve_refined(ls, xt, false, m, p, ridge, lane, b0, b1);
      float f0 = 0.0f, f1 = 0.0f;  // F[r] = sum_a x_w[r][a] W[a]
      for (int r = 0; r < m; ++r) {
        const float v = wave_sum(xt[lane * RRR_LS + r] * b0 + xt[(lane + 64) * RRR_LS + r] * b1);
        if (lane == (r & 63)) {
          if (r < 64) f0 = v;
          else f1 = v;
        }
      }
      b0 = f0;
      b1 = f1;
    }
    if (lane < m) f[lane * RRR_MAX + col] = b0;
    if (lane + 64 < m) f[(lane + 64) * RRR_MAX + col] = b1;
  }
}

// Z = y_w basis, then left = G^-1 x_w^T Z (primal) or x_w^T G^-1 Z (dual), in blocks of 16
// basis columns (one wave per column of a block; MULTI: more than one block).
template <bool MULTI>
__global__ __launch_bounds__(RRR_THREADS, 1) void rrr_solve_kernel(const float* __restrict__ x,
                                                                   const float* __restrict__ y,
                                                                   const float* __restrict__ w, int32_t m, int32_t p,
                                                                   int32_t d, int32_t rank, float ridge,
                                                                   const float* __restrict__ x_mean,
                                                                   const float* __restrict__ x_scale,
                                                                   const float* __restrict__ y_mean,
                                                                   float* __restrict__ ws,
                                                                   const float* __restrict__ basis,
                                                                   float* __restrict__ left) {
  __shared__ float ls[RRR_MAX * RRR_LS];  // L (lower)
  __shared__ float xt[RRR_MAX * RRR_LS];  // x_w^T
  __shared__ __align__(16) float zs[RRR_MAX][RRR_MAX_RANK];
  __shared__ __align__(16) float bs[RRR_MAX][RRR_MAX_RANK];
  const int t = threadIdx.x, i = t >> 3, c = t & 7, lane = t & 63, wv = t >> 6;
  const int64_t h = blockIdx.x;
  const bool dual = m < p;
  const int ng = dual ? m : p;
  const float* yh = y + h * m * d;
  const float* wh = w != nullptr ? w + h * m : nullptr;
  load_factor_and_xt(ws_slot(ws, h, 0), ng, x + h * m * p, wh, x_mean + h * p, x_scale + h * p, m, p, ls, xt);
  const float sw = i < m ? (wh != nullptr ? sqrtf(wh[i]) : 1.0f) : 0.0f;
  for (int j0 = 0; j0 < (MULTI ? rank : 1); j0 += RRR_MAX_RANK) {
  // thread (row i, columns c + 8 q): y_w in registers (loaded per block, so that it is not
  // held through the solves)
  float yw[16];
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int j = c + 8 * q;
    yw[q] = (i < m && j < d) ? (yh[i * d + j] - y_mean[h * d + j]) * sw : 0.0f;
  }
  // basis columns j0 .. j0 + 15 (zero past rank); the barrier also ends the previous
  // block's reads of zs
  for (int e = t; e < RRR_MAX * RRR_MAX_RANK; e += RRR_THREADS) {
    const int r = e / RRR_MAX_RANK, j = e % RRR_MAX_RANK;
    bs[r][j] = (r < d && j0 + j < rank) ? basis[(h * d + r) * rank + j0 + j] : 0.0f;
  }
  __syncthreads();
  // Z[i][*] = sum_k y_w[i][k] basis[k][*], reduced over the 8 lanes of the row
  {
    float z[RRR_MAX_RANK];
#pragma unroll
    for (int j = 0; j < RRR_MAX_RANK; ++j) z[j] = 0.0f;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const float4* br = reinterpret_cast<const float4*>(&bs[c + 8 * q][0]);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float4 bv = br[u];
        z[4 * u + 0] += yw[q] * bv.x;
        z[4 * u + 1] += yw[q] * bv.y;
        z[4 * u + 2] += yw[q] * bv.z;
        z[4 * u + 3] += yw[q] * bv.w;
      }
    }
#pragma unroll
    for (int j = 0; j < RRR_MAX_RANK; ++j) z[j] = sum8(z[j]);
    zs[i][c] = pick16(z, c);
    zs[i][c + 8] = pick16(z, c + 8);
  }
  __syncthreads();
  if (j0 + wv < rank) {
    const int j = j0 + wv;
    float b0 = zs[lane][wv], b1 = zs[lane + 64][wv];  // zero at rows >= m
    float o[4];
    if (dual) {
      ridge_solve_refined(ls, xt, true, m, p, ridge, lane, b0, b1);
      xt_times(xt, m, p, lane, b0, b1, o);
    } else {
      xt_times(xt, m, p, lane, b0, b1, o);
      ridge_solve_refined(ls, xt, false, m, p, ridge, lane, o[0], o[1]);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (lane + 64 * q < p) left[(h * p + lane + 64 * q) * rank + j] = o[q];
    }
  }
  }
}

// Per head: recovered = any non-finite value in the five state tensors; the output takes the
// previous state's values (prev non-null) or the zero correction (x_mean 0, x_scale 1,
// y_mean 0, left 0, basis 0) where recovered, the current ones elsewhere.  out may alias cur.
struct RrrState {
  const float* t[5];
};
struct RrrStateOut {
  float* t[5];
};
__global__ __launch_bounds__(256) void rrr_recover_kernel(RrrState cur, RrrState prev, RrrStateOut out, int32_t p,
                                                          int32_t d, int32_t rank, uint8_t* __restrict__ recovered) {
  const int64_t h = blockIdx.x;
  const int64_t n[5] = {p, p, d, static_cast<int64_t>(p) * rank, static_cast<int64_t>(d) * rank};
  int bad = 0;
#pragma unroll
  for (int k = 0; k < 5; ++k) {
    for (int64_t e = threadIdx.x; e < n[k]; e += blockDim.x) {
      const float v = cur.t[k][h * n[k] + e];
      bad |= !(fabsf(v) <= 3.402823466e38f);
    }
  }
  bad = __syncthreads_or(bad);
#pragma unroll
  for (int k = 0; k < 5; ++k) {
    for (int64_t e = threadIdx.x; e < n[k]; e += blockDim.x) {
      const int64_t o = h * n[k] + e;
      float v = cur.t[k][o];
      if (bad) v = prev.t[0] != nullptr ? prev.t[k][o] : (k == 1 ? 1.0f : 0.0f);
      out.t[k][o] = v;
    }
  }
  if (threadIdx.x == 0 && recovered != nullptr) recovered[h] = static_cast<uint8_t>(bad);
}

// ---- the fixed-count top-16 subspace basis of the N8 repair (top16_right_basis_triton,
// src/sparsepr/kernels/triton/rrr_eigensolver.py:14-128), for V [64][128] per head:
//   A = V V^T; Q0 = the reduced QR factor of C[i][j] = cos((i + 1/2)(j + 1) pi / 64);
//   8 times: Y = A Q, (X, s) = ns(Y^T Y), Q = Y X / sqrt(s);
//   B = V^T Q, (X, s) = ns(B^T B), basis = B X / sqrt(s);
// with ns(G): s = max(||G||_F, 1e-20), N = G / s, X0 = I, six times X <- X (3 I - N X X) / 2.
// The columns of C are DCT-II vectors, orthogonal with norm sqrt(32), so Householder QR
// (LAPACK's convention, which torch.linalg.qr follows) gives Q0 = C diag(sign) / sqrt(32) with
// the signs of R's diagonal below.  The result is not the exact eigenbasis, and where a Gram
// is ill-conditioned the six Newton-Schulz steps leave it short of orthonormal, as the
// reference's is.  One 256-thread workgroup per head, everything in LDS, fp32 with sequential
// sums.  V comes from the raw residual ((y - y_mean) sqrt(w)) when vals is null, else from
// vals (row stride vals_ld, head stride vals_hs).
constexpr int T16_M = 64, T16_D = 128, T16_R = 16;
constexpr uint32_t T16_SEED_NEGATIVE = 0x8E1Fu;  // R[j][j] < 0 for j = 0-4, 9-11, 15
constexpr int T16_POWER_ITERS = 8, T16_NS_ITERS = 6;  // the reference's defaults

// Newton-Schulz on the 16 x 16 Gram G held one entry per thread (thread t: entry (t / 16,
// t % 16)): leaves X ~ (G / s)^(-1/2) in x and returns sqrt(s).  x and tmp swap roles as
// the iterations go (every thread swaps alike); nrm and ubuf are scratch [16][17].
__device__ __forceinline__ float t16_newton_schulz(float g, int ns_iters, float (*nrm)[17], float (*&x)[17],
                                                   float (*&tmp)[17], float (*ubuf)[17], float* red) {
  const int t = threadIdx.x, a = t >> 4, b = t & 15, lane = t & 63, wv = t >> 6;
  const float sq = wave_sum(g * g);
  if (lane == 0) red[wv] = sq;
  __syncthreads();
  const float scale = fmaxf(sqrtf(((red[0] + red[1]) + red[2]) + red[3]), 1e-20f);
  nrm[a][b] = g / scale;
  x[a][b] = a == b ? 1.0f : 0.0f;
  __syncthreads();
  for (int it = 0; it < ns_iters; ++it) {
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < T16_R; ++k) s = fmaf(x[a][k], x[k][b], s);
    tmp[a][b] = s;
    __syncthreads();
    float u = 0.0f;
#pragma unroll
    for (int k = 0; k < T16_R; ++k) u = fmaf(nrm[a][k], tmp[k][b], u);
    ubuf[a][b] = (a == b ? 3.0f : 0.0f) - u;
    __syncthreads();
    float v = 0.0f;
#pragma unroll
    for (int k = 0; k < T16_R; ++k) v = fmaf(x[a][k], ubuf[k][b], v);
    tmp[a][b] = 0.5f * v;
    __syncthreads();
    float(*swap)[17] = x;
    x = tmp;
    tmp = swap;
  }
  return sqrtf(scale);
}

__global__ __launch_bounds__(256) void rrr_top16_kernel(const float* __restrict__ y, const float* __restrict__ w,
                                                        const float* __restrict__ y_mean,
                                                        const float* __restrict__ vals, int64_t vals_hs,
                                                        int32_t vals_ld, int32_t power_iters, int32_t ns_iters,
                                                        float* __restrict__ basis) {
  __shared__ float vs[T16_M][T16_D + 1];
  __shared__ float as[T16_M * (T16_M + 1)];  // A [64][65]; after the iterations B [128][17]
  __shared__ float qs[T16_M][T16_R + 1];
  __shared__ float ys[T16_M][T16_R + 1];
  __shared__ float sm[4][T16_R][T16_R + 1];
  __shared__ float red[4];
  const int t = threadIdx.x;
  const int64_t h = blockIdx.x;
  if (vals == nullptr) {
    const float* yh = y + h * T16_M * T16_D;
    const float* ym = y_mean + h * T16_D;
    for (int e = t; e < T16_M * T16_D; e += 256) {
      const int r = e >> 7, c = e & 127;
      vs[r][c] = (yh[e] - ym[c]) * (w != nullptr ? sqrtf(w[h * T16_M + r]) : 1.0f);
    }
  } else {
    const float* vh = vals + h * vals_hs;
    for (int e = t; e < T16_M * T16_D; e += 256) {
      const int r = e >> 7, c = e & 127;
      vs[r][c] = vh[static_cast<int64_t>(r) * vals_ld + c];
    }
  }
  {  // Q0
    const int i = t >> 2;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int j = (t & 3) + 4 * u;
      const double c = cos((i + 0.5) * (j + 1.0) * (3.14159265358979323846 / 64.0)) / sqrt(32.0);
      qs[i][j] = static_cast<float>((T16_SEED_NEGATIVE >> j) & 1u ? -c : c);
    }
  }
  __syncthreads();
  {  // A = V V^T: thread t owns rows t / 16 + 16 u and columns t % 16 + 16 v
    const int bi = t >> 4, bj = t & 15;
    float acc[4][4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[u][v] = 0.0f;
    for (int c = 0; c < T16_D; ++c) {
      float ri[4], rj[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        ri[u] = vs[bi + 16 * u][c];
        rj[u] = vs[bj + 16 * u][c];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[u][v] = fmaf(ri[u], rj[v], acc[u][v]);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int v = 0; v < 4; ++v) as[(bi + 16 * u) * (T16_M + 1) + bj + 16 * v] = acc[u][v];
  }
  __syncthreads();
  float(*nrm)[17] = sm[0];
  float(*xm)[17] = sm[1];
  float(*tmp)[17] = sm[2];
  float(*ubuf)[17] = sm[3];
  const int a = t >> 4, b = t & 15;
  const int ri = t >> 2, rc = t & 3;  // 64 x 16 products: row ri, columns rc + 4 u
  for (int it = 0; it < power_iters; ++it) {
    float yv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int k = 0; k < T16_M; ++k) {
      const float av = as[ri * (T16_M + 1) + k];
#pragma unroll
      for (int u = 0; u < 4; ++u) yv[u] = fmaf(av, qs[k][rc + 4 * u], yv[u]);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) ys[ri][rc + 4 * u] = yv[u];
    __syncthreads();
    float g = 0.0f;
    for (int r = 0; r < T16_M; ++r) g = fmaf(ys[r][a], ys[r][b], g);
    const float root = t16_newton_schulz(g, ns_iters, nrm, xm, tmp, ubuf, red);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      float s = 0.0f;
#pragma unroll
      for (int k = 0; k < T16_R; ++k) s = fmaf(ys[ri][k], xm[k][rc + 4 * u], s);
      qs[ri][rc + 4 * u] = s / root;
    }
    __syncthreads();
  }
  // B = V^T Q [128][16] into as (row stride 17): thread t owns row t / 2, columns 8 (t % 2) + v
  const int bc = t >> 1, bo = 8 * (t & 1);
  {
    float bv[8];
#pragma unroll
    for (int v = 0; v < 8; ++v) bv[v] = 0.0f;
    for (int r = 0; r < T16_M; ++r) {
      const float vv = vs[r][bc];
#pragma unroll
      for (int v = 0; v < 8; ++v) bv[v] = fmaf(vv, qs[r][bo + v], bv[v]);
    }
#pragma unroll
    for (int v = 0; v < 8; ++v) as[bc * (T16_R + 1) + bo + v] = bv[v];
  }
  __syncthreads();
  float g = 0.0f;
  for (int r = 0; r < T16_D; ++r) g = fmaf(as[r * (T16_R + 1) + a], as[r * (T16_R + 1) + b], g);
  const float root = t16_newton_schulz(g, ns_iters, nrm, xm, tmp, ubuf, red);
  float* out = basis + h * T16_D * T16_R;
#pragma unroll
  for (int v = 0; v < 8; ++v) {
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < T16_R; ++k) s = fmaf(as[bc * (T16_R + 1) + k], xm[k][bo + v], s);
    out[bc * T16_R + bo + v] = s / root;
  }
}

}  // namespace

extern "C" size_t spr_rrr_fit_workspace(int64_t bh) {
  return bh <= 0 ? 0 : static_cast<size_t>(bh) * RRR_SLOTS * RRR_MAT * sizeof(float);
}

namespace {
// The fit's launches; top16: the basis from rrr_top16_kernel instead of the exact eigenvectors.
int rrr_fit_launch(const float* x, const float* y, const float* weights, int64_t bh, int32_t m, int32_t p, int32_t d,
                   int32_t rank, float ridge, int32_t basis_source, bool top16, float* x_mean, float* x_scale,
                   float* y_mean, float* left, float* basis, void* workspace, size_t workspace_bytes,
                   hipStream_t stream) {
  SPR_REQUIRE(bh >= 0 && m >= 1 && p >= 1 && d >= 1, "spr_rrr_fit: bad size");
  SPR_REQUIRE(m <= RRR_MAX && d <= RRR_MAX, "spr_rrr_fit: m and d must be at most %d (got m=%d, d=%d)", RRR_MAX, m,
              d);
  SPR_REQUIRE(p <= 2 * RRR_MAX, "spr_rrr_fit: p must be at most %d (got %d)", 2 * RRR_MAX, p);
  SPR_REQUIRE(xt_rows(p) * xt_stride(m, p) <= RRR_MAX * RRR_LS,
              "spr_rrr_fit: p=%d features with m=%d rows exceed the LDS-resident dual solve (64 ceil(p / 64) (m | 1) "
              "must be at most %d)", p, m, RRR_MAX * RRR_LS);
  SPR_REQUIRE(rank >= 1 && rank <= RRR_MAX_FIT_RANK && rank <= d && rank <= m,
              "spr_rrr_fit: rank %d outside [1, min(64, d, m)]", rank);
  SPR_REQUIRE(ridge >= 0.0f, "spr_rrr_fit: ridge must be non-negative");
  SPR_REQUIRE(basis_source == 0 || basis_source == 1, "spr_rrr_fit: basis_source must be 0 (raw) or 1 (fitted)");
  SPR_REQUIRE(!top16 || (m == T16_M && d == T16_D && rank == T16_R),
              "spr_rrr_fit_top16: needs m = 64, d = 128 and rank 16 (got m=%d, d=%d, rank=%d)", m, d, rank);
  SPR_REQUIRE(bh <= 65535, "spr_rrr_fit: too many heads");
  if (bh == 0) return SPR_OK;
  SPR_REQUIRE(x && y && x_mean && x_scale && y_mean && left && basis && workspace, "spr_rrr_fit: null pointer");
  if (workspace_bytes < spr_rrr_fit_workspace(bh)) {
    spr_set_error("spr_rrr_fit: workspace too small (%zu < %zu)", workspace_bytes, spr_rrr_fit_workspace(bh));
    return SPR_EWORKSPACE;
  }
  float* ws = static_cast<float*>(workspace);
  const uint32_t nb = static_cast<uint32_t>(bh);
  const bool dual = m < p;
  const int32_t ng = dual ? m : p;
  const int32_t gkind = dual ? GRAM_DUAL : GRAM_PRIMAL;
  rrr_stats_kernel<<<dim3(nb), 256, 0, stream>>>(x, y, weights, m, p, d, x_mean, x_scale, y_mean);
  SPR_LAUNCHED("rrr_stats_kernel");
  if (top16) {
    rrr_gram_kernel<<<dim3(nb, 10), 256, 0, stream>>>(x, y, weights, m, p, d, ridge, x_mean, x_scale, y_mean, nullptr,
                                                      0, 0, gkind, gkind, ws);
    SPR_LAUNCHED("rrr_gram_kernel");
    launch_rrr_factor(dim3(nb, 1), stream, ws, ng, d, rank, 1, basis);
    SPR_LAUNCHED("rrr_factor_kernel");
    if (basis_source == 0) {
      rrr_top16_kernel<<<dim3(nb), 256, 0, stream>>>(y, weights, y_mean, nullptr, 0, 0, T16_POWER_ITERS,
                                                     T16_NS_ITERS, basis);
    } else {
      rrr_fitted_kernel<<<dim3(nb), RRR_THREADS, 0, stream>>>(x, y, weights, m, p, d, ridge, x_mean, x_scale, y_mean,
                                                              ws);
      SPR_LAUNCHED("rrr_fitted_kernel");
      rrr_top16_kernel<<<dim3(nb), 256, 0, stream>>>(nullptr, nullptr, nullptr, ws + 2 * RRR_MAT,
                                                     int64_t(RRR_SLOTS) * RRR_MAT, RRR_MAX, T16_POWER_ITERS,
                                                     T16_NS_ITERS, basis);
    }
    SPR_LAUNCHED("rrr_top16_kernel");
  } else if (basis_source == 0) {
    rrr_gram_kernel<<<dim3(nb, 20), 256, 0, stream>>>(x, y, weights, m, p, d, ridge, x_mean, x_scale, y_mean, nullptr,
                                                      0, 0, gkind, GRAM_RESIDUAL, ws);
    SPR_LAUNCHED("rrr_gram_kernel");
    launch_rrr_factor(dim3(nb, 2), stream, ws, ng, d, rank, 0, basis);
    SPR_LAUNCHED("rrr_factor_kernel");
  } else {
    rrr_gram_kernel<<<dim3(nb, 10), 256, 0, stream>>>(x, y, weights, m, p, d, ridge, x_mean, x_scale, y_mean, nullptr,
                                                      0, 0, gkind, gkind, ws);
    SPR_LAUNCHED("rrr_gram_kernel");
    launch_rrr_factor(dim3(nb, 1), stream, ws, ng, d, rank, 1, basis);
    SPR_LAUNCHED("rrr_factor_kernel");
    rrr_fitted_kernel<<<dim3(nb), RRR_THREADS, 0, stream>>>(x, y, weights, m, p, d, ridge, x_mean, x_scale, y_mean,
                                                            ws);
    SPR_LAUNCHED("rrr_fitted_kernel");
    rrr_gram_kernel<<<dim3(nb, 10), 256, 0, stream>>>(x, y, weights, m, p, d, ridge, x_mean, x_scale, y_mean,
                                                      ws + 2 * RRR_MAT, int64_t(RRR_SLOTS) * RRR_MAT, RRR_MAX,
                                                      GRAM_PLAIN, GRAM_PLAIN, ws);
    SPR_LAUNCHED("rrr_gram_kernel");
    launch_rrr_factor(dim3(nb, 1), stream, ws, ng, d, rank, 0, basis);
    SPR_LAUNCHED("rrr_factor_kernel");
  }
  if (rank > RRR_MAX_RANK) {
    rrr_solve_kernel<true><<<dim3(nb), RRR_THREADS, 0, stream>>>(x, y, weights, m, p, d, rank, ridge, x_mean, x_scale,
                                                         y_mean, ws, basis, left);
  } else {
    rrr_solve_kernel<false><<<dim3(nb), RRR_THREADS, 0, stream>>>(x, y, weights, m, p, d, rank, ridge, x_mean, x_scale,
                                                         y_mean, ws, basis, left);
  }
  SPR_LAUNCHED("rrr_solve_kernel");
  return SPR_OK;
}
}  // namespace

// x [bh, m, p], y [bh, m, d], weights [bh, m] fp32 (nullable: unit weights, unbiased std);
// outputs x_mean [bh, p], x_scale [bh, p], y_mean [bh, d], left [bh, p, rank], basis
// [bh, d, rank] (fp32).  basis_source 0: raw residual, 1: fitted values.  m, d <= 128;
// p <= 128, or m < p <= 256 with 64 ceil(p / 64) (m | 1) <= 16512; 1 <= rank <= min(64, d, m).
extern "C" int spr_rrr_fit_ex(const float* x, const float* y, const float* weights, int64_t bh, int32_t m, int32_t p,
                              int32_t d, int32_t rank, float ridge, int32_t basis_source, float* x_mean,
                              float* x_scale, float* y_mean, float* left, float* basis, void* workspace,
                              size_t workspace_bytes, hipStream_t stream) {
  return rrr_fit_launch(x, y, weights, bh, m, p, d, rank, ridge, basis_source, false, x_mean, x_scale, y_mean, left,
                        basis, workspace, workspace_bytes, stream);
}

// spr_rrr_fit_ex with the N8 repair's top-16 subspace basis (rrr_top16_kernel) in place of
// the exact eigenvectors: m = 64, d = 128, rank = 16.
extern "C" int spr_rrr_fit_top16(const float* x, const float* y, const float* weights, int64_t bh, int32_t m,
                                 int32_t p, int32_t d, int32_t rank, float ridge, int32_t basis_source, float* x_mean,
                                 float* x_scale, float* y_mean, float* left, float* basis, void* workspace,
                                 size_t workspace_bytes, hipStream_t stream) {
  return rrr_fit_launch(x, y, weights, bh, m, p, d, rank, ridge, basis_source, true, x_mean, x_scale, y_mean, left,
                        basis, workspace, workspace_bytes, stream);
}

// The top-16 subspace basis alone: values [bh, 64, 128] fp32 -> basis [bh, 128, 16] fp32.
extern "C" int spr_rrr_top16_basis(const float* values, int64_t bh, int32_t power_iters, int32_t inv_sqrt_iters,
                                   float* basis, hipStream_t stream) {
  SPR_REQUIRE(bh >= 0 && bh <= 65535, "spr_rrr_top16_basis: bad head count");
  SPR_REQUIRE(power_iters > 0 && inv_sqrt_iters > 0 && power_iters <= 4096 && inv_sqrt_iters <= 4096,
              "spr_rrr_top16_basis: iteration counts must be in [1, 4096]");
  if (bh == 0) return SPR_OK;
  SPR_REQUIRE(values && basis, "spr_rrr_top16_basis: null pointer");
  rrr_top16_kernel<<<dim3(static_cast<uint32_t>(bh)), 256, 0, stream>>>(nullptr, nullptr, nullptr, values,
                                                                       int64_t(T16_M) * T16_D, T16_D, power_iters,
                                                                       inv_sqrt_iters, basis);
  SPR_LAUNCHED("rrr_top16_kernel");
  return SPR_OK;
}

// The raw-residual fit (basis_source 0).
extern "C" int spr_rrr_fit(const float* x, const float* y, const float* weights, int64_t bh, int32_t m, int32_t p,
                           int32_t d, int32_t rank, float ridge, float* x_mean, float* x_scale, float* y_mean,
                           float* left, float* basis, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  return spr_rrr_fit_ex(x, y, weights, bh, m, p, d, rank, ridge, 0, x_mean, x_scale, y_mean, left, basis, workspace,
                        workspace_bytes, stream);
}

// Top-`rank` right singular basis of a [bh, m, d] (fp32): the eigenvectors of a^T a,
// ascending eigenvalue order.  m, d <= 128, 1 <= rank <= min(64, d).
extern "C" int spr_rrr_output_basis(const float* a, int64_t bh, int32_t m, int32_t d, int32_t rank, float* basis,
                                    void* workspace, size_t workspace_bytes, hipStream_t stream) {
  SPR_REQUIRE(bh >= 0 && m >= 1 && d >= 1 && m <= RRR_MAX && d <= RRR_MAX,
              "spr_rrr_output_basis: m, d must be in [1, %d]", RRR_MAX);
  SPR_REQUIRE(rank >= 1 && rank <= RRR_MAX_FIT_RANK && rank <= d, "spr_rrr_output_basis: rank %d outside [1, min(64, d)]",
              rank);
  SPR_REQUIRE(bh <= 65535, "spr_rrr_output_basis: too many heads");
  if (bh == 0) return SPR_OK;
  SPR_REQUIRE(a && basis && workspace, "spr_rrr_output_basis: null pointer");
  if (workspace_bytes < spr_rrr_fit_workspace(bh)) {
    spr_set_error("spr_rrr_output_basis: workspace too small (%zu < %zu)", workspace_bytes,
                  spr_rrr_fit_workspace(bh));
    return SPR_EWORKSPACE;
  }
  float* ws = static_cast<float*>(workspace);
  const uint32_t nb = static_cast<uint32_t>(bh);
  rrr_gram_kernel<<<dim3(nb, 10), 256, 0, stream>>>(nullptr, nullptr, nullptr, m, 1, d, 0.0f, nullptr, nullptr,
                                                    nullptr, a, int64_t(m) * d, d, GRAM_PLAIN, GRAM_PLAIN, ws);
  SPR_LAUNCHED("rrr_gram_kernel");
  launch_rrr_factor(dim3(nb, 1), stream, ws, 1, d, rank, 0, basis);
  SPR_LAUNCHED("rrr_factor_kernel");
  return SPR_OK;
}

// State tensors x_mean [bh, p], x_scale [bh, p], y_mean [bh, d], left [bh, p, rank],
// basis [bh, d, rank] (fp32); prev_* all null (zero correction) or all given; out_* may
// alias the current state; recovered [bh] u8 (nullable).
extern "C" int spr_rrr_recover(const float* x_mean, const float* x_scale, const float* y_mean, const float* left,
                               const float* basis, const float* prev_x_mean, const float* prev_x_scale,
                               const float* prev_y_mean, const float* prev_left, const float* prev_basis, int64_t bh,
                               int32_t p, int32_t d, int32_t rank, float* out_x_mean, float* out_x_scale,
                               float* out_y_mean, float* out_left, float* out_basis, uint8_t* recovered,
                               hipStream_t stream) {
  SPR_REQUIRE(bh >= 0 && p >= 1 && d >= 1 && rank >= 1, "spr_rrr_recover: bad size");
  SPR_REQUIRE(bh <= 2147483647, "spr_rrr_recover: too many heads");
  if (bh == 0) return SPR_OK;
  SPR_REQUIRE(x_mean && x_scale && y_mean && left && basis && out_x_mean && out_x_scale && out_y_mean && out_left &&
                  out_basis,
              "spr_rrr_recover: null pointer");
  const int given = (prev_x_mean != nullptr) + (prev_x_scale != nullptr) + (prev_y_mean != nullptr) +
                    (prev_left != nullptr) + (prev_basis != nullptr);
  SPR_REQUIRE(given == 0 || given == 5, "spr_rrr_recover: give all five previous tensors or none");
  const RrrState cur{{x_mean, x_scale, y_mean, left, basis}};
  const RrrState prev{{prev_x_mean, prev_x_scale, prev_y_mean, prev_left, prev_basis}};
  const RrrStateOut out{{out_x_mean, out_x_scale, out_y_mean, out_left, out_basis}};
  rrr_recover_kernel<<<dim3(static_cast<uint32_t>(bh)), 256, 0, stream>>>(cur, prev, out, p, d, rank, recovered);
  SPR_LAUNCHED("rrr_recover_kernel");
  return SPR_OK;
}

// mats fp32 [bh, n, n] symmetric (symmetrize = 1: use 0.5 (A + A^T)); vecs fp32 [bh, n, rank]:
// the eigenvectors of the `rank` largest eigenvalues in ascending order; vals fp32 [bh, rank]
// (nullable): their Rayleigh quotients, ascending.  1 <= n <= 128, 1 <= rank <= min(64, n).
extern "C" int spr_sym_top_eig(const float* mats, int64_t bh, int32_t n, int32_t rank, int32_t symmetrize,
                               float* vecs, float* vals, hipStream_t stream) {
  SPR_REQUIRE(bh >= 0 && n >= 1 && n <= RRR_MAX, "spr_sym_top_eig: n=%d outside [1, %d]", n, RRR_MAX);
  SPR_REQUIRE(rank >= 1 && rank <= 64 && rank <= n, "spr_sym_top_eig: rank %d outside [1, min(64, n)]", rank);
  SPR_REQUIRE(bh <= 65535, "spr_sym_top_eig: too many matrices");
  if (bh == 0) return SPR_OK;
  SPR_REQUIRE(mats && vecs, "spr_sym_top_eig: null pointer");
  if (rank <= RRR_MAX_RANK) {
    sym_top_eig_kernel<RRR_MAX_RANK><<<dim3(static_cast<uint32_t>(bh)), RRR_THREADS, 0, stream>>>(
        mats, n, rank, symmetrize, vecs, vals);
  } else {
    sym_top_eig_kernel<64><<<dim3(static_cast<uint32_t>(bh)), RRR_THREADS, 0, stream>>>(mats, n, rank, symmetrize,
                                                                                       vecs, vals);
  }
  SPR_LAUNCHED("sym_top_eig_kernel");
  return SPR_OK;
}
