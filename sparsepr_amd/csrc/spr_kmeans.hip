// Batched Euclidean k-means building blocks (one Lloyd iteration = assign ->
// counting-sort argsort -> segmented mean).
//
// Replaces, for the SparsePR path:
//   euclid_assign_triton / _euclid_assign_kernel   (flash_kmeans/assign_euclid_triton.py:803-917, :1238-1412)
//   euclid_assign_inline_xsq_triton               (sparsepr/kmeans_utils.py:775-893)
//   triton_centroid_update_sorted_euclid          (flash_kmeans/centroid_update_triton.py:316-386)
//   original_centroids(_triton)                   (kernels/triton/centroid_reduction.py:138-196)
//   role_cluster_step_q64 / k64                   (kernels/n8_ext/csrc/n8_ops.cu:198-269, :499-539)
//
// assign (bf16): crossT[c, x] = C . X^T on v_mfma_f32_32x32x16_bf16.  A = 32
//   centroids x 16 dims read from an LDS tile, B = 32 points x 16 dims kept in
//   registers for the whole kernel.  In the 32x32 accumulator a lane owns one
//   point (column l % 32) and 16 centroids, so the argmin is lane-local plus one
//   exchange with lane l ^ 32.  dist = max((x_sq + c_sq) - 2 cross, 0); the
//   lowest index wins among exact minima, as in the reference.
// mean: one workgroup per (batch, cluster) reads the cluster's rows in sorted
//   order and accumulates in fp64 (exact for bf16 inputs, so the result does
//   not depend on summation order); mean32 = float(sum / count); empty
//   clusters keep the previous centroid.
// role assign (fp32): exact FP32 distance, sequential fmaf over dims, lowest
//   index on ties (n8_ops.cu:189-196 better_pair).
#include <algorithm>

#include "spr_common.h"

namespace {

using spr::u32x4;

constexpr int ASSIGN_THREADS = 256;
constexpr int ASSIGN_POINTS_PER_WAVE = 64;  // two 32-point MFMA column fragments
constexpr int ASSIGN_POINTS = 4 * ASSIGN_POINTS_PER_WAVE;
constexpr int CCHUNK = 64;  // centroids per LDS tile

// x_sq_mode: 0 = fp32 sum of fp32 squares (inline-x_sq kernel),
//            1 = bf16-rounded squares summed in fp32, result rounded to bf16
//                (flash_kmeans x_sq buffer of x.dtype).
template <int D>
__global__ __launch_bounds__(ASSIGN_THREADS, 2) void kmeans_assign_bf16_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ c, const float* __restrict__ c_sq,
    const float* __restrict__ x_sq_in, int x_sq_mode, float* __restrict__ x_sq_out, int64_t n, int32_t k,
    int32_t* __restrict__ labels) {
  static_assert(D % 32 == 0 && D <= 256, "D must be a multiple of 32, at most 256");
  constexpr int KSTEPS = D / 16;
  constexpr int ROW_BYTES = D * 2 + 16;  // padded LDS row: conflict-free 16-byte reads
  constexpr int PIECES = CCHUNK * D / 8; // 16-byte pieces per centroid tile
  constexpr int PIECES_PER_THREAD = PIECES / ASSIGN_THREADS;
  static_assert(PIECES % ASSIGN_THREADS == 0, "tile pieces must divide evenly");

  __shared__ __attribute__((aligned(16))) uint8_t tile[2][CCHUNK * ROW_BYTES];
  __shared__ float tile_csq[2][CCHUNK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 31;
  const int half = lane >> 5;
  const int64_t b = blockIdx.y;
  const uint16_t* xb = x + b * n * D;
  const uint16_t* cb = c + static_cast<int64_t>(b) * k * D;
  const float* csqb = c_sq + static_cast<int64_t>(b) * k;

  // ---- points of this lane: two fragments of 32 points
  const int64_t p0 = static_cast<int64_t>(blockIdx.x) * ASSIGN_POINTS + wave * ASSIGN_POINTS_PER_WAVE + col;
  u32x4 xf[2][KSTEPS];
  float xsq[2];
#pragma unroll
  for (int f = 0; f < 2; ++f) {
    const int64_t p = p0 + 32 * f;
    const bool live = p < n;
    float part = 0.0f;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      u32x4 v = live ? *reinterpret_cast<const u32x4*>(xb + p * D + s * 16 + half * 8) : u32x4{0, 0, 0, 0};
      xf[f][s] = v;
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = spr::bf16_lo(w[e]);
        const float hi = spr::bf16_hi(w[e]);
        if (x_sq_mode == 1) {
          // squares rounded to bf16 (v_cvt_pk_bf16_f32, round to nearest even), summed in order
          const uint32_t sq2 = spr::pack_bf16x2_rne(lo * lo, hi * hi);
          part += spr::bf16_lo(sq2);
          part += spr::bf16_hi(sq2);
        } else {
          part = __builtin_fmaf(lo, lo, part);
          part = __builtin_fmaf(hi, hi, part);
        }
      }
    }
    const float other = __shfl_xor(part, 32, 64);
    float total = part + other;
    if (x_sq_mode == 1) total = spr::bf16_lo(spr::pack_bf16x2_rne(total, 0.0f));
    if (x_sq_in != nullptr) {
      total = live ? x_sq_in[b * n + p] : 0.0f;
    } else if (x_sq_out != nullptr && live && half == 0) {
      x_sq_out[b * n + p] = total;  // reused by later iterations over the same points
    }
    xsq[f] = total;
  }

  float best[2] = {3.4e38f, 3.4e38f};
  int32_t best_idx[2] = {0, 0};

  const int nchunks = static_cast<int>((k + CCHUNK - 1) / CCHUNK);
  u32x4 pre[PIECES_PER_THREAD];
  float pre_csq = 0.0f;

  auto fetch = [&](int chunk) {
#pragma unroll
    for (int i = 0; i < PIECES_PER_THREAD; ++i) {
      const int piece = tid + i * ASSIGN_THREADS;
      const int row = piece / (D / 8);
      const int vec = piece % (D / 8);
      const int64_t cidx = static_cast<int64_t>(chunk) * CCHUNK + row;
      pre[i] = cidx < k ? *reinterpret_cast<const u32x4*>(cb + cidx * D + vec * 8) : u32x4{0, 0, 0, 0};
    }
    if (tid < CCHUNK) {
      const int64_t cidx = static_cast<int64_t>(chunk) * CCHUNK + tid;
      pre_csq = cidx < k ? csqb[cidx] : __builtin_huge_valf();  // padding centroids never win
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int i = 0; i < PIECES_PER_THREAD; ++i) {
      const int piece = tid + i * ASSIGN_THREADS;
      const int row = piece / (D / 8);
      const int vec = piece % (D / 8);
      *reinterpret_cast<u32x4*>(&tile[buf][row * ROW_BYTES + vec * 16]) = pre[i];
    }
    if (tid < CCHUNK) tile_csq[buf][tid] = pre_csq;
  };

  fetch(0);
  stash(0);
  __syncthreads();

  for (int chunk = 0; chunk < nchunks; ++chunk) {
    const int buf = chunk & 1;
    if (chunk + 1 < nchunks) fetch(chunk + 1);
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      spr::f32x16 acc0 = {}, acc1 = {};
      const uint8_t* arow = &tile[buf][(blk * 32 + col) * ROW_BYTES + half * 16];
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(arow + s * 32);
        acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(spr::as_bf16x8(a), spr::as_bf16x8(xf[0][s]), acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(spr::as_bf16x8(a), spr::as_bf16x8(xf[1][s]), acc1, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int local = blk * 32 + 8 * i + 4 * half + j;
          const int32_t cidx = chunk * CCHUNK + local;
          const float csq = tile_csq[buf][local];
          // (x_sq + c_sq) - 2 cross with one rounding per step: 2 * cross is exact, so
          // fma(-2, cross, x_sq + c_sq) rounds exactly like the reference's subtraction.
          const float d0 = fmaxf(__builtin_fmaf(-2.0f, acc0[4 * i + j], __fadd_rn(xsq[0], csq)), 0.0f);
          const float d1 = fmaxf(__builtin_fmaf(-2.0f, acc1[4 * i + j], __fadd_rn(xsq[1], csq)), 0.0f);
          const bool t0 = d0 < best[0];
          const bool t1 = d1 < best[1];
          best[0] = t0 ? d0 : best[0];
          best_idx[0] = t0 ? cidx : best_idx[0];
          best[1] = t1 ? d1 : best[1];
          best_idx[1] = t1 ? cidx : best_idx[1];
        }
      }
    }
    if (chunk + 1 < nchunks) stash(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int f = 0; f < 2; ++f) {
    const float od = __shfl_xor(best[f], 32, 64);
    const int32_t oi = __shfl_xor(best_idx[f], 32, 64);
    if (od < best[f] || (od == best[f] && oi < best_idx[f])) {
      best[f] = od;
      best_idx[f] = oi;
    }
    const int64_t p = p0 + 32 * f;
    if (half == 0 && p < n) labels[b * n + p] = best_idx[f];
  }
}

// fp32 x -> TF32 (10 stored mantissa bits), nearest with ties away from zero: the
// operand rounding of tl.dot on fp32 inputs (input_precision "tf32", Triton's default).
__device__ __forceinline__ uint32_t tf32_rna_bits(float v) { return (__float_as_uint(v) + 0x1000u) & 0xFFFFE000u; }

// fp16 images of TF32 values.  v~ = tf32(v) has 11 significant bits, as many as fp16
// carries, so v~ 2^e is exact in fp16 wherever it lies in fp16's normal range.  The scale
// 2^e puts the largest magnitude of a point row (or of a centroid tile) in [2^14, 2^15);
// entries below 2^-29 of it become fp16 subnormals and keep only their leading bits, a
// change far below the fp32 rounding of the distance they enter.
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
__device__ __forceinline__ int tf32_scale_exp(float amax) {
  int e = 0;
  if (amax > 0.0f && amax < __builtin_huge_valf()) e = __builtin_amdgcn_frexp_expf(amax);  // amax < 2^e
  return 15 - e;
}
__device__ __forceinline__ uint32_t tf32_f16_bits(float v, int se) {
  const float t = __builtin_ldexpf(__uint_as_float(tf32_rna_bits(v)), se);
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(t));
}
__device__ __forceinline__ float tf32_abs(float v) { return fabsf(__uint_as_float(tf32_rna_bits(v))); }

// labels = argmin_k max((x_sq + c_sq) - 2 x.c, 0) for fp32 x and centroids, with the
// dot product of their TF32 roundings (exact products, fp32 accumulation): the
// flash-kmeans assign on fp32 inputs (assign_euclid_triton.py:897, kmeans_utils.py:829).
// x_sq (when not given) is the fp32 sum of the fp32 squares of x itself
// (kmeans_utils.py:812-814).  The layout follows kmeans_assign_bf16_kernel: 256 points
// per workgroup, 64-centroid LDS tiles, v_mfma_f32_32x32x16_f16 on the scaled fp16 images
// (one product per 16-dim step: every product of two TF32 values is exact in the fp32
// accumulator), and the accumulated dot taken back by the two exact power-of-two scales
// inside the distance's fused multiply-add.
template <int D>
__global__ __launch_bounds__(ASSIGN_THREADS, D > 64 ? 1 : 2) void kmeans_assign_tf32_kernel(
    const float* __restrict__ x, const float* __restrict__ c, const float* __restrict__ c_sq,
    const float* __restrict__ x_sq_in, float* __restrict__ x_sq_out, int64_t n, int32_t k,
    int32_t* __restrict__ labels) {
  static_assert(D % 16 == 0 && D <= 128, "D must be a multiple of 16, at most 128");
  constexpr int KSTEPS = D / 16;
  constexpr int ROW_BYTES = D * 2 + 16;     // padded fp16 LDS row
  constexpr int QUADS = CCHUNK * D / 4;     // 4-float pieces per centroid tile
  constexpr int QUADS_PER_THREAD = QUADS / ASSIGN_THREADS;
  static_assert(QUADS % ASSIGN_THREADS == 0, "tile pieces must divide evenly");

  __shared__ __attribute__((aligned(16))) uint8_t tile[2][CCHUNK * ROW_BYTES];
  __shared__ float tile_csq[2][CCHUNK];
  __shared__ int tile_exp[2];
  __shared__ float tile_max[ASSIGN_THREADS / 64];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 31;
  const int half = lane >> 5;
  const int64_t b = blockIdx.y;
  const float* xb = x + b * n * D;
  const float* cb = c + static_cast<int64_t>(b) * k * D;
  const float* csqb = c_sq + static_cast<int64_t>(b) * k;

  // ---- points of this lane: two fragments of 32 points, 8 dims per k-step; the row's
  // largest TF32 magnitude (both lanes of the row) sets its scale
  const int64_t p0 = static_cast<int64_t>(blockIdx.x) * ASSIGN_POINTS + wave * ASSIGN_POINTS_PER_WAVE + col;
  u32x4 xf[2][KSTEPS];
  float xsq[2];
  int xexp[2];
#pragma unroll
  for (int f = 0; f < 2; ++f) {
    const int64_t p = p0 + 32 * f;
    const bool live = p < n;
    float part = 0.0f, amax = 0.0f;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      const spr::f32x4* src = reinterpret_cast<const spr::f32x4*>(xb + p * D + s * 16 + half * 8);
      const spr::f32x4 v0 = live ? src[0] : spr::f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      const spr::f32x4 v1 = live ? src[1] : spr::f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      const float e[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        part = __fadd_rn(part, __fmul_rn(e[u], e[u]));
        amax = fmaxf(amax, tf32_abs(e[u]));
      }
    }
    amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
    xexp[f] = tf32_scale_exp(amax);
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {  // the row again (cached), now as scaled fp16
      const spr::f32x4* src = reinterpret_cast<const spr::f32x4*>(xb + p * D + s * 16 + half * 8);
      const spr::f32x4 v0 = live ? src[0] : spr::f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      const spr::f32x4 v1 = live ? src[1] : spr::f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      const float e[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
      uint32_t h[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) h[u] = tf32_f16_bits(e[u], xexp[f]);
      xf[f][s] = u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
    }
    const float other = __shfl_xor(part, 32, 64);
    float total = part + other;
    if (x_sq_in != nullptr) {
      total = live ? x_sq_in[b * n + p] : 0.0f;
    } else if (x_sq_out != nullptr && live && half == 0) {
      x_sq_out[b * n + p] = total;
    }
    xsq[f] = total;
  }

  float best[2] = {3.4e38f, 3.4e38f};
  int32_t best_idx[2] = {0, 0};
  const int nchunks = static_cast<int>((k + CCHUNK - 1) / CCHUNK);
  spr::f32x4 pre[QUADS_PER_THREAD];
  float pre_csq = 0.0f;

  auto fetch = [&](int chunk) {
#pragma unroll
    for (int i = 0; i < QUADS_PER_THREAD; ++i) {
      const int quad = tid + i * ASSIGN_THREADS;
      const int row = quad / (D / 4);
      const int vec = quad % (D / 4);
      const int64_t cidx = static_cast<int64_t>(chunk) * CCHUNK + row;
      pre[i] = cidx < k ? *reinterpret_cast<const spr::f32x4*>(cb + cidx * D + vec * 4)
                        : spr::f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    if (tid < CCHUNK) {
      const int64_t cidx = static_cast<int64_t>(chunk) * CCHUNK + tid;
      pre_csq = cidx < k ? csqb[cidx] : __builtin_huge_valf();  // padding centroids never win
    }
  };
  // Two barriers: the tile's largest magnitude (over every thread's pieces), then the
  // scaled fp16 tile.  The tile being written was last read before the barrier that
  // ended the previous chunk.
  auto stash = [&](int buf) {
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < QUADS_PER_THREAD; ++i) {
#pragma unroll
      for (int u = 0; u < 4; ++u) m = fmaxf(m, tf32_abs(pre[i][u]));
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if (lane == 0) tile_max[wave] = m;
    __syncthreads();
    float tm = tile_max[0];
#pragma unroll
    for (int w = 1; w < ASSIGN_THREADS / 64; ++w) tm = fmaxf(tm, tile_max[w]);
    const int et = tf32_scale_exp(tm);
#pragma unroll
    for (int i = 0; i < QUADS_PER_THREAD; ++i) {
      const int quad = tid + i * ASSIGN_THREADS;
      const int row = quad / (D / 4);
      const int vec = quad % (D / 4);
      uint32_t h[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) h[u] = tf32_f16_bits(pre[i][u], et);
      *reinterpret_cast<uint2*>(&tile[buf][row * ROW_BYTES + vec * 8]) = uint2{h[0] | (h[1] << 16),
                                                                              h[2] | (h[3] << 16)};
    }
    if (tid < CCHUNK) tile_csq[buf][tid] = pre_csq;
    if (tid == 0) tile_exp[buf] = et;
  };

  fetch(0);
  stash(0);
  __syncthreads();

  for (int chunk = 0; chunk < nchunks; ++chunk) {
    const int buf = chunk & 1;
    if (chunk + 1 < nchunks) fetch(chunk + 1);
    // -2 x.c = acc * (-2 2^-(point exponent + tile exponent)), exact
    const int et = tile_exp[buf];
    const float k0 = __builtin_ldexpf(-2.0f, -(xexp[0] + et));
    const float k1 = __builtin_ldexpf(-2.0f, -(xexp[1] + et));
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      spr::f32x16 acc0 = {}, acc1 = {};
      const int roff = (blk * 32 + col) * ROW_BYTES + half * 16;
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) {
        const f16x8_t a = __builtin_bit_cast(f16x8_t, *reinterpret_cast<const u32x4*>(&tile[buf][roff + s * 32]));
        acc0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, __builtin_bit_cast(f16x8_t, xf[0][s]), acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, __builtin_bit_cast(f16x8_t, xf[1][s]), acc1, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int local = blk * 32 + 8 * i + 4 * half + j;
          const int32_t cidx = chunk * CCHUNK + local;
          const float csq = tile_csq[buf][local];
          const float d0 = fmaxf(__builtin_fmaf(k0, acc0[4 * i + j], __fadd_rn(xsq[0], csq)), 0.0f);
          const float d1 = fmaxf(__builtin_fmaf(k1, acc1[4 * i + j], __fadd_rn(xsq[1], csq)), 0.0f);
          const bool t0 = d0 < best[0];
          const bool t1 = d1 < best[1];
          best[0] = t0 ? d0 : best[0];
          best_idx[0] = t0 ? cidx : best_idx[0];
          best[1] = t1 ? d1 : best[1];
          best_idx[1] = t1 ? cidx : best_idx[1];
        }
      }
    }
    if (chunk + 1 < nchunks) stash(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int f = 0; f < 2; ++f) {
    const float od = __shfl_xor(best[f], 32, 64);
    const int32_t oi = __shfl_xor(best_idx[f], 32, 64);
    if (od < best[f] || (od == best[f] && oi < best_idx[f])) {
      best[f] = od;
      best_idx[f] = oi;
    }
    const int64_t p = p0 + 32 * f;
    if (half == 0 && p < n) labels[b * n + p] = best_idx[f];
  }
}

// c_sq[b, k] = sum_d float(c)^2 in fp32, sequential over d.
template <typename T>
__global__ void centroid_sq_kernel(const T* __restrict__ c, int64_t rows, int32_t d, float* __restrict__ out) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  float s = 0.0f;
  for (int t = 0; t < d; ++t) {
    float v;
    if constexpr (sizeof(T) == 2) {
      v = spr::bf16_to_f32(c[r * d + t]);
    } else {
      v = c[r * d + t];
    }
    s = __builtin_fmaf(v, v, s);
  }
  out[r] = s;
}

// The assignment with the batch's centroids resident in LDS: a 1024-thread
// workgroup (four waves per SIMD) stages all k centroids once (padded rows, and
// -c_sq / 2 per centroid: zeros and -inf past k), then each wave walks 64-point
// blocks of the batch against them with no further barriers, centroid reloads or
// staging work.  The MFMA accumulator starts at -c_sq / 2, so it ends at
// x.c - c_sq / 2 and the nearest centroid of a step is its largest entry; the
// distance x_sq + c_sq - 2 x.c is formed once per step for its best candidate.
// Used while the padded centroids fit in LDS (k <= ASSIGN_RESIDENT_K at D = 128).
constexpr int ASSIGN_RESIDENT_K = 512;

constexpr int ASSIGN_RESIDENT_THREADS = 1024;

template <int D>
__global__ __launch_bounds__(ASSIGN_RESIDENT_THREADS, 1) void kmeans_assign_resident_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ c, const float* __restrict__ c_sq,
    const float* __restrict__ x_sq_in, int x_sq_mode, float* __restrict__ x_sq_out, int64_t n, int32_t k,
    int32_t* __restrict__ labels) {
  constexpr int KSTEPS = D / 16;
  constexpr int ROW_BYTES = D * 2 + 16;  // padded LDS row: conflict-free 16-byte reads
  extern __shared__ __attribute__((aligned(16))) uint8_t assign_smem[];
  const int kpad = (k + CCHUNK - 1) / CCHUNK * CCHUNK;
  uint8_t* cent = assign_smem;
  float* csq_l = reinterpret_cast<float*>(assign_smem + static_cast<int64_t>(kpad) * ROW_BYTES);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 31;
  const int half = lane >> 5;
  const int64_t b = blockIdx.y;
  const uint16_t* xb = x + b * n * D;
  const uint16_t* cb = c + static_cast<int64_t>(b) * k * D;
  const float* csqb = c_sq + static_cast<int64_t>(b) * k;

  for (int piece = tid; piece < kpad * (D / 8); piece += blockDim.x) {
    const int row = piece / (D / 8);
    const int vec = piece % (D / 8);
    const u32x4 v = row < k ? *reinterpret_cast<const u32x4*>(cb + static_cast<int64_t>(row) * D + vec * 8)
                            : u32x4{0, 0, 0, 0};
    *reinterpret_cast<u32x4*>(cent + row * ROW_BYTES + vec * 16) = v;
  }
  for (int r = tid; r < kpad; r += blockDim.x) csq_l[r] = r < k ? -0.5f * csqb[r] : -__builtin_huge_valf();
  __syncthreads();

  const int64_t blocks = (n + ASSIGN_POINTS_PER_WAVE - 1) / ASSIGN_POINTS_PER_WAVE;
  for (int64_t blk = static_cast<int64_t>(blockIdx.x) * (blockDim.x / 64) + wave; blk < blocks;
       blk += static_cast<int64_t>(gridDim.x) * (blockDim.x / 64)) {
    const int64_t p0 = blk * ASSIGN_POINTS_PER_WAVE + col;
    u32x4 xf[2][KSTEPS];
    float xsq[2];
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      const int64_t p = p0 + 32 * f;
      const bool live = p < n;
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s)
        xf[f][s] = live ? *reinterpret_cast<const u32x4*>(xb + p * D + s * 16 + half * 8) : u32x4{0, 0, 0, 0};
      if (x_sq_in != nullptr) {  // later Lloyd iterations: the norms of the first
        xsq[f] = live ? x_sq_in[b * n + p] : 0.0f;
        continue;
      }
      float part = 0.0f;
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) {
        const uint32_t w[4] = {xf[f][s].x, xf[f][s].y, xf[f][s].z, xf[f][s].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float lo = spr::bf16_lo(w[e]);
          const float hi = spr::bf16_hi(w[e]);
          if (x_sq_mode == 1) {
            const uint32_t sq2 = spr::pack_bf16x2_rne(lo * lo, hi * hi);
            part += spr::bf16_lo(sq2);
            part += spr::bf16_hi(sq2);
          } else {
            part = __builtin_fmaf(lo, lo, part);
            part = __builtin_fmaf(hi, hi, part);
          }
        }
      }
      const float other = __shfl_xor(part, 32, 64);
      float total = part + other;
      if (x_sq_mode == 1) total = spr::bf16_lo(spr::pack_bf16x2_rne(total, 0.0f));
      if (x_sq_out != nullptr && live && half == 0) x_sq_out[b * n + p] = total;
      xsq[f] = total;
    }

    // Per 32-centroid step each lane scans its 16 candidates (index c0 + 4 half +
    // 8i + j, ascending in (i, j)) for the step's largest accumulator entry
    // x.c - c_sq / 2 (the smallest unclamped distance), strict >, so the lowest
    // index wins among equal entries; the step's distance x_sq - 2 max (one
    // rounding) then meets the running best once.  The clamp max(r, 0) changes the
    // answer only when some distance is <= 0: all such candidates tie at 0 and the
    // lowest index among them wins, which a (rare, wave-uniform) rescan restores.
    float best[2] = {3.4e38f, 3.4e38f};
    int32_t best_idx[2] = {0, 0};
    for (int c0 = 0; c0 < kpad; c0 += 32) {
      // accumulator = -c_sq / 2 + x . c (row 8i + 4 half + j of the step: centroid c0 + that)
      const float* cs = csq_l + c0 + 4 * half;
      spr::f32x16 cinit;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const spr::f32x4 c4 = *reinterpret_cast<const spr::f32x4*>(cs + 8 * i);
#pragma unroll
        for (int j = 0; j < 4; ++j) cinit[4 * i + j] = c4[j];
      }
      spr::f32x16 acc0, acc1;
      const uint8_t* arow = cent + (c0 + col) * ROW_BYTES + half * 16;
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(arow + s * 32);
        acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(spr::as_bf16x8(a), spr::as_bf16x8(xf[0][s]),
                                                       s == 0 ? cinit : acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(spr::as_bf16x8(a), spr::as_bf16x8(xf[1][s]),
                                                       s == 0 ? cinit : acc1, 0, 0, 0);
      }
      // step-local argmax of the accumulator (the smallest c_sq - 2 x.c): four chains per
      // fragment, merged in ascending offset order, strict >, so the lowest offset wins ties
      float lb[2];
      int32_t lo[2];
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        const spr::f32x16& acc = f == 0 ? acc0 : acc1;
        float cb[4];
        int32_t co[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          cb[i] = acc[4 * i];
          co[i] = 8 * i;
#pragma unroll
          for (int j = 1; j < 4; ++j) {
            const bool t = acc[4 * i + j] > cb[i];
            co[i] = t ? 8 * i + j : co[i];
            cb[i] = fmaxf(acc[4 * i + j], cb[i]);
          }
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const bool t = cb[2 * h + 1] > cb[2 * h];
          co[2 * h] = t ? co[2 * h + 1] : co[2 * h];
          cb[2 * h] = fmaxf(cb[2 * h + 1], cb[2 * h]);
        }
        const bool t = cb[2] > cb[0];
        lo[f] = t ? co[2] : co[0];
        // the distance x_sq + c_sq - 2 x.c of the step's best, one rounding
        lb[f] = __builtin_fmaf(-2.0f, fmaxf(cb[2], cb[0]), xsq[f]);
      }
      if (__ballot(lb[0] <= 0.0f || lb[1] <= 0.0f) != 0ull) {
        // the clamp at 0: the first candidate whose distance is <= 0, in index order
#pragma unroll
        for (int f = 0; f < 2; ++f) {
          const spr::f32x16& acc = f == 0 ? acc0 : acc1;
          bool found = false;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const float r = __builtin_fmaf(-2.0f, acc[4 * i + j], xsq[f]);
              if (lb[f] <= 0.0f && !found && r <= 0.0f) {
                lo[f] = 8 * i + j;
                found = true;
              }
            }
          }
          lb[f] = fmaxf(lb[f], 0.0f);
        }
      }
      const int32_t base = c0 + 4 * half;
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        const bool t = lb[f] < best[f];
        best[f] = t ? lb[f] : best[f];
        best_idx[f] = t ? base + lo[f] : best_idx[f];
      }
    }
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      const float od = __shfl_xor(best[f], 32, 64);
      const int32_t oi = __shfl_xor(best_idx[f], 32, 64);
      if (od < best[f] || (od == best[f] && oi < best_idx[f])) {
        best[f] = od;
        best_idx[f] = oi;
      }
      const int64_t p = p0 + 32 * f;
      if (half == 0 && p < n) labels[b * n + p] = best_idx[f];
    }
  }
}


// The TF32 assignment with a batch's centroids resident in LDS: one workgroup per CU
// (768 or 512 threads, pipe_threads) stages the scaled fp16 images of the centroids'
// TF32 roundings once (padded rows; zeros and c_sq = +inf past k; the per-64-centroid
// tile exponents of kmeans_assign_tf32_kernel, so both kernels form the same exact
// products) and its waves walk 64-point blocks against them with no further barriers
// (v_mfma_f32_32x32x16_f16 on the scaled images).
//
// Per 32-centroid step each lane scans its 16 candidates (index c0 + 4 half + 8i + j,
// ascending in (i, j)) for the step's smallest c_sq - 2 cross (one fused multiply-add;
// 2 cross is exact), strict <, so the lowest index wins among equal minima; x_sq is
// added to the step's best only, and the result meets the running best once.  (The
// streamed kernel forms (x_sq + c_sq) - 2 cross per candidate: the two can differ only
// between candidates within a few fp32 ulp of x_sq + c_sq of each other.)  The clamp
// max(r, 0) changes the answer only when some r <= 0: all such candidates tie at 0 and
// the lowest index among them wins, which a (rare, wave-uniform) rescan of the step
// restores.  The MFMAs of step s + 1 are issued in the same instruction stream as the
// argmin of step s (interleaved by sched_group_barrier), so the matrix pipe and the VALU
// work at the same time within a wave.
//
// A workgroup walks a contiguous range of the (batch, block) space; where the range
// crosses into the next batch, the workgroup stages that batch's centroids in turn.
// Threads per workgroup: three waves per SIMD where the registers allow it (D <= 64: 165 and
// 168 VGPRs, the latter with 12 bytes of spill), two above.  At the N8 shapes 768 threads took
// the K assign (Kc 1000, D 48) from 658 to 590 us and the Q assign (Qc 300, D 64) from 358
// to 323 us against 512, with the same labels.
template <int D>
constexpr int pipe_threads() { return D <= 64 ? 768 : 512; }
constexpr size_t PIPE_LDS_LIMIT = 160 * 1024;

template <int D>
constexpr size_t pipe_lds_bytes(int64_t kpad) {
  return static_cast<size_t>(kpad) * (D * 2 + 16) + static_cast<size_t>(kpad) * 4 +
         static_cast<size_t>(kpad / CCHUNK) * 4;
}

template <int D>
__global__ __launch_bounds__(pipe_threads<D>(), 1) void kmeans_assign_tf32_resident_kernel(
    const float* __restrict__ x, const float* __restrict__ c, const float* __restrict__ c_sq,
    const float* __restrict__ x_sq_in, float* __restrict__ x_sq_out, int64_t batch, int64_t n, int32_t k,
    int32_t* __restrict__ labels) {
  static_assert(D % 16 == 0 && D <= 128, "D must be a multiple of 16, at most 128");
  constexpr int KSTEPS = D / 16;
  constexpr int ROW_BYTES = D * 2 + 16;  // padded LDS row: conflict-free 16-byte reads
  constexpr int PIPE_THREADS = pipe_threads<D>();
  constexpr int PIPE_WAVES = PIPE_THREADS / 64;
  extern __shared__ __attribute__((aligned(16))) uint8_t assign_smem[];
  const int kpad = (k + CCHUNK - 1) / CCHUNK * CCHUNK;  // a multiple of 64: an even number of steps
  uint8_t* cent = assign_smem;
  float* csq_l = reinterpret_cast<float*>(assign_smem + static_cast<int64_t>(kpad) * ROW_BYTES);
  int* cexp_l = reinterpret_cast<int*>(csq_l + kpad);  // scale exponent per 64-centroid tile

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 31;
  const int half = lane >> 5;

  const int64_t nblk = (n + ASSIGN_POINTS_PER_WAVE - 1) / ASSIGN_POINTS_PER_WAVE;  // 64-point blocks per batch
  const int64_t total = batch * nblk;
  const int64_t g_begin = total * blockIdx.x / gridDim.x;
  const int64_t g_end = total * (blockIdx.x + 1) / gridDim.x;

  for (int64_t g0 = g_begin; g0 < g_end;) {
    const int64_t b = g0 / nblk;
    const int64_t seg_end = std::min(g_end, (b + 1) * nblk);
    const float* csqb = c_sq + b * k;

    // ---- stage batch b's centroids (every wave is past the previous batch's blocks)
    __syncthreads();
    const float* cb = c + b * k * D;
    for (int t = wave; t < kpad / CCHUNK; t += PIPE_WAVES) {
      float m = 0.0f;
      for (int i = lane; i < CCHUNK * D / 4; i += 64) {
        const int row = t * CCHUNK + i / (D / 4);
        const spr::f32x4 v = row < k ? *reinterpret_cast<const spr::f32x4*>(cb + static_cast<int64_t>(row) * D +
                                                                          (i % (D / 4)) * 4)
                                     : spr::f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int u = 0; u < 4; ++u) m = fmaxf(m, tf32_abs(v[u]));
      }
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
      const int et = tf32_scale_exp(m);
      if (lane == 0) cexp_l[t] = et;
      for (int i = lane; i < CCHUNK * D / 4; i += 64) {
        const int row = t * CCHUNK + i / (D / 4);
        const int vec = i % (D / 4);
        const spr::f32x4 v = row < k ? *reinterpret_cast<const spr::f32x4*>(cb + static_cast<int64_t>(row) * D +
                                                                          vec * 4)
                                     : spr::f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        uint32_t h[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) h[u] = tf32_f16_bits(v[u], et);
        *reinterpret_cast<uint2*>(cent + row * ROW_BYTES + vec * 8) = uint2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
      }
    }

    for (int r = tid; r < kpad; r += PIPE_THREADS) csq_l[r] = r < k ? csqb[r] : __builtin_huge_valf();
    __syncthreads();

    for (int64_t g = g0 + wave; g < seg_end; g += PIPE_WAVES) {
      const int64_t p0 = (g - b * nblk) * ASSIGN_POINTS_PER_WAVE + col;
      u32x4 xf[2][KSTEPS];
      float xsq[2];
      int xexp[2] = {0, 0};
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        const int64_t p = p0 + 32 * f;
        const bool live = p < n;
        const float* xb = x + b * n * D;
        float part = 0.0f, amax = 0.0f;
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) {
          const spr::f32x4* src = reinterpret_cast<const spr::f32x4*>(xb + p * D + s * 16 + half * 8);
          const spr::f32x4 v0 = live ? src[0] : spr::f32x4{0.0f, 0.0f, 0.0f, 0.0f};
          const spr::f32x4 v1 = live ? src[1] : spr::f32x4{0.0f, 0.0f, 0.0f, 0.0f};
          const float e[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            part = __fadd_rn(part, __fmul_rn(e[u], e[u]));
            amax = fmaxf(amax, tf32_abs(e[u]));
          }
        }
        amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
        xexp[f] = tf32_scale_exp(amax);
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) {  // the row again (cached), now as scaled fp16
          const spr::f32x4* src = reinterpret_cast<const spr::f32x4*>(xb + p * D + s * 16 + half * 8);
          const spr::f32x4 v0 = live ? src[0] : spr::f32x4{0.0f, 0.0f, 0.0f, 0.0f};
          const spr::f32x4 v1 = live ? src[1] : spr::f32x4{0.0f, 0.0f, 0.0f, 0.0f};
          const float e[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
          uint32_t h[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) h[u] = tf32_f16_bits(e[u], xexp[f]);
          xf[f][s] = u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
        }
        const float other = __shfl_xor(part, 32, 64);
        float tot = part + other;
        if (x_sq_in != nullptr) {
          tot = live ? x_sq_in[b * n + p] : 0.0f;
        } else if (x_sq_out != nullptr && live && half == 0) {
          x_sq_out[b * n + p] = tot;
        }
        xsq[f] = tot;
      }

      float best[2] = {3.4e38f, 3.4e38f};
      int32_t best_idx[2] = {0, 0};

      // MFMAs of the 32 centroids from c0 into acc (both point fragments)
      auto mfma_step = [&](spr::f32x16 (&acc)[2], int c0) {
        const uint8_t* arow = cent + (c0 + col) * ROW_BYTES + half * 16;
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) {
          const u32x4 a = *reinterpret_cast<const u32x4*>(arow + s * 32);
#pragma unroll
          for (int f = 0; f < 2; ++f) {
            acc[f] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                            __builtin_bit_cast(f16x8_t, xf[f][s]),
                                                            s == 0 ? spr::f32x16{} : acc[f], 0, 0, 0);
          }
        }
      };
      // -2 x.c = acc * kf, kf = -2 2^-(point exponent + tile exponent) (exact)
      auto factors = [&](int c0, float (&kf)[2]) {
        const int et = cexp_l[c0 / CCHUNK];
        kf[0] = __builtin_ldexpf(-2.0f, -(xexp[0] + et));
        kf[1] = __builtin_ldexpf(-2.0f, -(xexp[1] + et));
      };
      // step-local (min, argmin) of c_sq - 2 x.c over acc (centroids c0 ..), then the best's
      // unclamped distance x_sq + (c_sq - 2 x.c)
      auto scan = [&](const spr::f32x16 (&acc)[2], int c0, const float (&kf)[2], float (&lb)[2],
                      int32_t (&lo)[2]) {
        const float* cs = csq_l + c0 + 4 * half;
        spr::f32x4 c4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) c4[i] = *reinterpret_cast<const spr::f32x4*>(cs + 8 * i);
        // eight independent chains (fragment f, row group i: offsets 8i .. 8i + 3), then a
        // merge in ascending offset order that takes a later chain only when strictly
        // smaller, so the lowest offset still wins among equal minima
        float cb[2][4];
        int32_t co[2][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
          for (int f = 0; f < 2; ++f) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float r = __builtin_fmaf(kf[f], acc[f][4 * i + j], c4[i][j]);  // c_sq - 2 x.c
              if (j == 0) {
                cb[f][i] = r;
                co[f][i] = 8 * i;
              } else {
                const bool t = r < cb[f][i];
                co[f][i] = t ? 8 * i + j : co[f][i];
                cb[f][i] = fminf(r, cb[f][i]);
              }
            }
          }
        }
#pragma unroll
        for (int f = 0; f < 2; ++f) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {  // (0, 1) and (2, 3)
            const bool t = cb[f][2 * h + 1] < cb[f][2 * h];
            co[f][2 * h] = t ? co[f][2 * h + 1] : co[f][2 * h];
            cb[f][2 * h] = fminf(cb[f][2 * h + 1], cb[f][2 * h]);
          }
          const bool t = cb[f][2] < cb[f][0];
          lo[f] = t ? co[f][2] : co[f][0];
          lb[f] = __fadd_rn(xsq[f], fminf(cb[f][2], cb[f][0]));  // the step best's distance
        }
      };
      // clamp rule and merge into the running best
      auto finish = [&](const spr::f32x16 (&acc)[2], int c0, const float (&kf)[2], float (&lb)[2],
                        int32_t (&lo)[2]) {
        if (__ballot(lb[0] <= 0.0f || lb[1] <= 0.0f) != 0ull) {
          // first candidate with r <= 0, in index order, at distance 0
          const float* cs = csq_l + c0 + 4 * half;
#pragma unroll
          for (int f = 0; f < 2; ++f) {
            bool found = false;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                const int off = 8 * i + j;
                const float r = __fadd_rn(xsq[f], __builtin_fmaf(kf[f], acc[f][4 * i + j], cs[off]));
                if (lb[f] <= 0.0f && !found && r <= 0.0f) {
                  lo[f] = off;
                  found = true;
                }
              }
            }
            lb[f] = fmaxf(lb[f], 0.0f);
          }
        }
        const int32_t base = c0 + 4 * half;
#pragma unroll
        for (int f = 0; f < 2; ++f) {
          const bool t = lb[f] < best[f];
          best[f] = t ? lb[f] : best[f];
          best_idx[f] = t ? base + lo[f] : best_idx[f];
        }
      };
      // the argmin of step cc (acc_c) with the MFMAs of step cn (acc_n) interleaved
      auto fused = [&](spr::f32x16 (&acc_n)[2], int cn, const spr::f32x16 (&acc_c)[2], int cc) {
        float kf[2], lb[2];
        int32_t lo[2];
        factors(cc, kf);
        mfma_step(acc_n, cn);
        scan(acc_c, cc, kf, lb, lo);
        // KSTEPS fragment reads and 4 c_sq reads first, then one MFMA per VALU group
        __builtin_amdgcn_sched_group_barrier(0x100, KSTEPS + 4, 0);
#pragma unroll
        for (int m = 0; m < 2 * KSTEPS; ++m) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 150 / (2 * KSTEPS), 0);
        }
        finish(acc_c, cc, kf, lb, lo);
      };

      spr::f32x16 acc_a[2], acc_b[2];
      mfma_step(acc_a, 0);
      int c0 = 0;
      for (; c0 + 64 < kpad; c0 += 64) {
        fused(acc_b, c0 + 32, acc_a, c0);
        fused(acc_a, c0 + 64, acc_b, c0 + 32);
      }
      fused(acc_b, c0 + 32, acc_a, c0);
      {
        float kf[2], lb[2];
        int32_t lo[2];
        factors(c0 + 32, kf);
        scan(acc_b, c0 + 32, kf, lb, lo);
        finish(acc_b, c0 + 32, kf, lb, lo);
      }
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        const float od = __shfl_xor(best[f], 32, 64);
        const int32_t oi = __shfl_xor(best_idx[f], 32, 64);
        if (od < best[f] || (od == best[f] && oi < best_idx[f])) {
          best[f] = od;
          best_idx[f] = oi;
        }
        const int64_t p = p0 + 32 * f;
        if (half == 0 && p < n) labels[b * n + p] = best_idx[f];
      }
    }
    g0 = seg_end;
  }
}

// Launches kmeans_assign_tf32_resident_kernel<D> when its LDS holds the padded
// centroids (*used = true); otherwise launches nothing (*used = false) and the caller
// takes the streamed kmeans_assign_tf32_kernel.  A grid of at most 256 workgroups (one
// per CU) splits the (batch, 64-point block) space evenly.
template <int D>
int launch_tf32_resident(const float* x, const float* c, const float* c_sq, const float* x_sq, float* x_sq_out,
                         int64_t batch, int64_t n, int32_t k, int32_t* labels, hipStream_t stream, bool* used) {
  *used = false;
  const int64_t kpad = spr::ceil_div(k, CCHUNK) * CCHUNK;
  const size_t lds = pipe_lds_bytes<D>(kpad);
  if (lds > PIPE_LDS_LIMIT) return SPR_OK;
  static bool lds_raised = false;  // dynamic LDS beyond 64 KB must be allowed once per process
  if (!lds_raised) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&kmeans_assign_tf32_resident_kernel<D>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             static_cast<int>(PIPE_LDS_LIMIT));
    if (e != hipSuccess) {
      spr_set_error("spr_kmeans_assign_tf32: hipFuncSetAttribute failed: %s", hipGetErrorString(e));
      return SPR_ELAUNCH;
    }
    lds_raised = true;
  }
  const int64_t blocks = batch * spr::ceil_div(n, ASSIGN_POINTS_PER_WAVE);
  constexpr int PIPE_THREADS = pipe_threads<D>();
  const int64_t grid = std::max<int64_t>(1, std::min<int64_t>(256, spr::ceil_div(blocks, PIPE_THREADS / 64)));
  kmeans_assign_tf32_resident_kernel<D><<<static_cast<uint32_t>(grid), PIPE_THREADS, lds, stream>>>(
      x, c, c_sq, x_sq, x_sq_out, batch, n, k, labels);
  SPR_LAUNCHED("kmeans_assign_tf32_resident_kernel");
  *used = true;
  return SPR_OK;
}

// ---------------------------------------------------------------- segmented mean
// Mean of one cluster from its fp64 sum: mean32 = float(sum / count) (empty ->
// previous centroid), out = mean32 in the centroid dtype, optional running
// sums/counts and max centroid shift.  Called by every thread of the workgroup;
// threads below D own one dim (`s` valid there).
template <typename T, int D>
__device__ void finalize_mean(double s, int32_t count, int64_t b, int32_t cl, int32_t k, const T* __restrict__ old,
                              float* __restrict__ mean32, T* __restrict__ out, float* __restrict__ shift_max,
                              float* __restrict__ sums_accum, int32_t* __restrict__ counts_accum,
                              float* __restrict__ c_sq_out, float* sq, float* cv) {
  const int tid = threadIdx.x;
  const int64_t o = (b * k + cl) * D;
  if (tid < D) {
    float prev;
    if constexpr (sizeof(T) == 2) {
      prev = spr::bf16_to_f32(old[o + tid]);
    } else {
      prev = old[o + tid];
    }
    const float m = count > 0 ? static_cast<float>(s / static_cast<double>(count)) : prev;
    if (mean32 != nullptr) mean32[o + tid] = m;
    float outv = m;
    if (out != nullptr) {
      if constexpr (sizeof(T) == 2) {
        const uint16_t bits = spr::f32_to_bf16(m);
        out[o + tid] = bits;
        outv = spr::bf16_to_f32(bits);
      } else {
        out[o + tid] = m;
      }
    }
    if (sums_accum != nullptr) sums_accum[o + tid] += static_cast<float>(s);
    const float diff = outv - prev;
    sq[tid] = diff * diff;
    cv[tid] = outv;
  }
  if (counts_accum != nullptr && tid == 0) counts_accum[b * k + cl] += count;
  if (shift_max != nullptr || c_sq_out != nullptr) {
    __syncthreads();
    if (shift_max != nullptr && tid == 0) {
      float acc = 0.0f;
      for (int t = 0; t < D; ++t) acc += sq[t];
      const float norm = sqrtf(acc);
      // The stored maximum only grows, so a shift not above a value read from it cannot be
      // the maximum: those workgroups skip the atomic.  Every workgroup of a launch
      // otherwise queued on the one address (about 24,000 at 1000 clusters x 24 heads).
      unsigned int* const sm = reinterpret_cast<unsigned int*>(shift_max);
      if (__float_as_uint(norm) > __hip_atomic_load(sm, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
        atomicMax(sm, __float_as_uint(norm));
    }
    // squared norm of the new centroid for the next assignment, in the order of
    // centroid_sq_kernel (sequential fma over d)
    if (c_sq_out != nullptr && tid == 64 % blockDim.x) {
      float acc = 0.0f;
      for (int t = 0; t < D; ++t) acc = __builtin_fmaf(cv[t], cv[t], acc);
      c_sq_out[b * k + cl] = acc;
    }
  }
}

// Slices of a cluster's rows (sorted order): every cluster with rows gets ceil(rows / MEAN_SLICE)
// slices of its own, so a large cluster is spread over many workgroups whatever the other
// clusters' sizes (on the C4 route's Q labels, the largest of 128 clusters holds 17,805 of
// 118,800 rows; slices sized from the average left it to two workgroups: 204 us per update
// against 134 us on uniform labels).
constexpr int MEAN_SLICE = 512;

// One workgroup per batch: slice_base[b][c] = the first slice of cluster c (exclusive scan of
// ceil(rows_c / MEAN_SLICE), c = 0 .. k; capped at maxs, the slices the workspace holds, so
// a malformed offsets table cannot index past it) and slice_rows[b][s] = {x, y, c, m}: rows
// [x, y) of cluster c, which has m slices (an empty range with m = 0 past the last slice).
// Offsets are clamped as the mean kernels clamp them.
__global__ __launch_bounds__(256) void mean_slice_plan_kernel(const int32_t* __restrict__ offsets, int64_t n,
                                                              int32_t k, int32_t maxs, int32_t* __restrict__ slice_base,
                                                              int4* __restrict__ slice_rows) {
  __shared__ int32_t wave_tot[4];
  const int64_t b = blockIdx.x;
  const int32_t* off = offsets + b * (k + 1);
  int32_t* sb = slice_base + b * (k + 1);
  int4* sr = slice_rows + b * static_cast<int64_t>(maxs);
  const int32_t n32 = static_cast<int32_t>(n);
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int per = (k + 255) / 256;
  const int c0 = min(t * per, k), c1 = min(c0 + per, k);
  auto slices_of = [&](int c, int32_t& start, int32_t& end) {
    start = min(max(off[c], 0), n32);
    end = min(max(off[c + 1], start), n32);
    return static_cast<int32_t>((static_cast<int64_t>(end) - start + MEAN_SLICE - 1) / MEAN_SLICE);
  };
  int64_t local = 0;
  for (int c = c0; c < c1; ++c) {
    int32_t a, e;
    local += slices_of(c, a, e);
  }
  int64_t incl = local;
  for (int o = 1; o < 64; o <<= 1) {
    const int64_t up = __shfl_up(incl, o, 64);
    if (lane >= o) incl += up;
  }
  if (lane == 63) wave_tot[wv] = static_cast<int32_t>(min(incl, static_cast<int64_t>(maxs)));
  __syncthreads();
  int64_t base = incl - local;
  for (int w = 0; w < wv; ++w) base += wave_tot[w];
  for (int c = c0; c < c1; ++c) {
    int32_t a, e;
    const int ns = slices_of(c, a, e);
    sb[c] = static_cast<int32_t>(min(base, static_cast<int64_t>(maxs)));
    for (int j = 0; j < ns; ++j) {
      const int64_t si = base + j;
      if (si < maxs) {
        const int64_t lo = a + static_cast<int64_t>(j) * MEAN_SLICE;  // 64-bit: no overflow near n = 2^31
        sr[si] = int4{static_cast<int32_t>(lo), static_cast<int32_t>(min<int64_t>(lo + MEAN_SLICE, e)), c, ns};
      }
    }
    base += ns;
  }
  __syncthreads();
  int64_t total = 0;
  for (int w = 0; w < 4; ++w) total += wave_tot[w];
  total = min(total, static_cast<int64_t>(maxs));
  if (t == 0) sb[k] = static_cast<int32_t>(total);
  for (int64_t si = total + t; si < maxs; si += 256) sr[si] = int4{0, 0, 0, 0};
}

// T: uint16_t (bf16) or float.  Workgroup (s, b) sums slice s of batch b (rows
// slice_rows[b][s] of the sorted order) in fp64.  The one slice of a cluster finalizes its
// mean directly; otherwise the sum goes to partial[b][s][D], and
// centroid_mean_finalize_kernel adds the cluster's slices in order (the result does not
// depend on the split).
template <typename T, int D>
__global__ __launch_bounds__(256) void centroid_mean_kernel(
    const T* __restrict__ x, const int32_t* __restrict__ sorted_idx, const int4* __restrict__ slice_rows, int64_t n,
    int32_t maxs, double* __restrict__ partial, const int32_t* __restrict__ offsets, const T* __restrict__ old,
    int32_t k, float* __restrict__ mean32, T* __restrict__ out, float* __restrict__ shift_max,
    float* __restrict__ sums_accum, int32_t* __restrict__ counts_accum, float* __restrict__ c_sq_out) {
  constexpr int E = 16 / sizeof(T);  // elements per 16-byte vector
  constexpr int VPR = D / E;         // vectors per row
  static_assert(D % E == 0 && VPR <= 256, "unsupported D");
  constexpr int R = 256 / VPR;       // row groups (threads past R * VPR idle)
  // rows per thread per pass: 8 for bf16 rows; 4 for fp32 (fewer registers, more waves: the
  // N8 means 142 -> 117 us at D 48 and 168 -> 140 us at D 64 against 8; 2 and 16 slower)
  constexpr int RPT = sizeof(T) == 4 ? 4 : 8;
  __shared__ double red[R][D + 1];
  __shared__ float sq[D], cv[D];

  const int tid = threadIdx.x;
  const int v = tid % VPR;
  const int rg = tid / VPR;
  const int64_t b = blockIdx.y;
  const int32_t n32 = static_cast<int32_t>(n);
  const int4 rr = slice_rows[b * maxs + blockIdx.x];
  if (rr.w == 0) return;  // past the last slice
  // the plan's ranges lie in [0, n); clamp anyway
  const int32_t start = min(max(rr.x, 0), n32);
  const int32_t end = min(max(rr.y, start), n32);
  const int32_t* idx = sorted_idx + b * n;
  const T* xb = x + b * n * D;
  double acc[E];
#pragma unroll
  for (int e = 0; e < E; ++e) acc[e] = 0.0;

  auto add_vec = [&](const u32x4& w) {
    if constexpr (sizeof(T) == 2) {
      const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[2 * e] += static_cast<double>(spr::bf16_lo(ws[e]));
        acc[2 * e + 1] += static_cast<double>(spr::bf16_hi(ws[e]));
      }
    } else {
      acc[0] += static_cast<double>(__uint_as_float(w.x));
      acc[1] += static_cast<double>(__uint_as_float(w.y));
      acc[2] += static_cast<double>(__uint_as_float(w.z));
      acc[3] += static_cast<double>(__uint_as_float(w.w));
    }
  };

  // Passes of R * RPT rows: each thread issues the loads of its RPT rows before
  // adding any of them, and the next pass's row indices are in flight while
  // the current rows are added.
  const bool worker = rg < R;
  constexpr int STEP = R * RPT;
  int32_t ix[RPT];
  auto load_ix = [&](int32_t base) {
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int32_t r = base + rg + R * i;
      ix[i] = (worker && r < end) ? idx[r] : -1;
    }
  };
  load_ix(start);
  for (int32_t base = start; base < end; base += STEP) {
    u32x4 w[RPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const uint32_t t = static_cast<uint32_t>(ix[i]);
      w[i] = t < static_cast<uint32_t>(n32) ? reinterpret_cast<const u32x4*>(xb + static_cast<int64_t>(t) * D)[v]
                                            : u32x4{0, 0, 0, 0};
    }
    if (base + STEP < end) load_ix(base + STEP);
#pragma unroll
    for (int i = 0; i < RPT; ++i) add_vec(w[i]);
  }
  if (worker) {
#pragma unroll
    for (int e = 0; e < E; ++e) red[rg][v * E + e] = acc[e];
  }
  __syncthreads();

  double s = 0.0;
  if (tid < D) {
    for (int g = 0; g < R; ++g) s += red[g][tid];
  }
  if (rr.w > 1) {
    if (tid < D) partial[(b * maxs + blockIdx.x) * D + tid] = s;
    return;
  }
  // the cluster's only slice: its rows are the whole cluster
  const int32_t cl = min(max(rr.z, 0), k - 1);
  finalize_mean<T, D>(s, end - start, b, cl, k, old, mean32, out, shift_max, sums_accum, counts_accum, c_sq_out,
                      sq, cv);
}

template <typename T, int D>
__global__ __launch_bounds__(256) void centroid_mean_finalize_kernel(
    const double* __restrict__ partial, const int32_t* __restrict__ slice_base, int32_t maxs,
    const int32_t* __restrict__ offsets, const T* __restrict__ old, int64_t n, int32_t k, float* __restrict__ mean32,
    T* __restrict__ out, float* __restrict__ shift_max, float* __restrict__ sums_accum,
    int32_t* __restrict__ counts_accum, float* __restrict__ c_sq_out) {
  __shared__ float sq[D], cv[D];
  const int64_t b = blockIdx.y;
  const int32_t cl = blockIdx.x;
  const int32_t* off = offsets + b * (k + 1);
  const int32_t* sb = slice_base + b * (k + 1);
  const int32_t n32 = static_cast<int32_t>(n);
  const int32_t c_start = min(max(off[cl], 0), n32);
  const int32_t c_end = min(max(off[cl + 1], c_start), n32);
  const int32_t s0 = min(max(sb[cl], 0), maxs);
  const int32_t s1 = min(max(sb[cl + 1], s0), maxs);
  // a cluster of one slice (the plan's rule) was finalized by that slice's workgroup
  if ((static_cast<int64_t>(c_end) - c_start + MEAN_SLICE - 1) / MEAN_SLICE == 1) return;
  double s = 0.0;
  if (threadIdx.x < D) {
    const double* p = partial + b * static_cast<int64_t>(maxs) * D + threadIdx.x;
    for (int32_t sp = s0; sp < s1; ++sp) s += p[static_cast<int64_t>(sp) * D];
  }
  finalize_mean<T, D>(s, c_end - c_start, b, cl, k, old, mean32, out, shift_max, sums_accum, counts_accum, c_sq_out,
                      sq, cv);
}

// ---------------------------------------------------------------- exact fp32 assign
template <int D>
__global__ __launch_bounds__(256) void role_assign_fp32_kernel(const float* __restrict__ f,
                                                               const float* __restrict__ c, int64_t n,
                                                               int32_t k, int32_t* __restrict__ labels,
                                                               float* __restrict__ best_dist) {
  constexpr int TILE = 64;
  __shared__ __attribute__((aligned(16))) float tile[TILE * D];
  const int64_t b = blockIdx.y;
  const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const bool live = p < n;
  float pt[D];
#pragma unroll
  for (int r = 0; r < D; r += 4) {
    u32x4 w = live ? *reinterpret_cast<const u32x4*>(f + (b * n + p) * D + r) : u32x4{0, 0, 0, 0};
    pt[r] = __uint_as_float(w.x);
    pt[r + 1] = __uint_as_float(w.y);
    pt[r + 2] = __uint_as_float(w.z);
    pt[r + 3] = __uint_as_float(w.w);
  }
  float bd = 3.402823466e38f;
  int32_t bi = 0x7fffffff;
  const float* cb = c + b * static_cast<int64_t>(k) * D;
  for (int32_t c0 = 0; c0 < k; c0 += TILE) {
    const int rows = (k - c0) < TILE ? (k - c0) : TILE;
    __syncthreads();
    for (int i = threadIdx.x; i < rows * D / 4; i += blockDim.x) {
      reinterpret_cast<u32x4*>(tile)[i] = reinterpret_cast<const u32x4*>(cb + static_cast<int64_t>(c0) * D)[i];
    }
    __syncthreads();
    for (int j = 0; j < rows; ++j) {
      const float* q = tile + j * D;
      float dist = 0.0f;
#pragma unroll
      for (int r = 0; r < D; ++r) {
        const float delta = __fsub_rn(pt[r], q[r]);
        dist = __builtin_fmaf(delta, delta, dist);
      }
      const int32_t idx = c0 + j;
      if (dist < bd || (dist == bd && idx < bi)) {
        bd = dist;
        bi = idx;
      }
    }
  }
  if (live) {
    labels[b * n + p] = bi;
    if (best_dist != nullptr) best_dist[b * n + p] = bd;
  }
}

}  // namespace

// ------------------------------------------------------------------ C ABI

// c_sq[rows] = sum_d c[rows, d]^2 (fp32); dtype 0 = bf16, 2 = fp32.
extern "C" int spr_centroid_sq(const void* c, int32_t dtype, int64_t rows, int32_t d, float* c_sq,
                               hipStream_t stream) {
  SPR_REQUIRE(rows >= 0 && d > 0, "spr_centroid_sq: bad size");
  if (rows == 0) return SPR_OK;
  SPR_REQUIRE(c && c_sq, "spr_centroid_sq: null pointer");
  const int blocks = static_cast<int>(spr::ceil_div(rows, 256));
  if (dtype == 0) {
    centroid_sq_kernel<uint16_t><<<blocks, 256, 0, stream>>>(static_cast<const uint16_t*>(c), rows, d, c_sq);
  } else if (dtype == 2) {
    centroid_sq_kernel<float><<<blocks, 256, 0, stream>>>(static_cast<const float*>(c), rows, d, c_sq);
  } else {
    SPR_REQUIRE(false, "spr_centroid_sq: unsupported dtype %d", dtype);
  }
  SPR_LAUNCHED("centroid_sq_kernel");
  return SPR_OK;
}

// labels[b, i] = argmin_k max((x_sq + c_sq) - 2 x.c, 0) for bf16 x [b, n, d],
// bf16 centroids [b, k, d], fp32 c_sq [b, k].  x_sq: fp32 [b, n] or null
// (computed inline with x_sq_mode 0 = fp32, 1 = bf16 buffer semantics).
extern "C" int spr_kmeans_assign_bf16(const void* x, const void* centroids, const float* c_sq, const float* x_sq,
                                      int32_t x_sq_mode, float* x_sq_out, int64_t batch, int64_t n, int32_t k, int32_t d,
                                      int32_t* labels, hipStream_t stream) {
  SPR_REQUIRE(batch >= 0 && n >= 0 && k >= 1, "spr_kmeans_assign_bf16: bad size");
  SPR_REQUIRE(batch <= 65535, "spr_kmeans_assign_bf16: batch %lld exceeds 65535", (long long)batch);
  SPR_REQUIRE(x_sq_mode == 0 || x_sq_mode == 1, "spr_kmeans_assign_bf16: x_sq_mode must be 0 or 1");
  if (batch == 0 || n == 0) return SPR_OK;
  SPR_REQUIRE(x && centroids && c_sq && labels, "spr_kmeans_assign_bf16: null pointer");
  SPR_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(centroids) % 16 == 0,
              "spr_kmeans_assign_bf16: x and centroids must be 16-byte aligned");
  dim3 grid(static_cast<uint32_t>(spr::ceil_div(n, ASSIGN_POINTS)), static_cast<uint32_t>(batch));
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const uint16_t* cp = static_cast<const uint16_t*>(centroids);
  if (d == 128 && k <= ASSIGN_RESIDENT_K) {
    // one resident workgroup per CU (256 CUs), sharing the batch's point blocks
    const int64_t kpad = spr::ceil_div(k, CCHUNK) * CCHUNK;
    const size_t lds = static_cast<size_t>(kpad) * (128 * 2 + 16) + static_cast<size_t>(kpad) * 4;
    constexpr int waves = ASSIGN_RESIDENT_THREADS / 64;
    const int64_t per_batch =
        std::max<int64_t>(1, std::min<int64_t>(spr::ceil_div(n, waves * ASSIGN_POINTS_PER_WAVE), 256 / batch));
    static bool lds_raised = false;  // dynamic LDS beyond 64 KB must be allowed once per process
    if (!lds_raised) {
      const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&kmeans_assign_resident_kernel<128>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize,
                                               ASSIGN_RESIDENT_K * (128 * 2 + 16) + ASSIGN_RESIDENT_K * 4);
      if (e != hipSuccess) {
        spr_set_error("spr_kmeans_assign_bf16: hipFuncSetAttribute failed: %s", hipGetErrorString(e));
        return SPR_ELAUNCH;
      }
      lds_raised = true;
    }
    kmeans_assign_resident_kernel<128><<<dim3(static_cast<uint32_t>(per_batch), static_cast<uint32_t>(batch)),
                                         ASSIGN_RESIDENT_THREADS, lds, stream>>>(xp, cp, c_sq, x_sq, x_sq_mode,
                                                                                  x_sq_out, n, k, labels);
    SPR_LAUNCHED("kmeans_assign_resident_kernel");
    return SPR_OK;
  }
  switch (d) {
    case 64:
      kmeans_assign_bf16_kernel<64><<<grid, ASSIGN_THREADS, 0, stream>>>(xp, cp, c_sq, x_sq, x_sq_mode, x_sq_out, n, k,
                                                                        labels);
      break;
    case 128:
      kmeans_assign_bf16_kernel<128><<<grid, ASSIGN_THREADS, 0, stream>>>(xp, cp, c_sq, x_sq, x_sq_mode, x_sq_out, n,
                                                                         k, labels);
      break;
    default:
      SPR_REQUIRE(false, "spr_kmeans_assign_bf16: head dim %d not supported (64, 128)", d);
  }
  SPR_LAUNCHED("kmeans_assign_bf16_kernel");
  return SPR_OK;
}

namespace {

// Original-space means of one or two tensors (x and, with JOINT, y) under one label
// traversal: workgroup (cl * nsplit + sp, b) sums slice sp of cluster cl's rows (sorted
// order) of x and y in fp64.  With nsplit == 1 it writes the fp32 means directly;
// otherwise partial[b][cl][sp][2][D] holds the slice sums and original_mean_finalize_kernel
// adds them in slice order.  Empty clusters take the fp32 fallback row, or 0 without one.
template <typename T, int D, bool JOINT>
__global__ __launch_bounds__(256) void original_mean_kernel(
    const T* __restrict__ x, const T* __restrict__ y, const int32_t* __restrict__ sorted_idx,
    const int32_t* __restrict__ offsets, int64_t n, int32_t k, int32_t nsplit, double* __restrict__ partial,
    const float* __restrict__ x_fb, const float* __restrict__ y_fb, float* __restrict__ x_out,
    float* __restrict__ y_out) {
  constexpr int E = 16 / sizeof(T);
  constexpr int VPR = D / E;
  static_assert(D % E == 0 && VPR <= 256, "unsupported D");
  constexpr int R = 256 / VPR;
  constexpr int RPT = JOINT ? 8 : 16;
  constexpr int NT = JOINT ? 2 : 1;
  __shared__ double red[NT][R][D + 1];
  const int tid = threadIdx.x;
  const int v = tid % VPR;
  const int rg = tid / VPR;
  const int64_t b = blockIdx.y;
  const int32_t cl = blockIdx.x / nsplit;
  const int32_t sp = blockIdx.x - cl * nsplit;
  const int32_t* off = offsets + b * (k + 1);
  const int32_t n32 = static_cast<int32_t>(n);
  const int32_t c_start = min(max(off[cl], 0), n32);
  const int32_t c_end = min(max(off[cl + 1], c_start), n32);
  const int32_t slice = (c_end - c_start + nsplit - 1) / nsplit;
  const int32_t start = min(c_start + sp * slice, c_end);
  const int32_t end = min(start + slice, c_end);
  const int32_t* idx = sorted_idx + b * n;
  const T* src[2] = {x + b * n * D, JOINT ? y + b * n * D : nullptr};

  double acc[NT][E];
#pragma unroll
  for (int q = 0; q < NT; ++q)
#pragma unroll
    for (int e = 0; e < E; ++e) acc[q][e] = 0.0;
  auto add_vec = [&](int q, const u32x4& w) {
    if constexpr (sizeof(T) == 2) {
      const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[q][2 * e] += static_cast<double>(spr::bf16_lo(ws[e]));
        acc[q][2 * e + 1] += static_cast<double>(spr::bf16_hi(ws[e]));
      }
    } else {
      acc[q][0] += static_cast<double>(__uint_as_float(w.x));
      acc[q][1] += static_cast<double>(__uint_as_float(w.y));
      acc[q][2] += static_cast<double>(__uint_as_float(w.z));
      acc[q][3] += static_cast<double>(__uint_as_float(w.w));
    }
  };
  const bool worker = rg < R;
  constexpr int STEP = R * RPT;
  int32_t ix[RPT];
  auto load_ix = [&](int32_t base) {
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int32_t r = base + rg + R * i;
      ix[i] = (worker && r < end) ? idx[r] : -1;
    }
  };
  load_ix(start);
  for (int32_t base = start; base < end; base += STEP) {
    u32x4 w[NT][RPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const uint32_t t = static_cast<uint32_t>(ix[i]);
#pragma unroll
      for (int q = 0; q < NT; ++q)
        w[q][i] = t < static_cast<uint32_t>(n32)
                      ? reinterpret_cast<const u32x4*>(src[q] + static_cast<int64_t>(t) * D)[v]
                      : u32x4{0, 0, 0, 0};
    }
    if (base + STEP < end) load_ix(base + STEP);
#pragma unroll
    for (int i = 0; i < RPT; ++i)
#pragma unroll
      for (int q = 0; q < NT; ++q) add_vec(q, w[q][i]);
  }
  if (worker) {
#pragma unroll
    for (int q = 0; q < NT; ++q)
#pragma unroll
      for (int e = 0; e < E; ++e) red[q][rg][v * E + e] = acc[q][e];
  }
  __syncthreads();
  if (tid < D) {
    const int32_t count = c_end - c_start;
#pragma unroll
    for (int q = 0; q < NT; ++q) {
      double s = 0.0;
      for (int g = 0; g < R; ++g) s += red[q][g][tid];
      if (nsplit > 1) {
        partial[(((b * k + cl) * nsplit + sp) * 2 + q) * D + tid] = s;
      } else {
        const float* fb = q == 0 ? x_fb : y_fb;
        float* o = q == 0 ? x_out : y_out;
        const int64_t at = (b * k + cl) * D + tid;
        o[at] = count > 0 ? static_cast<float>(s / static_cast<double>(count)) : (fb != nullptr ? fb[at] : 0.0f);
      }
    }
  }
}

template <int D>
__global__ __launch_bounds__(256) void original_mean_finalize_kernel(
    const double* __restrict__ partial, const int32_t* __restrict__ offsets, int64_t n, int32_t k, int32_t nsplit,
    int32_t ntensors, const float* __restrict__ x_fb, const float* __restrict__ y_fb, float* __restrict__ x_out,
    float* __restrict__ y_out) {
  const int64_t b = blockIdx.y;
  const int32_t cl = blockIdx.x;
  const int32_t* off = offsets + b * (k + 1);
  const int32_t n32 = static_cast<int32_t>(n);
  const int32_t c_start = min(max(off[cl], 0), n32);
  const int32_t c_end = min(max(off[cl + 1], c_start), n32);
  const int32_t count = c_end - c_start;
  for (int e = threadIdx.x; e < ntensors * D; e += blockDim.x) {
    const int q = e / D, c = e - q * D;
    double s = 0.0;
    for (int sp = 0; sp < nsplit; ++sp) s += partial[(((b * k + cl) * nsplit + sp) * 2 + q) * D + c];
    const float* fb = q == 0 ? x_fb : y_fb;
    float* o = q == 0 ? x_out : y_out;
    const int64_t at = (b * k + cl) * D + c;
    o[at] = count > 0 ? static_cast<float>(s / static_cast<double>(count)) : (fb != nullptr ? fb[at] : 0.0f);
  }
}

}  // namespace

// labels[b, i] = argmin_k max((x_sq + c_sq) - 2 tf32(x).tf32(c), 0) for fp32 x [b, n, d]
// and centroids [b, k, d], fp32 c_sq [b, k]; x_sq fp32 [b, n] or null (inline fp32).
extern "C" int spr_kmeans_assign_tf32(const float* x, const float* centroids, const float* c_sq, const float* x_sq,
                                      float* x_sq_out, int64_t batch, int64_t n, int32_t k, int32_t d,
                                      int32_t* labels, hipStream_t stream) {
  SPR_REQUIRE(batch >= 0 && n >= 0 && k >= 1, "spr_kmeans_assign_tf32: bad size");
  SPR_REQUIRE(batch <= 65535, "spr_kmeans_assign_tf32: batch %lld exceeds 65535", (long long)batch);
  if (batch == 0 || n == 0) return SPR_OK;
  SPR_REQUIRE(x && centroids && c_sq && labels, "spr_kmeans_assign_tf32: null pointer");
  SPR_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(centroids) % 16 == 0,
              "spr_kmeans_assign_tf32: x and centroids must be 16-byte aligned");
  dim3 grid(static_cast<uint32_t>(spr::ceil_div(n, ASSIGN_POINTS)), static_cast<uint32_t>(batch));
#define SPR_TF32_ASSIGN(DD)                                                                                      \
  do {                                                                                                           \
    bool used = false;                                                                                           \
    const int st = launch_tf32_resident<DD>(x, centroids, c_sq, x_sq, x_sq_out, batch, n, k, labels, stream,    \
                                            &used);                                                             \
    if (st != SPR_OK || used) return st;                                                                         \
    kmeans_assign_tf32_kernel<DD><<<grid, ASSIGN_THREADS, 0, stream>>>(x, centroids, c_sq, x_sq, x_sq_out, n, k, \
                                                                       labels);                                  \
  } while (0)
  switch (d) {
    case 16: SPR_TF32_ASSIGN(16); break;
    case 32: SPR_TF32_ASSIGN(32); break;
    case 48: SPR_TF32_ASSIGN(48); break;
    case 64: SPR_TF32_ASSIGN(64); break;
    case 80: SPR_TF32_ASSIGN(80); break;
    case 96: SPR_TF32_ASSIGN(96); break;
    case 112: SPR_TF32_ASSIGN(112); break;
    case 128: SPR_TF32_ASSIGN(128); break;
    default:
      SPR_REQUIRE(false, "spr_kmeans_assign_tf32: feature dim %d not supported (a multiple of 16 up to 128)", d);
  }
#undef SPR_TF32_ASSIGN
  SPR_LAUNCHED("kmeans_assign_tf32_kernel");
  return SPR_OK;
}

static int32_t mean_splits(int64_t n, int32_t k);

extern "C" size_t spr_original_centroids_workspace(int64_t batch, int64_t n, int32_t k, int32_t d) {
  const int32_t ns = mean_splits(n, k);
  return ns > 1 ? static_cast<size_t>(batch * k * ns * 2 * static_cast<int64_t>(d) * sizeof(double)) : 0;
}

// fp32 means of x (and y, nullable) rows per cluster from a stable label sort (sorted_idx,
// offsets of spr_argsort_labels); empty clusters take the fp32 fallback rows (nullable: 0).
// dtype 0 bf16 (d in {64, 128}) or 2 fp32 (d in {16, 32, 48, 64, 128}); y has x's dtype.
extern "C" int spr_original_centroids(const void* x, const void* y, int32_t dtype, const int32_t* sorted_idx,
                                      const int32_t* offsets, int64_t batch, int64_t n, int32_t k, int32_t d,
                                      const float* x_fallback, const float* y_fallback, float* x_out, float* y_out,
                                      void* workspace, size_t workspace_bytes, hipStream_t stream) {
  SPR_REQUIRE(batch >= 0 && n >= 0 && k >= 1, "spr_original_centroids: bad size");
  SPR_REQUIRE(batch <= 65535, "spr_original_centroids: batch %lld exceeds 65535", (long long)batch);
  SPR_REQUIRE((y == nullptr) == (y_out == nullptr), "spr_original_centroids: y and y_out go together");
  if (batch == 0) return SPR_OK;
  SPR_REQUIRE(sorted_idx && offsets && x_out, "spr_original_centroids: null pointer");
  SPR_REQUIRE(n == 0 || x, "spr_original_centroids: null x");
  const int32_t ns = mean_splits(n, k);
  const size_t need = spr_original_centroids_workspace(batch, n, k, d);
  if (workspace_bytes < need || (need > 0 && workspace == nullptr)) {
    spr_set_error("spr_original_centroids: workspace %zu < %zu bytes", workspace_bytes, need);
    return SPR_EWORKSPACE;
  }
  SPR_REQUIRE(static_cast<int64_t>(k) * ns < (int64_t(1) << 31), "spr_original_centroids: too many clusters");
  double* partial = static_cast<double*>(workspace);
  dim3 grid(static_cast<uint32_t>(k * ns), static_cast<uint32_t>(batch));
  dim3 fgrid(static_cast<uint32_t>(k), static_cast<uint32_t>(batch));
  const int ntensors = y != nullptr ? 2 : 1;
#define SPR_ORIG_CASE(T, DD)                                                                                      \
  do {                                                                                                            \
    if (y != nullptr)                                                                                             \
      original_mean_kernel<T, DD, true><<<grid, 256, 0, stream>>>(                                                \
          static_cast<const T*>(x), static_cast<const T*>(y), sorted_idx, offsets, n, k, ns, partial, x_fallback, \
          y_fallback, x_out, y_out);                                                                              \
    else                                                                                                          \
      original_mean_kernel<T, DD, false><<<grid, 256, 0, stream>>>(static_cast<const T*>(x), nullptr, sorted_idx, \
                                                                   offsets, n, k, ns, partial, x_fallback,       \
                                                                   nullptr, x_out, nullptr);                     \
    if (ns > 1)                                                                                                   \
      original_mean_finalize_kernel<DD><<<fgrid, 256, 0, stream>>>(partial, offsets, n, k, ns, ntensors,          \
                                                                   x_fallback, y_fallback, x_out, y_out);         \
  } while (0)
  if (dtype == 0) {
    switch (d) {
      case 64: SPR_ORIG_CASE(uint16_t, 64); break;
      case 128: SPR_ORIG_CASE(uint16_t, 128); break;
      default: SPR_REQUIRE(false, "spr_original_centroids: bf16 dim %d not supported (64, 128)", d);
    }
  } else if (dtype == 2) {
    switch (d) {
      case 16: SPR_ORIG_CASE(float, 16); break;
      case 32: SPR_ORIG_CASE(float, 32); break;
      case 48: SPR_ORIG_CASE(float, 48); break;
      case 64: SPR_ORIG_CASE(float, 64); break;
      case 128: SPR_ORIG_CASE(float, 128); break;
      default: SPR_REQUIRE(false, "spr_original_centroids: fp32 dim %d not supported (16, 32, 48, 64, 128)", d);
    }
  } else {
    SPR_REQUIRE(false, "spr_original_centroids: unsupported dtype %d", dtype);
  }
#undef SPR_ORIG_CASE
  SPR_LAUNCHED("original_mean_kernel");
  return SPR_OK;
}

// Segmented cluster means from a stable label sort (sorted_idx, offsets from
// spr_argsort_labels).  dtype 0 = bf16 rows / bf16 centroids, 2 = fp32.
// Outputs (each nullable): mean32 fp32 [b,k,d]; out (dtype) [b,k,d];
// shift_max (fp32 scalar, must start at 0; receives max_k ||out - old||);
// sums_accum fp32 [b,k,d] += sums; counts_accum int32 [b,k] += counts.
// Slices per cluster for the original-space means: about 512 rows each on average, at most
// 16.  (Per 1,000-row clusters of 64-dimension fp32 rows, 256-row slices and their finalize
// launch took 182 us against 169 us with one workgroup per cluster; 128-row slices were
// slower still.)
static int32_t mean_splits(int64_t n, int32_t k) {
  const int64_t avg = n / (k > 0 ? k : 1);
  return static_cast<int32_t>(std::min<int64_t>(16, std::max<int64_t>(1, (avg + 511) / 512)));
}

// Slices the per-cluster plan can hold: sum_c ceil(rows_c / MEAN_SLICE) <= n / MEAN_SLICE + k.
static int64_t mean_max_slices(int64_t n, int32_t k) { return (n + MEAN_SLICE - 1) / MEAN_SLICE + k; }
static size_t align16(size_t v) { return (v + 15) & ~static_cast<size_t>(15); }

// Workspace of spr_centroid_mean: fp64 slice sums [batch][maxs][d], the slice plan's cluster
// bases [batch][k + 1] and slices [batch][maxs] (rows, cluster, the cluster's slice count).
extern "C" size_t spr_centroid_mean_workspace(int64_t batch, int64_t n, int32_t k, int32_t d) {
  if (batch <= 0 || k < 1 || d < 1 || n < 0) return 0;
  const int64_t maxs = mean_max_slices(n, k);
  return align16(static_cast<size_t>(batch * maxs * d) * sizeof(double)) +
         align16(static_cast<size_t>(batch * (k + 1)) * sizeof(int32_t)) +
         align16(static_cast<size_t>(batch * maxs) * sizeof(int4));
}

extern "C" int spr_centroid_mean(const void* x, int32_t dtype, const int32_t* sorted_idx, const int32_t* offsets,
                                 const void* old, int64_t batch, int64_t n, int32_t k, int32_t d, float* mean32,
                                 void* out, float* shift_max, float* sums_accum, int32_t* counts_accum,
                                 float* c_sq_out, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  SPR_REQUIRE(batch >= 0 && n >= 0 && k >= 1, "spr_centroid_mean: bad size");
  SPR_REQUIRE(batch <= 65535, "spr_centroid_mean: batch %lld exceeds 65535", (long long)batch);
  if (batch == 0) return SPR_OK;
  SPR_REQUIRE(sorted_idx && offsets && old, "spr_centroid_mean: null pointer");
  SPR_REQUIRE(n == 0 || x, "spr_centroid_mean: null x");
  SPR_REQUIRE(n < (int64_t(1) << 31), "spr_centroid_mean: n too large");
  const int64_t maxs = mean_max_slices(n, k);
  SPR_REQUIRE(maxs < (int64_t(1) << 31), "spr_centroid_mean: too many clusters");
  const size_t need = spr_centroid_mean_workspace(batch, n, k, d);
  if (workspace_bytes < need || workspace == nullptr) {
    spr_set_error("spr_centroid_mean: workspace %zu < %zu bytes", workspace_bytes, need);
    return SPR_EWORKSPACE;
  }
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  double* partial = reinterpret_cast<double*>(ws);
  ws += align16(static_cast<size_t>(batch * maxs * d) * sizeof(double));
  int32_t* slice_base = reinterpret_cast<int32_t*>(ws);
  ws += align16(static_cast<size_t>(batch * (k + 1)) * sizeof(int32_t));
  int4* slice_rows = reinterpret_cast<int4*>(ws);
  const int32_t ms = static_cast<int32_t>(maxs);
  mean_slice_plan_kernel<<<dim3(static_cast<uint32_t>(batch)), 256, 0, stream>>>(offsets, n, k, ms, slice_base,
                                                                                 slice_rows);
  SPR_LAUNCHED("mean_slice_plan_kernel");
  dim3 grid(static_cast<uint32_t>(maxs), static_cast<uint32_t>(batch));
  dim3 fgrid(static_cast<uint32_t>(k), static_cast<uint32_t>(batch));
#define SPR_MEAN_CASE(T, DD)                                                                                 \
  do {                                                                                                       \
    centroid_mean_kernel<T, DD><<<grid, 256, 0, stream>>>(                                                   \
        static_cast<const T*>(x), sorted_idx, slice_rows, n, ms, partial, offsets, static_cast<const T*>(old), k, \
        mean32, static_cast<T*>(out), shift_max, sums_accum, counts_accum, c_sq_out);                         \
    centroid_mean_finalize_kernel<T, DD><<<fgrid, 256, 0, stream>>>(                                         \
        partial, slice_base, ms, offsets, static_cast<const T*>(old), n, k, mean32, static_cast<T*>(out),    \
        shift_max, sums_accum, counts_accum, c_sq_out);                                                      \
  } while (0)
  if (dtype == 0) {
    switch (d) {
      case 64: SPR_MEAN_CASE(uint16_t, 64); break;
      case 128: SPR_MEAN_CASE(uint16_t, 128); break;
      default: SPR_REQUIRE(false, "spr_centroid_mean: bf16 head dim %d not supported (64, 128)", d);
    }
  } else if (dtype == 2) {
    switch (d) {
      case 16: SPR_MEAN_CASE(float, 16); break;
      case 32: SPR_MEAN_CASE(float, 32); break;
      case 48: SPR_MEAN_CASE(float, 48); break;
      case 64: SPR_MEAN_CASE(float, 64); break;
      case 80: SPR_MEAN_CASE(float, 80); break;
      case 96: SPR_MEAN_CASE(float, 96); break;
      case 112: SPR_MEAN_CASE(float, 112); break;
      case 128: SPR_MEAN_CASE(float, 128); break;
      default: SPR_REQUIRE(false, "spr_centroid_mean: fp32 dim %d not supported (a multiple of 16 up to 128)", d);
    }
  } else {
    SPR_REQUIRE(false, "spr_centroid_mean: unsupported dtype %d", dtype);
  }
#undef SPR_MEAN_CASE
  SPR_LAUNCHED("centroid_mean_kernel");
  return SPR_OK;
}

// Exact-FP32 nearest centroid for fp32 features [b, n, d], centroids [b, k, d].
extern "C" int spr_role_assign_fp32(const float* features, const float* centroids, int64_t batch, int64_t n,
                                    int32_t k, int32_t d, int32_t* labels, float* best_dist,
                                    hipStream_t stream) {
  SPR_REQUIRE(batch >= 0 && n >= 0 && k >= 1, "spr_role_assign_fp32: bad size");
  SPR_REQUIRE(batch <= 65535, "spr_role_assign_fp32: batch exceeds 65535");
  if (batch == 0 || n == 0) return SPR_OK;
  SPR_REQUIRE(features && centroids && labels, "spr_role_assign_fp32: null pointer");
  dim3 grid(static_cast<uint32_t>(spr::ceil_div(n, 256)), static_cast<uint32_t>(batch));
  switch (d) {
    case 16: role_assign_fp32_kernel<16><<<grid, 256, 0, stream>>>(features, centroids, n, k, labels, best_dist); break;
    case 32: role_assign_fp32_kernel<32><<<grid, 256, 0, stream>>>(features, centroids, n, k, labels, best_dist); break;
    case 48: role_assign_fp32_kernel<48><<<grid, 256, 0, stream>>>(features, centroids, n, k, labels, best_dist); break;
    case 64: role_assign_fp32_kernel<64><<<grid, 256, 0, stream>>>(features, centroids, n, k, labels, best_dist); break;
    default: SPR_REQUIRE(false, "spr_role_assign_fp32: dim %d not supported (16, 32, 48, 64)", d);
  }
  SPR_LAUNCHED("role_assign_fp32_kernel");
  return SPR_OK;
}
