// Role-coordinate projection with row RMS normalisation (N8's Q role features), and the
// K (or V) role projection with one RMS scale per head.
//
// Replaces:
//   _role_projection_rms_kernel + role_projection_rms_triton
//       (src/sparsepr/kernels/triton/role_projection.py:16-55, :58-103)
//   _role_k_projection_normalize_fp32 / _role_kv_projection_normalize_fp32, torch.compile'd
//       under role_kv_matmul_precision (src/sparsepr/models/common/n8_v6.py:77-149), and
//       normalize_feature_scale(project_tokens(...)) (operator_kmeans.py:540-550)
//
//   p = x . F~, out = p / sqrt(max(sum_r p_r^2 / R, 1e-12))
// for x bf16 [bh, n, d] and the factor F fp32 [bh, d, R]; F~ is F as the fp32 matmul sees it:
//   PREC 0 ("high", and tl.dot(..., input_precision="tf32")): rounded to TF32 (nearest, ties
//          away; a bf16 x is exact in TF32), split into bf16 hi + lo with hi + lo == F~;
//   PREC 1 ("highest", plain fp32): F itself, split into bf16 hi + mid + lo (8 significant
//          bits each, 24 in all) with hi + mid + lo == F;
//   PREC 2 ("medium", bf16 operands): F rounded to bf16 (nearest even).
// Each product of a bf16 x with a bf16 piece is exact, so only the fp32 summation order
// differs from the reference's.
//
// Layout: workgroups of four waves per head, as many as stay resident, each walking token
// blocks of its head (rp_tokens); F~^T hi / lo of the head
// sit in LDS (R rows padded to a multiple of 32, d columns, 16-byte pieces swizzled
// by row).  A wave computes P^T = F~^T X^T for 32 tokens per step: A = F~^T fragments
// from LDS, B = X^T fragments straight from HBM (lane = token, 16 contiguous bytes per
// 16-dim step, the next block's prefetched), so each lane ends up with R / 2 values of
// one token and the row's sum of squares needs one exchange between the two half-waves.
#include <algorithm>

#include "spr_common.h"

namespace {

using spr::f32x16;
using spr::u32x4;

constexpr int RP_THREADS = 256;
constexpr int RP_WAVES = RP_THREADS / 64;
// Tokens per block (a workgroup takes several blocks of its head): 256 for the row-normalised
// projection (MODE 0) and the K projection's scaling pass (MODE 2), 1024 for its sum pass
// (MODE 1: one fp64 partial per block, which MODE 2 sums in block order).  Measured in the N8
// step against 512 for all: Q projection 0.39 -> 0.36 ms, K projection 0.64 -> 0.61 ms.
constexpr int rp_tokens(int mode) { return mode == 1 ? 1024 : 256; }
constexpr int RP_MAX_R = 128;

__device__ __forceinline__ float tf32_rna(float x) {
  return __uint_as_float((__float_as_uint(x) + 0x1000u) & 0xffffe000u);
}

__device__ __forceinline__ float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// D = head dim (D / 8 sixteen-byte pieces per F~^T row); RB = rank padded to 32, in 32-row blocks.
// MODE 0: rows normalised by their RMS.  MODE 1: no output; the workgroup's sum of p^2 goes to
// partial[head][block] (fp64).  MODE 2: p divided by the head's scale sqrt(max(mean p^2, ...))
// formed from the partials in block order (the same on every workgroup); block 0 stores it.
// MODE 2 writes (weight p) / scale into columns out_col .. out_col + R of rows out_ld floats long.
// NP = bf16 pieces of F~ (PREC 0: 2, 1: 3, 2: 1).
template <int D, int RB, int MODE, int PREC>
__global__ __launch_bounds__(RP_THREADS) void role_projection_kernel(const uint16_t* __restrict__ x,
                                                                     const float* __restrict__ factor, int64_t n,
                                                                     int32_t rank, float* __restrict__ out,
                                                                     int32_t out_ld, int32_t out_col, float weight,
                                                                     double* __restrict__ partial,
                                                                     float* __restrict__ head_scale) {
  constexpr int64_t RP_TOKENS = rp_tokens(MODE);
  constexpr int KSTEPS = D / 16;
  constexpr int ROWB = D * 2;  // bytes per F~^T row (bf16)
  constexpr int RP = RB * 32;
  constexpr int NP = PREC == 0 ? 2 : (PREC == 1 ? 3 : 1);
  __shared__ __attribute__((aligned(16))) uint8_t fpc[NP][RP * ROWB];
  const int64_t b = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 31;
  const int half = lane >> 5;

  // F~^T pieces into LDS: element (r, k) of row r at piece (k / 8) ^ (r % (D / 8)), slot k % 8.
  // Each piece is the top 16 bits (a bf16) of what the earlier pieces leave, so the pieces
  // sum to F~ exactly (the remainders are exact in fp32).
  const float* fb = factor + b * D * rank;
  for (int i = tid; i < RP * D / 2; i += RP_THREADS) {
    const int r = i / (D / 2), k = 2 * (i % (D / 2));
    float v[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const float f = r < rank ? fb[static_cast<int64_t>(k + u) * rank + r] : 0.0f;
      v[u] = PREC == 0 ? tf32_rna(f) : (PREC == 2 ? spr::bf16_to_f32(spr::f32_to_bf16(f)) : f);
    }
    const int off = r * ROWB + ((((k >> 3) ^ (r % (D / 8))) << 4) | ((k & 7) << 1));
#pragma unroll
    for (int pc = 0; pc < NP; ++pc) {
      const uint32_t h0 = __float_as_uint(v[0]) & 0xffff0000u, h1 = __float_as_uint(v[1]) & 0xffff0000u;
      *reinterpret_cast<uint32_t*>(fpc[pc] + off) = (h0 >> 16) | h1;
      v[0] -= __uint_as_float(h0);
      v[1] -= __uint_as_float(h1);
    }
  }
  __syncthreads();

  const uint16_t* xb = x + b * n * D;
  float* ob = out + b * n * (MODE == 2 ? out_ld : rank);
  __shared__ double red_l[RP_WAVES];
  float div = 1.0f;
  if (MODE == 2) {
    // the head's scale: fp64 sum of the partials in block order, then as the reference
    // rounds it: fp32 mean, sqrt, clamp at 1e-8
    const int64_t nparts = (n + rp_tokens(1) - 1) / rp_tokens(1);  // the first pass's blocks
    double tot = 0.0;
    for (int64_t i = 0; i < nparts; ++i) tot += partial[b * nparts + i];
    div = fmaxf(sqrtf(static_cast<float>(tot / (static_cast<double>(n) * rank))), 1.0e-8f);
    if (blockIdx.x == 0 && tid == 0) head_scale[b] = div;
  }
  // Token blocks of RP_TOKENS: this workgroup takes blocks blockIdx.x, + gridDim.x, ... of its
  // head (the grid holds as many workgroups per head as stay resident at once, so no second
  // round of workgroups trails the first).  MODE 1 writes one partial per block.
  const int64_t nvb = (n + RP_TOKENS - 1) / RP_TOKENS;
  // X^T fragments of a 32-token block: lane = token, 16 bytes per 16-dim step (zero past the end)
  auto load_x = [&](u32x4 (&xf)[KSTEPS], int64_t t0, int64_t t_end) {
    const int64_t t = t0 + col;
    const bool live = t < t_end;
    const uint16_t* xr = xb + (live ? t : t0) * D + 8 * half;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      xf[s] = *reinterpret_cast<const u32x4*>(xr + 16 * s);
      if (!live) xf[s] = u32x4{0, 0, 0, 0};
    }
  };
  // this wave's next 32-token block after (vb, t0): the next one of the block, else the
  // first of the workgroup's next block; vb = nvb when there is none
  auto skip_empty = [&](int64_t& vb, int64_t& t0) {  // a short last block may hold none of this wave's rows
    while (vb < nvb && t0 >= min((vb + 1) * RP_TOKENS, n)) {
      vb += gridDim.x;
      t0 = vb * RP_TOKENS + 32 * wave;
    }
  };
  auto advance = [&](int64_t& vb, int64_t& t0) {
    t0 += 32 * RP_WAVES;
    skip_empty(vb, t0);
  };
  int64_t vb = blockIdx.x, t0 = vb * RP_TOKENS + 32 * wave;
  skip_empty(vb, t0);
  u32x4 xn[KSTEPS];
  if (vb < nvb) load_x(xn, t0, min((vb + 1) * RP_TOKENS, n));
  double wsum = 0.0;  // MODE 1: this lane's sum of p^2 over the current block
  for (int64_t cur = blockIdx.x; cur < nvb; cur += gridDim.x) {
    const int64_t t_end = min((cur + 1) * RP_TOKENS, n);
    while (vb == cur) {
      const int64_t t = t0 + col;
      const bool live = t < t_end;
      u32x4 xf[KSTEPS];
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) xf[s] = xn[s];
      const int64_t t_row = t0;
      // the next block's loads are in flight during this block's MFMAs and stores
      advance(vb, t0);
      if (vb < nvb) load_x(xn, t0, min((vb + 1) * RP_TOKENS, n));
      f32x16 acc[RB];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        acc[rb] = f32x16{};
        const int r = 32 * rb + col;
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) {
          const int off = r * ROWB + (((2 * s + half) ^ (r % (D / 8))) << 4);
#pragma unroll
          for (int pc = 0; pc < NP; ++pc) {
            const u32x4 a = *reinterpret_cast<const u32x4*>(fpc[pc] + off);
            acc[rb] =
                __builtin_amdgcn_mfma_f32_32x32x16_bf16(spr::as_bf16x8(a), spr::as_bf16x8(xf[s]), acc[rb], 0, 0, 0);
          }
        }
      }
      // lane (token col, half) holds p_r for r = 32 rb + 8 (e / 4) + 4 half + e % 4 (zero past rank)
      float ss = 0.0f;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
        for (int e = 0; e < 16; ++e) ss = __builtin_fmaf(acc[rb][e], acc[rb][e], ss);
      }
      if (MODE == 1) {
        wsum += live ? static_cast<double>(ss) : 0.0;
        continue;
      }
      ss = sum_xor32(ss);
      const float inv = 1.0f / sqrtf(fmaxf(ss / static_cast<float>(rank), 1.0e-12f));
      auto nrm = [&](float v) { return MODE == 0 ? v * inv : (weight * v) / div; };
      if (live) {
        const int64_t tt = t_row + col;
        float* orow = MODE == 2 ? ob + tt * out_ld + out_col : ob + tt * rank;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int r0 = 32 * rb + 8 * g + 4 * half;
            if (r0 + 3 < rank && (rank & 3) == 0 && (MODE != 2 || ((out_ld | out_col) & 3) == 0)) {
              *reinterpret_cast<float4*>(orow + r0) = make_float4(nrm(acc[rb][4 * g]), nrm(acc[rb][4 * g + 1]),
                                                                  nrm(acc[rb][4 * g + 2]), nrm(acc[rb][4 * g + 3]));
            } else {
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                if (r0 + i < rank) orow[r0 + i] = nrm(acc[rb][4 * g + i]);
              }
            }
          }
        }
      }
    }
    if (MODE == 1) {
      // lanes in order, then waves in order: the same fp64 sum on every run
      for (int o = 1; o < 64; o <<= 1) wsum += __shfl_xor(wsum, o, 64);
      if (lane == 0) red_l[wave] = wsum;
      __syncthreads();
      if (tid == 0) {
        double tsum = 0.0;
        for (int w = 0; w < RP_WAVES; ++w) tsum += red_l[w];
        partial[b * nvb + cur] = tsum;
      }
      __syncthreads();
      wsum = 0.0;
    }
  }
}

}  // namespace

// Compute units of the calling thread's current device (queried once per device).
static int rp_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

// Workgroups per head: as many as stay resident together (per_cu per CU, from the
// occupancy calculator), shared evenly by the heads, at most one per token block.
static uint32_t rp_groups_per_head(int64_t bh, int64_t n, int per_cu, int tokens) {
  const int64_t resident = static_cast<int64_t>(std::max(per_cu, 1)) * rp_cu_count();
  const int64_t nvb = (n + tokens - 1) / tokens;
  return static_cast<uint32_t>(std::max<int64_t>(1, std::min<int64_t>(nvb, resident / std::max<int64_t>(bh, 1))));
}

// Resident workgroups per CU of role_projection_kernel<D, RB, MODE, PREC> (queried once per
// instantiation; 1 if the query fails).
template <int D, int RB, int MODE, int PREC>
static int rp_occupancy() {
  static int cached = 0;
  if (cached == 0) {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, role_projection_kernel<D, RB, MODE, PREC>, RP_THREADS, 0) !=
            hipSuccess ||
        nb <= 0)
      nb = 1;
    cached = nb;
  }
  return cached;
}

template <int MODE, int PREC>
static void launch_role_projection(int64_t bh, hipStream_t stream, const uint16_t* xp, const float* factor,
                                   int64_t n, int32_t d, int32_t rank, float* out, int32_t out_ld, int32_t out_col,
                                   float weight, double* partial, float* head_scale) {
  const int rb = (rank + 31) / 32;
#define SPR_RP(DD, RBB)                                                                                      \
  role_projection_kernel<DD, RBB, MODE, PREC>                                                                \
      <<<dim3(rp_groups_per_head(bh, n, (rp_occupancy<DD, RBB, MODE, PREC>()), rp_tokens(MODE)), \
              static_cast<uint32_t>(bh)),                                                                    \
         RP_THREADS, 0, stream>>>(xp, factor, n, rank, out, out_ld, out_col, weight, partial, head_scale)
  if (d == 128) {
    if (rb == 1) SPR_RP(128, 1); else if (rb == 2) SPR_RP(128, 2); else if (rb == 3) SPR_RP(128, 3); else SPR_RP(128, 4);
  } else {
    if (rb == 1) SPR_RP(64, 1); else if (rb == 2) SPR_RP(64, 2); else if (rb == 3) SPR_RP(64, 3); else SPR_RP(64, 4);
  }
#undef SPR_RP
}

extern "C" int spr_role_projection_rms(const void* x, const float* factor, int64_t bh, int64_t n, int32_t d,
                                       int32_t rank, float* out, hipStream_t stream) {
  SPR_REQUIRE(bh >= 0 && n >= 0, "spr_role_projection_rms: bad size");
  SPR_REQUIRE(d == 64 || d == 128, "spr_role_projection_rms: head dim must be 64 or 128 (got %d)", d);
  SPR_REQUIRE(rank >= 1 && rank <= RP_MAX_R, "spr_role_projection_rms: rank must be in [1, %d] (got %d)", RP_MAX_R,
              rank);
  if (bh == 0 || n == 0) return SPR_OK;
  SPR_REQUIRE(x && factor && out, "spr_role_projection_rms: null pointer");
  SPR_REQUIRE(bh <= 65535, "spr_role_projection_rms: too many heads");
  launch_role_projection<0, 0>(bh, stream, static_cast<const uint16_t*>(x), factor, n, d, rank, out, rank, 0, 1.0f,
                               nullptr, nullptr);
  SPR_LAUNCHED("role_projection_kernel");
  return SPR_OK;
}

extern "C" size_t spr_role_k_projection_workspace(int64_t bh, int64_t n) {
  return static_cast<size_t>(bh) * static_cast<size_t>((n + rp_tokens(1) - 1) / rp_tokens(1)) * sizeof(double);
}

extern "C" int spr_role_k_projection_ex(const void* x, const float* factor, int64_t bh, int64_t n, int32_t d,
                                        int32_t rank, int32_t precision, float weight, float* out, int32_t out_ld,
                                        int32_t out_col, float* key_scale, void* workspace, size_t workspace_bytes,
                                        hipStream_t stream) {
  SPR_REQUIRE(bh >= 0 && n >= 0, "spr_role_k_projection: bad size");
  SPR_REQUIRE(d == 64 || d == 128, "spr_role_k_projection: head dim must be 64 or 128 (got %d)", d);
  SPR_REQUIRE(rank >= 1 && rank <= RP_MAX_R, "spr_role_k_projection: rank must be in [1, %d] (got %d)", RP_MAX_R,
              rank);
  SPR_REQUIRE(precision >= 0 && precision <= 2, "spr_role_k_projection: precision must be 0, 1 or 2 (got %d)",
              precision);
  SPR_REQUIRE(out_col >= 0 && out_ld >= out_col + rank, "spr_role_k_projection: columns %d + %d exceed rows of %d",
              out_col, rank, out_ld);
  if (bh == 0) return SPR_OK;
  SPR_REQUIRE(n >= 1, "spr_role_k_projection: no tokens");
  SPR_REQUIRE(x && factor && out && key_scale, "spr_role_k_projection: null pointer");
  SPR_REQUIRE(bh <= 65535, "spr_role_k_projection: too many heads");
  if (workspace == nullptr || workspace_bytes < spr_role_k_projection_workspace(bh, n)) {
    spr_set_error("spr_role_k_projection: workspace of %zu bytes needed", spr_role_k_projection_workspace(bh, n));
    return SPR_EWORKSPACE;
  }
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  double* part = static_cast<double*>(workspace);
#define SPR_KP(PP)                                                                                             \
  do {                                                                                                         \
    launch_role_projection<1, PP>(bh, stream, xp, factor, n, d, rank, nullptr, 0, 0, 1.0f, part, nullptr);   \
    SPR_LAUNCHED("role_projection_kernel<sum of squares>");                                                    \
    launch_role_projection<2, PP>(bh, stream, xp, factor, n, d, rank, out, out_ld, out_col, weight, part,     \
                                  key_scale);                                                                  \
    SPR_LAUNCHED("role_projection_kernel<head scale>");                                                        \
  } while (0)
  if (precision == 0) SPR_KP(0); else if (precision == 1) SPR_KP(1); else SPR_KP(2);
#undef SPR_KP
  return SPR_OK;
}

extern "C" int spr_role_k_projection(const void* x, const float* factor, int64_t bh, int64_t n, int32_t d,
                                     int32_t rank, float* out, float* key_scale, void* workspace,
                                     size_t workspace_bytes, hipStream_t stream) {
  return spr_role_k_projection_ex(x, factor, bh, n, d, rank, 0, 1.0f, out, rank, 0, key_scale, workspace,
                                  workspace_bytes, stream);
}
