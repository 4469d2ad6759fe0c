// SVG-EAR routing scores: per (query head, query centroid, key cluster) the log
// value-error score of N8's default selector and the log attention mass.
//
// Replaces:
//   _svg_ear_value_error_kernel + svg_ear_value_error_scores_triton
//       (src/sparsepr/kernels/triton/svg_ear.py:95-192, :453-531)
//   _svg_ear_grouped_value_error_kernel + svg_ear_grouped_value_error_scores_triton
//       (svg_ear.py:195-286, :534-600): the same scores, one K/V walk per GQA group
//   _attention_mass_score_kernel + attention_mass_scores_triton (svg_ear.py:7-92, :372-450)
//
// Scores, for query centroid q and the tokens t of key cluster c (k, v bf16):
//   l_t = (q~ . k_t) / sqrt(D), q~ = q rounded to TF32 (the reference's tl.dot
//         input_precision="tf32"), l_c = (q . kc) / sqrt(D) (+ Jensen term)
//   value error: m = max(l_c, max_t l_t), w_c = e^(l_c - m), w_t = e^(l_t - m),
//       E = sum_t max(w_c^2 |vc|^2 + w_t^2 |v_t|^2 - 2 w_t w_c (v_t . vc), 0)
//       score = log(max(E / n_c, 1e-30)) + 2 m;  -inf for an empty cluster
//   attention mass: score = log(max(sum_t e^(l_t - m), 1e-30)) + m, m = max_t l_t
// The running max is kept per 32-token chunk with the reference's rescaling
// (E *= alpha^2, w_c *= alpha; the mass sum *= alpha).
//
// Layout.  A first kernel writes the centroid logits l_c [query head, centroid,
// cluster] (fp32 dot products over d, sequential, 128 rows x 32 clusters per workgroup)
// into the score buffer; the score kernel overwrites each entry with its score.
// The score kernel runs one workgroup of four waves per (query head, 8
// consecutive key clusters); wave w scores query rows 32 w .. 32 w + 31 of each
// group of 128 (a loop covers more centroids).  The clusters' tokens are one
// contiguous run, walked in 32-token chunks (a chunk never spans two clusters).
// Per chunk: every thread holds 32 bytes of K and of V (token tid / 8, dims
// 16 (tid % 8) .. + 15), prefetched during the previous chunk; it stores the K
// bytes into a swizzled LDS tile (16-byte piece p of token row t at slot
// p ^ (t % 16): the MFMA fragment reads hit 16 distinct slots per 16 lanes) and
// reduces |v_t|^2 and v_t . vc over the token's 8 threads (DPP) into LDS.  After one
// barrier S^T = K Q~^T comes from 16 bf16 MFMAs per wave: q~ is split into bf16
// hi + lo with hi + lo == q~ exactly (q~ has 11 significant bits, hi the top 8,
// lo the next 3), so every product is the reference's TF32 product exactly and
// only the fp32 summation order differs.  Two LDS buffers alternate by chunk.
// The token runs come from a block prefix sum of the sizes and are clamped to
// the stored tokens, so no size vector can make the kernel read outside K or V.
#include <type_traits>

#include "spr_common.h"

namespace {

using spr::f32x16;
using spr::u32x4;

constexpr int SE_D = 128;
constexpr int SE_THREADS = 256;
constexpr int SE_WAVES = SE_THREADS / 64;
constexpr int SE_CHUNK = 32;  // tokens per chunk: one 32-row MFMA block
constexpr int SE_KSTEPS = SE_D / 16;
constexpr float SE_LOG2E = 1.4426950408889634f;

// Round to TF32 (10 stored mantissa bits), to nearest with ties away from zero.
__device__ __forceinline__ float tf32_rna(float x) {
  return __uint_as_float((__float_as_uint(x) + 0x1000u) & 0xffffe000u);
}

__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * SE_LOG2E); }

__device__ __forceinline__ float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, uint8_t* lds, int32_t voff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, 0);
#endif
}

// Workgroup barrier after this wave's LDS accesses completed, with no wait on the
// vector memory counter: LDS DMA of later chunks stays in flight across it (its
// landing is waited for explicitly).  The memory clobber keeps the compiler from
// moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// sum over lanes 8 i .. 8 i + 7 (quad_perm [1, 0, 3, 2], [2, 3, 0, 1], then row_half_mirror)
__device__ __forceinline__ float oct_sum(float v) {
  v += dpp_mov<0xB1>(v);
  v += dpp_mov<0x4E>(v);
  return v + dpp_mov<0x141>(v);
}

// max / sum over lanes l and l ^ 32: v_permlane32_swap of x with itself gives the
// lower half-wave's value in the first result and the upper half's in the second on
// every lane, so both lanes of a pair combine the same two operands in the same order.
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

constexpr int SE_ROW = SE_D * 2;  // bytes per bf16 token row
// key clusters per workgroup (4 was faster on synthetic cluster sizes but 2 % slower on the
// routed clusters of the C4 bench, and within noise in the N8 step; 2 and 16 were slower)
constexpr int SE_CPW = 8;
constexpr int CL_CLUSTERS = 32;   // clusters per centroid-logit workgroup
constexpr int CL_ROWS = 2 * (SE_THREADS / 4);  // query rows per centroid-logit workgroup

// l_c = (q . kc) / sqrt(D) (+ 0.5 min(sum_d q_d^2 var_d / D, cap)) for CL_ROWS query rows x
// CL_CLUSTERS clusters per workgroup: thread -> query rows tid / 4 and tid / 4 + CL_ROWS / 2,
// clusters 8 (tid % 4) .. + 7 (each centroid read from LDS serves two rows); fp32 fma chains
// over d in order.  Written to out [qh, qn, kn].
__global__ __launch_bounds__(SE_THREADS) void svg_ear_centroid_logit_kernel(
    const float* __restrict__ qc, const float* __restrict__ kcent, const float* __restrict__ var_k, float cap,
    int32_t qn, int32_t kn, int32_t group, float* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) float kc_l[CL_CLUSTERS][SE_D];
  __shared__ __attribute__((aligned(16))) float var_l[CL_CLUSTERS][SE_D];
  const int64_t qh = blockIdx.z;
  const int64_t kh = qh / group;
  const int cb = blockIdx.x * CL_CLUSTERS;
  const int ncl = min(CL_CLUSTERS, kn - cb);
  const int tid = threadIdx.x;
  const float scale = 1.0f / 11.313708498984761f;
  for (int i = tid; i < CL_CLUSTERS * SE_D / 4; i += SE_THREADS) {
    const int c = i / (SE_D / 4), d = 4 * (i % (SE_D / 4));
    const bool live = c < ncl;
    const int64_t o = (kh * kn + cb + c) * SE_D + d;
    *reinterpret_cast<float4*>(&kc_l[c][d]) =
        live ? *reinterpret_cast<const float4*>(kcent + o) : float4{0.0f, 0.0f, 0.0f, 0.0f};
    *reinterpret_cast<float4*>(&var_l[c][d]) =
        (live && var_k != nullptr) ? *reinterpret_cast<const float4*>(var_k + o) : float4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  __syncthreads();
  const int r0 = blockIdx.y * CL_ROWS + tid / 4;
  const int r1 = r0 + CL_ROWS / 2;
  const int c0 = 8 * (tid % 4);
  if (r0 >= qn) return;
  const float* qrow0 = qc + (qh * qn + r0) * SE_D;
  const float* qrow1 = qc + (qh * qn + min(r1, qn - 1)) * SE_D;  // a row past qn computes, stores nothing
  float dot0[8], s20[8], dot1[8], s21[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) dot0[j] = s20[j] = dot1[j] = s21[j] = 0.0f;
  for (int d0 = 0; d0 < SE_D; d0 += 4) {
    const float4 qa = *reinterpret_cast<const float4*>(qrow0 + d0);
    const float4 qb = *reinterpret_cast<const float4*>(qrow1 + d0);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float4 kv = *reinterpret_cast<const float4*>(&kc_l[c0 + j][d0]);
      dot0[j] = __builtin_fmaf(qa.x, kv.x, dot0[j]);
      dot0[j] = __builtin_fmaf(qa.y, kv.y, dot0[j]);
      dot0[j] = __builtin_fmaf(qa.z, kv.z, dot0[j]);
      dot0[j] = __builtin_fmaf(qa.w, kv.w, dot0[j]);
      dot1[j] = __builtin_fmaf(qb.x, kv.x, dot1[j]);
      dot1[j] = __builtin_fmaf(qb.y, kv.y, dot1[j]);
      dot1[j] = __builtin_fmaf(qb.z, kv.z, dot1[j]);
      dot1[j] = __builtin_fmaf(qb.w, kv.w, dot1[j]);
      if (var_k != nullptr) {
        const float4 vv = *reinterpret_cast<const float4*>(&var_l[c0 + j][d0]);
        s20[j] = __builtin_fmaf(qa.x * qa.x, vv.x, s20[j]);
        s20[j] = __builtin_fmaf(qa.y * qa.y, vv.y, s20[j]);
        s20[j] = __builtin_fmaf(qa.z * qa.z, vv.z, s20[j]);
        s20[j] = __builtin_fmaf(qa.w * qa.w, vv.w, s20[j]);
        s21[j] = __builtin_fmaf(qb.x * qb.x, vv.x, s21[j]);
        s21[j] = __builtin_fmaf(qb.y * qb.y, vv.y, s21[j]);
        s21[j] = __builtin_fmaf(qb.z * qb.z, vv.z, s21[j]);
        s21[j] = __builtin_fmaf(qb.w * qb.w, vv.w, s21[j]);
      }
    }
  }
  auto store = [&](int r, const float (&dot)[8], const float (&s2)[8]) {
    float* orow = out + (qh * qn + r) * kn + cb + c0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (c0 + j < ncl) {
        float l = dot[j] * scale;
        if (var_k != nullptr) l += 0.5f * fminf(s2[j] / static_cast<float>(SE_D), cap);
        orow[j] = l;
      }
    }
  };
  store(r0, dot0, s20);
  if (r1 < qn) store(r1, dot1, s21);
}

template <int MODE>  // 0: value error (scores holds l_c on entry), 1: attention mass
__global__ __launch_bounds__(SE_THREADS) void svg_ear_score_kernel(
    const float* __restrict__ qc, const uint16_t* __restrict__ ks, const uint16_t* __restrict__ vs,
    const float* __restrict__ vcent, const int32_t* __restrict__ k_sizes, int32_t qn, int32_t kn, int64_t t_stored,
    int32_t group, float* __restrict__ scores) {
  // four K and four V tiles as separate arrays: the chunk loop is unrolled by four so that
  // every LDS read names a tile the compiler can tell apart from the ones being DMA'd
  // (otherwise it waits for all DMA in flight before each read)
  __shared__ __attribute__((aligned(1024))) uint8_t k_l0[SE_CHUNK * SE_ROW];
  __shared__ __attribute__((aligned(1024))) uint8_t k_l1[SE_CHUNK * SE_ROW];
  __shared__ __attribute__((aligned(1024))) uint8_t k_l2[SE_CHUNK * SE_ROW];
  __shared__ __attribute__((aligned(1024))) uint8_t k_l3[SE_CHUNK * SE_ROW];
  __shared__ __attribute__((aligned(1024))) uint8_t v_l0[SE_CHUNK * SE_ROW];
  __shared__ __attribute__((aligned(1024))) uint8_t v_l1[SE_CHUNK * SE_ROW];
  __shared__ __attribute__((aligned(1024))) uint8_t v_l2[SE_CHUNK * SE_ROW];
  __shared__ __attribute__((aligned(1024))) uint8_t v_l3[SE_CHUNK * SE_ROW];
  __shared__ __attribute__((aligned(16))) float vn2_l[2][SE_CHUNK];
  __shared__ __attribute__((aligned(16))) float cdv_l[2][SE_CHUNK];
  __shared__ float vc_l[SE_CPW][SE_D];
  __shared__ float vc2_l[SE_CPW];
  __shared__ float cl_l[SE_CPW][32 * SE_WAVES];
  __shared__ int32_t start_l[SE_CPW];  // first stored token of each cluster's run (clamped)
  __shared__ int32_t len_l[SE_CPW];    // tokens in each run (clamped)
  __shared__ int32_t nxt_l[SE_CPW];    // next cluster with tokens (ncl if none)
  __shared__ int64_t red_l[SE_WAVES];

  const int c_begin = blockIdx.x * SE_CPW;
  const int ncl = min(SE_CPW, kn - c_begin);
  const int64_t qh = blockIdx.y;
  const int64_t kh = qh / group;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 31;
  const int half = lane >> 5;
  const float scale = 1.0f / 11.313708498984761f;  // 1 / sqrt(128), as the fp32 quotient

  // ---- token runs of clusters c_begin .. c_begin + ncl - 1 (negative sizes count as 0)
  const int32_t* sz = k_sizes + kh * kn;
  int64_t part = 0;
  for (int j = tid; j < c_begin; j += SE_THREADS) part += max(sz[j], 0);
  for (int o = 32; o > 0; o >>= 1) part += __shfl_xor(part, o, 64);
  if (lane == 0) red_l[wave] = part;
  if (MODE == 0) {
    for (int i = tid; i < SE_CPW * SE_D; i += SE_THREADS) {
      const int j = i / SE_D;
      vc_l[j][i % SE_D] = j < ncl ? vcent[(kh * kn + c_begin + j) * SE_D + i % SE_D] : 0.0f;
    }
  }
  __syncthreads();
  if (tid == 0) {
    int64_t cum = 0;
    for (int w = 0; w < SE_WAVES; ++w) cum += red_l[w];
    for (int j = 0; j < SE_CPW; ++j) {
      const int64_t a = min(cum, t_stored);
      if (j < ncl) cum += max(sz[c_begin + j], 0);
      start_l[j] = static_cast<int32_t>(a);
      len_l[j] = static_cast<int32_t>(min(cum, t_stored) - a);
    }
    int next = ncl;
    for (int j = SE_CPW - 1; j >= 0; --j) {
      nxt_l[j] = next;
      if (j < ncl && len_l[j] > 0) next = j;
    }
  }
  if (MODE == 0) {
    for (int j = wave; j < SE_CPW; j += SE_WAVES) {
      const float a = vc_l[j][2 * lane], b = vc_l[j][2 * lane + 1];
      const float s = wave_sum(__builtin_fmaf(a, a, b * b));
      if (lane == 0) vc2_l[j] = s;
    }
  }
  __syncthreads();
  auto cl_len = [&](int j) { return len_l[j]; };
  // empty clusters score -inf
  for (int j = 0; j < ncl; ++j) {
    if (cl_len(j) <= 0) {
      for (int q = tid; q < qn; q += SE_THREADS) scores[(qh * qn + q) * kn + c_begin + j] = -__builtin_huge_valf();
    }
  }
  const int j_first = cl_len(0) > 0 ? 0 : nxt_l[0];
  if (j_first >= ncl) return;

  // ---- K/V chunks land in LDS by DMA: 32 token rows of 256 bytes per tile; wave w moves rows
  // 4 w .. 4 w + 3 and 16 + 4 w .. + 3 (1 KB per instruction).  In the K tile the lane that
  // fills slot p of row t fetches piece p ^ (t % 16) (the swizzle of the MFMA reads); V is
  // stored as is.  Rows past the cluster's run hold the next cluster's tokens (masked in the
  // scores); rows past the stored tokens read as zero (buffer bounds).
  const __amdgpu_buffer_rsrc_t k_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(ks + kh * t_stored * SE_D), 0, static_cast<int32_t>(t_stored * SE_ROW), 0x00020000);
  const __amdgpu_buffer_rsrc_t v_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(MODE == 0 ? vs + kh * t_stored * SE_D : ks), 0, static_cast<int32_t>(t_stored * SE_ROW),
      0x00020000);
  auto dma = [&](int j, int c0, uint8_t* kd, uint8_t* vd) {
    const int slot = lane & 15;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r0 = 4 * wave + 16 * i;
      const int row = r0 + (lane >> 4);
      const int32_t off = (start_l[j] + c0 + row) * SE_ROW;
      lds_dma16(k_rsrc, kd + r0 * SE_ROW, off + ((slot ^ (row & 15)) << 4));
      if (MODE == 0) lds_dma16(v_rsrc, vd + r0 * SE_ROW, off + (slot << 4));
    }
  };
  constexpr int DMA_PER_CHUNK = MODE == 0 ? 4 : 2;  // per wave
  // |v_t|^2 and v_t . vc of chunk (j, c0) from V tile b into vn2_l / cdv_l[p]: token tid / 8,
  // dims 16 (tid % 8) .. + 15, reduced over the token's 8 lanes
  auto vstats = [&](int j, const uint8_t* vt, int p) {
    const int pt = tid >> 3, pp = 2 * (tid & 7);
    const uint8_t* vr = vt + pt * SE_ROW + pp * 16;
    const float* cc = vc_l[j] + 8 * pp;
    float pn = 0.0f, pc = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const u32x4 v4 = *reinterpret_cast<const u32x4*>(vr + 16 * i);
      const uint32_t w[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = spr::bf16_lo(w[e]), hi = spr::bf16_hi(w[e]);
        pn = __builtin_fmaf(lo, lo, pn);
        pn = __builtin_fmaf(hi, hi, pn);
        pc = __builtin_fmaf(lo, cc[8 * i + 2 * e], pc);
        pc = __builtin_fmaf(hi, cc[8 * i + 2 * e + 1], pc);
      }
    }
    pn = oct_sum(pn);
    pc = oct_sum(pc);
    if ((tid & 7) == 0) {
      vn2_l[p][pt] = pn;
      cdv_l[p][pt] = pc;
    }
  };
  // next (cluster, chunk) of the walk; j = ncl when done
  auto advance = [&](int& j, int& c0) {
    c0 += SE_CHUNK;
    if (c0 >= cl_len(j)) {
      c0 = 0;
      j = nxt_l[j];
    }
  };

  for (int q0 = 0; q0 < qn; q0 += 32 * SE_WAVES) {
    const int q = q0 + 32 * wave + col;
    const bool q_live = q < qn;
    const bool wave_live = q0 + 32 * wave < qn;
    const float* qrow = qc + (qh * qn + (q_live ? q : 0)) * SE_D;

    // B fragments: q~ dims 16 s + 8 half + 0..7 as bf16 hi and lo
    u32x4 qhi[SE_KSTEPS], qlo[SE_KSTEPS];
#pragma unroll
    for (int s = 0; s < SE_KSTEPS; ++s) {
      float v[8];
      if (q_live) {
        const float4 a = *reinterpret_cast<const float4*>(qrow + 16 * s + 8 * half);
        const float4 b = *reinterpret_cast<const float4*>(qrow + 16 * s + 8 * half + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = 0.0f;
      }
      uint32_t h[4], l[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float t0 = tf32_rna(v[2 * i]), t1 = tf32_rna(v[2 * i + 1]);
        const float h0 = __uint_as_float(__float_as_uint(t0) & 0xffff0000u);
        const float h1 = __uint_as_float(__float_as_uint(t1) & 0xffff0000u);
        h[i] = (__float_as_uint(h0) >> 16) | (__float_as_uint(h1) & 0xffff0000u);
        // t - h has at most 3 significant bits: exact in fp32 and in bf16
        l[i] = (__float_as_uint(t0 - h0) >> 16) | (__float_as_uint(t1 - h1) & 0xffff0000u);
      }
      qhi[s] = u32x4{h[0], h[1], h[2], h[3]};
      qlo[s] = u32x4{l[0], l[1], l[2], l[3]};
    }
    // every wave is done with the previous query group (its tiles, statistics and cl_l)
    __syncthreads();
    if (MODE == 0) {
      // centroid logits of this query group (written by svg_ear_centroid_logit_kernel)
      for (int i = tid; i < SE_CPW * 32 * SE_WAVES; i += SE_THREADS) {
        const int j = i / (32 * SE_WAVES), r = q0 + i % (32 * SE_WAVES);
        cl_l[j][i % (32 * SE_WAVES)] = (j < ncl && r < qn) ? scores[(qh * qn + r) * kn + c_begin + j] : 0.0f;
      }
      __syncthreads();  // every wave has read l_c before any score of the group is written
    }

    float m = 0.0f, cw = 1.0f, esum = 0.0f;
    int j = j_first, c0 = 0;       // chunk computed
    int jv = j_first, cv = 0;      // chunk whose V statistics come next
    int jd = j_first, cd = 0;      // next chunk to DMA
    int issued = 0, step = 0;      // chunks DMA'd / computed in this query group
    // chunks 0 .. 2 into tiles 0 .. 2 (named arrays, as in the loop)
    auto prologue_dma = [&](uint8_t* kd, uint8_t* vd) {
      if (jd < ncl) {
        dma(jd, cd, kd, vd);
        ++issued;
        advance(jd, cd);
      }
    };
    prologue_dma(k_l0, v_l0);
    prologue_dma(k_l1, v_l1);
    prologue_dma(k_l2, v_l2);
    // chunk 0 landed (this wave's DMA), then every wave's; its V statistics
    if (issued == 3) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * DMA_PER_CHUNK) : "memory");
    } else if (issued == 2) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(DMA_PER_CHUNK) : "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    lds_barrier();
    if (MODE == 0) vstats(jv, v_l0, 0);
    advance(jv, cv);
    // S^T of the chunk in tile kt: 16 MFMAs (hi and lo halves of q~ per 16-dim step)
    auto smma = [&](f32x16& acc, const uint8_t* kt) {
      acc = f32x16{};
#pragma unroll
      for (int s = 0; s < SE_KSTEPS; ++s) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(kt + col * SE_ROW + (((2 * s + half) ^ (col & 15)) << 4));
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(spr::as_bf16x8(a), spr::as_bf16x8(qhi[s]), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(spr::as_bf16x8(a), spr::as_bf16x8(qlo[s]), acc, 0, 0, 0);
      }
    };
    f32x16 acc_a, acc_b;
    if (wave_live) smma(acc_a, k_l0);
    // One chunk step s: DMAs chunk s + 3 into kd / vd, takes the V statistics of chunk
    // s + 1 from vt1 into buf ^ 1, issues the MFMAs of chunk s + 1 (tile kt1) into
    // acc_next and folds chunk s (acc_cur, statistics buf) into the running state: the
    // matrix unit works on s + 1 while the VALU works on s.  Returns false when the walk
    // is done.
    auto chunk_step = [&](const uint8_t* kt1, const uint8_t* vt1, uint8_t* kd, uint8_t* vd, const int buf,
                          f32x16& acc_cur, f32x16& acc_next) {
      if (j >= ncl) return false;
      const int cn = min(SE_CHUNK, cl_len(j) - c0);
      const int jc = j;
      const bool first = c0 == 0;
      const bool last = c0 + SE_CHUNK >= cl_len(j);
      // chunk step + 1 landed (this wave's DMA; the one of step + 2 may still be in flight),
      // then every wave's; every wave is past step - 1, so its tiles and statistics are free
      if (issued > step + 2) {
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(DMA_PER_CHUNK) : "memory");
      } else {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
      lds_barrier();
      if (jd < ncl) {
        dma(jd, cd, kd, vd);
        ++issued;
        advance(jd, cd);
      }
      const bool has_next = jv < ncl;
      if (has_next) {
        if (MODE == 0) vstats(jv, vt1, buf ^ 1);
        advance(jv, cv);
      }
      advance(j, c0);
      ++step;
      if (wave_live) {
        if (has_next) smma(acc_next, kt1);
        if (first) {
          m = MODE == 0 ? cl_l[jc][32 * wave + col] : -__builtin_huge_valf();
          cw = 1.0f;
          esum = 0.0f;
        }
        f32x16* acc = &acc_cur;
        constexpr int NB = 1;
        // element e of block b is token 32 b + 8 (e / 4) + 4 half + e % 4 of the chunk
        // The chunk's 16 elements per lane, straight-line.  A full chunk (the common case)
        // needs no mask; in a partial one a token past the end (its rows hold the next
        // cluster's tokens or zeros) gets exponent -inf (weight 0) and its error term is
        // cleared bitwise, so no value of those rows reaches the sums.
        auto update = [&](auto masked) {
          constexpr bool MASKED = decltype(masked)::value;
          auto live = [&](int b, int e) { return 32 * b + 8 * (e / 4) + 4 * half + (e % 4) < cn; };
          // max over the raw dot products, scaled once: fl(a s) is monotone in a for s > 0,
          // so this is the max of the scaled logits
          float cmax = -__builtin_huge_valf();
#pragma unroll
          for (int b = 0; b < NB; ++b) {
#pragma unroll
            for (int e = 0; e < 16; ++e) cmax = fmaxf(cmax, (!MASKED || live(b, e)) ? acc[b][e] : -__builtin_huge_valf());
          }
          cmax = max_xor32(cmax) * scale;
          const float m_new = fmaxf(m, cmax);
          const float alpha = exp_fast(m - m_new);
          // e^(l - m_new) = 2^(dot * scale * log2 e - m_new * log2 e), one fma per element
          const float c1 = scale * SE_LOG2E;
          const float negm = -m_new * SE_LOG2E;
          float add = 0.0f;
          if (MODE == 0) {
            cw *= alpha;
            esum *= alpha * alpha;
            const float base = cw * cw * vc2_l[jc];
            const float two_cw = 2.0f * cw;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                const int t0 = 32 * b + 8 * i + 4 * half;
                const float4 vn = *reinterpret_cast<const float4*>(&vn2_l[buf][t0]);
                const float4 cd = *reinterpret_cast<const float4*>(&cdv_l[buf][t0]);
                const float vna[4] = {vn.x, vn.y, vn.z, vn.w};
                const float cda[4] = {cd.x, cd.y, cd.z, cd.w};
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                  const bool lv = !MASKED || live(b, 4 * i + r);
                  const float x = __builtin_fmaf(acc[b][4 * i + r], c1, negm);
                  const float tw = __builtin_amdgcn_exp2f(lv ? x : -__builtin_huge_valf());
                  // w_c^2 |vc|^2 + w_t (w_t |v|^2 - 2 w_c v.vc)
                  const float err =
                      fmaxf(__builtin_fmaf(tw, __builtin_fmaf(tw, vna[r], -two_cw * cda[r]), base), 0.0f);
                  add += MASKED ? __int_as_float(__float_as_int(err) & -static_cast<int>(lv)) : err;
                }
              }
            }
          } else {
            esum *= alpha;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
#pragma unroll
              for (int e = 0; e < 16; ++e) {
                const bool lv = !MASKED || live(b, e);
                add += __builtin_amdgcn_exp2f(lv ? __builtin_fmaf(acc[b][e], c1, negm) : -__builtin_huge_valf());
              }
            }
          }
          esum += add;
          m = m_new;
        };
        if (cn == SE_CHUNK) {
          update(std::false_type{});
        } else {
          update(std::true_type{});
        }
        if (last) {
          const float total = sum_xor32(esum);
          if (q_live && half == 0) {
            const float score = MODE == 0
                                    ? logf(fmaxf(total / static_cast<float>(cl_len(jc)), 1.0e-30f)) + 2.0f * m
                                    : logf(fmaxf(total, 1.0e-30f)) + m;
            scores[(qh * qn + q) * kn + c_begin + jc] = score;
          }
        }
      }
      return true;
    };
    while (chunk_step(k_l1, v_l1, k_l3, v_l3, 0, acc_a, acc_b) && chunk_step(k_l2, v_l2, k_l0, v_l0, 1, acc_b, acc_a) &&
           chunk_step(k_l3, v_l3, k_l1, v_l1, 0, acc_a, acc_b) && chunk_step(k_l0, v_l0, k_l2, v_l2, 1, acc_b, acc_a)) {
    }
  }
}

// ---------------------------------------------------------------- compensation
// svg_ear_compensation_triton (svg_ear.py:289-369 kernel, :603-678 wrapper): the sparse
// output (numerator, denominator 1, running max = its LSE) extended by the centroid
// approximation of the key clusters the map did not select.  One workgroup per (64 query
// rows, head); thread t owns row t / 4 and dims 32 (t % 4) .. + 31.  Key clusters go in
// blocks of BK (the reference's BLOCK_K), their TF32-rounded K and V centroids staged in
// LDS: the logit of a cluster is the quad's partial TF32 dot products summed over the four
// lanes (DPP) / sqrt(D) + log(max(count, 1)); per block the running max moves and the state
// is rescaled, the weights (TF32-rounded, as the reference's tl.dot sees them) times the V
// centroids are summed apart and then added (N3: all valid clusters added, the selected
// ones subtracted, as the reference orders it).  fp32 throughout.
__device__ __forceinline__ float quad_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));  // [1,0,3,2]
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));  // [2,3,0,1]
  return v;
}
constexpr int SC_BQ = 64;
constexpr int SC_PART = SE_D / 4;
__device__ __forceinline__ float ldf(const uint16_t* p) { return spr::bf16_to_f32(*p); }  // bf16
__device__ __forceinline__ float ldf(const float* p) { return *p; }
template <typename T>
struct TypeTag {
  using type = T;
};
template <int BK, bool N3, typename TQ, typename TS>
__global__ __launch_bounds__(256) void svg_ear_compensation_kernel(
    const TQ* __restrict__ q, const TS* __restrict__ sparse, const float* __restrict__ lse,
    const int32_t* __restrict__ qlabels, const uint8_t* __restrict__ dmap, int32_t qc1,
    const float* __restrict__ kc, const float* __restrict__ counts, const float* __restrict__ vc, int64_t tokens,
    int32_t kn, float scale, float* __restrict__ out) {
  constexpr int D = SE_D;
  __shared__ __attribute__((aligned(16))) float kcs[BK][D];
  __shared__ __attribute__((aligned(16))) float vcs[BK][D];
  __shared__ float lcnt[BK];
  __shared__ int32_t cvalid[BK];
  const int t = threadIdx.x, qi = t >> 2, d0 = SC_PART * (t & 3);
  const int64_t h = blockIdx.y;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * SC_BQ + qi;
  const bool live = row < tokens;
  const int64_t r = live ? row : tokens - 1;  // rows past the end read the last row, store nothing
  float qv[SC_PART], acc[SC_PART];
#pragma unroll
  for (int j = 0; j < SC_PART; ++j) {
    qv[j] = tf32_rna(ldf(q + (h * tokens + r) * D + d0 + j));
    acc[j] = ldf(sparse + (h * tokens + r) * D + d0 + j);
  }
  float denom = 1.0f;
  float row_max = lse[h * tokens + r];
  const int32_t drow = min(max(qlabels[h * tokens + r] + 1, 0), qc1 - 1);
  const uint8_t* dm = dmap + (h * qc1 + drow) * static_cast<int64_t>(kn + 1) + 1;
  for (int k0 = 0; k0 < kn; k0 += BK) {
    __syncthreads();  // the previous block's centroids are read
    for (int e = t; e < BK * D; e += 256) {
      const int k = e / D, dd = e - k * D, kk = k0 + k;
      kcs[k][dd] = kk < kn ? tf32_rna(kc[(h * kn + kk) * D + dd]) : 0.0f;
      vcs[k][dd] = kk < kn ? tf32_rna(vc[(h * kn + kk) * D + dd]) : 0.0f;
    }
    if (t < BK) {
      const int kk = k0 + t;
      const float c = kk < kn ? counts[h * kn + kk] : 0.0f;
      lcnt[t] = logf(fmaxf(c, 1.0f));
      cvalid[t] = (kk < kn && c > 0.0f) ? 1 : 0;
    }
    __syncthreads();
    float lg[BK];
    uint32_t take = 0, selm = 0;  // bit k: cluster k0 + k added / (N3) selected and added
    float bmax = -__builtin_huge_valf();
#pragma unroll
    for (int k = 0; k < BK; ++k) {
      float pdot = 0.0f;
#pragma unroll
      for (int j = 0; j < SC_PART; j += 4) {
        const spr::f32x4 kv = *reinterpret_cast<const spr::f32x4*>(&kcs[k][d0 + j]);
#pragma unroll
        for (int u = 0; u < 4; ++u) pdot = __builtin_fmaf(qv[j + u], kv[u], pdot);
      }
      lg[k] = quad_sum(pdot) * scale + lcnt[k];
      const bool act = live && cvalid[k] != 0;
      const bool sel = k0 + k < kn ? dm[k0 + k] != 0 : true;
      const bool tk = N3 ? act : (act && !sel);
      take |= static_cast<uint32_t>(tk) << k;
      selm |= static_cast<uint32_t>(N3 && act && sel) << k;
      if (tk) bmax = fmaxf(bmax, lg[k]);
    }
    const float new_max = fmaxf(row_max, bmax);
    const float old = exp_fast(row_max - new_max);  // NaN when both are -inf, as the reference's
    float wsum = 0.0f, ssum = 0.0f;
    float dota[SC_PART], dots[SC_PART];
#pragma unroll
    for (int j = 0; j < SC_PART; ++j) dota[j] = dots[j] = 0.0f;
#pragma unroll
    for (int k = 0; k < BK; ++k) {
      const float w = (take >> k) & 1u ? exp_fast(lg[k] - new_max) : 0.0f;
      const float ws = (selm >> k) & 1u ? w : 0.0f;
      wsum += w;
      ssum += ws;
      const float wt = tf32_rna(w), wst = tf32_rna(ws);
#pragma unroll
      for (int j = 0; j < SC_PART; j += 4) {
        const spr::f32x4 vv = *reinterpret_cast<const spr::f32x4*>(&vcs[k][d0 + j]);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          dota[j + u] = __builtin_fmaf(wt, vv[u], dota[j + u]);
          if constexpr (N3) dots[j + u] = __builtin_fmaf(wst, vv[u], dots[j + u]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < SC_PART; ++j) {
      acc[j] = acc[j] * old + dota[j];
      if constexpr (N3) acc[j] -= dots[j];
    }
    denom = N3 ? (denom * old + wsum) - ssum : denom * old + wsum;
    row_max = new_max;
  }
  if (live) {
    const float inv_den = 1.0f / fmaxf(denom, 1e-30f);
    float* orow = out + (h * tokens + row) * D + d0;
#pragma unroll
    for (int j = 0; j < SC_PART; j += 4) {
      *reinterpret_cast<spr::f32x4*>(orow + j) =
          spr::f32x4{acc[j] * inv_den, acc[j + 1] * inv_den, acc[j + 2] * inv_den, acc[j + 3] * inv_den};
    }
  }
}

}  // namespace

// q [bh, tokens, 128] (q_dtype 0 bf16 / 2 fp32), sparse [bh, tokens, 128] (sparse_dtype 0 / 2),
// lse fp32 [bh, tokens], qlabels int32 [bh, tokens], dmap uint8 [bh, qc1, kn + 1] (row
// qlabel + 1, column cluster + 1), kcentroids / vcentroids fp32 [bh, kn, 128], kcounts fp32
// [bh, kn] -> out fp32 [bh, tokens, 128].  reformulation 0 "skipped", 1 "n3_residual";
// block_k 16 or 32.
extern "C" int spr_svg_ear_compensation(const void* q, int32_t q_dtype, const void* sparse, int32_t sparse_dtype,
                                        const float* lse, const int32_t* qlabels, const uint8_t* dmap, int32_t qc1,
                                        const float* kcentroids, const float* kcounts, const float* vcentroids,
                                        int64_t bh, int64_t tokens, int32_t d, int32_t kn, int32_t reformulation,
                                        int32_t block_k, float* out, hipStream_t stream) {
  SPR_REQUIRE(bh >= 0 && tokens >= 0 && kn >= 0 && qc1 >= 1, "spr_svg_ear_compensation: bad size");
  SPR_REQUIRE(d == SE_D, "spr_svg_ear_compensation: requires DIM=128, got %d", d);
  SPR_REQUIRE(reformulation == 0 || reformulation == 1, "spr_svg_ear_compensation: reformulation must be 0 or 1");
  SPR_REQUIRE(block_k == 16 || block_k == 32, "spr_svg_ear_compensation: block_k must be 16 or 32 (got %d)", block_k);
  SPR_REQUIRE((q_dtype == 0 || q_dtype == 2) && (sparse_dtype == 0 || sparse_dtype == 2),
              "spr_svg_ear_compensation: q and sparse must be bf16 (0) or fp32 (2)");
  SPR_REQUIRE(bh <= 65535, "spr_svg_ear_compensation: too many heads");
  if (bh == 0 || tokens == 0) return SPR_OK;
  SPR_REQUIRE(q && sparse && lse && qlabels && dmap && out && (kn == 0 || (kcentroids && kcounts && vcentroids)),
              "spr_svg_ear_compensation: null pointer");
  const dim3 grid(static_cast<uint32_t>(spr::ceil_div(tokens, SC_BQ)), static_cast<uint32_t>(bh));
  const float scale = 1.0f / sqrtf(static_cast<float>(d));
  auto go = [&](auto bk, auto n3, auto tq, auto ts) {
    using TQ = typename decltype(tq)::type;
    using TS = typename decltype(ts)::type;
    svg_ear_compensation_kernel<decltype(bk)::value, decltype(n3)::value, TQ, TS><<<grid, 256, 0, stream>>>(
        static_cast<const TQ*>(q), static_cast<const TS*>(sparse), lse, qlabels, dmap, qc1, kcentroids, kcounts,
        vcentroids, tokens, kn, scale, out);
  };
  auto by_types = [&](auto bk, auto n3) {
    using BF = TypeTag<uint16_t>;
    using F32 = TypeTag<float>;
    if (q_dtype == 0) {
      if (sparse_dtype == 0) go(bk, n3, BF{}, BF{}); else go(bk, n3, BF{}, F32{});
    } else {
      if (sparse_dtype == 0) go(bk, n3, F32{}, BF{}); else go(bk, n3, F32{}, F32{});
    }
  };
  auto by_mode = [&](auto bk) {
    if (reformulation == 1) by_types(bk, std::true_type{}); else by_types(bk, std::false_type{});
  };
  if (block_k == 16) by_mode(std::integral_constant<int, 16>{}); else by_mode(std::integral_constant<int, 32>{});
  SPR_LAUNCHED("svg_ear_compensation_kernel");
  return SPR_OK;
}

extern "C" size_t spr_svg_ear_scores_flops(int64_t q_heads, int32_t qn, int64_t tokens) {
  return static_cast<size_t>(2) * q_heads * qn * tokens * SE_D;
}

extern "C" int spr_svg_ear_scores(const float* q_centroids, const uint16_t* k_sorted, const uint16_t* v_sorted,
                                  const float* k_centroids, const float* v_centroids, const float* var_k_diag,
                                  float jensen_var_cap, const int32_t* k_sizes, int64_t q_heads, int32_t qn,
                                  int32_t kn, int64_t kv_heads, int64_t t_stored, int32_t d, int32_t group,
                                  int32_t mode, float* scores, hipStream_t stream) {
  SPR_REQUIRE(mode == 0 || mode == 1, "spr_svg_ear_scores: mode must be 0 (value error) or 1 (attention mass)");
  SPR_REQUIRE(d == SE_D, "spr_svg_ear_scores: head dim must be 128 (got %d)", d);
  SPR_REQUIRE(qn >= 1 && kn >= 1 && kv_heads >= 1 && group >= 1 && t_stored >= 1,
              "spr_svg_ear_scores: bad size");
  SPR_REQUIRE(q_heads == kv_heads * group, "spr_svg_ear_scores: q_heads %lld != kv_heads %lld * group %d",
              static_cast<long long>(q_heads), static_cast<long long>(kv_heads), group);
  SPR_REQUIRE(q_heads <= 65535 && kn <= (1 << 30) && qn <= (1 << 22), "spr_svg_ear_scores: grid too large");
  SPR_REQUIRE(t_stored < (int64_t(1) << 31) / (2 * SE_D) - SE_CHUNK,
              "spr_svg_ear_scores: at most %lld stored tokens per head",
              static_cast<long long>((int64_t(1) << 31) / (2 * SE_D) - SE_CHUNK - 1));
  SPR_REQUIRE(q_centroids && k_sorted && k_sizes && scores, "spr_svg_ear_scores: null pointer");
  if (mode == 0) {
    SPR_REQUIRE(v_sorted && k_centroids && v_centroids, "spr_svg_ear_scores: value error needs V and centroids");
    SPR_REQUIRE(!(jensen_var_cap > 0.0f) || var_k_diag != nullptr,
                "spr_svg_ear_scores: Jensen-aware routing requires var_k_diag");
  }
  const dim3 grid(static_cast<uint32_t>((kn + SE_CPW - 1) / SE_CPW), static_cast<uint32_t>(q_heads));
  if (mode == 0) {
    const bool jensen = jensen_var_cap > 0.0f;
    svg_ear_centroid_logit_kernel<<<dim3(static_cast<uint32_t>((kn + CL_CLUSTERS - 1) / CL_CLUSTERS),
                                         static_cast<uint32_t>((qn + CL_ROWS - 1) / CL_ROWS),
                                         static_cast<uint32_t>(q_heads)),
                                    SE_THREADS, 0, stream>>>(q_centroids, k_centroids, jensen ? var_k_diag : nullptr,
                                                             jensen ? jensen_var_cap : 0.0f, qn, kn, group, scores);
    SPR_LAUNCHED("svg_ear_centroid_logit_kernel");
    svg_ear_score_kernel<0><<<grid, SE_THREADS, 0, stream>>>(q_centroids, k_sorted, v_sorted, v_centroids, k_sizes,
                                                             qn, kn, t_stored, group, scores);
    SPR_LAUNCHED("svg_ear_score_kernel<value>");
  } else {
    svg_ear_score_kernel<1><<<grid, SE_THREADS, 0, stream>>>(q_centroids, k_sorted, nullptr, nullptr, k_sizes, qn,
                                                             kn, t_stored, group, scores);
    SPR_LAUNCHED("svg_ear_score_kernel<mass>");
  }
  return SPR_OK;
}
