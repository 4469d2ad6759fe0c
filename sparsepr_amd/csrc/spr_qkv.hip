// Model-edge fusions in front of the attention: Q/K RMSNorm, rotary embedding and the
// attention layout, one pass over the projected Q/K/V.
//
// Replaces:
//   wan_qkv_norm_rope_layout     (kernels/n8_ext/csrc/n8_ops.cu:16-105, host :356-413)
//     q, k, v [B, L, C = H D] -> [B, H, L, D]; RMSNorm over all C channels of a token with
//     model-dtype weights [C]; the normalised values are rounded to the model dtype, then
//     rotated in complex pairs (2i, 2i + 1) of each head by the fp32 table
//     (freq_real, freq_imag) [L, D / 2]; V is relaid out unchanged.
//   cosmos25_qkv_norm_rope_bshd  (n8_ops.cu:107-187, host :415-497)
//     q, k, v [B, S, C = H D] -> [B, S, H, D]; RMSNorm over each head's D values with fp32
//     weights [D]; rounded to the model dtype, then rotated in halves (d with d +- D / 2,
//     the first half negated) by fp32 angles [S, 1, 1, D] through sincosf; V copied.
//
// Arithmetic (fp32, contraction off, every fused multiply-add written out):
//   ss = sum of squares (per-thread fmaf chains, then a fixed reduction tree);
//   inv = 1 / sqrt(ss / n + eps) (correctly rounded division and square root);
//   r = round_T((x * inv) * w);
//   Wan:    out0 = round_T(fmaf(r0, fr, -(r1 * fi))), out1 = round_T(fmaf(r0, fi, r1 * fr));
//   Cosmos: out = round_T(fmaf(r, cos, (sign * r_pair) * sin)).
// The summation order differs from the reference's, so an output can differ from it by
// one unit in the last place of the model dtype where a value sits on a rounding boundary.
//
// Both are HBM-bound: 16-byte vectors of 8 channels, q and k kept in registers between
// the sum of squares and the write, one workgroup per token (Cosmos: every head of the
// token loaded before any arithmetic, its sines and cosines computed once into LDS).
#pragma clang fp contract(off)

#include "spr_common.h"

namespace {

constexpr int QKV_THREADS = 256;

template <int DT>
struct Elem;
template <>
struct Elem<0> {  // bf16
  using S = uint16_t;
  __device__ static float to_f(S s) { return spr::bf16_to_f32(s); }
  __device__ static S from_f(float f) { return spr::f32_to_bf16(f); }
};
template <>
struct Elem<1> {  // fp16
  using S = uint16_t;
  __device__ static float to_f(S s) { return static_cast<float>(__builtin_bit_cast(_Float16, s)); }
  __device__ static S from_f(float f) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f)); }
};
template <>
struct Elem<2> {  // fp32
  using S = float;
  __device__ static float to_f(S s) { return s; }
  __device__ static S from_f(float f) { return f; }
};

// 8 consecutive elements <-> float[8] (16 bytes for 16-bit types, 32 for fp32).
template <int DT>
__device__ __forceinline__ void load8(const typename Elem<DT>::S* p, float (&x)[8]) {
  if constexpr (DT == 2) {
    const spr::f32x4 a = reinterpret_cast<const spr::f32x4*>(p)[0];
    const spr::f32x4 b = reinterpret_cast<const spr::f32x4*>(p)[1];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = a[e];
      x[e + 4] = b[e];
    }
  } else {
    const spr::u32x4 r = *reinterpret_cast<const spr::u32x4*>(p);
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = Elem<DT>::to_f(static_cast<uint16_t>(w[e] & 0xFFFFu));
      x[2 * e + 1] = Elem<DT>::to_f(static_cast<uint16_t>(w[e] >> 16));
    }
  }
}
template <int DT>
__device__ __forceinline__ void store8(typename Elem<DT>::S* p, const float (&x)[8]) {
  if constexpr (DT == 2) {
    reinterpret_cast<spr::f32x4*>(p)[0] = spr::f32x4{x[0], x[1], x[2], x[3]};
    reinterpret_cast<spr::f32x4*>(p)[1] = spr::f32x4{x[4], x[5], x[6], x[7]};
  } else {
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      w[e] = static_cast<uint32_t>(Elem<DT>::from_f(x[2 * e])) |
             (static_cast<uint32_t>(Elem<DT>::from_f(x[2 * e + 1])) << 16);
    }
    *reinterpret_cast<spr::u32x4*>(p) = spr::u32x4{w[0], w[1], w[2], w[3]};
  }
}
template <int DT>
__device__ __forceinline__ void copy8(const typename Elem<DT>::S* src, typename Elem<DT>::S* dst) {
  if constexpr (DT == 2) {
    reinterpret_cast<spr::u32x4*>(dst)[0] = reinterpret_cast<const spr::u32x4*>(src)[0];
    reinterpret_cast<spr::u32x4*>(dst)[1] = reinterpret_cast<const spr::u32x4*>(src)[1];
  } else {
    *reinterpret_cast<spr::u32x4*>(dst) = *reinterpret_cast<const spr::u32x4*>(src);
  }
}
template <int DT>
__device__ __forceinline__ float round_t(float x) {
  return Elem<DT>::to_f(Elem<DT>::from_f(x));
}

__device__ __forceinline__ float inv_rms(float ss, float n, float eps) {
  return __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, n), eps)));
}

// Sum over the workgroup (4 waves), every thread gets the total; two values at once.
__device__ __forceinline__ void block_sum2(float& a, float& b, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    a += __shfl_xor(a, o, 64);
    b += __shfl_xor(b, o, 64);
  }
  const int wv = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    red[2 * wv] = a;
    red[2 * wv + 1] = b;
  }
  __syncthreads();
  a = (red[0] + red[2]) + (red[4] + red[6]);
  b = (red[1] + red[3]) + (red[5] + red[7]);
}

// ---- Wan: one workgroup per (b, t) token row; NV vectors of 8 channels per thread.
template <int DT, int NV>
__global__ __launch_bounds__(QKV_THREADS) void wan_qkv_kernel(
    const typename Elem<DT>::S* __restrict__ q, const typename Elem<DT>::S* __restrict__ k,
    const typename Elem<DT>::S* __restrict__ v, const typename Elem<DT>::S* __restrict__ qw,
    const typename Elem<DT>::S* __restrict__ kw, const float* __restrict__ freq_real,
    const float* __restrict__ freq_imag, int64_t tokens, int32_t channels, int32_t heads, int32_t head_dim,
    float eps, typename Elem<DT>::S* __restrict__ q_out, typename Elem<DT>::S* __restrict__ k_out,
    typename Elem<DT>::S* __restrict__ v_out) {
  using S = typename Elem<DT>::S;
  __shared__ float red[8];
  const int64_t row = blockIdx.x;
  const int64_t b = row / tokens;
  const int64_t t = row - b * tokens;
  const int nvec = channels >> 3;
  const S* qr = q + row * channels;
  const S* kr = k + row * channels;
  float qv[NV][8], kv[NV][8];
  float qss = 0.0f, kss = 0.0f;
#pragma unroll
  for (int u = 0; u < NV; ++u) {
    const int vi = threadIdx.x + u * QKV_THREADS;
    if (vi < nvec) {
      load8<DT>(qr + vi * 8, qv[u]);
      load8<DT>(kr + vi * 8, kv[u]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        qss = __builtin_fmaf(qv[u][e], qv[u][e], qss);
        kss = __builtin_fmaf(kv[u][e], kv[u][e], kss);
      }
    }
  }
  block_sum2(qss, kss, red);
  const float q_inv = inv_rms(qss, static_cast<float>(channels), eps);
  const float k_inv = inv_rms(kss, static_cast<float>(channels), eps);
  const int half = head_dim >> 1;
#pragma unroll
  for (int u = 0; u < NV; ++u) {
    const int vi = threadIdx.x + u * QKV_THREADS;
    if (vi >= nvec) continue;
    const int c0 = vi * 8;
    const int h = c0 / head_dim;
    const int d0 = c0 - h * head_dim;
    const int64_t o = ((b * heads + h) * tokens + t) * head_dim + d0;
    copy8<DT>(v + row * channels + c0, v_out + o);
    float wq[8], wk[8];
    load8<DT>(qw + c0, wq);
    load8<DT>(kw + c0, wk);
    const spr::f32x4 fr = *reinterpret_cast<const spr::f32x4*>(freq_real + t * half + d0 / 2);
    const spr::f32x4 fi = *reinterpret_cast<const spr::f32x4*>(freq_imag + t * half + d0 / 2);
    float qo[8], ko[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float q0 = round_t<DT>((qv[u][2 * e] * q_inv) * wq[2 * e]);
      const float q1 = round_t<DT>((qv[u][2 * e + 1] * q_inv) * wq[2 * e + 1]);
      const float k0 = round_t<DT>((kv[u][2 * e] * k_inv) * wk[2 * e]);
      const float k1 = round_t<DT>((kv[u][2 * e + 1] * k_inv) * wk[2 * e + 1]);
      qo[2 * e] = __builtin_fmaf(q0, fr[e], -(q1 * fi[e]));
      qo[2 * e + 1] = __builtin_fmaf(q0, fi[e], q1 * fr[e]);
      ko[2 * e] = __builtin_fmaf(k0, fr[e], -(k1 * fi[e]));
      ko[2 * e + 1] = __builtin_fmaf(k0, fi[e], k1 * fr[e]);
    }
    store8<DT>(q_out + o, qo);
    store8<DT>(k_out + o, ko);
  }
}

// Wan for head dims that are not a multiple of 8: one workgroup per token, pairs.
template <int DT>
__global__ __launch_bounds__(QKV_THREADS) void wan_qkv_pairs_kernel(
    const typename Elem<DT>::S* __restrict__ q, const typename Elem<DT>::S* __restrict__ k,
    const typename Elem<DT>::S* __restrict__ v, const typename Elem<DT>::S* __restrict__ qw,
    const typename Elem<DT>::S* __restrict__ kw, const float* __restrict__ freq_real,
    const float* __restrict__ freq_imag, int64_t tokens, int32_t channels, int32_t heads, int32_t head_dim,
    float eps, typename Elem<DT>::S* __restrict__ q_out, typename Elem<DT>::S* __restrict__ k_out,
    typename Elem<DT>::S* __restrict__ v_out) {
  using E = Elem<DT>;
  __shared__ float red[8];
  const int64_t row = blockIdx.x;
  const int64_t b = row / tokens;
  const int64_t t = row - b * tokens;
  const int64_t base = row * channels;
  float qss = 0.0f, kss = 0.0f;
  for (int c = threadIdx.x; c < channels; c += QKV_THREADS) {
    const float a = E::to_f(q[base + c]), bb = E::to_f(k[base + c]);
    qss = __builtin_fmaf(a, a, qss);
    kss = __builtin_fmaf(bb, bb, kss);
  }
  block_sum2(qss, kss, red);
  const float q_inv = inv_rms(qss, static_cast<float>(channels), eps);
  const float k_inv = inv_rms(kss, static_cast<float>(channels), eps);
  const int half = head_dim >> 1;
  for (int c = threadIdx.x; c < channels; c += QKV_THREADS) {
    const int h = c / head_dim;
    v_out[((b * heads + h) * tokens + t) * head_dim + (c - h * head_dim)] = v[base + c];
  }
  for (int pr = threadIdx.x; pr < channels / 2; pr += QKV_THREADS) {
    const int h = pr / half;
    const int ph = pr - h * half;
    const int c0 = h * head_dim + 2 * ph;
    const float fr = freq_real[t * half + ph], fi = freq_imag[t * half + ph];
    const float q0 = round_t<DT>((E::to_f(q[base + c0]) * q_inv) * E::to_f(qw[c0]));
    const float q1 = round_t<DT>((E::to_f(q[base + c0 + 1]) * q_inv) * E::to_f(qw[c0 + 1]));
    const float k0 = round_t<DT>((E::to_f(k[base + c0]) * k_inv) * E::to_f(kw[c0]));
    const float k1 = round_t<DT>((E::to_f(k[base + c0 + 1]) * k_inv) * E::to_f(kw[c0 + 1]));
    const int64_t o = ((b * heads + h) * tokens + t) * head_dim + 2 * ph;
    q_out[o] = E::from_f(__builtin_fmaf(q0, fr, -(q1 * fi)));
    q_out[o + 1] = E::from_f(__builtin_fmaf(q0, fi, q1 * fr));
    k_out[o] = E::from_f(__builtin_fmaf(k0, fr, -(k1 * fi)));
    k_out[o + 1] = E::from_f(__builtin_fmaf(k0, fi, k1 * fr));
  }
}

// ---- Cosmos2.5: one workgroup of 256 threads per (b, s) token; a head's D values on
// LPH = D / 8 lanes (8 consecutive dims each), 64 / LPH heads per wave, HPB heads per pass
// over the workgroup and up to NI passes per lane, all loaded into registers before any
// arithmetic so that the token's loads are in flight together.  The lane holding dims
// d .. d + 7 of the first half pairs with lane ^ (LPH / 2) holding d + D / 2 ...  The
// token's D sines and cosines are computed once (one angle per thread) into LDS while the
// loads are outstanding, and serve every head.
template <int DT, int D, int NI>
__global__ __launch_bounds__(QKV_THREADS) void cosmos_qkv_kernel(
    const typename Elem<DT>::S* __restrict__ q, const typename Elem<DT>::S* __restrict__ k,
    const typename Elem<DT>::S* __restrict__ v, const float* __restrict__ qw, const float* __restrict__ kw,
    const float* __restrict__ angles, int64_t tokens, int32_t heads, float eps,
    typename Elem<DT>::S* __restrict__ q_out, typename Elem<DT>::S* __restrict__ k_out,
    typename Elem<DT>::S* __restrict__ v_out) {
  constexpr int LPH = D / 8;
  constexpr int HPW = 64 / LPH;
  constexpr int HPB = HPW * (QKV_THREADS / 64);
  static_assert(LPH >= 2 && LPH <= 64 && (LPH & (LPH - 1)) == 0, "D / 8 must be a power of two");
  __shared__ float cs_s[D], sn_s[D];
  const int64_t row = blockIdx.x;  // b * tokens + s
  const int64_t s = row % tokens;
  const int lane = threadIdx.x & 63;
  const int h0 = (threadIdx.x >> 6) * HPW + lane / LPH;
  const int d0 = (lane % LPH) * 8;
  const float sign = d0 < D / 2 ? -1.0f : 1.0f;
  for (int hb = 0; hb < heads; hb += NI * HPB) {
    float x[NI][8], y[NI][8];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int h = hb + h0 + i * HPB;
      if (h < heads) {
        const int64_t base = (row * heads + h) * D + d0;
        load8<DT>(q + base, x[i]);
        load8<DT>(k + base, y[i]);
        copy8<DT>(v + base, v_out + base);
      }
    }
    if (hb == 0) {
      for (int e = threadIdx.x; e < D; e += QKV_THREADS) sincosf(angles[s * D + e], &sn_s[e], &cs_s[e]);
      __syncthreads();
    }
    float cs[8], sn[8], wq[8], wk[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      cs[e] = cs_s[d0 + e];
      sn[e] = sn_s[d0 + e];
      wq[e] = qw[d0 + e];
      wk[e] = kw[d0 + e];
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int h = hb + h0 + i * HPB;
      if (h >= heads) continue;  // a head's lane group is all in or all out
      float qss = 0.0f, kss = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        qss = __builtin_fmaf(x[i][e], x[i][e], qss);
        kss = __builtin_fmaf(y[i][e], y[i][e], kss);
      }
#pragma unroll
      for (int o = 1; o < LPH; o <<= 1) {  // within the head's lane group
        qss += __shfl_xor(qss, o, 64);
        kss += __shfl_xor(kss, o, 64);
      }
      const float q_inv = inv_rms(qss, static_cast<float>(D), eps);
      const float k_inv = inv_rms(kss, static_cast<float>(D), eps);
      float qo[8], ko[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float xr = round_t<DT>((x[i][e] * q_inv) * wq[e]);
        const float yr = round_t<DT>((y[i][e] * k_inv) * wk[e]);
        const float xp = __shfl_xor(xr, LPH / 2, 64);
        const float yp = __shfl_xor(yr, LPH / 2, 64);
        qo[e] = __builtin_fmaf(xr, cs[e], (sign * xp) * sn[e]);
        ko[e] = __builtin_fmaf(yr, cs[e], (sign * yp) * sn[e]);
      }
      const int64_t base = (row * heads + h) * D + d0;
      store8<DT>(q_out + base, qo);
      store8<DT>(k_out + base, ko);
    }
  }
}

// Cosmos2.5 for other even head dims: one wave per (b, s, h) row, lanes over the dims.
template <int DT>
__global__ __launch_bounds__(QKV_THREADS) void cosmos_qkv_rows_kernel(
    const typename Elem<DT>::S* __restrict__ q, const typename Elem<DT>::S* __restrict__ k,
    const typename Elem<DT>::S* __restrict__ v, const float* __restrict__ qw, const float* __restrict__ kw,
    const float* __restrict__ angles, int64_t rows, int64_t tokens, int32_t heads, int32_t head_dim, float eps,
    typename Elem<DT>::S* __restrict__ q_out, typename Elem<DT>::S* __restrict__ k_out,
    typename Elem<DT>::S* __restrict__ v_out) {
  using E = Elem<DT>;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * (QKV_THREADS / 64) + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int lane = threadIdx.x & 63;
  const int64_t s = (r / heads) % tokens;
  const int64_t base = r * head_dim;
  float qss = 0.0f, kss = 0.0f;
  for (int d = lane; d < head_dim; d += 64) {
    const float a = E::to_f(q[base + d]), b = E::to_f(k[base + d]);
    qss = __builtin_fmaf(a, a, qss);
    kss = __builtin_fmaf(b, b, kss);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    qss += __shfl_xor(qss, o, 64);
    kss += __shfl_xor(kss, o, 64);
  }
  const float q_inv = inv_rms(qss, static_cast<float>(head_dim), eps);
  const float k_inv = inv_rms(kss, static_cast<float>(head_dim), eps);
  const int half = head_dim >> 1;
  for (int d = lane; d < head_dim; d += 64) {
    const int pd = d < half ? d + half : d - half;
    const float sign = d < half ? -1.0f : 1.0f;
    const float x = round_t<DT>((E::to_f(q[base + d]) * q_inv) * qw[d]);
    const float xp = round_t<DT>((E::to_f(q[base + pd]) * q_inv) * qw[pd]);
    const float y = round_t<DT>((E::to_f(k[base + d]) * k_inv) * kw[d]);
    const float yp = round_t<DT>((E::to_f(k[base + pd]) * k_inv) * kw[pd]);
    float sn, cs;
    sincosf(angles[s * head_dim + d], &sn, &cs);
    q_out[base + d] = E::from_f(__builtin_fmaf(x, cs, (sign * xp) * sn));
    k_out[base + d] = E::from_f(__builtin_fmaf(y, cs, (sign * yp) * sn));
    v_out[base + d] = v[base + d];
  }
}

template <int DT>
int launch_wan(const void* q, const void* k, const void* v, const void* qw, const void* kw, const float* fr,
               const float* fi, int64_t batch, int64_t tokens, int32_t channels, int32_t heads, float eps, void* qo,
               void* ko, void* vo, hipStream_t stream) {
  using S = typename Elem<DT>::S;
  const int32_t head_dim = channels / heads;
  const uint32_t rows = static_cast<uint32_t>(batch * tokens);
  const int nvec = channels / 8;
#define SPR_WAN(NV)                                                                                              \
  wan_qkv_kernel<DT, NV><<<rows, QKV_THREADS, 0, stream>>>(                                                      \
      static_cast<const S*>(q), static_cast<const S*>(k), static_cast<const S*>(v), static_cast<const S*>(qw), \
      static_cast<const S*>(kw), fr, fi, tokens, channels, heads, head_dim, eps, static_cast<S*>(qo),          \
      static_cast<S*>(ko), static_cast<S*>(vo))
  if (head_dim % 8 == 0 && nvec <= 4 * QKV_THREADS) {
    if (nvec <= QKV_THREADS) SPR_WAN(1);
    else if (nvec <= 2 * QKV_THREADS) SPR_WAN(2);
    else SPR_WAN(4);
  } else {
    wan_qkv_pairs_kernel<DT><<<rows, QKV_THREADS, 0, stream>>>(
        static_cast<const S*>(q), static_cast<const S*>(k), static_cast<const S*>(v), static_cast<const S*>(qw),
        static_cast<const S*>(kw), fr, fi, tokens, channels, heads, head_dim, eps, static_cast<S*>(qo),
        static_cast<S*>(ko), static_cast<S*>(vo));
  }
#undef SPR_WAN
  SPR_LAUNCHED("wan_qkv_kernel");
  return SPR_OK;
}

template <int DT>
int launch_cosmos(const void* q, const void* k, const void* v, const float* qw, const float* kw, const float* ang,
                  int64_t batch, int64_t tokens, int32_t heads, int32_t head_dim, float eps, void* qo, void* ko,
                  void* vo, hipStream_t stream) {
  using S = typename Elem<DT>::S;
  const uint32_t token_rows = static_cast<uint32_t>(batch * tokens);
  // passes per lane: heads / (heads per pass = 4 waves x 512 / D heads), at most 4 kept in
  // registers at once (more heads take further rounds of the same loop)
  const int hpb = 4 * (512 / head_dim);
  const int passes = static_cast<int>(spr::ceil_div(heads, hpb));
#define SPR_COSMOS(DD)                                                                                          \
  do {                                                                                                          \
    if (passes <= 1) SPR_COSMOS_NI(DD, 1);                                                                      \
    else if (passes == 2) SPR_COSMOS_NI(DD, 2);                                                                 \
    else if (passes == 3) SPR_COSMOS_NI(DD, 3);                                                                 \
    else SPR_COSMOS_NI(DD, 4);                                                                                  \
  } while (0)
#define SPR_COSMOS_NI(DD, NI)                                                                                   \
  cosmos_qkv_kernel<DT, DD, NI><<<token_rows, QKV_THREADS, 0, stream>>>(                                        \
      static_cast<const S*>(q), static_cast<const S*>(k), static_cast<const S*>(v), qw, kw, ang, tokens, heads, \
      eps, static_cast<S*>(qo), static_cast<S*>(ko), static_cast<S*>(vo))
  if (head_dim == 64) {
    SPR_COSMOS(64);
  } else if (head_dim == 128) {
    SPR_COSMOS(128);
  } else if (head_dim == 256) {
    SPR_COSMOS(256);
  } else {
    const int64_t rows = batch * tokens * heads;
    const uint32_t blocks = static_cast<uint32_t>(spr::ceil_div(rows, QKV_THREADS / 64));
    cosmos_qkv_rows_kernel<DT><<<blocks, QKV_THREADS, 0, stream>>>(
        static_cast<const S*>(q), static_cast<const S*>(k), static_cast<const S*>(v), qw, kw, ang, rows, tokens,
        heads, head_dim, eps, static_cast<S*>(qo), static_cast<S*>(ko), static_cast<S*>(vo));
  }
#undef SPR_COSMOS_NI
#undef SPR_COSMOS
  SPR_LAUNCHED("cosmos_qkv_kernel");
  return SPR_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

// q, k, v [batch, tokens, channels] of dtype (0 bf16, 1 fp16, 2 fp32), weights [channels]
// of the same dtype, freq_real / freq_imag fp32 [tokens, head_dim / 2]; outputs
// [batch, heads, tokens, head_dim].  All device pointers, contiguous, 16-byte aligned.
extern "C" int spr_wan_qkv_norm_rope_layout(const void* q, const void* k, const void* v, const void* q_weight,
                                            const void* k_weight, const float* freq_real, const float* freq_imag,
                                            int32_t dtype, int64_t batch, int64_t tokens, int32_t channels,
                                            int32_t heads, float epsilon, void* q_out, void* k_out, void* v_out,
                                            hipStream_t stream) {
  SPR_REQUIRE(batch >= 0 && tokens >= 0 && channels >= 1, "spr_wan_qkv_norm_rope_layout: bad size");
  SPR_REQUIRE(heads > 0 && channels % heads == 0, "Wan channels must divide num_heads");
  SPR_REQUIRE((channels / heads) % 2 == 0, "Wan head_dim must be even");
  SPR_REQUIRE(dtype >= 0 && dtype <= 2, "spr_wan_qkv_norm_rope_layout: dtype %d not in {0, 1, 2}", dtype);
  SPR_REQUIRE(batch * tokens < (int64_t(1) << 31), "spr_wan_qkv_norm_rope_layout: too many rows");
  if (batch == 0 || tokens == 0) return SPR_OK;
  SPR_REQUIRE(q && k && v && q_weight && k_weight && freq_real && freq_imag && q_out && k_out && v_out,
              "spr_wan_qkv_norm_rope_layout: null pointer");
  SPR_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(q_weight) && aligned16(k_weight) &&
                  aligned16(freq_real) && aligned16(freq_imag) && aligned16(q_out) && aligned16(k_out) &&
                  aligned16(v_out),
              "spr_wan_qkv_norm_rope_layout: pointers must be 16-byte aligned");
  switch (dtype) {
    case 0: return launch_wan<0>(q, k, v, q_weight, k_weight, freq_real, freq_imag, batch, tokens, channels, heads,
                                 epsilon, q_out, k_out, v_out, stream);
    case 1: return launch_wan<1>(q, k, v, q_weight, k_weight, freq_real, freq_imag, batch, tokens, channels, heads,
                                 epsilon, q_out, k_out, v_out, stream);
    default: return launch_wan<2>(q, k, v, q_weight, k_weight, freq_real, freq_imag, batch, tokens, channels, heads,
                                  epsilon, q_out, k_out, v_out, stream);
  }
}

// q, k, v [batch, tokens, heads * head_dim] of dtype, weights fp32 [head_dim], angles fp32
// [tokens, head_dim]; outputs [batch, tokens, heads, head_dim] (the input layout).
extern "C" int spr_cosmos25_qkv_norm_rope_bshd(const void* q, const void* k, const void* v, const float* q_weight,
                                               const float* k_weight, const float* rope_angles, int32_t dtype,
                                               int64_t batch, int64_t tokens, int32_t heads, int32_t head_dim,
                                               float epsilon, void* q_out, void* k_out, void* v_out,
                                               hipStream_t stream) {
  SPR_REQUIRE(batch >= 0 && tokens >= 0 && heads > 0, "Cosmos2.5 channels must divide num_heads");
  SPR_REQUIRE(head_dim > 0 && head_dim % 2 == 0, "Cosmos2.5 head_dim must be positive and even");
  SPR_REQUIRE(epsilon > 0.0f, "Cosmos2.5 RMSNorm epsilon must be positive");
  SPR_REQUIRE(dtype >= 0 && dtype <= 2, "spr_cosmos25_qkv_norm_rope_bshd: dtype %d not in {0, 1, 2}", dtype);
  SPR_REQUIRE(batch * tokens < (int64_t(1) << 31) && batch * tokens * heads < (int64_t(1) << 37),
              "spr_cosmos25_qkv_norm_rope_bshd: too many rows");
  if (batch == 0 || tokens == 0) return SPR_OK;
  SPR_REQUIRE(q && k && v && q_weight && k_weight && rope_angles && q_out && k_out && v_out,
              "spr_cosmos25_qkv_norm_rope_bshd: null pointer");
  SPR_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(q_out) && aligned16(k_out) &&
                  aligned16(v_out),
              "spr_cosmos25_qkv_norm_rope_bshd: tensors must be 16-byte aligned");
  switch (dtype) {
    case 0: return launch_cosmos<0>(q, k, v, q_weight, k_weight, rope_angles, batch, tokens, heads, head_dim,
                                    epsilon, q_out, k_out, v_out, stream);
    case 1: return launch_cosmos<1>(q, k, v, q_weight, k_weight, rope_angles, batch, tokens, heads, head_dim,
                                    epsilon, q_out, k_out, v_out, stream);
    default: return launch_cosmos<2>(q, k, v, q_weight, k_weight, rope_angles, batch, tokens, heads, head_dim,
                                     epsilon, q_out, k_out, v_out, stream);
  }
}
