// Shared helpers for the SparsePR HIP kernels (gfx950 / CDNA4 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

// Status codes returned by every extern "C" entry point.
enum {
  SPR_OK = 0,
  SPR_EINVAL = 1,      // bad argument (shape, size, null pointer, unsupported config)
  SPR_ELAUNCH = 2,     // HIP launch / runtime error
  SPR_EWORKSPACE = 3,  // workspace too small
};

void spr_set_error(const char* fmt, ...);

#define SPR_REQUIRE(cond, ...)         \
  do {                                 \
    if (!(cond)) {                     \
      spr_set_error(__VA_ARGS__);      \
      return SPR_EINVAL;               \
    }                                  \
  } while (0)

#define SPR_LAUNCHED(name)                                                   \
  do {                                                                       \
    hipError_t e_ = hipGetLastError();                                       \
    if (e_ != hipSuccess) {                                                  \
      spr_set_error("%s: launch failed: %s", name, hipGetErrorString(e_));   \
      return SPR_ELAUNCH;                                                    \
    }                                                                        \
  } while (0)

namespace spr {

// ---------------------------------------------------------------- vector types
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;

struct alignas(16) u32x4 {
  uint32_t x, y, z, w;
};

// ---------------------------------------------------------------- bf16 <-> f32
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// fp32 -> bf16, round to nearest even, in one instruction (v_cvt_pk_bf16_f32 under
// the default rounding mode; denormals preserved; a NaN stays a NaN).
typedef __bf16 bf16x2_hw __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2_rne(float lo, float hi) {
  const bf16x2_hw v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) { return pack_bf16x2_rne(lo, hi); }

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// ---------------------------------------------------------------- fp16 <-> f32
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// ---------------------------------------------------------------- exp
// e^x in fp32 with a fixed evaluation order, used where results must be
// reproducible bit for bit on the CPU (top-p block selection).  Cody-Waite
// range reduction with a two-part ln2, degree-7 Taylor polynomial (Horner,
// fused multiply-adds), exact scaling by 2^n applied as 2^(n - n/2) * 2^(n/2) so
// that n = 128 (x up to ln(FLT_MAX) ~ 88.72) stays finite.  x < -87 -> 0 (every
// nonzero result is normal, so the scaling never rounds); x > 89 -> inf, and
// x in (ln(FLT_MAX), 89] overflows to inf in the scaling.
__device__ __forceinline__ float canonical_expf(float x) {
  if (x != x) return x;
  if (x < -87.0f) return 0.0f;
  if (x > 89.0f) return __builtin_huge_valf();
  const float log2e = 1.44269504088896341f;
  const float ln2_hi = 0.693145751953125f;
  const float ln2_lo = 1.428606765330187045e-06f;
  float n = __builtin_rintf(x * log2e);
  float r = __builtin_fmaf(-n, ln2_hi, x);
  r = __builtin_fmaf(-n, ln2_lo, r);
  float p = 1.98412698412698413e-04f;
  p = __builtin_fmaf(p, r, 1.38888888888888889e-03f);
  p = __builtin_fmaf(p, r, 8.33333333333333333e-03f);
  p = __builtin_fmaf(p, r, 4.16666666666666667e-02f);
  p = __builtin_fmaf(p, r, 1.66666666666666667e-01f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const int ni = static_cast<int>(n);
  const int nb = ni >> 1, na = ni - nb;  // both in [-63, 64]
  const float sa = __uint_as_float(static_cast<uint32_t>(na + 127) << 23);
  const float sb = __uint_as_float(static_cast<uint32_t>(nb + 127) << 23);
  return (p * sa) * sb;  // exact power-of-two scaling
}

// ---------------------------------------------------------------- misc
__host__ __device__ __forceinline__ int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace spr
