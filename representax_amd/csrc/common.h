// Shared device helpers for the representax quantized-linear kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

namespace rpx {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// bf16 <-> f32. Conversion to bf16 is round-to-nearest-even
// (v_cvt_pk_bf16_f32 on gfx950).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __builtin_bit_cast(float, static_cast<uint32_t>(b) << 16);
}
__device__ __forceinline__ float bf16lo_to_f32(uint32_t w) {
  return __builtin_bit_cast(float, w << 16);
}
__device__ __forceinline__ float bf16hi_to_f32(uint32_t w) {
  return __builtin_bit_cast(float, w & 0xFFFF0000u);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  f32x2_t v = {lo, hi};
  bf16x2_t r = __builtin_convertvector(v, bf16x2_t);
  return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return static_cast<uint16_t>(pack_bf16x2(f, 0.0f) & 0xFFFFu);
}
// Round a float to the nearest bf16 value, returned as float.
__device__ __forceinline__ float round_bf16(float f) {
  return __builtin_bit_cast(float, pack_bf16x2(f, 0.0f) << 16);
}

// ---------------------------------------------------------------------------
// OCP fp8 encode: float32 -> code, round to nearest even, non-saturating
// (e4m3fn: overflow/inf -> NaN 0x7F; e5m2: overflow/inf -> inf 0x7C).
// Integer-only so that it is identical on every device and on the host.
// ---------------------------------------------------------------------------
template <int EB, int MB, int BIAS, bool HAS_INF>
__host__ __device__ __forceinline__ uint32_t f32_to_fp8_code(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7FFFFFFFu;
  const uint32_t nan_code = HAS_INF ? 0x7Fu : 0x7Fu;
  const uint32_t inf_code = HAS_INF ? (((1u << EB) - 1u) << MB) : 0x7Fu;
  const uint32_t max_code = HAS_INF ? inf_code - 1u : 0x7Eu;
  if (a > 0x7F800000u) return sign | nan_code;
  if (a == 0x7F800000u) return sign | inf_code;
  const int emin = 1 - BIAS;
  int e_eff = (a >= 0x00800000u) ? static_cast<int>(a >> 23) - 127 : -126;
  uint32_t sig = (a & 0x007FFFFFu) | ((a >= 0x00800000u) ? 0x00800000u : 0u);
  int e_t = e_eff > emin ? e_eff : emin;
  int shift = (23 - MB) + (e_t - e_eff);
  if (shift > 31) shift = 31;
  uint32_t units = sig >> shift;
  uint32_t rem = sig & ((1u << shift) - 1u);
  uint32_t half = 1u << (shift - 1);
  if (rem > half || (rem == half && (units & 1u))) units += 1u;
  if (units == 0u) return sign;
  int code = ((e_t + BIAS - 1) << MB) + static_cast<int>(units);
  if (code > static_cast<int>(max_code)) return sign | (HAS_INF ? inf_code : nan_code);
  return sign | static_cast<uint32_t>(code);
}
__host__ __device__ __forceinline__ uint32_t f32_to_e4m3fn(float f) {
  return f32_to_fp8_code<4, 3, 7, false>(f);
}
__host__ __device__ __forceinline__ uint32_t f32_to_e5m2(float f) {
  return f32_to_fp8_code<5, 2, 15, true>(f);
}

// Correctly rounded f32 quotient x / s given r = RN(1 / s): one Newton
// correction of q = x * r (Markstein's theorem), exact whenever no
// intermediate overflows or underflows. Scales outside [1e-30, 1e30] (where r
// could leave the normal range), |x| < 1e-28 (where the residual could),
// non-finite results and tiny results take the IEEE divide instead.
__host__ __device__ __forceinline__ float div_rn(float x, float s, float r) {
  if (!(s >= 1.0e-30f && s <= 1.0e30f) || __builtin_fabsf(x) < 1.0e-28f) return x / s;
  float q = x * r;
  const float e = __builtin_fmaf(-q, s, x);
  q = __builtin_fmaf(e, r, q);
  const float aq = __builtin_fabsf(q);
  if (!(aq <= 1.0e30f) || aq < 1.0e-30f) q = x / s;
  return q;
}

enum Fp8Format : int { kE4M3FN = 0, kE5M2 = 1 };
enum DType : int { kF32 = 0, kBF16 = 1 };

__host__ __device__ __forceinline__ float fp8_max(int fmt) {
  return fmt == kE4M3FN ? 448.0f : 57344.0f;
}

// ---------------------------------------------------------------------------
// Host-side error state (thread local), read back through rpx_last_error().
// ---------------------------------------------------------------------------
void set_error(const std::string& msg);
int fail_invalid(const std::string& msg);
int check_hip(hipError_t err, const char* what);

constexpr int kOk = 0;
constexpr int kErrInvalid = 1;
constexpr int kErrHip = 2;
constexpr int kErrDevice = 3;

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace rpx
