// Shared helpers for the gfx950 MoE kernels: element conversions, launch checks and
// the status plumbing of the C-ABI.  Wave size is 64 on CDNA4 throughout.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "../../include/mintext_moe.h"

#define MTX_WAVE 64

namespace mtx {

// Last HIP error seen by an entry point (process-wide; diagnostics only).
extern int g_last_hip_error;

inline int check_launch() {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    g_last_hip_error = (int)e;
    return MTX_ERR_HIP;
  }
  return MTX_OK;
}

// Compute units of the current device (cached per device; 0 if the query fails).
inline int device_cu_count() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cache[dev] = n;
  }
  return cache[dev];
}

inline int dtype_size(int dt) {
  switch (dt) {
    case MTX_F32: return 4;
    case MTX_BF16: return 2;
    case MTX_FP8E4M3: return 1;
    default: return 0;
  }
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline int64_t round_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

// ---- scalar conversions (device) -------------------------------------------------------
// bf16 stored as uint16_t bit patterns; float -> bf16 is round-to-nearest-even with NaN kept.
__device__ __forceinline__ float bf16_to_f32(uint16_t v) {
  return __uint_as_float(((uint32_t)v) << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
}

// float -> OCP e4m3fn, round-to-nearest-even, saturating to +-448 (NaN stays NaN).
// Written from the format definition: 1 sign, 4 exponent (bias 7), 3 mantissa bits,
// no infinities, S.1111.111 is NaN; subnormals have exponent field 0 (scale 2^-6).
__device__ __forceinline__ uint8_t f32_to_e4m3(float f) {
  uint32_t u = __float_as_uint(f);
  uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint8_t)(sign | 0x7f);         // NaN
  if (a >= 0x43e00000u) return (uint8_t)(sign | 0x7e);        // >= 448 -> 448 (saturate)
  if (a < 0x3c800000u) {                                      // < 2^-6: subnormal range
    // value / 2^-9 rounded to nearest even integer m in [0, 8]; m == 8 is the min normal.
    float af = __uint_as_float(a);
    float q = af * 512.0f;                                    // exact (power-of-two scale)
    float r = __builtin_rintf(q);                             // RNE
    return (uint8_t)(sign | (uint8_t)r);
  }
  // normal: keep 3 mantissa bits with RNE on the dropped 20 bits
  uint32_t mant = a & 0x7fffffu;
  int32_t exp = (int32_t)(a >> 23) - 127 + 7;                 // e4m3 biased exponent (>= 1)
  uint32_t keep = mant >> 20;
  uint32_t rest = mant & 0xfffffu;
  uint32_t half = 0x80000u;
  if (rest > half || (rest == half && (keep & 1u))) {
    keep += 1;
    if (keep == 8) { keep = 0; exp += 1; }
  }
  if (exp > 15 || (exp == 15 && keep == 7)) return (uint8_t)(sign | 0x7e);  // saturate
  return (uint8_t)(sign | (uint8_t)(exp << 3) | (uint8_t)keep);
}

// Four values -> four e4m3fn codes (byte i = value i) with the same results as f32_to_e4m3:
// the value is clamped to +-448 and converted by v_cvt_pk_fp8_f32 (OCP e4m3, RNE on gfx950,
// checked against f32_to_e4m3 over every f32 with |x| in [2^-30, 2^10)); NaN keeps its sign.
__device__ __forceinline__ uint32_t e4m3_pack4(float a, float b, float c, float d) {
  auto cl = [](float x) { return fminf(fmaxf(x, -448.0f), 448.0f); };
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(cl(a), cl(b), 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(cl(c), cl(d), w, true);
  uint32_t q = (uint32_t)w;
  const float v[4] = {a, b, c, d};
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (__builtin_expect(v[i] != v[i], 0))
      q = (q & ~(0xffu << (8 * i))) | ((uint32_t)(f32_to_e4m3(v[i])) << (8 * i));
  return q;
}

__device__ __forceinline__ float e4m3_to_f32(uint8_t v) {
  uint32_t sign = (v & 0x80u) ? 0x80000000u : 0u;
  uint32_t e = (v >> 3) & 0xfu, m = v & 7u;
  if (e == 0xf && m == 7) return __uint_as_float(sign | 0x7fc00000u);
  if (e == 0) { float r = (float)m * 0.001953125f; return sign ? -r : r; }
  return __uint_as_float(sign | ((e - 7 + 127) << 23) | (m << 20));
}

// Load/store of one element of a runtime dtype as float.
__device__ __forceinline__ float load_as_f32(const void* p, int64_t i, int dt) {
  if (dt == MTX_F32) return ((const float*)p)[i];
  if (dt == MTX_BF16) return bf16_to_f32(((const uint16_t*)p)[i]);
  return e4m3_to_f32(((const uint8_t*)p)[i]);
}
__device__ __forceinline__ void store_from_f32(void* p, int64_t i, int dt, float v) {
  if (dt == MTX_F32) ((float*)p)[i] = v;
  else if (dt == MTX_BF16) ((uint16_t*)p)[i] = f32_to_bf16(v);
  else ((uint8_t*)p)[i] = f32_to_e4m3(v);
}

__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + expf(-g)); }

}  // namespace mtx
